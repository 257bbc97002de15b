"""Pins the oracle (CPU restatement of Reels.jl's int8 LoRA linear) before the GPU results are
compared with it: known-answer vectors, a second independent restatement, closed forms and invariants
chosen so that a dropped term, wrong sign, wrong index or transposed operand fails a test.
CPU only."""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "wan21_block_tiny_int8.npz")
F32 = np.float32


def bf(vals):
    return oracle.f32_to_bf16(np.asarray(vals, F32))


# ---- Philox4x32-10: Random123 known-answer vectors ---------------------------------------------
@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, want):
    assert [int(v) for v in oracle.philox(ctr, key)] == want


def test_normal_generator_moments_and_outliers():
    z = oracle.bf16_to_f32(oracle.normal_bf16(7, (1 << 20,), 1.0)).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    w = oracle.bf16_to_f32(oracle.normal_bf16(8, (1 << 20,), 0.02, outlier_rate=1e-3))
    frac = np.mean(np.abs(w) == oracle.bf16_to_f32(bf([0.4]))[0])
    assert 0.0007 < frac < 0.0013  # 0.1% outliers at exactly +-20 sigma
    assert np.array_equal(oracle.normal_bf16(7, (1000,), 1.0), oracle.normal_bf16(7, (1000,), 1.0))


# ---- bf16 conversions (src/models/interface.jl:13-25) ----------------------------------------
def test_bf16_exhaustive_round_trip():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(h)
    assert np.array_equal(oracle.f32_to_bf16(f), h)
    assert np.array_equal(oracle.c_f32_to_bf16(f), h)


def test_bf16_rounding_matches_rne_and_torch():
    import torch
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 1 << 32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    f = bits.view(F32)
    f = f[np.isfinite(f)]
    ours = oracle.f32_to_bf16(f)
    assert np.array_equal(ours, oracle.c_f32_to_bf16(f))
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    # ties to even on exact halfway points
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000], np.uint32).view(F32)
    assert list(oracle.f32_to_bf16(ties)) == [0x3F80, 0x3F82, 0xBF80, 0xBF82]


# ---- pack: quantize_frozen_matrix (src/layers/quantization.jl:35-44) -------------------------
def _pack_both(w32):
    q1, s1, st1 = oracle.pack(w32, "f32")
    q2, s2, st2 = oracle.numpy_pack(w32)
    assert st1 == st2
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    return q1, s1, st1


def test_pack_two_restatements_agree_bitwise():
    w = oracle.normal_bf16(11, (1024, 5120), 0.02, outlier_rate=1e-3)
    w32 = oracle.bf16_to_f32(w)
    q, s, st = _pack_both(w32)
    qb, sb, stb = oracle.pack(w, "bf16")  # bf16 input path = f32 of the same values
    assert st == 0 and np.array_equal(q, qb) and np.array_equal(s, sb)
    f = oracle.normal_f32(12, (512, 1536), 1.0)
    _pack_both(f)
    # f16 input path = f32 of the same values
    h16 = f.astype(np.float16)
    q16, s16, _ = oracle.pack(h16.view(np.uint16), "f16")
    q32, s32, _ = oracle.pack(h16.astype(F32), "f32")
    assert np.array_equal(q16, q32) and np.array_equal(s16, s32)


def test_pack_closed_forms():
    rows = np.zeros((8, 10), F32)
    # absmax 127 -> scale exactly 1: codes are rint(w), ties to even
    rows[0] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.0, 126.5, -126.5]
    # absmax 254 -> scale exactly 2
    rows[1, :6] = [254, 5, 7, -5, 1, 3]
    # zero row -> scale 1, codes 0 (quantization.jl:40)
    # single spike
    rows[3, 4] = 0.3
    # constant row
    rows[4] = -0.7
    # negative absmax
    rows[5, :2] = [-3, 1]
    # 20-sigma outlier among small values
    rows[6] = [0.01, -0.02, 0.4, 0.0, 0.015, -0.005, 0.02, 0.0, -0.01, 0.003]
    rows[7] = np.float32(1e-30)  # tiny but normal
    q, s, st = _pack_both(rows)
    assert st == 0
    assert list(q[0]) == [127, 2, 4, -2, -4, 0, 2, 0, 126, -126] and s[0] == 1.0
    assert list(q[1, :6]) == [127, 2, 4, -2, 0, 2] and s[1] == 2.0
    assert s[2] == 1.0 and not q[2].any()
    assert s[3] == F32(0.3) / F32(127) and list(q[3]) == [0, 0, 0, 0, 127, 0, 0, 0, 0, 0]
    assert np.all(q[4] == -127)
    assert q[5, 0] == -127 and q[5, 1] == 42  # 127/3 = 42.33
    assert q[6, 2] == 127 and s[6] == F32(0.4) / F32(127)
    assert np.all(q[7] == 127)


def test_pack_denormals_are_not_flushed():
    ulp = np.array([1], np.uint32).view(F32)[0]  # smallest denormal
    w = np.array([[127 * ulp, 64 * ulp, 0, -127 * ulp],    # scale = 1 ulp exactly
                  [10 * ulp, 5 * ulp, 10 * ulp, 5 * ulp]],  # scale rounds to 0 -> +-Inf -> 127
                 F32)
    q, s, st = _pack_both(w)
    assert st == 0
    assert s[0] == ulp and list(q[0]) == [127, 64, 0, -127]
    assert s[1] == 0.0 and list(q[1]) == [127, 127, 127, 127]
    # scale 0 with a zero weight gives 0/0 = NaN -> Int8(NaN) throws
    _, _, st = _pack_both(np.array([[10 * ulp, 0.0]], F32))
    assert st == 1


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_pack_nonfinite_is_an_error(bad):
    w = np.ones((3, 6), F32)
    w[1, 2] = bad
    q, s, st = _pack_both(w)
    assert st == 1
    assert np.all(q[0] == 127) and np.all(q[2] == 127)  # other rows unaffected


def test_pack_invariants():
    w = oracle.bf16_to_f32(oracle.normal_bf16(13, (777, 333), 0.02, outlier_rate=5e-3))
    q, s, st = _pack_both(w)
    assert st == 0
    assert q.min() >= -127 and q.max() <= 127           # never -128
    assert np.all((np.sign(q) == np.sign(w)) | (q == 0))
    assert np.all(np.abs(q).max(axis=1) == 127)          # every non-zero row reaches 127
    # |w - q s| <= s/2 up to the f32 rounding of w/s (at most half an ulp of a value < 128)
    err = np.abs(w.astype(np.float64) - q * s[:, None].astype(np.float64))
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 2.0 ** -17))


@pytest.mark.parametrize("shape,seed", [((7, 5), 950), ((512, 1536), 951)])
def test_pack_reconstruction_tolerance_of_reference(shape, seed):
    # test/unit/quantization.jl:3-8: randn weights, Array(quantized) ≈ weight rtol=1e-2
    # atol=1e-2 (Julia isapprox: norm(a - b) <= max(atol, rtol * max(norm(a), norm(b))))
    w = oracle.normal_f32(seed, shape, 1.0)
    q, s, st = _pack_both(w)
    deq = oracle.dequant(q, s, "f32")
    assert np.linalg.norm(deq - w) <= max(1e-2, 1e-2 * max(np.linalg.norm(deq), np.linalg.norm(w)))


def test_pack_golden_real_wan_weights():
    g = np.load(GOLDEN)
    names = sorted({k[:-2] for k in g.files if k.endswith("_q")})
    assert len(names) == 10
    for n in names:
        q, s, st = _pack_both(g[n + "_w"])
        assert st == 0
        assert np.array_equal(q, g[n + "_q"]), n
        assert np.array_equal(s.view(np.uint32), g[n + "_s"].view(np.uint32)), n


# ---- dequantization (quantization.jl:25-29, 61-64) --------------------------------------------
def test_dequant_closed_forms():
    q = np.array([[-127, -1, 0, 1, 127, 63]], np.int8)
    s = np.array([0.003141], F32)
    f32 = oracle.dequant(q, s, "f32")
    assert np.array_equal(f32, (q.astype(F32) * s[0]).astype(F32))
    b16 = oracle.dequant(q, s, "bf16")
    assert np.array_equal(b16, oracle.f32_to_bf16(q.astype(F32) * s[0]))
    h16 = oracle.dequant(q, s, "f16").view(np.float16)
    want = q.astype(np.float16) * np.float16(s[0])  # numpy f16 multiply rounds once
    assert np.array_equal(h16, want)


# ---- forward (lora.jl:56-95) ------------------------------------------------------------------
def _small_int_case(M=5, K=7, N=6, r=3, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.integers(-3, 4, size=(M, K)).astype(F32)
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(F32)
    A = rng.integers(-2, 3, size=(K, r)).astype(F32)
    B = rng.integers(-2, 3, size=(r, N)).astype(F32)
    bias = rng.integers(-5, 6, size=N).astype(F32)
    return x, q, s, A, B, bias


def test_forward_brute_force_integers():
    x, q, s, A, B, bias = _small_int_case()
    c = 2.0
    y, h = oracle.lora_forward(bf(x), q, s, bf(A), bf(B), c, bias=bf(bias))
    xi = x.astype(np.int64)
    want_h = xi @ A.astype(np.int64)
    want = (xi @ q.astype(np.int64).T) * s.astype(np.float64) + c * (want_h @ B.astype(np.int64)) + bias
    assert np.array_equal(h, want_h.astype(np.float64))
    assert np.array_equal(y, want)
    # row selection returns the same rows
    y2, _ = oracle.lora_forward(bf(x), q, s, bf(A), bf(B), c, bias=bf(bias), rows=[4, 0])
    assert np.array_equal(y2, want[[4, 0]])


def test_forward_zero_B_is_base_and_merged_weight_identity():
    # test/unit/lora.jl:6 (B = 0 gives the base product exactly) and :8 (merged weight)
    x = oracle.normal_bf16(21, (9, 16), 1.0)
    w = oracle.normal_bf16(22, (12, 16), 0.02)
    q, s, _ = oracle.pack(w)
    A = oracle.normal_bf16(23, (16, 4), 0.1)
    y0, _ = oracle.lora_forward(x, q, s, A, np.zeros((4, 12), np.uint16), 0.5)
    base, _ = oracle.lora_forward(x, q, s, None, None, 0.0)
    assert np.array_equal(y0, base)
    B = oracle.normal_bf16(24, (4, 12), 0.1)
    y, _ = oracle.lora_forward(x, q, s, A, B, 0.5)
    merged = q.astype(np.float64) * s.astype(np.float64)[:, None] + 0.5 * (
        oracle.bf16_to_f32(A).astype(np.float64) @ oracle.bf16_to_f32(B).astype(np.float64)).T
    np.testing.assert_allclose(y, oracle.bf16_to_f32(x).astype(np.float64) @ merged.T, rtol=1e-12,
                               atol=1e-12)


# ---- backward (lora.jl:106-118): exact finite differences of the linear forward --------------
def _loss(x, q, s, A, B, c, dy):
    y, _ = oracle.lora_forward(x, q, s, A, B, c)
    return float(np.sum(y * oracle.bf16_to_f32(dy).astype(np.float64)))


def test_backward_matches_finite_differences():
    # The loss sum(y .* dy) is linear in A, in B and in x, so a difference quotient between two
    # bf16 values is exact up to f64 rounding (the reference's own check, test/unit/lora.jl:12-21,
    # uses a central difference with rtol 2e-2).
    M, K, N, r, c = 6, 8, 5, 3, 1.5
    x = oracle.normal_bf16(31, (M, K), 1.0)
    w = oracle.normal_bf16(32, (N, K), 0.1)
    q, s, _ = oracle.pack(w)
    A = oracle.normal_bf16(33, (K, r), 0.3)
    B = oracle.normal_bf16(34, (r, N), 0.3)
    dy = oracle.normal_bf16(35, (M, N), 1.0)
    g = oracle.lora_backward(dy, x, q, s, A, B, c)
    base = _loss(x, q, s, A, B, c, dy)

    def quotient(arr, idx, name):
        a = arr.copy()
        old = oracle.bf16_to_f32(a[idx:idx + 1] if a.ndim == 1 else a[idx][None])[0]
        new = bf([old + 0.25])[0]
        a[idx] = new
        step = float(oracle.bf16_to_f32(np.array([new], np.uint16))[0]) - float(old)
        args = dict(x=x, A=A, B=B)
        args[name] = a
        return (_loss(args["x"], q, s, args["A"], args["B"], c, dy) - base) / step

    for idx in [(0, 0), (K - 1, r - 1), (3, 1)]:
        assert np.isclose(quotient(A, idx, "A"), g["dA"][idx], rtol=1e-9, atol=1e-9)
    for idx in [(0, 0), (r - 1, N - 1), (1, 2)]:
        assert np.isclose(quotient(B, idx, "B"), g["dB"][idx], rtol=1e-9, atol=1e-9)
    for idx in [(0, 0), (M - 1, K - 1), (2, 5)]:
        assert np.isclose(quotient(x, idx, "x"), g["dx"][idx], rtol=1e-9, atol=1e-9)
    # column / row selection returns the same entries
    g2 = oracle.lora_backward(dy, x, q, s, A, B, c, rows=[5, 1], kcols=[7, 0], ncols=[4, 2])
    assert np.array_equal(g2["dx"], g["dx"][[5, 1]])
    assert np.array_equal(g2["dA"], g["dA"][[7, 0]])
    assert np.array_equal(g2["dB"], g["dB"][:, [4, 2]])


def test_bias_gradient_is_the_difference_quotient_of_the_forward():
    # The forward adds the bias per output channel (lora.jl:64-67 via mixed_add, linear.jl:7-13),
    # so sum(y .* dy) is affine in the bias: a difference quotient in bias[n] is exact and equals
    # the oracle's bias gradient. A gradient summed over the wrong axis (over n instead of m) or
    # with the LoRA scale applied would fail it.
    M, K, N, r, c = 7, 8, 5, 3, 1.5
    x = oracle.normal_bf16(41, (M, K), 1.0)
    w = oracle.normal_bf16(42, (N, K), 0.1)
    q, s, _ = oracle.pack(w)
    A = oracle.normal_bf16(43, (K, r), 0.3)
    B = oracle.normal_bf16(44, (r, N), 0.3)
    dy = oracle.normal_bf16(45, (M, N), 1.0)
    bias = oracle.normal_bf16(46, (N,), 0.5)
    d = oracle.bf16_to_f32(dy).astype(np.float64)

    def loss(b):
        y, _ = oracle.lora_forward(x, q, s, A, B, c, b)
        return float(np.sum(y * d))

    base = loss(bias)
    g = oracle.bias_gradient(dy)
    assert g.shape == (N,)
    for n in range(N):
        b2 = bias.copy()
        old = float(oracle.bf16_to_f32(bias[n:n + 1])[0])
        b2[n] = bf([old + 0.5])[0]
        step = float(oracle.bf16_to_f32(b2[n:n + 1])[0]) - old
        assert np.isclose((loss(b2) - base) / step, g[n], rtol=1e-9, atol=1e-9)
    # column selection, and the binary16 / float32 decodes of the same values
    assert np.array_equal(oracle.bias_gradient(dy, cols=[4, 0]), g[[4, 0]])
    vals = oracle.bf16_to_f32(dy)
    assert np.array_equal(oracle.bias_gradient(vals, elt="f32"), g)
    assert np.array_equal(oracle.bias_gradient(oracle.f32_to_f16(vals), elt="f16"),
                          oracle.f16_to_f32(oracle.f32_to_f16(vals)).astype(np.float64).sum(0))


def test_backward_brute_force_integers():
    x, q, s, A, B, _ = _small_int_case(seed=3)
    dy = np.random.default_rng(4).integers(-3, 4, size=(x.shape[0], q.shape[0])).astype(F32)
    c = 0.5
    g = oracle.lora_backward(bf(dy), bf(x), q, s, bf(A), bf(B), c)
    X, D = x.astype(np.float64), dy.astype(np.float64)
    Wd = q.astype(np.float64) * s.astype(np.float64)[:, None]
    Af, Bf = A.astype(np.float64), B.astype(np.float64)
    u = D @ Bf.T
    assert np.array_equal(g["dx"], D @ Wd + c * u @ Af.T)
    assert np.array_equal(g["dA"], c * X.T @ u)
    assert np.array_equal(g["dB"], c * (X @ Af).T @ D)


# ---- gelu_tanh (src/layers/linear.jl:61-68) ----------------------------------------------------
def test_gelu_closed_forms_and_derivative():
    xs = np.array([0.0, 1.0, -1.0, 3.0, -3.0, 0.5, 10.0, -10.0], F32)
    y = oracle.bf16_to_f32(oracle.gelu_tanh(bf(xs)))
    assert y[0] == 0.0
    xb = oracle.bf16_to_f32(bf(xs)).astype(np.float64)
    k = np.sqrt(2 / np.pi)
    ref = 0.5 * xb * (1 + np.tanh(k * (xb + 0.044715 * xb ** 3)))
    assert np.allclose(y, ref, rtol=2 ** -7, atol=1e-6)
    # gelu(x) - gelu(-x) = x
    for i, j in [(1, 2), (3, 4)]:
        assert np.isclose(y[i] - y[j], xb[i], rtol=2 ** -6)
    # derivative: central differences of the f64 formula
    grid = np.linspace(-4, 4, 81).astype(F32)
    ones = bf(np.ones_like(grid))
    d = oracle.bf16_to_f32(oracle.gelu_tanh_backward(bf(grid), ones)).astype(np.float64)
    gb = oracle.bf16_to_f32(bf(grid)).astype(np.float64)
    f = lambda v: 0.5 * v * (1 + np.tanh(k * (v + 0.044715 * v ** 3)))
    fd = (f(gb + 1e-5) - f(gb - 1e-5)) / 2e-5
    assert np.allclose(d, fd, rtol=2 ** -7, atol=2 ** -8)


# ---- the reference's own fp16 int8 forward (reported beside ours) --------------------------------
# Each rounding point of oracle.reference_fp16_forward is pinned by an input whose exact result and
# rounded result differ, with the expected values worked out by hand (binary16: 11-bit significand,
# ties to even, largest finite 65504, values >= 65520 round to Inf).
def _ref16(x, q, s, A, B, c, bias=None):
    return oracle.reference_fp16_forward(bf(x), np.asarray(q, np.int8), np.asarray(s, F32),
                                         bf(A), bf(B), c, None if bias is None else bf(bias))


def test_reference_fp16_exact_small_integers_equal_brute_force():
    # every product and sum is exact in binary16 (|y| < 32 on a 1/4 grid), so the restatement must
    # equal the f64 brute force exactly; M, K, N, r all distinct so a transposed operand fails
    rng = np.random.default_rng(3)
    M, K, N, r, c = 5, 7, 3, 2, 0.5
    x = rng.integers(-2, 3, (M, K)).astype(F32)
    q = rng.integers(-7, 8, (N, K)).astype(np.int8)
    s = np.array([0.25, 0.5, 0.125], F32)
    A = rng.integers(-2, 3, (K, r)).astype(F32)
    B = rng.integers(-2, 3, (r, N)).astype(F32)
    want = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            want[m, n] = sum(float(x[m, k]) * float(q[n, k]) * float(s[n]) for k in range(K))
            h = [sum(float(x[m, k]) * float(A[k, j]) for k in range(K)) for j in range(r)]
            want[m, n] += c * sum(h[j] * float(B[j, n]) for j in range(r))
    got = _ref16(x, q, s, A, B, c)
    assert got.shape == (M, N)
    assert np.array_equal(got.astype(np.float64), want)


def test_reference_fp16_weight_is_f16_of_q_times_f16_scale():
    # s = 1/3: Float16(s) = 0.333251953125; Wd = Float16(q * Float16(s)). One-hot x picks out
    # column k = 1 of Wd for token 0; token 1 picks column 0 (all zero codes).
    q = np.zeros((5, 3), np.int8)
    q[:, 1] = [1, 3, 5, 7, -127]
    s = np.full(5, 1.0 / 3.0, F32)
    x = np.array([[0, 1, 0], [1, 0, 0]], F32)
    zA, zB = np.zeros((3, 1), F32), np.zeros((1, 5), F32)
    got = _ref16(x, q, s, zA, zB, 1.0)
    # 3 * 0.333251953125 = 1 - 2^-12, a tie between 1 - 2^-11 and 1 -> 1.0 (even);
    # 5 -> 1706.25 * 2^-10 -> 1.666015625; 7 -> 1194.375 * 2^-9 -> 2.33203125;
    # -127 -> -1354.34 * 2^-5 -> -42.3125 (rounding 5/3, 7/3, 127/3 directly gives 1.6669921875,
    # 2.333984375, -42.34375)
    assert got[0].tolist() == [0.333251953125, 1.0, 1.666015625, 2.33203125, -42.3125]
    assert got[1].tolist() == [0.0] * 5


def test_reference_fp16_output_rounds_ties_to_even_and_overflows():
    # s = 1, q = 1: Wd = 1. y = x0 + x1 in f32, then rounded to binary16
    q = np.ones((1, 2), np.int8)
    s = np.ones(1, F32)
    x = np.array([[2048, 1], [2048, 3], [2048, 2], [65280, 224], [65280, 240], [65280, 239]], F32)
    zA, zB = np.zeros((2, 1), F32), np.zeros((1, 1), F32)
    got = _ref16(x, q, s, zA, zB, 1.0)[:, 0]
    # 2049 -> 2048 (tie, even), 2051 -> 2052 (tie, even), 2050 exact; 65504 is the largest
    # finite binary16, 65520 rounds to Inf, 65519 rounds down to 65504
    assert got.tolist() == [2048.0, 2052.0, 2050.0, 65504.0, np.inf, 65504.0]


def test_reference_fp16_lora_roundings_bias_and_final_add():
    z = np.zeros((1, 2), np.int8)
    one = np.ones(1, F32)
    # h = Float16(x A) = Float16(2049) = 2048; Float16(h B) = Float16(3 * 2048) = 6144 exactly;
    # adapter = 0.25 * 6144. Without the rounding of h: Float16(6147) = 6148 -> 1537
    got = _ref16([[2048, 1]], z, one, [[1], [1]], [[3]], 0.25)
    assert got.tolist() == [[1536.0]]
    # Float16(h B) with h = [2048, 1] exact, B = [1, 1]: 2049 -> 2048
    got = _ref16([[1]], np.zeros((1, 1), np.int8), one, [[2048, 1]], [[1], [1]], 1.0)
    assert got.tolist() == [[2048.0]]
    # the bias is added in binary16 (mixed_add of two Float16 arrays): 2048 + 1 -> 2048;
    # the scaled adapter is Float32 and its add is not rounded to binary16: 2048 + 1 = 2049
    q1 = np.ones((1, 1), np.int8)
    got = _ref16([[2048]], q1, one, [[0]], [[0]], 1.0, bias=[1])
    assert got.tolist() == [[2048.0]]
    got = _ref16([[2048]], q1, one, [[1]], [[1]], 1.0 / 2048)
    assert got.tolist() == [[2049.0]]


def test_reference_fp16_path_error_is_small_on_wan_like_inputs():
    x = oracle.normal_bf16(41, (64, 256), 1.0)
    w = oracle.normal_bf16(42, (128, 256), 0.02)
    q, s, _ = oracle.pack(w)
    A = oracle.normal_bf16(43, (256, 16), 0.01)
    B = oracle.normal_bf16(44, (16, 128), 0.01)
    y, _ = oracle.lora_forward(x, q, s, A, B, 1.0)
    y16 = oracle.reference_fp16_forward(x, q, s, A, B, 1.0)
    rel = np.abs(y16 - y).max() / np.abs(y).max()
    assert 1e-6 < rel < 1e-2


# ---- the reference's CPU path restated for timing (oracle/cpu_path.py) --------------------------
def test_cpu_path_matches_the_f64_oracle():
    # The bench's CPU baseline must compute the reference's Float32 path: compare it with the f64
    # oracle on the same float32 values (M, K, N, r all distinct so a transposed operand fails)
    import torch
    from oracle import cpu_path
    M, K, N, r, c = 33, 40, 24, 4, 0.75
    x = oracle.normal_f32(51, (M, K), 1.0)
    w = oracle.normal_f32(52, (N, K), 0.02)
    q, s, _ = oracle.pack(w, "f32")
    A = oracle.normal_f32(53, (K, r), 0.1)
    B = oracle.normal_f32(54, (r, N), 0.1)
    dy = oracle.normal_f32(55, (M, N), 1.0)
    t = torch.from_numpy
    y = cpu_path.forward(t(x), t(q), t(s), t(A), t(B), c).numpy()
    dx, dA, dB = (v.numpy() for v in cpu_path.backward(t(x), t(dy), t(q), t(s), t(A), t(B), c))
    yo, _ = oracle.lora_forward(x, q, s, A, B, c, elt="f32")
    go = oracle.lora_backward(dy, x, q, s, A, B, c, elt="f32")
    for got, ref in ((y, yo), (dx, go["dx"]), (dA, go["dA"]), (dB, go["dB"])):
        assert got.shape == ref.shape
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    assert cpu_path.flops(M, K, N, r) == 4.0 * M * N * K + 6.0 * M * r * (K + N)


def test_cpu_path_time_linear():
    # the per-linear timing behind the configs' CPU baselines: both legs timed, finite, positive
    from oracle import cpu_path
    tf, tb = cpu_path.time_linear(64, 48, 40, 4, reps=2)
    assert 0.0 < tf < 60.0 and 0.0 < tb < 60.0
    tf, tb = cpu_path.time_linear(64, 48, 40, 4, warm=0)
    assert 0.0 < tf < 60.0 and 0.0 < tb < 60.0


# ---- the fp16 element path (the reference's Float16 compute) -----------------------------------
def h16(a):
    """IEEE binary16 patterns of the values a (numpy's rounding)."""
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def test_f16_decode_exhaustive_against_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # -0 kept


def test_f16_rounding_against_numpy():
    rng = np.random.default_rng(61)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(100000) * 1e-5).astype(np.float32),          # subnormal range
        (rng.standard_normal(50000) * 3e4).astype(np.float32),            # near the top
        np.array([65504, 65519.99, 65520, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14,
                  2 ** -14 - 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 0.0, -0.0], np.float32)])
    # exact halfway cases between adjacent binary16 values: ties to even
    base = rng.integers(0, 0x7bff, size=20000).astype(np.uint16)
    lo = base.view(np.float16).astype(np.float64)
    hi = (base + 1).view(np.float16).astype(np.float64)
    vals = np.concatenate([vals, ((lo + hi) / 2).astype(np.float32)])
    with np.errstate(over="ignore"):  # 65520 and above round to +-inf on purpose
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(vals), want)


def test_f16_forward_backward_equal_bf16_path_on_shared_values():
    # small integers are exact in both formats: the two element paths must give the same f64
    x, q, s, A, B, bias = _small_int_case(seed=7)
    dy = np.random.default_rng(8).integers(-3, 4, size=(x.shape[0], q.shape[0])).astype(F32)
    c = 0.75
    yb, hb = oracle.lora_forward(bf(x), q, s, bf(A), bf(B), c, bias=bf(bias))
    yh, hh = oracle.lora_forward(h16(x), q, s, h16(A), h16(B), c, bias=h16(bias), elt="f16")
    assert np.array_equal(yb, yh) and np.array_equal(hb, hh)
    gb = oracle.lora_backward(bf(dy), bf(x), q, s, bf(A), bf(B), c)
    gh = oracle.lora_backward(h16(dy), h16(x), q, s, h16(A), h16(B), c, elt="f16")
    for k in ("dx", "dA", "dB"):
        assert np.array_equal(gb[k], gh[k]), k


def test_f16_forward_uses_the_binary16_values():
    # values with more than 8 significant bits: the f16 decode is exact where bf16 would round
    x = np.array([[1 + 2 ** -10, -3 - 2 ** -9]], np.float32)
    q = np.array([[1, 1]], np.int8)
    s = np.array([1.0], np.float32)
    y, _ = oracle.lora_forward(h16(x), q, s, None, None, 0.0, elt="f16")
    assert y[0, 0] == (1 + 2 ** -10) + (-3 - 2 ** -9)


def test_f16_gelu_closed_forms():
    xs = np.array([0.0, 1.0, -1.0, 3.0, -3.0, 0.5, 8.0, -8.0], F32)
    y = oracle.f16_to_f32(oracle.gelu_tanh(h16(xs), elt="f16")).astype(np.float64)
    assert y[0] == 0.0
    k = np.sqrt(2 / np.pi)
    xb = xs.astype(np.float64)
    ref = 0.5 * xb * (1 + np.tanh(k * (xb + 0.044715 * xb ** 3)))
    assert np.allclose(y, ref, rtol=2 ** -10, atol=1e-6)
    for i, j in [(1, 2), (3, 4)]:
        assert np.isclose(y[i] - y[j], xb[i], rtol=2 ** -9)
    grid = np.linspace(-4, 4, 81).astype(F32)
    d = oracle.f16_to_f32(oracle.gelu_tanh_backward(h16(grid), h16(np.ones_like(grid)),
                                                    elt="f16")).astype(np.float64)
    gx = grid.astype(np.float16).astype(np.float64)
    f = lambda v: 0.5 * v * (1 + np.tanh(k * (v + 0.044715 * v ** 3)))
    fd = (f(gx + 1e-5) - f(gx - 1e-5)) / 2e-5
    assert np.allclose(d, fd, rtol=2 ** -10, atol=2 ** -12)


def test_f32_forward_backward_equal_bf16_path_on_shared_values():
    # bf16-exact values passed as float32: the f32 element path decodes them to the same f64
    x, q, s, A, B, bias = _small_int_case(seed=9)
    dy = np.random.default_rng(10).integers(-3, 4, size=(x.shape[0], q.shape[0])).astype(F32)
    c = 0.75
    yb, hb = oracle.lora_forward(bf(x), q, s, bf(A), bf(B), c, bias=bf(bias))
    yf, hf = oracle.lora_forward(x, q, s, A, B, c, bias=bias, elt="f32")
    assert np.array_equal(yb, yf) and np.array_equal(hb, hf)
    gb = oracle.lora_backward(bf(dy), bf(x), q, s, bf(A), bf(B), c)
    gf = oracle.lora_backward(dy, x, q, s, A, B, c, elt="f32")
    for k in ("dx", "dA", "dB"):
        assert np.array_equal(gb[k], gf[k]), k


def test_f32_forward_uses_the_float32_values():
    # 24 significant bits survive the f32 decode (bf16 and f16 would round them away)
    x = np.array([[1 + 2 ** -20, -3 - 2 ** -21]], np.float32)
    q = np.array([[1, 1]], np.int8)
    s = np.array([1.0], np.float32)
    y, _ = oracle.lora_forward(x, q, s, None, None, 0.0, elt="f32")
    assert y[0, 0] == float(np.float32(1 + 2 ** -20)) + float(np.float32(-3 - 2 ** -21))


def test_f32_gelu_is_the_unrounded_bf16_gelu():
    # the f32 path returns gelu in f32 (linear.jl:61-68 with T = Float32: no cast back); the
    # bf16 path is the same value rounded to nearest even, and both meet the closed forms
    xs = np.linspace(-6, 6, 241).astype(F32)
    xs = oracle.bf16_to_f32(oracle.f32_to_bf16(xs))  # inputs both paths represent exactly
    yf = oracle.gelu_tanh(xs, elt="f32")
    assert yf.dtype == np.float32
    assert np.array_equal(oracle.f32_to_bf16(yf), oracle.gelu_tanh(bf(xs)))
    k = np.sqrt(2 / np.pi)
    xb = xs.astype(np.float64)
    ref = 0.5 * xb * (1 + np.tanh(k * (xb + 0.044715 * xb ** 3)))
    assert np.allclose(yf, ref, rtol=1e-6, atol=1e-7)
    assert yf[np.argmin(np.abs(xs))] == 0.0
    d = oracle.gelu_tanh_backward(xs, np.ones_like(xs), elt="f32").astype(np.float64)
    f = lambda v: 0.5 * v * (1 + np.tanh(k * (v + 0.044715 * v ** 3)))
    fd = (f(xb + 1e-6) - f(xb - 1e-6)) / 2e-6
    assert np.allclose(d, fd, rtol=1e-5, atol=1e-6)


# ---- attention (src/layers/attention.jl) ------------------------------------------------------
def _np_attention(q, k, v, mask=None, causal=False):
    """Second restatement, numpy only: softmax over visible keys per (batch, head, query)."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    sc = float(np.float32(1) / np.sqrt(np.float32(D)))
    s = np.einsum("bqhd,bkhd->bhqk", q, k) * sc
    vis = np.ones((Sq, Sk), bool) if mask is None else mask.astype(bool).copy()
    if causal:
        vis &= np.arange(Sk)[None, :] <= np.arange(Sq)[:, None]
    s = np.where(vis[None, None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    lse = (m + np.log(e.sum(-1, keepdims=True)))[..., 0]
    p = e / e.sum(-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", p, v), lse


def _att_inputs(rng, B, Sq, Sk, H, D, scale=1.0):
    f = lambda *sh: (rng.standard_normal(sh) * scale).astype(np.float32)
    return f(B, Sq, H, D), f(B, Sk, H, D), f(B, Sk, H, D)


def test_attention_zero_queries_average_the_visible_values():
    # q = 0: every visible score is 0, so the weights are uniform (closed form)
    rng = np.random.default_rng(1)
    _, k, v = _att_inputs(rng, 2, 5, 7, 3, 8)
    q = np.zeros((2, 5, 3, 8), np.float32)
    mask = rng.random((5, 7)) < 0.6
    mask[:, 0] = True
    out, lse = oracle.attention_forward(q, k, v, mask=mask, elt="f32")
    for i in range(5):
        vis = mask[i]
        assert np.allclose(out[:, i], v[:, vis].astype(np.float64).mean(axis=1), rtol=0, atol=1e-12)
        assert np.allclose(lse[:, :, i], np.log(vis.sum()), rtol=0, atol=1e-12)


def test_attention_causal_first_query_is_the_first_value():
    # causal, query 0 sees key 0 only: output v[0], lse = its score
    rng = np.random.default_rng(2)
    q, k, v = _att_inputs(rng, 1, 6, 6, 2, 16)
    out, lse = oracle.attention_forward(q, k, v, causal=True, elt="f32")
    assert np.array_equal(out[:, 0], v[:, 0].astype(np.float64))
    sc = float(np.float32(1) / np.sqrt(np.float32(16)))
    s00 = (q[0, 0].astype(np.float64) * k[0, 0]).sum(-1) * sc
    assert np.allclose(lse[0, :, 0], s00, rtol=0, atol=1e-12)


def test_attention_matches_numpy_restatement():
    rng = np.random.default_rng(3)
    for (B, Sq, Sk, H, D, causal, masked) in [(1, 7, 9, 2, 4, False, True), (2, 9, 9, 3, 8, True, False),
                                              (1, 5, 3, 1, 16, False, False)]:
        q, k, v = _att_inputs(rng, B, Sq, Sk, H, D)
        mask = None
        if masked:
            mask = rng.random((Sq, Sk)) < 0.7
            mask[:, 1] = True
        out, lse = oracle.attention_forward(q, k, v, mask=mask, causal=causal, elt="f32")
        ro, rl = _np_attention(q, k, v, mask, causal)
        assert np.allclose(out, ro, rtol=1e-12, atol=1e-12)
        assert np.allclose(lse, rl, rtol=1e-12, atol=1e-12)


def test_attention_mask_and_causal_equivalences():
    # an all-visible mask is no mask; the lower-triangular mask is causal (layers.jl:70, 97-100)
    rng = np.random.default_rng(4)
    q, k, v = _att_inputs(rng, 1, 6, 6, 2, 8)
    base = oracle.attention_forward(q, k, v, elt="f32")
    full = oracle.attention_forward(q, k, v, mask=np.ones((6, 6), bool), elt="f32")
    assert np.array_equal(base[0], full[0]) and np.array_equal(base[1], full[1])
    tri = np.tril(np.ones((6, 6), bool))
    c1 = oracle.attention_forward(q, k, v, causal=True, elt="f32")
    c2 = oracle.attention_forward(q, k, v, mask=tri, elt="f32")
    assert np.array_equal(c1[0], c2[0]) and np.array_equal(c1[1], c2[1])
    # a query with no visible key: NaN output and lse, as the reference's online softmax
    m = np.ones((6, 6), bool)
    m[2] = False
    out, lse = oracle.attention_forward(q, k, v, mask=m, elt="f32")
    assert np.isnan(out[0, 2]).all() and np.isnan(lse[0, :, 2]).all()
    assert np.isfinite(out[0, [0, 1, 3, 4, 5]]).all()


def test_attention_16bit_inputs_decode_exactly():
    # bf16 / f16 patterns are decoded exactly: the same values given as f32 give the same result
    rng = np.random.default_rng(5)
    q, k, v = _att_inputs(rng, 1, 4, 5, 2, 8)
    qb, kb, vb = (oracle.f32_to_bf16(a) for a in (q, k, v))
    ob, lb = oracle.attention_forward(qb, kb, vb, elt="bf16")
    of, lf = oracle.attention_forward(*(oracle.bf16_to_f32(a) for a in (qb, kb, vb)), elt="f32")
    assert np.array_equal(ob, of) and np.array_equal(lb, lf)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_backward_matches_finite_differences(causal):
    # objective sum(out .* dy), central differences of the f64 forward (as layers.jl:62-67)
    rng = np.random.default_rng(6)
    B, Sq, Sk, H, D = 1, 4, 5 if not causal else 4, 2, 4
    q, k, v = _att_inputs(rng, B, Sq, Sk, H, D)
    dy = rng.standard_normal(q.shape).astype(np.float32)
    mask = None if causal else (rng.random((Sq, Sk)) < 0.8) | (np.arange(Sk)[None, :] == 0)
    dq, dk, dv = oracle.attention_backward(q, k, v, dy, mask=mask, causal=causal, elt="f32")

    def objective(qq, kk, vv):
        o, _ = oracle.attention_forward(qq, kk, vv, mask=mask, causal=causal, elt="f32")
        return float((o * dy.astype(np.float64)).sum())

    for name, arr, grad in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for idx in [(0, 1, 0, 2), (0, 2, 1, 3), (0, 3, 1, 0)]:
            hi, lo = arr.copy(), arr.copy()
            hi[idx] += np.float32(1e-2)
            lo[idx] -= np.float32(1e-2)
            step = float(hi[idx]) - float(lo[idx])
            args_hi = {"q": (hi, k, v), "k": (q, hi, v), "v": (q, k, hi)}[name]
            args_lo = {"q": (lo, k, v), "k": (q, lo, v), "v": (q, k, lo)}[name]
            fd = (objective(*args_hi) - objective(*args_lo)) / step
            assert abs(fd - grad[idx]) <= 1e-4 + 1e-4 * abs(fd), (name, idx, fd, grad[idx])


def test_cpu_path_attention_matches_the_f64_oracle():
    # the attention CPU baseline (the reference's f32 tiled attention, attention.jl:106-221)
    # against the f64 oracle; tiles smaller than the sizes so several blocks and a ragged last
    # block are exercised
    import torch
    from oracle import cpu_path
    Sq, Sk, D = 70, 90, 32
    rng = np.random.default_rng(9)
    q, k, v, dy = (rng.standard_normal(s).astype(F32) for s in ((Sq, D), (Sk, D), (Sk, D), (Sq, D)))
    t = torch.from_numpy
    out, lse = cpu_path.attention_forward(t(q), t(k), t(v), query_block=32, key_block=40)
    dq, dk, dv = cpu_path.attention_backward(t(q), t(k), t(v), t(dy), out, lse, 32, 40)
    r4 = lambda a: a.reshape(1, a.shape[0], 1, D)
    oo, lo = oracle.attention_forward(r4(q), r4(k), r4(v), elt="f32")
    go = oracle.attention_backward(r4(q), r4(k), r4(v), r4(dy), elt="f32")
    assert np.abs(out.numpy() - oo[0, :, 0]).max() <= 1e-5 * np.abs(oo).max()
    assert np.abs(lse.numpy() - lo[0, 0]).max() <= 1e-5
    for got, ref in zip((dq, dk, dv), go):
        assert np.abs(got.numpy() - ref[0, :, 0]).max() <= 1e-4 * np.abs(ref).max()


def test_attention_sampled_equals_the_full_oracle():
    # the blockwise f64 restatement used at full size agrees with the loop oracle on every query
    # and key it is asked for, in several blocks (block smaller than Sq), bf16 and f32 inputs
    rng = np.random.default_rng(77)
    B, Sq, Sk, H, D = 2, 70, 53, 3, 16
    f = lambda *sh: rng.standard_normal(sh).astype(F32)
    q, k, v, dy = (oracle.f32_to_bf16(a) for a in (f(B, Sq, H, D), f(B, Sk, H, D),
                                                   f(B, Sk, H, D), f(B, Sq, H, D)))
    out, lse = oracle.attention_forward(q, k, v)
    dq, dk, dv = oracle.attention_backward(q, k, v, dy)
    qr, kc = [0, 17, 69], [0, 30, 52]
    for (b, h) in [(0, 0), (1, 2)]:
        r = oracle.attention_sampled(q, k, v, dy, b, h, qr, kc, block=16)
        np.testing.assert_allclose(r["out"], out[b, qr, h], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["lse"], lse[b, h, qr], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(r["dq"], dq[b, qr, h], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(r["dk"], dk[b, kc, h], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(r["dv"], dv[b, kc, h], rtol=1e-9, atol=1e-12)
    qf, kf, vf, dyf = (oracle.bf16_to_f32(a) for a in (q, k, v, dy))
    r = oracle.attention_sampled(qf, kf, vf, dyf, 1, 1, [5], [7], elt="f32")
    np.testing.assert_allclose(r["dv"], dv[1, [7], 1], rtol=1e-9, atol=1e-12)
