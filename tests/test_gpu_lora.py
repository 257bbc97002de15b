"""GPU parity of the int8 LoRA linear forward and backward (lora_forward / lora_backward,
src/layers/lora.jl:56-118) against the f64 oracle on the same seeded inputs.

Tolerance (bf16 compute, stated in tests/_util.assert_parity): normwise max|e|/max|ref| <= 1e-2
and elementwise |e| <= 1e-2 (|ref| + rms(ref)). The restated reference fp16 path's error against
the same oracle is printed beside ours. At the full Wan-14B size the rows / columns checked
against the oracle are sampled, and size-independent properties cover the rest (exact scaling by
2, bitwise reproducibility)."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_bits, bf16_f32, rel_errors, to_dev

pytestmark = pytest.mark.gpu


def make_case(M, K, N, r, alpha, seed=0, bias=False, w_sigma=0.02, ab_sigma=0.01):
    x = oracle.normal_bf16(seed + 1, (M, K), 1.0)
    w = oracle.normal_bf16(seed + 2, (N, K), w_sigma)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    A = oracle.normal_bf16(seed + 3, (K, r), ab_sigma) if r else None
    B = oracle.normal_bf16(seed + 4, (r, N), ab_sigma) if r else None
    dy = oracle.normal_bf16(seed + 5, (M, N), 1.0)
    b = oracle.normal_bf16(seed + 6, (N,), 0.1) if bias else None
    c = float(np.float32(alpha) / np.float32(r)) if r else 0.0
    return dict(x=x, q=q, s=s, A=A, B=B, dy=dy, bias=b, c=c, M=M, K=K, N=N, r=r)


def run_gpu(dev, cs, save_h=True, h_for_bwd=True):
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x = to_dev(cs["x"], dev)
    A = to_dev(cs["A"], dev) if cs["r"] else None
    B = to_dev(cs["B"], dev) if cs["r"] else None
    bias = to_dev(cs["bias"], dev) if cs["bias"] is not None else None
    y, h = i8lora_forward(x, W, A, B, bias, cs["c"], save_h=save_h and cs["r"] > 0)
    dy = to_dev(cs["dy"], dev)
    dx, dA, dB = i8lora_backward(dy, x, W, A, B, cs["c"], h=h if h_for_bwd else None)
    torch.cuda.synchronize(dev)
    out = dict(y=bf16_f32(y), dx=bf16_f32(dx))
    if h is not None:
        out["h"] = bf16_f32(h)
    if dA is not None:
        out["dA"] = dA.cpu().numpy()
        out["dB"] = dB.cpu().numpy()
    return out


def check_full(dev, cs, label):
    print(f"[lora] {label}: M={cs['M']} K={cs['K']} N={cs['N']} r={cs['r']}", flush=True)
    g = run_gpu(dev, cs)
    y, h = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], cs["bias"])
    assert_parity(g["y"], y, f"{label} y")
    if cs["r"]:
        assert_parity(g["h"], h, f"{label} h")
        ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"])
        assert_parity(g["dA"], ref["dA"], f"{label} dA")
        assert_parity(g["dB"], ref["dB"], f"{label} dB")
    else:
        ref = {"dx": oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"],
                                          np.zeros((cs["K"], 0), np.uint16),
                                          np.zeros((0, cs["N"]), np.uint16), 0.0,
                                          want=("dx",))["dx"]}
    assert_parity(g["dx"], ref["dx"], f"{label} dx")
    if cs["r"] and cs["bias"] is None:
        y16 = oracle.reference_fp16_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"])
        print(f"[lora] {label}: reference fp16 path normwise/elementwise error "
              f"{rel_errors(y16, y)[0]:.3e}/{rel_errors(y16, y)[1]:.3e} vs ours "
              f"{rel_errors(g['y'], y)[0]:.3e}/{rel_errors(g['y'], y)[1]:.3e}")
    return g


def test_cfg1_cpu_runnable_case(dev):
    # W 1536x1536 ~N(0,0.02) packed per channel; x 1024x1536 ~N(0,1); rank 16, alpha 16;
    # A, B ~N(0, 0.01); dY ~N(0,1)
    check_full(dev, make_case(1024, 1536, 1536, 16, 16.0, seed=100), "cfg1")


def test_reference_gpu_test_shape_ragged(dev):
    # the shape of test/gpu/lora.jl:111-134: weight 7x5, rank 3, alpha 6, 4 tokens (generic path)
    check_full(dev, make_case(4, 5, 7, 3, 6.0, seed=110, w_sigma=1.0, ab_sigma=1.0), "ragged7x5")


@pytest.mark.parametrize("M,K,N,r,bias", [
    (77, 1536, 1536, 32, False),    # skinny token count, tail tile
    (333, 512, 768, 16, True),      # bias, partial tiles in every dimension
    (256, 256, 256, 64, False),     # rank 64
    (300, 384, 320, 128, True),     # rank 128, N not a multiple of 256
    (130, 1536, 8960, 32, False),   # FFN-in shape
    (100, 8960, 1536, 32, False),   # FFN-out shape
    (65, 48, 80, 16, False),        # K not a multiple of 64
    (200, 512, 528, 32, True),      # K % 64 == 0, N % 64 != 0: int8 GEMM forward, general dX
    (200, 528, 512, 16, False),     # N % 64 == 0, K % 64 != 0: general forward, int8 GEMM dX
    (100, 64, 192, 32, True),       # one k-step forward (LoRA operands copied up front), three in dX
    (260, 128, 64, 16, False),      # two k-steps forward, one in dX
    (96, 256, 320, 32, True),       # 4 and 5 k-steps: the output staging around the LoRA stage
    (150, 640, 384, 48, True),      # rank 48: LoRA operands read from global memory
    (50, 256, 256, 0, True),        # base-only linear(::DenseLayer) with bias
    (40, 24, 20, 2, True),          # ragged: generic path with bias
    (1100, 2048, 2560, 32, True),   # 50 / 40 tiles of 256 x 256: reductions split in both GEMMs
    (400, 2048, 2560, 32, True),    # row-wave tiles: 128 rows x 64 tokens forward, 64 x 64 dX
    (352, 1024, 4608, 24, False),   # row-wave tiles with a padded rank
])
def test_shapes(dev, M, K, N, r, bias):
    check_full(dev, make_case(M, K, N, r, float(r) if r else 1.0, seed=M + K + N + r,
                              bias=bias), f"shape{M}x{K}x{N}r{r}")


@pytest.mark.parametrize("r", [1, 4, 8, 24, 160])
def test_any_rank_on_a_wan_shape(dev, r):
    """Any positive rank (the reference accepts any rank and per-layer rank_overrides,
    src/config/schema.jl:117-123, lora.jl:13-28; its own tests use r = 3) takes the MFMA path:
    the LoRA panels are zero-padded to a multiple of 16 in the workspace, ranks above 128 run in
    chunks. 5120 x 5120 at 4096 tokens, alpha = r: sampled rows of y and dx, h in full, sampled
    dA / dB columns against the oracle, with h saved by the forward and recomputed."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    M, K, N = 4096, 5120, 5120
    cs = make_case(M, K, N, r, float(r), seed=800 + r)
    print(f"[lora] rank {r} on {M}x{K}x{N}", flush=True)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x, dy = to_dev(cs["x"], dev), to_dev(cs["dy"], dev)
    A, B = to_dev(cs["A"], dev), to_dev(cs["B"], dev)
    y, h = i8lora_forward(x, W, A, B, None, cs["c"], save_h=True)
    dx, dA, dB = i8lora_backward(dy, x, W, A, B, cs["c"], h=h)
    dx_r, dA_r, dB_r = i8lora_backward(dy, x, W, A, B, cs["c"], h=None)  # h recomputed
    torch.cuda.synchronize(dev)
    assert h.shape == (M, r)
    assert torch.equal(dx, dx_r) and torch.equal(dA, dA_r) and torch.equal(dB, dB_r)
    rng = np.random.default_rng(r)
    rows = np.concatenate([rng.choice(M - 8, 24, replace=False), np.arange(M - 8, M)])
    kc, nc = rng.choice(K, 32, replace=False), rng.choice(N, 32, replace=False)
    yo, ho = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], rows=rows)
    go = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                              rows=rows, kcols=kc, ncols=nc)
    assert_parity(bf16_f32(y)[rows], yo, f"rank {r} y")
    assert_parity(bf16_f32(h)[rows], ho, f"rank {r} h")
    assert_parity(bf16_f32(dx)[rows], go["dx"], f"rank {r} dx")
    assert_parity(dA.cpu().numpy()[kc], go["dA"], f"rank {r} dA")
    assert_parity(dB.cpu().numpy()[:, nc], go["dB"], f"rank {r} dB")


def test_recompute_h_equals_saved_h(dev):
    cs = make_case(200, 512, 256, 32, 32.0, seed=7)
    a = run_gpu(dev, cs, h_for_bwd=True)
    b = run_gpu(dev, cs, h_for_bwd=False)
    for k in ("dx", "dA", "dB"):
        assert np.array_equal(a[k], b[k]), k


def test_backward_bitwise_reproducible(dev):
    cs = make_case(3000, 1536, 1536, 32, 32.0, seed=8)
    a = run_gpu(dev, cs)
    b = run_gpu(dev, cs)
    for k in ("y", "h", "dx", "dA", "dB"):
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 13824), (13824, 5120)])
def test_wan14b_projection_full_size(dev, K, N):
    """The Wan-2.1-14B block projections at 32760 tokens (q/k/v/o 5120 -> 5120, ffn.0 5120 ->
    13824, ffn.2 13824 -> 5120; r = 32, alpha 32): sampled rows (including the partial last tile)
    and sampled dA/dB columns against the oracle; exact doubling y(2x) = 2 y(x),
    dx(2dy) = 2 dx(dy), dA(2dy) = 2 dA, dB(2dy) = 2 dB over the whole output (power-of-two
    scaling is exact in every f32 sum and bf16 rounding)."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    M, r = 32760, 32
    cs = make_case(M, K, N, r, 32.0, seed=500 + K + 2 * N)
    print(f"[lora] wan14b projection {K}->{N} at {M} tokens", flush=True)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x, dy = to_dev(cs["x"], dev), to_dev(cs["dy"], dev)
    A, B = to_dev(cs["A"], dev), to_dev(cs["B"], dev)
    y, h = i8lora_forward(x, W, A, B, None, cs["c"], save_h=True)
    dx, dA, dB = i8lora_backward(dy, x, W, A, B, cs["c"], h=h)
    y2, _ = i8lora_forward(x * 2, W, A, B, None, cs["c"])
    dx2, dA2, dB2 = i8lora_backward(dy * 2, x, W, A, B, cs["c"], h=h)
    torch.cuda.synchronize(dev)
    assert torch.equal(y2, y * 2)
    assert torch.equal(dx2, dx * 2)
    assert torch.equal(dA2, dA * 2) and torch.equal(dB2, dB * 2)
    rng = np.random.default_rng(5)
    rows = np.concatenate([rng.choice(M - 64, 40, replace=False), np.arange(M - 24, M)])
    kcols = rng.choice(K, 48, replace=False)
    ncols = rng.choice(N, 48, replace=False)
    yr, _ = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], rows=rows)
    ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                               rows=rows, kcols=kcols, ncols=ncols)
    assert_parity(bf16_f32(y)[rows], yr, f"wan14b {K}->{N} y (sampled rows)")
    assert_parity(bf16_f32(dx)[rows], ref["dx"], f"wan14b {K}->{N} dx (sampled rows)")
    assert_parity(dA.cpu().numpy()[kcols], ref["dA"], f"wan14b {K}->{N} dA (sampled k)")
    assert_parity(dB.cpu().numpy()[:, ncols], ref["dB"], f"wan14b {K}->{N} dB (sampled n)")


def test_mirror_api_and_autograd(dev):
    import torch
    from reels_amd import (I8LoRALinearFunction, LoRALinear, linear, DenseLayer, lora_backward,
                           lora_forward, quantize_frozen_matrix, set_adapter_enabled)
    w = to_dev(oracle.normal_bf16(600, (384, 256), 0.02), dev)
    qm = quantize_frozen_matrix(w)
    layer = LoRALinear(qm, rank=16, alpha=16, generator=torch.Generator(device=dev).manual_seed(1))
    x = to_dev(oracle.normal_bf16(601, (3, 50, 256), 1.0), dev)  # trailing dims kept
    # B = 0 at construction: the layer equals the base linear exactly (test/unit/lora.jl:6)
    assert torch.equal(layer(x), linear(DenseLayer(qm), x))
    layer.B = to_dev(oracle.normal_bf16(602, (16, 384), 0.05), dev)
    set_adapter_enabled(layer, False)
    assert torch.equal(layer(x), linear(DenseLayer(qm), x))
    set_adapter_enabled(layer, True)
    y = lora_forward(layer, x)
    dy = to_dev(oracle.normal_bf16(603, (3, 50, 384), 1.0), dev)
    g = lora_backward(layer, x, dy)
    assert g["dx"].shape == x.shape and g["A"].shape == (256, 16) and g["B"].shape == (16, 384)
    # autograd rule returns the same gradients as the explicit backward
    xa = x.reshape(-1, 256).clone().requires_grad_(True)
    A = layer.A.clone().requires_grad_(True)
    B = layer.B.clone().requires_grad_(True)
    out = I8LoRALinearFunction.apply(xa, A, B, qm.values, qm.scales, None, layer.lora_scale)
    assert torch.equal(out, y.reshape(-1, 384))
    out.backward(dy.reshape(-1, 384))
    assert torch.equal(xa.grad, g["dx"].reshape(-1, 256))
    assert torch.equal(A.grad, g["A"].to(torch.bfloat16))
    assert torch.equal(B.grad, g["B"].to(torch.bfloat16))


def test_autograd_trainable_bias_gets_its_gradient(dev):
    """A trainable bias (LoRALinear train_bias) gets the pullback of mixed_add: dy summed over
    the tokens (linear.jl:7-13), checked against the f64 column sum; x, A and B get the same
    gradients as the explicit backward."""
    import torch
    from reels_amd import I8LoRALinearFunction, QuantizedMatrix, i8lora_backward
    M, K, N, r = 300, 256, 384, 16
    cs = make_case(M, K, N, r, 16.0, seed=640, bias=True)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x = to_dev(cs["x"], dev).requires_grad_(True)
    A = to_dev(cs["A"], dev).requires_grad_(True)
    B = to_dev(cs["B"], dev).requires_grad_(True)
    bias = to_dev(cs["bias"], dev).requires_grad_(True)
    dy = to_dev(cs["dy"], dev)
    y = I8LoRALinearFunction.apply(x, A, B, W.values, W.scales, bias, cs["c"])
    y.backward(dy)
    torch.cuda.synchronize(dev)
    want = oracle.bf16_to_f32(cs["dy"]).astype(np.float64).sum(0)
    assert bias.grad is not None and bias.grad.dtype == torch.bfloat16
    assert_parity(bf16_f32(bias.grad), want, "autograd dbias")
    dx, dA, dB = i8lora_backward(dy, x.detach(), W, A.detach(), B.detach(), cs["c"])
    assert torch.equal(x.grad, dx)
    assert torch.equal(A.grad, dA.to(torch.bfloat16)) and torch.equal(B.grad, dB.to(torch.bfloat16))


def test_autograd_f32_master_adapters_get_f32_gradients(dev):
    """f32 master copies of A and B (the reference's AdamW keeps f32 state, optimizer.jl:9-24)
    with bf16 activations: the kernels run on bf16 roundings of the masters and the gradients
    come back as the kernels' f32 values, not rounded to bf16."""
    import torch
    from reels_amd import I8LoRALinearFunction, QuantizedMatrix, i8lora_backward, i8lora_forward
    M, K, N, r = 200, 256, 384, 16
    cs = make_case(M, K, N, r, 16.0, seed=650)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x = to_dev(cs["x"], dev).requires_grad_(True)
    A32 = (to_dev(cs["A"], dev).float() * (1.0 + 2.0 ** -12)).requires_grad_(True)  # not bf16 values
    B32 = (to_dev(cs["B"], dev).float() * (1.0 - 2.0 ** -12)).requires_grad_(True)
    dy = to_dev(cs["dy"], dev)
    y = I8LoRALinearFunction.apply(x, A32, B32, W.values, W.scales, None, cs["c"])
    y.backward(dy)
    torch.cuda.synchronize(dev)
    assert A32.grad.dtype == torch.float32 and B32.grad.dtype == torch.float32
    Ab, Bb = A32.detach().to(torch.bfloat16), B32.detach().to(torch.bfloat16)
    y2, _ = i8lora_forward(x.detach(), W, Ab, Bb, None, cs["c"])
    dx, dA, dB = i8lora_backward(dy, x.detach(), W, Ab, Bb, cs["c"])
    assert torch.equal(y, y2) and torch.equal(x.grad, dx)
    assert torch.equal(A32.grad, dA) and torch.equal(B32.grad, dB)
    ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], bf16_bits(Ab), bf16_bits(Bb), cs["c"])
    assert_parity(A32.grad.cpu().numpy(), ref["dA"], "f32 master dA")
    assert_parity(B32.grad.cpu().numpy(), ref["dB"], "f32 master dB")


@pytest.mark.parametrize("n", [1, 1000, 8960 * 64 + 3])
def test_gelu_tanh(dev, n):
    from reels_amd import gelu_tanh, gelu_tanh_backward
    xb = oracle.normal_bf16(700 + n, (n,), 2.0)
    dyb = oracle.normal_bf16(701 + n, (n,), 1.0)
    x, dy = to_dev(xb, dev), to_dev(dyb, dev)
    y = bf16_f32(gelu_tanh(x))
    dx = bf16_f32(gelu_tanh_backward(x, dy))
    yo = oracle.bf16_to_f32(oracle.gelu_tanh(xb))
    dxo = oracle.bf16_to_f32(oracle.gelu_tanh_backward(xb, dyb))
    # f32 tanh of the device and of the host libm may differ in the last bits: allow one bf16
    # ulp (2^-7 relative) and require most elements to be bit-identical
    assert np.all(np.abs(y - yo) <= 2.0 ** -7 * np.abs(yo) + 1e-30)
    assert np.mean(y == yo) > 0.99
    assert np.all(np.abs(dx - dxo) <= 2.0 ** -6 * np.abs(dxo) + 2.0 ** -12 * np.abs(dxo).max())
    assert np.mean(dx == dxo) > 0.95


def test_gelu_tanh_unaligned_operands(dev):
    """Operands that are not 16-byte aligned take the one-element-per-thread path: the same bits
    as the 16-byte path on aligned copies."""
    import torch
    from reels_amd import gelu_tanh, gelu_tanh_backward
    n = 4099
    xb = oracle.normal_bf16(711, (n + 1,), 2.0)
    dyb = oracle.normal_bf16(712, (n + 1,), 1.0)
    x, dy = to_dev(xb, dev), to_dev(dyb, dev)
    xu, dyu = x[1:], dy[1:]
    assert xu.data_ptr() % 16 != 0
    xa, dya = xu.clone(), dyu.clone()
    assert torch.equal(gelu_tanh(xu), gelu_tanh(xa))
    assert torch.equal(gelu_tanh_backward(xu, dyu), gelu_tanh_backward(xa, dya))


@pytest.mark.parametrize("K,N", [(8960, 1536), (1536, 8960)])
def test_tokens_beyond_2gib_of_activations(dev, K, N):
    # 120000 tokens x 8960 bf16 is 2.15 GB: the GEMM whose reduction is 8960 wide (forward for
    # 8960->1536, dX for 1536->8960) runs as two token chunks (119808 + 192 tokens). y and dx
    # are row-independent, so rows on both sides of the chunk boundary are checked against the
    # oracle run on just those rows.
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    from tests._util import bf16_bits
    M, r = 120000, 32
    print(f"[lora] chunked tokens M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device=dev).manual_seed(K + N)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    dy = torch.randn((M, N), generator=g, device=dev).to(torch.bfloat16)
    w = oracle.normal_bf16(K + N, (N, K), 0.02)
    q, s, _ = oracle.pack(w, "bf16")
    A = oracle.normal_bf16(K + N + 1, (K, r), 0.01)
    B = oracle.normal_bf16(K + N + 2, (r, N), 0.01)
    W = QuantizedMatrix(to_dev(q, dev, "raw"), to_dev(s, dev, "raw"))
    Ad, Bd = to_dev(A, dev), to_dev(B, dev)
    y, h = i8lora_forward(x, W, Ad, Bd, None, 1.0, save_h=True)
    dx, _, _ = i8lora_backward(dy, x, W, Ad, Bd, 1.0, h=h, want_dA=False, want_dB=False)
    torch.cuda.synchronize(dev)
    rows = np.array([0, 1, 119806, 119807, 119808, 119809, 119999])
    rt = torch.from_numpy(rows).to(dev)
    xr, dyr = bf16_bits(x[rt]), bf16_bits(dy[rt])
    yo, _ = oracle.lora_forward(xr, q, s, A, B, 1.0)
    dxo = oracle.lora_backward(dyr, xr, q, s, A, B, 1.0, want=("dx",))["dx"]
    assert_parity(bf16_f32(y[rt]), yo, f"chunked {K}->{N} y (rows across the chunk boundary)")
    assert_parity(bf16_f32(dx[rt]), dxo, f"chunked {K}->{N} dx (rows across the chunk boundary)")
