"""GPU parity of the int8 pack kernel (quantize_frozen_matrix, src/layers/quantization.jl:35-44):
codes and scales must equal the oracle's bit for bit."""
import ctypes

import numpy as np
import pytest

import oracle
from tests._util import to_dev

pytestmark = pytest.mark.gpu
F32 = np.float32


def gpu_pack(dev, w, kind):
    """Runs reels_hip_i8_pack on w (numpy: float32, or uint16 bits for bf16 / f16)."""
    import torch
    from reels_amd import _lib
    if kind == "f32":
        t = torch.from_numpy(np.ascontiguousarray(w, F32)).to(dev)
        code = _lib.F32
    else:
        t = torch.from_numpy(np.ascontiguousarray(w).view(np.int16)).to(dev)
        code = _lib.BF16 if kind == "bf16" else _lib.F16
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.int8, device=dev)
    s = torch.empty((N,), dtype=torch.float32, device=dev)
    st = torch.full((1,), 7, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = _lib.lib().reels_hip_i8_pack(ctypes.c_void_p(t.data_ptr()), code, N, K, K,
                                      ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                                      ctypes.c_void_p(st.data_ptr()), stream)
    assert rc == 0, _lib.lib().reels_hip_last_error()
    torch.cuda.synchronize(dev)
    return q.cpu().numpy(), s.cpu().numpy(), int(st.item())


def check(dev, w, kind, expect_status=0):
    print(f"[pack] kind={kind} shape={w.shape}", flush=True)
    q, s, st = gpu_pack(dev, w, kind)
    qo, so, sto = oracle.pack(w, kind)
    assert st == sto == expect_status
    assert np.array_equal(q, qo), f"codes differ at {np.argwhere(q != qo)[:5]}"
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    return q, s


@pytest.mark.parametrize("N,K", [(1024, 5120), (333, 1536), (64, 8960), (40, 13824), (8, 20480),
                                 (5, 16), (3, 37), (17, 24)])
def test_pack_bf16_random_with_outliers(dev, N, K):
    w = oracle.normal_bf16(100 + K, (N, K), 0.02, outlier_rate=1e-3)
    check(dev, w, "bf16")


@pytest.mark.parametrize("N,K", [(256, 1536), (9, 5120), (7, 5), (12, 40000)])
def test_pack_f32_and_f16(dev, N, K):
    f = oracle.normal_f32(200 + K, (N, K), 1.0)
    check(dev, f, "f32")
    check(dev, f.astype(np.float16).view(np.uint16), "f16")


def _special_rows(width):
    ulp = np.array([1], np.uint32).view(F32)[0]
    rows = np.zeros((9, width), F32)
    rows[0, :10] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.0, 126.5, -126.5]
    rows[1, :6] = [254, 5, 7, -5, 1, 3]
    rows[3, 4] = 0.3
    rows[4] = -0.7
    rows[5, :2] = [-3, 1]
    rows[6, :10] = [0.01, -0.02, 0.4, 0.0, 0.015, -0.005, 0.02, 0.0, -0.01, 0.003]
    rows[7, :4] = [127 * ulp, 64 * ulp, 0, -127 * ulp]
    rows[8] = 10 * ulp
    rows[8, 1::2] = 5 * ulp
    return rows


@pytest.mark.parametrize("width", [10, 16, 64])
def test_pack_closed_form_and_denormal_rows(dev, width):
    rows = _special_rows(width)
    q, s = check(dev, rows, "f32")
    assert list(q[0, :10]) == [127, 2, 4, -2, -4, 0, 2, 0, 126, -126] and s[0] == 1.0
    assert list(q[1, :6]) == [127, 2, 4, -2, 0, 2] and s[1] == 2.0
    assert s[2] == 1.0 and not q[2].any()
    assert s[8] == 0.0 and np.all(q[8] == 127)  # denormal scale rounds to 0: +-Inf -> 127


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("width", [6, 32])
def test_pack_nonfinite_sets_status(dev, bad, width):
    w = np.ones((3, width), F32)
    w[1, 2] = bad
    check(dev, w, "f32", expect_status=1)
    wb = oracle.f32_to_bf16(w)
    check(dev, wb, "bf16", expect_status=1)


def test_pack_real_wan_weights_golden(dev):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "wan21_block_tiny_int8.npz"))
    for n in sorted({k[:-2] for k in g.files if k.endswith("_q")}):
        q, s, st = gpu_pack(dev, g[n + "_w"], "f32")
        assert st == 0
        assert np.array_equal(q, g[n + "_q"]), n
        assert np.array_equal(s.view(np.uint32), g[n + "_s"].view(np.uint32)), n


def test_pack_strided_rows_and_mirror_api(dev):
    import torch
    from reels_amd import quantize_frozen_matrix
    w = oracle.normal_bf16(300, (64, 1600), 0.02, outlier_rate=1e-2)
    full = to_dev(w, dev)
    view = full[:, 32:32 + 1536]  # ld_w = 1600 > K = 1536
    qm = quantize_frozen_matrix(view)
    qo, so, _ = oracle.pack(np.ascontiguousarray(w[:, 32:32 + 1536]), "bf16")
    assert np.array_equal(qm.values.cpu().numpy(), qo)
    assert np.array_equal(qm.scales.cpu().numpy(), so)
    bad = full.clone()
    bad[3, 5] = float("nan")
    with pytest.raises(ValueError, match="InexactError"):
        quantize_frozen_matrix(bad)
    assert qm.values.dtype == torch.int8 and qm.shape == (64, 1536)


@pytest.mark.parametrize("N,K", [(13824, 5120), (5120, 13824)])
def test_pack_wan14b_ffn_matrices_full(dev, N, K):
    # full-size 14B FFN weights with 0.1% outliers at 20 sigma, bit-exact
    w = oracle.normal_bf16(400 + N, (N, K), 0.02, outlier_rate=1e-3)
    check(dev, w, "bf16")


def test_pack_near_ties_take_exact_division(dev):
    # rows whose w/s lands on or within a few ulps of a half-integer for arbitrary scales: the
    # kernel's multiply shortcut must hand these to the IEEE division (codes bit-exact)
    rng = np.random.default_rng(77)
    rows = []
    for _ in range(512):
        absmax = np.float32(rng.uniform(1e-3, 10.0))
        s = np.float32(absmax / np.float32(127.0))
        k = rng.integers(-126, 126, size=63).astype(np.float64)
        d = rng.choice([0.0, 1e-7, -1e-7, 2e-6, -2e-6, 3e-5, -3e-5, 1e-3], size=63)
        vals = ((k + 0.5 + d) * np.float64(s)).astype(F32)
        vals = np.clip(vals, -absmax, absmax)
        rows.append(np.concatenate([[absmax], vals]).astype(F32))
    w = np.stack(rows)
    check(dev, w, "f32")
    check(dev, oracle.f32_to_bf16(w), "bf16")


def test_pack_one_launch_beyond_2_32_elements(dev):
    """One pack launch over 860160 rows x 5120 (4.4e9 elements, above 2^32; the 40-layer
    14B weight set is packed in launches of this order), bf16 ~N(0, 0.02) with 0.1% outliers at
    +-20 sigma: the first and last 64 rows and 192 random rows bit-exact against the oracle."""
    import torch
    from reels_amd import _lib
    rows, K = 860160, 5120
    assert rows * K > 2 ** 32
    print(f"[pack] one launch {rows} x {K} = {rows * K} elements", flush=True)
    gen = torch.Generator(device=dev).manual_seed(91)
    w = torch.empty((rows, K), dtype=torch.bfloat16, device=dev)
    step = 32768
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        c = torch.randn((r1 - r0, K), generator=gen, device=dev).mul_(0.02)
        u = torch.rand((r1 - r0, K), generator=gen, device=dev)
        c = torch.where(u < 0.001, torch.where(u < 0.0005, -0.4, 0.4), c)
        w[r0:r1] = c.to(torch.bfloat16)
        del c, u
    q = torch.empty((rows, K), dtype=torch.int8, device=dev)
    s = torch.empty((rows,), dtype=torch.float32, device=dev)
    st = torch.full((1,), 7, dtype=torch.int32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.lib().reels_hip_i8_pack(p(w), _lib.BF16, rows, K, K, p(q), p(s), p(st),
                                      ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _lib.check("reels_hip_i8_pack", rc)
    torch.cuda.synchronize(dev)
    assert int(st.item()) == 0
    rng = np.random.default_rng(92)
    idx = np.unique(np.concatenate([np.arange(64), np.arange(rows - 64, rows),
                                    rng.integers(0, rows, 192)]))
    ix = torch.as_tensor(idx, device=dev)
    wb = w[ix].view(torch.int16).cpu().numpy().view(np.uint16)
    qg, sg = q[ix].cpu().numpy(), s[ix].cpu().numpy()
    del w, q, s
    torch.cuda.empty_cache()
    qo, so, sto = oracle.pack(wb, "bf16")
    assert sto == 0
    assert np.array_equal(qg, qo), f"codes differ in rows {idx[np.unique(np.argwhere(qg != qo)[:, 0])][:5]}"
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32))
