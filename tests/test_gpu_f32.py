"""GPU parity of the fp32 entry points (reels_hip_i8lora_fwd_f32 / _bwd_f32 / gelu_tanh_f32): the
reference's Float32 compute with int8 frozen weights (_dequantize_for_compute with T = Float32,
src/layers/quantization.jl:61-64; lora_forward / lora_backward in Float32, lora.jl:56-118),
checked against the f64 oracle (elt="f32") on the same seeded float32 inputs.

Tolerance: fp32 compute with f32 sums over at most 5120 terms keeps the error near 2^-24 times a
small multiple of sqrt(K); the bar here is normwise and elementwise 1e-5 (tests/_util.assert_parity
with tol=1e-5), a thousand times tighter than the bf16 bar. Covered: the fp32-MFMA GEMM (K, N
multiples of 4, aligned), the fp32 projection and split-M gradient kernels, the generic kernels
(K or N not a multiple of 4), and the mirror API with autograd."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity

pytestmark = pytest.mark.gpu
TOL = 1e-5


def f32v(seed, shape, sigma):
    """Seeded N(0, sigma^2) float32 values with all 24 significant bits in use."""
    return (np.random.default_rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def make_case(M, K, N, r, alpha, seed=0, bias=False, w_sigma=0.02, ab_sigma=0.01):
    x = f32v(seed + 1, (M, K), 1.0)
    w = f32v(seed + 2, (N, K), w_sigma)
    q, s, st = oracle.pack(w, "f32")
    assert st == 0
    A = f32v(seed + 3, (K, r), ab_sigma) if r else None
    B = f32v(seed + 4, (r, N), ab_sigma) if r else None
    dy = f32v(seed + 5, (M, N), 1.0)
    b = f32v(seed + 6, (N,), 0.1) if bias else None
    c = float(np.float32(alpha) / np.float32(r)) if r else 0.0
    return dict(x=x, q=q, s=s, A=A, B=B, dy=dy, bias=b, c=c, M=M, K=K, N=N, r=r)


def todev(a, d):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(d)


def run_gpu(d, cs):
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    W = QuantizedMatrix(todev(cs["q"], d), todev(cs["s"], d), torch.float32)
    x = todev(cs["x"], d)
    A = todev(cs["A"], d) if cs["r"] else None
    B = todev(cs["B"], d) if cs["r"] else None
    bias = todev(cs["bias"], d) if cs["bias"] is not None else None
    y, h = i8lora_forward(x, W, A, B, bias, cs["c"], save_h=cs["r"] > 0)
    assert y.dtype == torch.float32
    dx, dA, dB = i8lora_backward(todev(cs["dy"], d), x, W, A, B, cs["c"], h=h)
    assert dx.dtype == torch.float32
    torch.cuda.synchronize(d)
    out = dict(y=y.cpu().numpy(), dx=dx.cpu().numpy())
    if h is not None:
        out["h"] = h.cpu().numpy()
        out["dA"], out["dB"] = dA.cpu().numpy(), dB.cpu().numpy()
    return out


def check(d, cs, label):
    print(f"[f32] {label}: M={cs['M']} K={cs['K']} N={cs['N']} r={cs['r']}", flush=True)
    g = run_gpu(d, cs)
    y, h = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], cs["bias"],
                               elt="f32")
    assert_parity(g["y"], y, f"{label} y", tol=TOL)
    if cs["r"]:
        assert_parity(g["h"], h, f"{label} h", tol=TOL)
        ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                                   elt="f32")
        assert_parity(g["dA"], ref["dA"], f"{label} dA", tol=TOL)
        assert_parity(g["dB"], ref["dB"], f"{label} dB", tol=TOL)
    else:
        z = np.zeros((cs["K"], 0), np.float32), np.zeros((0, cs["N"]), np.float32)
        ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], z[0], z[1], 0.0,
                                   want=("dx",), elt="f32")
    assert_parity(g["dx"], ref["dx"], f"{label} dx", tol=TOL)
    return g


@pytest.mark.parametrize("M,K,N,r,bias", [
    (1024, 1536, 1536, 16, False),  # the CPU-runnable workload's shape
    (333, 512, 768, 16, True),      # bias, partial tiles in every dimension
    (300, 384, 320, 128, True),     # rank 128
    (130, 1536, 8960, 32, False),   # FFN-in shape
    (77, 100, 36, 3, True),         # rank 3, K not a multiple of the 32-wide k-step
    (65, 48, 80, 16, False),        # a single partial k-step
    (50, 256, 256, 0, True),        # base-only linear with bias
    (40, 22, 20, 5, True),          # K not a multiple of 4: generic kernels
    (33, 64, 30, 2, False),         # N not a multiple of 4: generic kernels
])
def test_f32_shapes(dev, M, K, N, r, bias):
    check(dev, make_case(M, K, N, r, float(r) if r else 1.0, seed=700 + M + K + N + r, bias=bias),
          f"f32 {M}x{K}x{N}r{r}")


def test_f32_wan14b_q_sampled(dev):
    # 2048 tokens of the 14B q projection; rows and columns sampled against the oracle
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    cs = make_case(2048, 5120, 5120, 32, 32.0, seed=750)
    print("[f32] 2048x5120x5120 r32 (sampled)", flush=True)
    W = QuantizedMatrix(todev(cs["q"], dev), todev(cs["s"], dev), torch.float32)
    x, A, B = todev(cs["x"], dev), todev(cs["A"], dev), todev(cs["B"], dev)
    y, h = i8lora_forward(x, W, A, B, None, cs["c"], save_h=True)
    dx, dA, dB = i8lora_backward(todev(cs["dy"], dev), x, W, A, B, cs["c"], h=h)
    torch.cuda.synchronize(dev)
    rows = np.array([0, 1, 127, 128, 1023, 2000, 2047])
    yr, hr = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], rows=rows,
                                 elt="f32")
    ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                               rows=rows, kcols=[0, 77, 5119], ncols=[1, 4096, 5119], elt="f32")
    assert_parity(y.cpu().numpy()[rows], yr, "f32 14b-q y (sampled rows)", tol=TOL)
    assert_parity(h.cpu().numpy()[rows], hr, "f32 14b-q h (sampled rows)", tol=TOL)
    assert_parity(dx.cpu().numpy()[rows], ref["dx"], "f32 14b-q dx (sampled rows)", tol=TOL)
    assert_parity(dA.cpu().numpy()[[0, 77, 5119]], ref["dA"], "f32 14b-q dA (sampled)", tol=TOL)
    assert_parity(dB.cpu().numpy()[:, [1, 4096, 5119]], ref["dB"], "f32 14b-q dB (sampled)",
                  tol=TOL)
    # size-independent: scaling x by 2 scales y, h, dA exactly (powers of two are exact in f32)
    y2, h2 = i8lora_forward(x * 2, W, A, B, None, cs["c"], save_h=True)
    torch.cuda.synchronize(dev)
    assert torch.equal(y2, y * 2) and torch.equal(h2, h * 2)


def test_f32_backward_bitwise_reproducible(dev):
    cs = make_case(600, 512, 768, 32, 32.0, seed=760)
    a, b = run_gpu(dev, cs), run_gpu(dev, cs)
    for k in ("y", "h", "dx", "dA", "dB"):
        assert np.array_equal(a[k], b[k]), k


def test_f32_mirror_api_autograd_and_transfer(dev):
    import torch
    from reels_amd import (I8LoRALinearFunction, LoRALinear, frozen_weight_transfer,
                           lora_backward, lora_forward, move_weight)
    t = frozen_weight_transfer("hip", "fp32", quantization="int8")
    w = todev(f32v(770, (384, 256), 0.02), dev)
    W = move_weight(w, t)
    assert W.compute_dtype == torch.float32
    q, s, _ = oracle.pack(w.cpu().numpy(), "f32")
    assert np.array_equal(W.values.cpu().numpy(), q)
    layer = LoRALinear(W, rank=16, alpha=32.0)
    assert layer.A.dtype == torch.float32 and layer.B.dtype == torch.float32
    layer.B = todev(f32v(771, (16, 384), 0.05), dev)
    x = todev(f32v(772, (3, 50, 256), 1.0), dev)
    y, h = lora_forward(layer, x, save_h=True)
    assert y.dtype == torch.float32 and y.shape == (3, 50, 384)
    dy = todev(f32v(773, (3, 50, 384), 1.0), dev)
    g = lora_backward(layer, x, dy, h=h)
    A = layer.A.clone().requires_grad_(True)
    B = layer.B.clone().requires_grad_(True)
    xx = x.reshape(-1, 256).clone().requires_grad_(True)
    out = I8LoRALinearFunction.apply(xx, A, B, W.values, W.scales, None, layer.lora_scale)
    out.backward(dy.reshape(-1, 384))
    torch.cuda.synchronize(dev)
    assert torch.equal(out.reshape(3, 50, 384), y)
    assert torch.equal(xx.grad.reshape(3, 50, 256), g["dx"])
    assert torch.equal(A.grad, g["A"]) and torch.equal(B.grad, g["B"])
    # the forward against the oracle through the layer API
    yo, _ = oracle.lora_forward(x.reshape(-1, 256).cpu().numpy(), q, s, layer.A.cpu().numpy(),
                                layer.B.cpu().numpy(), layer.lora_scale, elt="f32")
    assert_parity(y.reshape(-1, 384).cpu().numpy(), yo, "f32 layer y", tol=TOL)


@pytest.mark.parametrize("n", [1, 1000, 65537])
def test_f32_gelu_tanh(dev, n):
    import torch
    from reels_amd import gelu_tanh, gelu_tanh_backward
    xs, dys = f32v(780 + n, (n,), 2.0), f32v(781 + n, (n,), 1.0)
    y = gelu_tanh(todev(xs, dev)).cpu().numpy()
    dx = gelu_tanh_backward(todev(xs, dev), todev(dys, dev)).cpu().numpy()
    assert y.dtype == np.float32 and dx.dtype == np.float32
    yo, dxo = oracle.gelu_tanh(xs, elt="f32"), oracle.gelu_tanh_backward(xs, dys, elt="f32")
    # Device and host f32 tanh may differ in their last bits (t = tanh(...) within a couple of
    # ulps of magnitude <= 1, i.e. 2^-23 absolute). For x < 0, 1 + t cancels, so y = 0.5 x (1 + t)
    # inherits an absolute error up to 0.5 |x| 2^-23 (about 16 ulps of y near x = -2), and the
    # derivative 0.5 (1 + t) + 0.5 x (1 - t^2) k (1 + 3 a x^2) one up to
    # (1 + |x| + 0.14 |x|^3) 2^-23 times |dy|. Allowed: 8 ulps of the result, or those bounds.
    x64 = np.abs(xs.astype(np.float64))
    for got, want, what in ((y, yo, "y"), (dx, dxo, "dx")):
        e = np.abs(got.astype(np.float64) - want.astype(np.float64))
        ok = e <= 8 * np.spacing(np.abs(want)).astype(np.float64) + 2.0 ** -40
        if what == "y":
            ok |= e <= x64 * 2.0 ** -22
        else:
            ok |= e <= (1 + x64 + 0.14 * x64 ** 3) * 2.0 ** -22 * np.abs(dys.astype(np.float64))
        bad = np.flatnonzero(~ok)
        assert bad.size == 0, (what, [(int(i), float(got[i]), float(want[i]), float(xs[i]))
                                      for i in bad[:6]])
