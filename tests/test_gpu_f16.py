"""GPU parity of the fp16 entry points (reels_hip_i8lora_fwd_f16 / _bwd_f16 / gelu_tanh_f16):
the reference's own int8 compute precision (Float16; src/layers/quantization.jl:61-62,
lora.jl:56-118, linear.jl:61-68), checked against the f64 oracle on the same seeded binary16
inputs (oracle elt="f16") at the tolerance of tests/_util.assert_parity (normwise and
elementwise 1e-2). Every path is covered: the dequantized-weight GEMM (K, N multiples of 64),
both int8-weight GEMMs, the generic kernels, and the mirror API with autograd."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, rel_errors

pytestmark = pytest.mark.gpu


def f16(seed, shape, sigma, outlier_rate=0.0):
    """Seeded N(0, sigma^2) values as binary16 patterns (uint16)."""
    v = oracle.bf16_to_f32(oracle.normal_bf16(seed, shape, 1.0, outlier_rate=outlier_rate))
    v = v * np.float32(sigma) * np.float32(1.0 + 2 ** -9)  # not bf16-representable any more
    return v.astype(np.float16).view(np.uint16)


def dev16(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16).to(dev)


def host16(t):
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f32(bits):
    return oracle.f16_to_f32(bits)


def make_case(M, K, N, r, alpha, seed=0, bias=False, w_sigma=0.02, ab_sigma=0.01, dy_sigma=1.0):
    x = f16(seed + 1, (M, K), 1.0)
    w = f16(seed + 2, (N, K), w_sigma, outlier_rate=1e-3)
    q, s, st = oracle.pack(f32(w), "f32")
    assert st == 0
    A = f16(seed + 3, (K, r), ab_sigma) if r else None
    B = f16(seed + 4, (r, N), ab_sigma) if r else None
    dy = f16(seed + 5, (M, N), dy_sigma)
    b = f16(seed + 6, (N,), 0.1) if bias else None
    c = float(np.float32(alpha) / np.float32(r)) if r else 0.0
    return dict(x=x, q=q, s=s, A=A, B=B, dy=dy, bias=b, c=c, M=M, K=K, N=N, r=r)


def run_gpu(dev, cs):
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    W = QuantizedMatrix(torch.from_numpy(cs["q"]).to(dev), torch.from_numpy(cs["s"]).to(dev),
                        torch.float16)
    x = dev16(cs["x"], dev)
    A = dev16(cs["A"], dev) if cs["r"] else None
    B = dev16(cs["B"], dev) if cs["r"] else None
    bias = dev16(cs["bias"], dev) if cs["bias"] is not None else None
    y, h = i8lora_forward(x, W, A, B, bias, cs["c"], save_h=cs["r"] > 0)
    assert y.dtype == torch.float16
    dx, dA, dB = i8lora_backward(dev16(cs["dy"], dev), x, W, A, B, cs["c"], h=h)
    assert dx.dtype == torch.float16
    torch.cuda.synchronize(dev)
    out = dict(y=f32(host16(y)), dx=f32(host16(dx)))
    if h is not None:
        out["h"] = f32(host16(h))
        out["dA"], out["dB"] = dA.cpu().numpy(), dB.cpu().numpy()
    return out


def check(dev, cs, label):
    print(f"[f16] {label}: M={cs['M']} K={cs['K']} N={cs['N']} r={cs['r']}", flush=True)
    g = run_gpu(dev, cs)
    y, h = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], cs["bias"],
                               elt="f16")
    assert_parity(g["y"], y, f"{label} y")
    if cs["r"]:
        assert_parity(g["h"], h, f"{label} h")
        ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                                   elt="f16")
        assert_parity(g["dA"], ref["dA"], f"{label} dA")
        assert_parity(g["dB"], ref["dB"], f"{label} dB")
    else:
        z = np.zeros((cs["K"], 0), np.uint16), np.zeros((0, cs["N"]), np.uint16)
        ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], z[0], z[1], 0.0,
                                   want=("dx",), elt="f16")
    assert_parity(g["dx"], ref["dx"], f"{label} dx")
    return g


@pytest.mark.parametrize("M,K,N,r,bias", [
    (1024, 1536, 1536, 16, False),  # the CPU-runnable workload's shape, dequantized-weight path
    (333, 512, 768, 16, True),      # bias, partial tiles
    (300, 384, 320, 128, True),     # rank 128
    (130, 1536, 8960, 32, False),   # FFN-in shape
    (200, 512, 528, 32, True),      # int8-weight GEMM forward, general dX
    (200, 528, 512, 16, False),     # general forward, int8-weight GEMM dX
    (65, 48, 80, 16, False),        # K not a multiple of 64
    (50, 256, 256, 0, True),        # base-only linear with bias
    (40, 24, 20, 5, True),          # rank 5: generic kernels
    (1100, 2048, 2560, 32, True),   # split reductions in both GEMMs
    (512, 1536, 1536, 32, False),   # row-wave tiles of 64 rows x 64 tokens in both directions
    (77, 1536, 1536, 16, True),     # row-wave tiles on part of the GPU (72 tiles)
])
def test_f16_shapes(dev, M, K, N, r, bias):
    check(dev, make_case(M, K, N, r, float(r) if r else 1.0, seed=900 + M + K + N + r, bias=bias),
          f"f16 {M}x{K}x{N}r{r}")


def test_f16_larger_block_sampled(dev):
    # 4096 tokens of the 14B q projection: rows sampled against the oracle
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    cs = make_case(4096, 5120, 5120, 32, 32.0, seed=950)
    print("[f16] 4096x5120x5120 r32 (sampled rows)", flush=True)
    W = QuantizedMatrix(torch.from_numpy(cs["q"]).to(dev), torch.from_numpy(cs["s"]).to(dev),
                        torch.float16)
    x, A, B = dev16(cs["x"], dev), dev16(cs["A"], dev), dev16(cs["B"], dev)
    y, h = i8lora_forward(x, W, A, B, None, cs["c"], save_h=True)
    dx, dA, dB = i8lora_backward(dev16(cs["dy"], dev), x, W, A, B, cs["c"], h=h)
    torch.cuda.synchronize(dev)
    rows = np.array([0, 1, 255, 256, 2047, 4000, 4095])
    yr, _ = oracle.lora_forward(cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"], rows=rows,
                                elt="f16")
    ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                               rows=rows, kcols=[0, 77, 5119], ncols=[1, 4096, 5119], elt="f16")
    assert_parity(f32(host16(y))[rows], yr, "f16 14b-q y (sampled rows)")
    assert_parity(f32(host16(dx))[rows], ref["dx"], "f16 14b-q dx (sampled rows)")
    assert_parity(dA.cpu().numpy()[[0, 77, 5119]], ref["dA"], "f16 14b-q dA (sampled)")
    assert_parity(dB.cpu().numpy()[:, [1, 4096, 5119]], ref["dB"], "f16 14b-q dB (sampled)")


def test_f16_mirror_api_autograd_and_transfer(dev):
    import torch
    from reels_amd import (I8LoRALinearFunction, LoRALinear, frozen_weight_transfer,
                           lora_backward, lora_forward, move_weight)
    t = frozen_weight_transfer("hip", "fp16", quantization="int8")
    w = dev16(f16(970, (384, 256), 0.02), dev)
    W = move_weight(w, t)
    assert W.compute_dtype == torch.float16
    q, s, _ = oracle.pack(f32(host16(w)), "f32")
    assert np.array_equal(W.values.cpu().numpy(), q)
    layer = LoRALinear(W, rank=16, alpha=32.0)
    assert layer.A.dtype == torch.float16 and layer.B.dtype == torch.float16
    layer.B = dev16(f16(971, (16, 384), 0.05), dev)
    x = dev16(f16(972, (3, 50, 256), 1.0), dev)
    y, h = lora_forward(layer, x, save_h=True)
    assert y.dtype == torch.float16 and y.shape == (3, 50, 384)
    dy = dev16(f16(973, (3, 50, 384), 1.0), dev)
    g = lora_backward(layer, x, dy, h=h)
    A = layer.A.clone().requires_grad_(True)
    B = layer.B.clone().requires_grad_(True)
    xx = x.reshape(-1, 256).clone().requires_grad_(True)
    out = I8LoRALinearFunction.apply(xx, A, B, W.values, W.scales, None, layer.lora_scale)
    out.backward(dy.reshape(-1, 384))
    torch.cuda.synchronize(dev)
    assert torch.equal(out.reshape(3, 50, 384).view(torch.int16), y.view(torch.int16))
    assert torch.equal(xx.grad.reshape(3, 50, 256).view(torch.int16), g["dx"].view(torch.int16))
    assert torch.equal(A.grad, g["A"].to(torch.float16))
    assert torch.equal(B.grad, g["B"].to(torch.float16))


@pytest.mark.parametrize("n", [1, 1000, 65537])
def test_f16_gelu_tanh(dev, n):
    from reels_amd import gelu_tanh, gelu_tanh_backward
    xb, dyb = f16(980 + n, (n,), 2.0), f16(981 + n, (n,), 1.0)
    y = host16(gelu_tanh(dev16(xb, dev)))
    dx = host16(gelu_tanh_backward(dev16(xb, dev), dev16(dyb, dev)))
    yo, dxo = oracle.gelu_tanh(xb, elt="f16"), oracle.gelu_tanh_backward(xb, dyb, elt="f16")
    # Device and host f32 tanh may differ in the last bits: one binary16 ulp, or 2^-22 absolute
    # in the subnormal range (quantum 2^-24). For x < -2 the derivative
    # 0.5 (1 + t) + 0.5 x (1 - t^2) k (1 + 3 a x^2) cancels in f32 (t = tanh(...) -> -1; the
    # reference differentiates the same f32 formula): its absolute error there is up to
    # ~17 * 2^-23 * |dy| against the oracle's f64, so 2^-18 |dy| is allowed in that region.
    xf, dyf = f32(xb).astype(np.float64), f32(dyb).astype(np.float64)
    for got, want, what in ((y, yo, "y"), (dx, dxo, "dx")):
        d = np.abs(got.astype(np.int32) - want.astype(np.int32))
        e = np.abs(f32(got).astype(np.float64) - f32(want).astype(np.float64))
        close = e <= 2.0 ** -22
        if what == "dx":
            close |= (xf < -2) & (e <= 2.0 ** -18 * np.abs(dyf))
        bad = np.flatnonzero(~((d <= 1) | close))
        assert bad.size == 0, (what, [(int(i), hex(got[i]), hex(want[i]), float(f32(xb)[i]),
                                       float(f32(dyb)[i])) for i in bad[:6]])


@pytest.mark.parametrize("dy_sigma", [1e-3, 1e-4])
@pytest.mark.parametrize("M,K,N,r", [
    (96, 256, 320, 8),     # rank not a multiple of 16
    (200, 512, 528, 32),   # N % 64 != 0: int8-weight dX GEMM over a reduction of 528
    (200, 528, 512, 16),   # K % 64 != 0, N % 64 == 0: int8-weight dX GEMM over 512
    (65, 48, 80, 16),      # K, N not multiples of 64
    (40, 24, 20, 2),       # ragged: generic kernels
])
def test_small_output_gradients_keep_binary16_precision(dev, M, K, N, r, dy_sigma):
    """Output gradients of 1e-3 and 1e-4 times per-channel scales of ~1e-4 give dy * s far below
    binary16's normal range (6.1e-5). The reference multiplies dy by its binary16 weight
    Float16(q) * Float16(s) (quantization.jl:61-62, 75-76) with f32 accumulation, so dx keeps
    binary16's relative precision; so must every path here (the bar is the usual 1e-2)."""
    cs = make_case(M, K, N, r, float(r), seed=M + K + N + r + int(1 / dy_sigma), dy_sigma=dy_sigma)
    print(f"[f16] small dy sigma={dy_sigma:g}: M={M} K={K} N={N} r={r}", flush=True)
    g = run_gpu(dev, cs)
    ref = oracle.lora_backward(cs["dy"], cs["x"], cs["q"], cs["s"], cs["A"], cs["B"], cs["c"],
                               elt="f16")
    assert_parity(g["dx"], ref["dx"], f"small dy {dy_sigma:g} {M}x{K}x{N}r{r} dx")
    assert_parity(g["dB"], ref["dB"], f"small dy {dy_sigma:g} {M}x{K}x{N}r{r} dB")
    if dy_sigma >= 1e-3:
        # at 1e-4, u = f16(dy B^T) (~4e-6) is itself a binary16 subnormal: the reference's f16
        # B' * dy (lora.jl:113) rounds it the same way, the f64 oracle does not
        assert_parity(g["dA"], ref["dA"], f"small dy {dy_sigma:g} {M}x{K}x{N}r{r} dA")
