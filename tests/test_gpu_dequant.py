"""GPU parity of the dequantization for compute (reels_hip_i8_dequant; _dequantize_for_compute /
_host_dequantize, src/layers/quantization.jl:25-29, 54-64): every element bit-identical to the
oracle's dequant (f32 fl32(q s), f16 f16(q f16(s)), bf16 bf16(fl32(q s))), plain and transposed.
The bf16 forms are the weights the LoRA linear's bf16 GEMMs multiply."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

KIND = {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16}


def _packed(seed, N, K, sigma=0.02):
    w = oracle.normal_bf16(seed, (N, K), sigma, outlier_rate=1e-3)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    return q, s


def _gpu_dequant(dev, q, s, mode, transpose, ld=None):
    import torch
    from reels_amd import QuantizedMatrix
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[mode]
    N, K = q.shape
    qd = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    if ld is not None:  # a strided view: rows of ld codes, the first K used
        wide = torch.zeros((N, ld), dtype=torch.int8, device=dev)
        wide[:, :K] = qd
        qd = wide[:, :K]
    W = QuantizedMatrix(qd, torch.from_numpy(s).to(dev), dt)
    out = W.dequantize(transpose=transpose)
    torch.cuda.synchronize(dev)
    o = out.cpu()
    return o.numpy() if mode == "f32" else o.view(torch.int16).numpy().view(np.uint16)


def _check(dev, q, s, mode, transpose, ld=None):
    print(f"[dequant] {mode} transpose={transpose} shape={q.shape} ld={ld}", flush=True)
    got = _gpu_dequant(dev, q, s, mode, transpose, ld)
    ref = oracle.dequant(q, s, mode)
    if transpose:
        ref = np.ascontiguousarray(ref.T)
    assert got.shape == ref.shape
    gb = got.view(np.uint32 if mode == "f32" else np.uint16)
    rb = ref.view(np.uint32 if mode == "f32" else np.uint16)
    assert np.array_equal(gb, rb), f"{mode}: first differences at {np.argwhere(gb != rb)[:5]}"


# (N, K): fast bf16 row kernel (K % 16 == 0), fast transpose (N, K % 64 == 0), generic paths
# (192, 320): five 64-column tiles, so the transpose's second block holds one tile of its four
@pytest.mark.parametrize("N,K", [(256, 1536), (1024, 5120), (128, 64), (333, 1536), (7, 5),
                                 (65, 48), (40, 8960), (192, 320)])
@pytest.mark.parametrize("mode", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("transpose", [False, True])
def test_dequant_bit_exact(dev, N, K, mode, transpose):
    q, s = _packed(500 + N + K, N, K)
    _check(dev, q, s, mode, transpose)


def test_dequant_full_14b_ffn_weight_bf16(dev):
    # the largest weight the LoRA linear dequantizes: 14B ffn.0, 13824 x 5120, both layouts
    q, s = _packed(777, 13824, 5120)
    _check(dev, q, s, "bf16", False)
    _check(dev, q, s, "bf16", True)


@pytest.mark.parametrize("mode", ["bf16", "f16", "f32"])
def test_dequant_strided_rows_and_special_scales(dev, mode):
    q, s = _packed(901, 64, 128)
    _check(dev, q, s, mode, False, ld=160)   # row stride 160 (fast-path alignment kept)
    _check(dev, q, s, mode, True, ld=136)    # row stride not a multiple of 16: generic kernel
    # codes with special scales (dequantization takes any float32 scale): 0, denormal, f16
    # denormal, 2362 and 65504 whose products overflow f16 to +-Inf (no NaN: every scale finite)
    ulp = float(np.array([1], np.uint32).view(np.float32)[0])
    ss = np.array([0.0, 3 * ulp, 1e-6, 2362.0, 65504.0, 1.0], np.float32)
    qq = np.random.default_rng(902).integers(-127, 128, size=(6, 48)).astype(np.int8)
    qq[:, :3] = [-127, 0, 127]
    _check(dev, qq, ss, mode, False)
    _check(dev, qq, ss, mode, True)
