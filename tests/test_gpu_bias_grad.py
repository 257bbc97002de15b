"""GPU parity of the trainable bias's gradient (reels_hip_i8lora_bwd_bias, _f16, _f32).

LoRALinear trains its bias when train_bias is set (src/layers/lora.jl:37-38); the forward adds it
with mixed_add (lora.jl:64-67, src/layers/linear.jl:7-13), whose pullback sums dy over the
tokens. The library sums in f32 in a fixed order, so the result is checked against the f64
oracle (oracle.bias_gradient) with a tolerance of 1e-5 (f32 sums of up to 32760 terms), and
bitwise between repeated calls and between the two places it is computed: inside the dB gradient
pass (dB requested) and in a pass of its own (dB not requested, r = 0).
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests._util import assert_parity, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _case(M, K, N, r, seed, elt="bf16"):
    x = oracle.normal_bf16(seed + 1, (M, K), 1.0)
    w = oracle.normal_bf16(seed + 2, (N, K), 0.02)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    A = oracle.normal_bf16(seed + 3, (K, r), 0.01) if r else None
    B = oracle.normal_bf16(seed + 4, (r, N), 0.01) if r else None
    dy = oracle.normal_bf16(seed + 5, (M, N), 1.0)
    if elt == "f16":
        cv = lambda a: None if a is None else oracle.f32_to_f16(oracle.bf16_to_f32(a))
        x, A, B, dy = cv(x), cv(A), cv(B), cv(dy)
    elif elt == "f32":
        cv = lambda a: None if a is None else oracle.bf16_to_f32(a)
        x, A, B, dy = cv(x), cv(A), cv(B), cv(dy)
    return dict(x=x, q=q, s=s, A=A, B=B, dy=dy, M=M, K=K, N=N, r=r, elt=elt)


def _dev_t(a, dev, elt):
    import torch
    if a is None:
        return None
    if elt == "bf16":
        return to_dev(a, dev)
    if elt == "f16":
        return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _bwd(dev, cs, want_dx=True, want_dA=True, want_dB=True):
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    e = cs["elt"]
    x, A, B, dy = (_dev_t(cs[k], dev, e) for k in ("x", "A", "B", "dy"))
    c = float(np.float32(16.0) / np.float32(cs["r"])) if cs["r"] else 0.0
    res = i8lora_backward(dy, x, W, A, B, c, want_dx=want_dx, want_dA=want_dA, want_dB=want_dB,
                          want_dbias=True)
    torch.cuda.synchronize(dev)
    return res


@pytest.mark.parametrize("M,K,N,r,label", [
    (4096, 1536, 1536, 32, "dequantized-weight path"),
    (77, 5120, 5120, 32, "few-token path"),
    (333, 5120, 5120, 32, "split-reduction path"),
    (1000, 768, 2048, 160, "rank above one chunk of 128"),
    (300, 100, 100, 4, "generic path (K, N not multiples of 16)"),
    (130, 256, 384, 0, "base-only linear"),
])
def test_bias_gradient_matches_oracle_and_is_reproducible(dev, M, K, N, r, label):
    print(f"[bias] {label}: M={M} K={K} N={N} r={r}", flush=True)
    cs = _case(M, K, N, r, seed=700 + M)
    res = _bwd(dev, cs)
    dbias = res[3].cpu().numpy()
    assert_parity(dbias, oracle.bias_gradient(cs["dy"]), f"{label} dbias", tol=TOL)
    again = _bwd(dev, cs)[3].cpu().numpy()
    assert np.array_equal(dbias.view(np.uint32), again.view(np.uint32)), "not reproducible"
    # computed in a pass of its own (no dB pass to ride on): the same bits
    alone = _bwd(dev, cs, want_dx=False, want_dA=False, want_dB=False)[3].cpu().numpy()
    assert np.array_equal(dbias.view(np.uint32), alone.view(np.uint32)), \
        "fused and standalone column sums differ"


@pytest.mark.parametrize("elt", ["f16", "f32"])
def test_bias_gradient_other_precisions(dev, elt):
    cs = _case(2048, 512, 1024, 16, seed=760, elt=elt)
    res = _bwd(dev, cs)
    dbias = res[3].cpu().numpy()
    assert_parity(dbias, oracle.bias_gradient(cs["dy"], elt=elt), f"{elt} dbias", tol=TOL)
    alone = _bwd(dev, cs, want_dx=False, want_dA=False, want_dB=False)[3].cpu().numpy()
    assert np.array_equal(dbias.view(np.uint32), alone.view(np.uint32))


def test_bias_gradient_other_outputs_unchanged(dev):
    """reels_hip_i8lora_bwd_bias gives reels_hip_i8lora_bwd's dx, dA, dB bit for bit."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward
    cs = _case(2048, 1536, 1536, 32, seed=780)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x, A, B, dy = (to_dev(cs[k], dev) for k in ("x", "A", "B", "dy"))
    a = i8lora_backward(dy, x, W, A, B, 0.5)
    b = i8lora_backward(dy, x, W, A, B, 0.5, want_dbias=True)
    torch.cuda.synchronize(dev)
    for t0, t1 in zip(a, b[:3]):
        assert torch.equal(t0.view(torch.int16) if t0.dtype == torch.bfloat16 else t0.view(torch.int32),
                           t1.view(torch.int16) if t1.dtype == torch.bfloat16 else t1.view(torch.int32))


def test_bias_gradient_empty_tokens_is_zero(dev):
    import torch
    from reels_amd import _lib
    N = 64
    dbias = torch.full((N,), 7.0, dtype=torch.float32, device=dev)
    dy = torch.empty((0, N), dtype=torch.bfloat16, device=dev)
    q = torch.zeros((N, 32), dtype=torch.int8, device=dev)
    s = torch.ones((N,), dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.lib().reels_hip_i8lora_bwd_bias(p(dy), None, None, p(q), p(s), None, None, 0, 32,
                                              N, 0, 0.0, None, None, None, p(dbias), None, 0,
                                              None)
    _lib.check("reels_hip_i8lora_bwd_bias", rc)
    torch.cuda.synchronize(dev)
    assert torch.count_nonzero(dbias).item() == 0


def test_bias_gradient_wan14b_full_size(dev):
    """Wan-14B q projection at 32760 tokens: sampled columns against the f64 sums, every column
    against the exact doubling identity dbias(2 dy) = 2 dbias(dy)."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward
    M, K, N, r = 32760, 5120, 5120, 32
    print(f"[bias] wan14b M={M} K={K} N={N} r={r}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    dy = torch.randn((M, N), generator=g, device=dev).to(torch.bfloat16)
    W = QuantizedMatrix(torch.randint(-127, 128, (N, K), generator=g, device=dev,
                                      dtype=torch.int8),
                        torch.full((N,), 0.02 / 127, device=dev))
    A = (0.01 * torch.randn((K, r), generator=g, device=dev)).to(torch.bfloat16)
    B = (0.01 * torch.randn((r, N), generator=g, device=dev)).to(torch.bfloat16)
    db = i8lora_backward(dy, x, W, A, B, 1.0, want_dx=False, want_dbias=True)[3]
    db2 = i8lora_backward(dy * 2, x, W, A, B, 1.0, want_dx=False, want_dbias=True)[3]
    torch.cuda.synchronize(dev)
    assert torch.equal(db2, 2 * db)
    cols = np.array([0, 1, 127, 128, 2047, 4095, 5119])
    dyc = dy[:, torch.as_tensor(cols, device=dev)].contiguous()
    dyn = dyc.view(torch.int16).cpu().numpy().view(np.uint16)
    assert_parity(db.cpu().numpy()[cols], oracle.bias_gradient(dyn), "wan14b dbias", tol=TOL)


def test_autograd_bias_gradient_is_the_library_result(dev):
    """The autograd rule's bias gradient comes from the library's column sums."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward
    from reels_amd.layers import I8LoRALinearFunction
    cs = _case(640, 512, 768, 16, seed=790)
    W = QuantizedMatrix(to_dev(cs["q"], dev, "raw"), to_dev(cs["s"], dev, "raw"))
    x, A, B, dy = (to_dev(cs[k], dev) for k in ("x", "A", "B", "dy"))
    bias = torch.zeros((cs["N"],), dtype=torch.float32, device=dev, requires_grad=True)
    y = I8LoRALinearFunction.apply(x, A, B, W.values, W.scales, bias.to(torch.bfloat16), 1.0)
    y.backward(dy)
    want = i8lora_backward(dy, x, W, A, B, 1.0, want_dbias=True)[3]
    torch.cuda.synchronize(dev)
    assert torch.equal(bias.grad, want.to(torch.bfloat16).float())
