"""The FFN's GELU fused with its projections: the first projection's forward followed by the GELU
(reels_hip_i8lora_fwd_gelu) and the second projection's backward with the GELU's pullback
(reels_hip_i8lora_bwd_gelu), each with its f16 form. Where the GEMM is the unsplit
dequantized-weight GEMM the GELU (or its pullback) runs in its epilogue; elsewhere (few tokens,
split reductions) the separate pass runs after it. Either way every output must equal the two
separate calls bit for bit: the linear, then gelu_tanh (or the linear's backward, then
gelu_tanh_backward). The separate calls are checked against the oracle in test_gpu_lora.py
(shapes, ranks, test_gelu_tanh); one case here also samples rows of the composition against the
oracle."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_f32, to_dev

pytestmark = pytest.mark.gpu


def _case(dev, M, K, N, r, seed, dt):
    import torch
    from reels_amd import QuantizedMatrix
    w = oracle.normal_bf16(seed, (N, K), 0.02)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    cast = (lambda a: to_dev(a, dev)) if dt == "bf16" else \
        (lambda a: torch.from_numpy(oracle.bf16_to_f32(a)).to(torch.float16).to(dev))
    W = QuantizedMatrix(to_dev(q, dev, "raw"), to_dev(s, dev, "raw"),
                        torch.bfloat16 if dt == "bf16" else torch.float16)
    host = dict(x=oracle.normal_bf16(seed + 1, (M, K), 1.0), A=oracle.normal_bf16(seed + 2, (K, r), 0.01),
                B=oracle.normal_bf16(seed + 3, (r, N), 0.01), bias=oracle.normal_bf16(seed + 4, (N,), 0.1),
                q=q, s=s)
    d = {k: cast(host[k]) for k in ("x", "A", "B", "bias")}
    d["W"] = W
    return host, d


# (M, K, N, r, dtype): the second projection's dX (M x N outputs) runs the fused epilogue in the
# first three (unsplit GEMM: at least 128 output tiles of 256 x 256, partial row and column tiles
# in the second); the rest take the separate pass (few tokens, split reduction)
SHAPES = [(4096, 1536, 8960, 32, "bf16"), (1000, 1536, 8960, 32, "bf16"),
          (2048, 1024, 4096, 16, "f16"), (77, 1536, 1536, 16, "bf16"), (300, 1536, 8960, 32, "bf16"),
          (512, 1024, 2048, 8, "f16")]


@pytest.mark.parametrize("M,K,N,r,dt", SHAPES)
def test_fused_gelu_forward_equals_the_separate_calls(dev, M, K, N, r, dt):
    """y, g and h of i8lora_forward_gelu against i8lora_forward then gelu_tanh: the forward's
    M x N outputs run the fused epilogue in the first three shapes (unsplit GEMM), the separate
    pass in the rest."""
    import torch
    from reels_amd import gelu_tanh, i8lora_forward, i8lora_forward_gelu
    print(f"[gelu-fused fwd] M={M} K={K} N={N} r={r} {dt}", flush=True)
    host, d = _case(dev, M, K, N, r, 700 + M + N, dt)
    c = 0.75
    y, g, h = i8lora_forward_gelu(d["x"], d["W"], d["A"], d["B"], d["bias"], c, save_h=True)
    y2, h2 = i8lora_forward(d["x"], d["W"], d["A"], d["B"], d["bias"], c, save_h=True)
    g2 = gelu_tanh(y2)
    torch.cuda.synchronize(dev)
    assert torch.equal(y, y2), "y differs from i8lora_forward"
    assert torch.equal(h, h2), "h differs from i8lora_forward"
    assert torch.equal(g, g2), "g differs from gelu_tanh(y)"
    if M == 1000:
        # sampled rows of g against the oracle's GELU of the oracle's rounded linear output
        rows = np.unique(np.concatenate([np.arange(0, M, 97), [M - 1]]))
        yo, _ = oracle.lora_forward(host["x"][rows], host["q"], host["s"], host["A"], host["B"], c,
                                    bias=host["bias"])
        assert_parity(bf16_f32(y)[rows], yo, "y vs oracle")
        go = oracle.bf16_to_f32(oracle.gelu_tanh(oracle.f32_to_bf16(bf16_f32(y)[rows])))
        got = bf16_f32(g)[rows]
        # the device's and the host's f32 tanh may differ in the last bits: one bf16 ulp
        assert np.all(np.abs(got - go) <= 2.0 ** -7 * np.abs(go) + 1e-30), "g vs the oracle's GELU of y"


def test_fused_gelu_forward_rejects_a_missing_output(dev):
    import ctypes
    from reels_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    rc = L.reels_hip_i8lora_fwd_gelu(fake, fake, fake, None, None, None, 4, 64, 64, 0, 1.0, fake,
                                     None, None, None, 0, None)
    assert rc == -1 and b"NULL g" in L.reels_hip_last_error()


@pytest.mark.parametrize("M,K,N,r,dt", SHAPES)
def test_fused_gelu_pullback_equals_the_separate_calls(dev, M, K, N, r, dt):
    import torch
    from reels_amd import gelu_tanh, gelu_tanh_backward, i8lora_backward, i8lora_backward_gelu, i8lora_forward
    print(f"[gelu-fused] M={M} K={K} N={N} r={r} {dt}", flush=True)
    # forward of the chain: ffn.0-like projection K -> N, then the GELU
    host, d = _case(dev, M, K, N, r, 900 + M + N, dt)
    c = 1.0
    y, _ = i8lora_forward(d["x"], d["W"], d["A"], d["B"], d["bias"], c)
    g = gelu_tanh(y)
    # backward of the ffn.2-like projection N -> K (weight [K][N]) whose input is g: its dx is the
    # GELU's output gradient
    host2, d2 = _case(dev, M, N, K, r, 1900 + M + N, dt)
    dy = torch.from_numpy(oracle.bf16_to_f32(oracle.normal_bf16(2900 + M, (M, K), 1.0))).to(dev).to(g.dtype)
    dgx, dA, dB, dbias = i8lora_backward_gelu(dy, g, y, d2["W"], d2["A"], d2["B"], c, h=None,
                                              want_dbias=True)
    dz, dA2, dB2, dbias2 = i8lora_backward(dy, g, d2["W"], d2["A"], d2["B"], c, h=None, want_dbias=True)
    dgx2 = gelu_tanh_backward(y, dz)
    torch.cuda.synchronize(dev)
    assert torch.equal(dgx, dgx2), "dgx differs from gelu_tanh_backward(y, dx)"
    assert torch.equal(dA, dA2) and torch.equal(dB, dB2) and torch.equal(dbias, dbias2)
    again = i8lora_backward_gelu(dy, g, y, d2["W"], d2["A"], d2["B"], c, h=None)
    torch.cuda.synchronize(dev)
    assert torch.equal(again[0], dgx), "a repeated call gives other bits"
    if M == 1000:
        # sampled rows against the oracle: dz of the second projection, then the GELU's pullback
        # of the rounded dz at the rounded y
        rows = np.unique(np.concatenate([np.arange(0, M, 97), [M - 1]]))
        gb, yb, dyb = (oracle.f32_to_bf16(bf16_f32(t)) for t in (g, y, dy))
        go = oracle.lora_backward(dyb[rows], gb[rows], host2["q"], host2["s"], host2["A"],
                                  host2["B"], c, want=("dx",))
        assert_parity(bf16_f32(dz)[rows], go["dx"], "dz vs oracle")
        pull = oracle.bf16_to_f32(oracle.gelu_tanh_backward(yb[rows], oracle.f32_to_bf16(bf16_f32(dz)[rows])))
        got = bf16_f32(dgx)[rows]
        tol = 2.0 ** -6 * np.abs(pull) + 2.0 ** -12 * np.abs(pull).max()
        assert np.all(np.abs(got - pull) <= tol), "fused pullback vs oracle"


def test_fused_gelu_pullback_rejects_a_missing_gelu_input(dev):
    import ctypes
    from reels_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    rc = L.reels_hip_i8lora_bwd_gelu(fake, fake, None, fake, fake, None, None, None, 4, 64, 64, 0,
                                     1.0, fake, None, None, None, None, 0, None)
    assert rc == -1 and b"NULL gx" in L.reels_hip_last_error()
