"""reels_hip_i8lora_fwd_noalloc: the forward that allocates nothing (its scratch is a device array
inside the library). Called through the C ABI and checked against reels_hip_i8lora_fwd on the
same inputs, two calls in a row with the second smaller (the scratch keeps the first call's
contents), and against the f64 oracle. Where reels_hip_i8lora_fwd also multiplies the int8 codes
(K not a multiple of 64) the two must agree bit for bit; where it takes the dequantized-weight
path (K, N multiples of 64) both must meet the bf16 tolerance of tests/_util.assert_parity."""
import ctypes

import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_bits, bf16_f32, to_dev

pytestmark = pytest.mark.gpu


def _case(M, K, N, r, seed):
    x = oracle.normal_bf16(seed + 1, (M, K), 1.0)
    w = oracle.normal_bf16(seed + 2, (N, K), 0.02, outlier_rate=1e-3)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    A = oracle.normal_bf16(seed + 3, (K, r), 0.01)
    B = oracle.normal_bf16(seed + 4, (r, N), 0.01)
    bias = oracle.normal_bf16(seed + 5, (N,), 0.1)
    return x, q, s, A, B, bias


def _run(dev, L, fn, x, q, s, A, B, bias, M, K, N, r, c):
    import torch
    from reels_amd import _lib
    t = {k: to_dev(v, dev) for k, v in dict(x=x, A=A, B=B, bias=bias).items()}
    qd, sd = to_dev(q, dev, "raw"), to_dev(s, dev, "raw")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    h = torch.empty((M, r), dtype=torch.bfloat16, device=dev)
    p = lambda a: ctypes.c_void_p(a.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if fn == "noalloc":
        rc = L.reels_hip_i8lora_fwd_noalloc(p(t["x"]), p(qd), p(sd), p(t["A"]), p(t["B"]),
                                            p(t["bias"]), M, K, N, r, c, p(y), p(h), st)
        _lib.check("reels_hip_i8lora_fwd_noalloc", rc)
    else:
        nb = int(L.reels_hip_i8lora_workspace_bytes(M, K, N, r, _lib.WS_FWD))
        ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
        rc = L.reels_hip_i8lora_fwd(p(t["x"]), p(qd), p(sd), p(t["A"]), p(t["B"]), p(t["bias"]),
                                    M, K, N, r, c, p(y), p(h), p(ws), nb, st)
        _lib.check("reels_hip_i8lora_fwd", rc)
    torch.cuda.synchronize(dev)
    return bf16_bits(y), bf16_bits(h)


def test_noalloc_forward_matches_the_workspace_forward(dev):
    from reels_amd import _lib
    L = _lib.lib()
    # call 1: a Wan-like shape (the workspace forward takes the dequantized-weight path);
    # call 2, smaller: K = 528 (both multiply the int8 codes: bit-identical); call 3 repeats
    # call 1 after the scratch held call 2's contents; rank 24 pads the panels to 32
    for (M, K, N, r, seed, exact) in [(2048, 1536, 1536, 32, 10, False),
                                      (300, 528, 512, 24, 20, True),
                                      (2048, 1536, 1536, 32, 10, False)]:
        print(f"[noalloc] M={M} K={K} N={N} r={r}", flush=True)
        x, q, s, A, B, bias = _case(M, K, N, r, seed)
        c = float(np.float32(r) / np.float32(r))
        y0, h0 = _run(dev, L, "noalloc", x, q, s, A, B, bias, M, K, N, r, c)
        y1, h1 = _run(dev, L, "workspace", x, q, s, A, B, bias, M, K, N, r, c)
        assert np.array_equal(h0, h1), "h differs from the workspace forward"
        f0, f1 = oracle.bf16_to_f32(y0), oracle.bf16_to_f32(y1)
        if exact:
            assert np.array_equal(y0, y1), "y differs from the workspace forward"
        else:
            assert_parity(f0, f1.astype(np.float64), "noalloc y vs workspace y")
        rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 16)), [M - 1]]))
        yo, ho = oracle.lora_forward(x[rows], q, s, A, B, c, bias)
        assert_parity(f0[rows], yo, "noalloc y vs oracle")
        assert_parity(oracle.bf16_to_f32(h0)[rows], ho, "noalloc h vs oracle")


def test_noalloc_rejects_sizes_beyond_its_scratch(dev):
    import torch
    from reels_amd import _lib
    L = _lib.lib()
    # h alone: 300000 tokens x 64 ranks x 2 bytes = 38.4 MB > 32 MiB: rejected before any launch,
    # so these tiny buffers are never read
    M, K, N, r = 300000, 64, 64, 64
    buf = torch.zeros((1024,), dtype=torch.uint8, device=dev)
    p = ctypes.c_void_p(buf.data_ptr())
    assert L.reels_hip_i8lora_workspace_bytes(M, K, N, r, _lib.WS_FWD_NOALLOC) > 32 << 20
    rc = L.reels_hip_i8lora_fwd_noalloc(p, p, p, p, p, None, M, K, N, r, 1.0, p, p, None)
    assert rc == -1
    assert b"scratch" in L.reels_hip_last_error()
    # the entry point still works afterwards
    x, q, s, A, B, bias = _case(64, 64, 64, 16, 30)
    y0, _ = _run(dev, L, "noalloc", x, q, s, A, B, bias, 64, 64, 64, 16, 1.0)
    y1, _ = _run(dev, L, "workspace", x, q, s, A, B, bias, 64, 64, 64, 16, 1.0)
    assert_parity(oracle.bf16_to_f32(y0), oracle.bf16_to_f32(y1).astype(np.float64),
                  "noalloc y after a rejected call")


@pytest.mark.parametrize("M,K,N,r", [(77, 5120, 5120, 32), (2048, 1536, 1536, 32)])
def test_noalloc_forward_under_graph_capture(dev, M, K, N, r):
    """The caller this entry point is for: warmed up once, then captured with torch.cuda.graph
    (global capture mode, under which an allocation on the capturing thread fails the capture)
    and replayed several times with eager work and synchronisations between the replays; every
    replay equals the eager call bit for bit. 77 tokens take the few-token kernel, 2048 the
    int8 GEMM."""
    import torch
    from reels_amd import _lib
    L = _lib.lib()
    x, q, s, A, B, bias = _case(M, K, N, r, 40 + M)
    c = 1.0
    t = {k: to_dev(v, dev) for k, v in dict(x=x, A=A, B=B, bias=bias).items()}
    qd, sd = to_dev(q, dev, "raw"), to_dev(s, dev, "raw")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    h = torch.empty((M, r), dtype=torch.bfloat16, device=dev)
    p = lambda a: ctypes.c_void_p(a.data_ptr())

    def call():
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        rc = L.reels_hip_i8lora_fwd_noalloc(p(t["x"]), p(qd), p(sd), p(t["A"]), p(t["B"]),
                                            p(t["bias"]), M, K, N, r, c, p(y), p(h), st)
        _lib.check("reels_hip_i8lora_fwd_noalloc", rc)

    print(f"[noalloc] graph capture M={M} K={K} N={N} r={r}", flush=True)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    y_ref, h_ref = y.clone(), h.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(3):
        y.zero_()
        h.zero_()
        torch.cuda.synchronize(dev)
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(y, y_ref), f"replay {i}: y differs from the eager call"
        assert torch.equal(h, h_ref), f"replay {i}: h differs from the eager call"
        call()  # eager work between the replays
        torch.cuda.synchronize(dev)
        assert torch.equal(y, y_ref)
