"""The reference's own CPU path for the int8 LoRA linear, restated for timing (the cpu_baseline
leg of bench.py). TEST/BENCH INFRASTRUCTURE ONLY: never part of the product path.

Reels.jl runs int8 weights on the CPU in Float32 only (array_transfer(:cpu, :bf16) throws,
src/models/interface.jl:38-41). Per call it materialises Float32.(q) .* s
(src/layers/quantization.jl:63-64) and hands it to BLAS sgemm (OpenBLAS in the reference's
Manifest), then runs the rank-r GEMMs and broadcasts of src/layers/lora.jl:56-95 and the explicit
backward of lora.jl:106-118. This module performs the same sequence with torch's CPU BLAS (the
multithreaded fp32 GEMM available on this image) on float32 tensors.
"""
from __future__ import annotations

import time

import torch


def materialize(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """_dequantize_for_compute(values, scales, Float32): a new [N][K] f32 array per call."""
    return q.to(torch.float32) * s[:, None]


def forward(x, q, s, A, B, c):
    """lora_forward for Float32 (lora.jl:56-95): y = Wd x + c B (A x). x [M][K], A [K][r],
    B [r][N] (the physical layouts of the Julia arrays)."""
    Wd = materialize(q, s)
    y = x @ Wd.t()
    ax = x @ A
    return y + c * (ax @ B)


def backward(x, dy, q, s, A, B, c):
    """lora_backward (lora.jl:106-118): ax = A x; dA = c (B' dy) x'; dB = c dy ax';
    dx = Wd' dy + c A' (B' dy)."""
    ax = x @ A
    bdy = dy @ B.t()
    dA = c * (x.t() @ bdy)
    dB = c * (ax.t() @ dy)
    Wd = materialize(q, s)
    dx = dy @ Wd + c * (bdy @ A.t())
    return dx, dA, dB


def flops(M: int, K: int, N: int, r: int) -> float:
    """Algorithmic flops of one linear's forward + dX + dA + dB: 4MNK + 6Mr(K+N)."""
    return 4.0 * M * N * K + 6.0 * M * r * (K + N)


def time_block(projections, M: int, r: int, seed: int = 0):
    """Times one pass (forward then backward) of every (K, N) projection at M tokens.
    Returns (seconds, flops)."""
    g = torch.Generator().manual_seed(seed)
    data = []
    for (K, N) in projections:
        x = torch.randn((M, K), generator=g)
        dy = torch.randn((M, N), generator=g)
        q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        s = torch.rand((N,), generator=g) * 1e-3 + 1e-4
        A = torch.randn((K, r), generator=g) * 0.01
        B = torch.randn((r, N), generator=g) * 0.01
        data.append((x, dy, q, s, A, B))
    c = 1.0
    total = 0.0
    t0 = time.perf_counter()
    for (x, dy, q, s, A, B) in data:
        forward(x, q, s, A, B, c)
    for (x, dy, q, s, A, B) in reversed(data):
        backward(x, dy, q, s, A, B, c)
    t1 = time.perf_counter()
    for (K, N) in projections:
        total += flops(M, K, N, r)
    return t1 - t0, total


def time_linear(K: int, N: int, M: int, r: int, seed: int = 0, reps: int = 1, warm: int = 1):
    """Times the forward and, separately, the backward of one (K, N) linear at M tokens (the best
    of reps runs each, after warm untimed runs). Returns (forward seconds, backward seconds)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g)
    dy = torch.randn((M, N), generator=g)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand((N,), generator=g) * 1e-3 + 1e-4
    A = torch.randn((K, r), generator=g) * 0.01
    B = torch.randn((r, N), generator=g) * 0.01
    c = 1.0
    tf = tb = float("inf")
    for i in range(warm + reps):
        t0 = time.perf_counter()
        forward(x, q, s, A, B, c)
        t1 = time.perf_counter()
        backward(x, dy, q, s, A, B, c)
        t2 = time.perf_counter()
        if i >= warm:
            tf, tb = min(tf, t1 - t0), min(tb, t2 - t1)
    return tf, tb


def attention_forward(q, k, v, query_block: int = 128, key_block: int = 128):
    """memory_efficient_attention on the CPU (attention.jl:106-172) for one head without a mask:
    f32 tiles of query_block x key_block scores on BLAS, an online softmax per query block.
    q [Sq][D], k and v [Sk][D] float32. Returns (out [Sq][D], lse [Sq])."""
    Sq, D = q.shape
    scale = 1.0 / float(torch.tensor(float(D), dtype=torch.float32).sqrt())
    out = torch.empty_like(q)
    lse = torch.empty((Sq,), dtype=torch.float32)
    for q0 in range(0, Sq, query_block):
        qb = q[q0:q0 + query_block]
        mx = torch.full((qb.shape[0],), float("-inf"))
        norm = torch.zeros((qb.shape[0],))
        acc = torch.zeros((qb.shape[0], D))
        for k0 in range(0, k.shape[0], key_block):
            s = (qb @ k[k0:k0 + key_block].t()) * scale
            nm = torch.maximum(mx, s.max(dim=1).values)
            prev = torch.exp(mx - nm)
            p = torch.exp(s - nm[:, None])
            norm = prev * norm + p.sum(dim=1)
            acc = acc * prev[:, None] + p @ v[k0:k0 + key_block]
            mx = nm
        out[q0:q0 + query_block] = acc / norm[:, None]
        lse[q0:q0 + query_block] = mx + torch.log(norm)
    return out, lse


def attention_backward(q, k, v, dy, out, lse, query_block: int = 128, key_block: int = 128):
    """memory_efficient_attention_backward on the CPU (attention.jl:174-221), one head, no mask:
    score tiles recomputed from q, k and the cached lse. Returns (dq, dk, dv)."""
    Sq, D = q.shape
    scale = 1.0 / float(torch.tensor(float(D), dtype=torch.float32).sqrt())
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    for q0 in range(0, Sq, query_block):
        qb, dyb = q[q0:q0 + query_block], dy[q0:q0 + query_block]
        corr = (dyb * out[q0:q0 + query_block]).sum(dim=1)
        lb = lse[q0:q0 + query_block]
        g = torch.zeros_like(qb)
        for k0 in range(0, k.shape[0], key_block):
            kb, vb = k[k0:k0 + key_block], v[k0:k0 + key_block]
            p = torch.exp((qb @ kb.t()) * scale - lb[:, None])
            ds = p * (dyb @ vb.t() - corr[:, None])
            g += (ds @ kb) * scale
            dk[k0:k0 + key_block] += (ds.t() @ qb) * scale
            dv[k0:k0 + key_block] += p.t() @ dyb
        dq[q0:q0 + query_block] = g
    return dq, dk, dv
