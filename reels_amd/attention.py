"""Host mirror of memory_efficient_attention and memory_efficient_attention_backward
(src/layers/attention.jl:106-221 CPU, 225-371 CUDA) over the HIP kernels of
``reels_amd/csrc/attention.hip`` (C ABI ``reels_hip_attention_fwd`` / ``_bwd``).

Tensors are torch tensors in the row-major form of the reference's ``(head_dim, heads, tokens,
batch)`` arrays: ``q`` ``[B][Sq][H][D]``, ``k`` and ``v`` ``[B][Sk][H][D]``; ``mask`` is the
reference's ``(key_tokens, query_tokens)`` Bool array as a ``[Sq][Sk]`` bool tensor (True =
visible). bfloat16, float16 or float32, any head dim up to 128, on the ROCm device (bfloat16 and
float16 with head dim 64 or 128 take the tuned kernels, the rest the generic ones); the output
has the input dtype (``promote_type`` of equal types) and the cache keeps the f32 log-sum-exp.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import NamedTuple, Optional

import numpy as np
import torch

from . import _lib
from .layers import _need_device, _ptr, _stream

_DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


@dataclass
class TiledAttentionCache:
    """attention.jl:9-17: what the backward needs (logsumexp per query, the output, the mask)."""
    logsumexp: torch.Tensor          # [B][H][Sq] float32
    output: torch.Tensor             # [B][Sq][H][D]
    mask: Optional[torch.Tensor]     # [Sq][Sk] uint8 on the device, or None
    scale: float
    query_block: int
    key_block: int
    causal: bool


class AttentionResult(NamedTuple):
    output: torch.Tensor
    cache: TiledAttentionCache


class AttentionGradients(NamedTuple):
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor


def _check(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """The reference's shape checks (attention.jl:111-118), then this path's own limits."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need_device(t, n)
        if t.dim() != 4:
            raise ValueError(f"{n} must be 4-d [batch][tokens][heads][head_dim], got {tuple(t.shape)}")
    if not (q.shape[3] == k.shape[3] == v.shape[3]):
        raise ValueError("q, k, and v head dimensions differ")
    if not (q.shape[2] == k.shape[2] == v.shape[2]):
        raise ValueError("q, k, and v head counts differ")
    if k.shape[1] != v.shape[1]:
        raise ValueError("k and v token counts differ")
    if not (q.shape[0] == k.shape[0] == v.shape[0]):
        raise ValueError("q, k, and v batch counts differ")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DT:
        raise TypeError(f"q, k, v must share one dtype, bfloat16, float16 or float32 (got "
                        f"{q.dtype}, {k.dtype}, {v.dtype})")
    if not 1 <= q.shape[3] <= 128:
        raise ValueError(f"head_dim must be between 1 and 128 on this path, got {q.shape[3]}")
    return q.contiguous(), k.contiguous(), v.contiguous()


def _device_mask(mask, Sq: int, Sk: int, device) -> Optional[torch.Tensor]:
    if mask is None:
        return None
    m = torch.as_tensor(mask)
    if tuple(m.shape) != (Sq, Sk):
        raise ValueError("attention mask shape differs")
    return m.to(device=device, dtype=torch.uint8).contiguous()


def memory_efficient_attention(q, k, v, mask=None, causal: bool = False, query_block: int = 128,
                               key_block: int = 128) -> AttentionResult:
    """attention.jl:106-172 (CPU) / 225-304 (CUDA): exact attention with an online softmax.
    query_block and key_block are the reference's tile sizes; they do not change the result
    and only need to be positive, as there."""
    q, k, v = _check(q, k, v)
    if query_block <= 0 or key_block <= 0:
        raise ValueError("attention tile sizes must be positive")
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    m = _device_mask(mask, Sq, Sk, q.device)
    out = torch.empty_like(q)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    _lib.check("reels_hip_attention_fwd", L.reels_hip_attention_fwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(m), int(bool(causal)), B, Sq, Sk, H, D, _DT[q.dtype],
        _ptr(out), _ptr(lse), _stream(q.device)))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # attention.jl:129
    return AttentionResult(out, TiledAttentionCache(lse, out, m, scale, int(query_block),
                                                    int(key_block), bool(causal)))


def memory_efficient_attention_backward(q, k, v, dy, cache: TiledAttentionCache) -> AttentionGradients:
    """attention.jl:174-221 (CPU) / 306-371 (CUDA): dq, dk, dv, recomputing the probabilities
    from the cached log-sum-exp."""
    q, k, v = _check(q, k, v)
    _need_device(dy, "dy")
    if tuple(dy.shape) != tuple(cache.output.shape):
        raise ValueError("attention output gradient shape differs")
    if dy.dtype != q.dtype:
        raise TypeError(f"dy must be {q.dtype}, got {dy.dtype}")
    dy = dy.contiguous()
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    L = _lib.lib()
    wsb = L.reels_hip_attention_workspace_bytes(B, Sq, H)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=q.device)
    _lib.check("reels_hip_attention_bwd", L.reels_hip_attention_bwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(cache.output.contiguous()), _ptr(dy),
        _ptr(cache.logsumexp.contiguous()), _ptr(cache.mask), int(cache.causal), B, Sq, Sk, H, D,
        _DT[q.dtype], _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ctypes.c_size_t(wsb),
        _stream(q.device)))
    return AttentionGradients(dq, dk, dv)
