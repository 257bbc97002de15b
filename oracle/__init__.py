"""Oracle for the int8 frozen-weight LoRA linear: a CPU restatement of Reels.jl's algorithm.

TEST INFRASTRUCTURE ONLY. tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check or time against it. The product path
(``reels_amd``) never imports it and fails loudly when its HIP library is missing.

Two independent restatements live here:
  * ``liboracle.so`` (oracle.c): pack, dequant, f64 LoRA forward/backward, GELU, Philox inputs;
  * ``numpy_pack`` (this file): a second, numpy-only restatement of quantize_frozen_matrix
    (src/layers/quantization.jl:35-44) that must agree with the C one bit for bit.
Parity status per function is documented in oracle.h and in the test files that pin it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.oracle_pack.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp]
        L.oracle_pack.restype = ctypes.c_int
        L.oracle_dequant.argtypes = [vp, vp, i64, i64, ctypes.c_int, vp]
        ci = ctypes.c_int
        L.oracle_lora_forward.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                          ctypes.c_float, vp, i64, vp, vp, ci]
        L.oracle_lora_backward.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                           ctypes.c_float, vp, i64, vp, i64, vp, i64, vp, vp, vp,
                                           ci]
        L.oracle_gelu_tanh.argtypes = [vp, vp, i64, ci]
        L.oracle_gelu_tanh_backward.argtypes = [vp, vp, vp, i64, ci]
        L.oracle_f16_to_f32_array.argtypes = [vp, vp, i64]
        L.oracle_f32_to_f16_array.argtypes = [vp, vp, i64]
        L.oracle_attention_forward.argtypes = [vp, vp, vp, vp, ci, i64, i64, i64, i64, i64, ci,
                                               vp, vp]
        L.oracle_attention_backward.argtypes = [vp, vp, vp, vp, vp, ci, i64, i64, i64, i64, i64,
                                                ci, vp, vp, vp]
        L.oracle_philox4x32_10.argtypes = [vp, vp, vp]
        L.oracle_normal_bf16.argtypes = [ctypes.c_uint64, ctypes.c_uint32, i64, ctypes.c_double,
                                         ctypes.c_double, ctypes.c_double, vp]
        L.oracle_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_uint32, i64, ctypes.c_double, vp]
        L.oracle_f32_to_bf16_array.argtypes = [vp, vp, i64]
        L.oracle_bf16_to_f32_array.argtypes = [vp, vp, i64]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---- bf16 helpers (src/models/interface.jl:13-25) -------------------------------------------
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """numpy mirror of bfloat16_values: (bits + 0x7fff + ((bits >> 16) & 1)) >> 16."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def c_f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_bf16_array(_p(f), _p(out), f.size)
    return out


# ---- pack --------------------------------------------------------------------------------------
def pack(w: np.ndarray, dtype: str = "auto"):
    """C restatement of quantize_frozen_matrix (quantization.jl:35-44).

    w: [N][K] float32, or uint16 holding bf16 ("bf16") / f16 ("f16") bits.
    Returns (q int8 [N][K], s float32 [N], status) with status 1 on non-finite input."""
    if dtype == "auto":
        dtype = "f32" if w.dtype == np.float32 else "bf16"
    code = {"f32": 0, "bf16": 1, "f16": 2}[dtype]
    w = np.ascontiguousarray(w)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    st = lib().oracle_pack(_p(w), code, N, K, K, _p(q), _p(s))
    if st < 0:
        raise ValueError("oracle_pack: bad arguments")
    return q, s, st


def numpy_pack(w32: np.ndarray):
    """Independent numpy restatement of quantize_frozen_matrix (quantization.jl:35-44).

    w32: float32 [N][K]. Returns (q, s, status)."""
    host = np.ascontiguousarray(w32, dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore", under="ignore"):
        maxima = np.max(np.abs(host), axis=1)  # np.max propagates NaN like Julia's maximum
        scales = (maxima / np.float32(127.0)).astype(np.float32)
        scales[maxima == np.float32(0.0)] = np.float32(1.0)
        ratio = (host / scales[:, None]).astype(np.float32)
        # Base.clamp(x, lo, hi) = ifelse(x > hi, hi, ifelse(x < lo, lo, x)): NaN passes through
        clamped = np.where(ratio > 127.0, np.float32(127.0),
                           np.where(ratio < -127.0, np.float32(-127.0), ratio))
        rounded = np.rint(clamped)  # ties to even
    bad = ~np.isfinite(rounded)
    status = int(bad.any())
    q = np.where(bad, 0, rounded).astype(np.int8)
    return q, scales.astype(np.float32), status


def dequant(q, s, mode: str = "f32"):
    code = {"f32": 0, "f16": 1, "bf16": 2}[mode]
    q = _c(q, np.int8)
    s = _c(s, np.float32)
    N, K = q.shape
    out = np.empty((N, K), np.float32 if mode == "f32" else np.uint16)
    lib().oracle_dequant(_p(q), _p(s), N, K, code, _p(out))
    return out


# ---- forward / backward -----------------------------------------------------------------------
_ELT = {"bf16": 0, "f16": 1, "f32": 2}
# storage of activations, adapters and bias: 16-bit codes for bf16 / f16, float32 values for f32
_STORE = {"bf16": np.uint16, "f16": np.uint16, "f32": np.float32}


def lora_forward(x, q, s, A, B, c, bias=None, rows=None, elt="bf16"):
    """f64 restatement of lora_forward (lora.jl:56-95). x, A, B, bias: 16-bit patterns (uint16)
    of bf16 or, with elt="f16", IEEE binary16, or float32 values with elt="f32". Returns
    (y [len(rows)][N] f64, h [len(rows)][r] f64)."""
    st = _STORE[elt]
    x = _c(x, st); q = _c(q, np.int8); s = _c(s, np.float32)
    A = _c(A, st); B = _c(B, st); bias = _c(bias, st)
    M, K = x.shape
    N = q.shape[0]
    r = A.shape[1] if A is not None and A.size else 0
    if A is None:
        A = np.zeros((K, 0), st); B = np.zeros((0, N), st)
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    nrows = M if rws is None else len(rws)
    y = np.empty((nrows, N), np.float64)
    h = np.empty((nrows, max(r, 1)), np.float64)
    lib().oracle_lora_forward(_p(x), _p(q), _p(s), _p(A), _p(B), _p(bias), M, K, N, r,
                              float(c), _p(rws), nrows, _p(y), _p(h), _ELT[elt])
    return y, h[:, :r]


def lora_backward(dy, x, q, s, A, B, c, rows=None, kcols=None, ncols=None,
                  want=("dx", "dA", "dB"), elt="bf16"):
    """f64 restatement of lora_backward (lora.jl:106-118). Returns dict of requested grads:
    dx [len(rows)][K], dA [len(kcols)][r], dB [r][len(ncols)]."""
    st = _STORE[elt]
    dy = _c(dy, st); x = _c(x, st); q = _c(q, np.int8); s = _c(s, np.float32)
    A = _c(A, st); B = _c(B, st)
    M, K = x.shape
    N = q.shape[0]
    r = A.shape[1]
    rws = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    kc = None if kcols is None else np.ascontiguousarray(kcols, dtype=np.int64)
    nc = None if ncols is None else np.ascontiguousarray(ncols, dtype=np.int64)
    nrows = M if rws is None else len(rws)
    nk = K if kc is None else len(kc)
    nn = N if nc is None else len(nc)
    dx = np.empty((nrows, K), np.float64) if "dx" in want else None
    dA = np.empty((nk, r), np.float64) if "dA" in want else None
    dB = np.empty((r, nn), np.float64) if "dB" in want else None
    lib().oracle_lora_backward(_p(dy), _p(x), _p(q), _p(s), _p(A), _p(B), M, K, N, r, float(c),
                               _p(rws), nrows, _p(kc), nk, _p(nc), nn, _p(dx), _p(dA), _p(dB),
                               _ELT[elt])
    return {"dx": dx, "dA": dA, "dB": dB}


def bias_gradient(dy, cols=None, elt="bf16"):
    """f64 gradient of a trainable bias (LoRALinear with train_bias, lora.jl:37-38): the forward
    adds it per output channel with mixed_add (lora.jl:64-67, linear.jl:7-13), so its cotangent
    is dy summed over the tokens, dbias[n] = sum_m dy[m][n]. dy: [M][N] 16-bit patterns (bf16 or,
    with elt="f16", binary16) or float32 values (elt="f32"). Returns [len(cols)] f64."""
    dy = np.ascontiguousarray(dy)
    if elt == "bf16":
        d = bf16_to_f32(dy.astype(np.uint16))
    elif elt == "f16":
        d = f16_to_f32(dy.astype(np.uint16))
    else:
        d = dy.astype(np.float32)
    if cols is not None:
        d = d[:, np.asarray(cols, dtype=np.int64)]
    return d.astype(np.float64).sum(axis=0)


def gelu_tanh(x, elt="bf16"):
    x = _c(x, _STORE[elt])
    y = np.empty_like(x)
    lib().oracle_gelu_tanh(_p(x), _p(y), x.size, _ELT[elt])
    return y


def gelu_tanh_backward(x, dy, elt="bf16"):
    x = _c(x, _STORE[elt]); dy = _c(dy, _STORE[elt])
    dx = np.empty_like(x)
    lib().oracle_gelu_tanh_backward(_p(x), _p(dy), _p(dx), x.size, _ELT[elt])
    return dx


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(f), _p(out), f.size)
    return out


# ---- seeded inputs ----------------------------------------------------------------------------
def philox(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, np.uint32)
    lib().oracle_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def normal_bf16(seed: int, shape, sigma: float, stream: int = 0, outlier_rate: float = 0.0,
                outlier_sigma: float = 20.0) -> np.ndarray:
    """Seeded N(0, sigma^2) values rounded to bf16 (returned as uint16 bits)."""
    n = int(np.prod(shape))
    out = np.empty(n, np.uint16)
    lib().oracle_normal_bf16(seed, stream, n, sigma, outlier_rate, outlier_sigma, _p(out))
    return out.reshape(shape)


def normal_f32(seed: int, shape, sigma: float, stream: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().oracle_normal_f32(seed, stream, n, sigma, _p(out))
    return out.reshape(shape)


# ---- the reference's own fp16 int8 path (for reporting its error beside ours) -----------------
def reference_fp16_forward(x, q, s, A, B, c, bias=None):
    """Restatement of the reference's fp16 + int8 lora_forward (its only GPU precision for int8):
    Wd = Float16(q) .* Float16(s) (quantization.jl:61-62); y = Wd * x and the adapter GEMMs with
    f16 inputs, f32 accumulation and f16 outputs (assumed cuBLAS HGEMM behaviour: only an import
    of CUDA.jl could pin it); bias added in Float16; the Float32 scale alpha/r promotes the adapter
    to Float32 and mixed_add returns Float32 (lora.jl:86-94, linear.jl:7-13).
    x, A, B, bias: bf16 bits; returns float32 [M][N]."""
    f16 = np.float16
    x16 = bf16_to_f32(x).astype(f16)
    A16 = bf16_to_f32(A).astype(f16)            # [K][r]
    B16 = bf16_to_f32(B).astype(f16)            # [r][N]
    Wd = (q.astype(f16) * np.asarray(s, np.float32).astype(f16)[:, None]).astype(f16)  # [N][K]
    with np.errstate(over="ignore"):  # binary16 overflow to Inf is part of the semantics
        y = (x16.astype(np.float32) @ Wd.astype(np.float32).T).astype(f16)
        if bias is not None:
            y = (y.astype(np.float32) + bf16_to_f32(bias).astype(f16).astype(np.float32)).astype(f16)
        h = (x16.astype(np.float32) @ A16.astype(np.float32)).astype(f16)
        ad = (h.astype(np.float32) @ B16.astype(np.float32)).astype(f16)
    adapter = np.float32(c) * ad.astype(np.float32)
    return y.astype(np.float32) + adapter


def _att_args(q, k, v, mask, elt):
    st = _STORE[elt]
    q = _c(q, st); k = _c(k, st); v = _c(v, st)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    assert k.shape == (B, Sk, H, D) and v.shape == (B, Sk, H, D)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    assert m is None or m.shape == (Sq, Sk)
    return q, k, v, m, B, Sq, Sk, H, D


def attention_forward(q, k, v, mask=None, causal=False, elt="bf16"):
    """f64 restatement of memory_efficient_attention (attention.jl:106-172). q [B][Sq][H][D], k and
    v [B][Sk][H][D] (16-bit patterns as uint16, or float32 with elt="f32"); mask [Sq][Sk] bool
    (True = visible) or None. Returns (out [B][Sq][H][D] f64, lse [B][H][Sq] f64)."""
    q, k, v, m, B, Sq, Sk, H, D = _att_args(q, k, v, mask, elt)
    out = np.empty((B, Sq, H, D), np.float64)
    lse = np.empty((B, H, Sq), np.float64)
    lib().oracle_attention_forward(_p(q), _p(k), _p(v), _p(m), int(bool(causal)), B, Sq, Sk, H, D,
                                   _ELT[elt], _p(out), _p(lse))
    return out, lse


def attention_backward(q, k, v, dy, mask=None, causal=False, elt="bf16"):
    """f64 restatement of memory_efficient_attention_backward (attention.jl:174-221): returns
    (dq, dk, dv) in the q / k / v layouts."""
    q, k, v, m, B, Sq, Sk, H, D = _att_args(q, k, v, mask, elt)
    dy = _c(dy, _STORE[elt])
    assert dy.shape == q.shape
    dq = np.empty(q.shape, np.float64)
    dk = np.empty(k.shape, np.float64)
    dv = np.empty(v.shape, np.float64)
    lib().oracle_attention_backward(_p(q), _p(k), _p(v), _p(dy), _p(m), int(bool(causal)), B, Sq,
                                    Sk, H, D, _ELT[elt], _p(dq), _p(dk), _p(dv))
    return dq, dk, dv


def attention_sampled(q, k, v, dy, b, h, qrows=(), kcols=(), elt="bf16", block=1024):
    """f64 attention without mask or causal order (attention.jl:106-221, the Wan self-attention
    case) of one (batch b, head h), for sizes where the whole score matrix does not fit:
    out, lse and dq for the query rows ``qrows``, and dk, dv for the key columns ``kcols``.
    q, dy [B][Sq][H][D], k, v [B][Sk][H][D] as 16-bit patterns (bf16 or f16) or float32 values
    (elt="f32"). dk and dv need every query's softmax and correction sum(dy .* out)
    (attention.jl:190), so the queries are streamed in blocks of ``block`` rows through torch's
    CPU f64 matrix products (all host threads). Returns a dict with "out" [nq][D], "lse" [nq],
    "dq" [nq][D], "dk" [nk][D], "dv" [nk][D] (f64 numpy)."""
    import torch

    def dec(a, S):
        a = np.ascontiguousarray(a[b, :, h, :])
        if elt == "bf16":
            f = bf16_to_f32(a.astype(np.uint16))
        elif elt == "f16":
            f = f16_to_f32(a.astype(np.uint16))
        else:
            f = a.astype(np.float32)
        return torch.from_numpy(f.astype(np.float64))

    Sq, Sk, D = q.shape[1], k.shape[1], q.shape[3]
    Q, Kt, V, dY = dec(q, Sq), dec(k, Sk), dec(v, Sk), dec(dy, Sq)
    sc = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # 1 / sqrt(Float32(D)), attention.jl:129
    res = {}

    def rows_of(Qb, dYb):
        S = (Qb @ Kt.T) * sc
        m = S.max(dim=1, keepdim=True).values
        E = torch.exp(S - m)
        l = E.sum(dim=1, keepdim=True)
        P = E / l
        out = P @ V
        corr = (dYb * out).sum(dim=1, keepdim=True)
        return P, out, (m + torch.log(l)).squeeze(1), corr

    qrows = np.asarray(qrows, dtype=np.int64)
    if qrows.size:
        ix = torch.from_numpy(qrows)
        P, out, lse, corr = rows_of(Q[ix], dY[ix])
        dS = P * (dY[ix] @ V.T - corr)
        res["out"], res["lse"] = out.numpy(), lse.numpy()
        res["dq"] = (sc * (dS @ Kt)).numpy()
    kcols = np.asarray(kcols, dtype=np.int64)
    if kcols.size:
        kx = torch.from_numpy(kcols)
        Vc = V[kx]
        dk = torch.zeros((kcols.size, D), dtype=torch.float64)
        dv = torch.zeros((kcols.size, D), dtype=torch.float64)
        for i0 in range(0, Sq, block):
            Qb, dYb = Q[i0:i0 + block], dY[i0:i0 + block]
            P, _, _, corr = rows_of(Qb, dYb)
            Pc = P[:, kx]
            dSc = Pc * (dYb @ Vc.T - corr)
            dv += Pc.T @ dYb
            dk += sc * (dSc.T @ Qb)
        res["dk"], res["dv"] = dk.numpy(), dv.numpy()
    return res
