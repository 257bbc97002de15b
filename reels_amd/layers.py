"""Host-side mirror of Reels.jl's int8 frozen-weight layer API over the HIP C ABI.

Names, argument meaning and error behaviour follow src/layers/quantization.jl,
src/layers/lora.jl and src/layers/linear.jl. Arrays are torch tensors holding the same memory the
reference's column-major Julia arrays hold: a Julia matrix of size (a, b) is a torch tensor of
shape (b, a). So Julia x::(K, M) is x[M][K]; LoRA A::(r, K) is A[K][r]; B::(N, r) is B[r][N];
QuantizedMatrix.values (logically (N, K)) is stored [N][K] (K contiguous), the layout of the
SafeTensors I8 format (src/checkpoints/safetensors.jl:52-58).

Every compute call runs the HIP kernels; there is no PyTorch or CPU fallback. Device tensors must
live on a ROCm device; CPU tensors raise.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

_DTYPE_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a ROCm device tensor (got {t.device}); the int8 path "
                         "runs only on the GPU")


# activation types of the LoRA linear and the suffix of their C entry points: bfloat16 (this
# library's default), float16 (the reference's int8 compute precision) and float32 (the
# reference's Float32 compute, its only CPU precision)
_ACT_SUFFIX = {torch.bfloat16: "", torch.float16: "_f16", torch.float32: "_f32"}


def _act_dtype(t: torch.Tensor, name: str) -> torch.dtype:
    _need_device(t, name)
    if t.dtype not in _ACT_SUFFIX:
        raise TypeError(f"{name} must be bfloat16, float16 or float32, got {t.dtype}")
    return t.dtype


def _contig(t: Optional[torch.Tensor], dtype: torch.dtype, name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    _need_device(t, name)
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    return t.contiguous()


# ---- storage ---------------------------------------------------------------------------------
@dataclass
class QuantizedMatrix:
    """Per-output-channel symmetric int8 storage of a frozen weight (quantization.jl:5-9).

    values: int8 [N][K]; scales: float32 [N]; compute_dtype: the dtype produced when the weight
    is materialised (the reference's type parameter T)."""

    values: torch.Tensor
    scales: torch.Tensor
    compute_dtype: torch.dtype = torch.bfloat16

    @property
    def shape(self):  # Base.size (quantization.jl:16): (out, in)
        return tuple(self.values.shape)

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def dequantize(self, dtype: Optional[torch.dtype] = None, transpose: bool = False,
                   stream=None) -> torch.Tensor:
        """_materialize_weight / _dequantize_for_compute (quantization.jl:54-64) on the GPU
        (reels_hip_i8_dequant): float32 fl32(q s), float16 f16(q f16(s)), bfloat16
        bf16(fl32(q s)) - the weight the int8 LoRA linear multiplies. [N][K], or [K][N] with
        transpose. (The host-side _host_dequantize, quantization.jl:25-29, agrees for float32
        and bfloat16; for float16 it rounds fl32(q s) instead of multiplying by f16(s).)"""
        d = dtype or self.compute_dtype
        if d not in _DTYPE_CODE:
            raise TypeError(f"unsupported dtype {d}")
        _need_device(self.values, "values")
        N, K = self.values.shape
        q = self.values if self.values.stride(1) == 1 else self.values.contiguous()
        sc = self.scales
        if sc.dtype != torch.float32 or sc.device != q.device or sc.shape != (N,):
            raise ValueError("scales must be a float32 vector of length N on the codes' device")
        sc = sc.contiguous()
        out = torch.empty((K, N) if transpose else (N, K), dtype=d, device=q.device)
        st = _stream(q.device) if stream is None else stream
        _lib.check("reels_hip_i8_dequant", _lib.lib().reels_hip_i8_dequant(
            ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(sc.data_ptr()), N, K,
            q.stride(0), _DTYPE_CODE[d], int(transpose), ctypes.c_void_p(out.data_ptr()), st))
        return out


def quantize_frozen_matrix(weight: torch.Tensor, T: Optional[torch.dtype] = None,
                           stream=None) -> QuantizedMatrix:
    """quantize_frozen_matrix (quantization.jl:35-44) on the GPU, bit-exact.

    weight: [N][K] float32 / bfloat16 / float16 device tensor (rows = output channels).
    T: the compute dtype tagged on the result, eltype(weight) by default as in the reference.
    Raises ValueError (the reference's InexactError from Int8(NaN)) on non-finite weights."""
    _need_device(weight, "weight")
    if weight.dim() != 2:
        raise ValueError("weight must be a matrix")
    if weight.dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported weight dtype {weight.dtype}")
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    N, K = weight.shape
    values = torch.empty((N, K), dtype=torch.int8, device=weight.device)
    scales = torch.empty((N,), dtype=torch.float32, device=weight.device)
    status = torch.empty((1,), dtype=torch.int32, device=weight.device)
    st = _stream(weight.device) if stream is None else stream
    _lib.check("reels_hip_i8_pack", _lib.lib().reels_hip_i8_pack(
        _ptr(weight), _DTYPE_CODE[weight.dtype], N, K, weight.stride(0), _ptr(values),
        _ptr(scales), _ptr(status), st))
    if int(status.item()) != 0:
        raise ValueError("InexactError: Int8(NaN) — weight contains non-finite values")
    return QuantizedMatrix(values, scales, T or weight.dtype)  # T = eltype(weight) by default


# ---- raw entry points -------------------------------------------------------------------------
# The C ABI sees only pointers, so every shape, dtype and device is checked here before a launch:
# a mismatched tensor would otherwise be read out of bounds on the device.
def _check_shape(t: Optional[torch.Tensor], shape, name: str) -> None:
    if t is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _check_codes(weight: QuantizedMatrix) -> None:
    q, s = weight.values, weight.scales
    if q.dtype != torch.int8 or q.dim() != 2:
        raise ValueError(f"weight values must be an int8 matrix, got {q.dtype} {tuple(q.shape)}")
    if s.dtype != torch.float32 or tuple(s.shape) != (q.shape[0],) or s.device != q.device:
        raise ValueError("weight scales must be a float32 vector of length N on the codes' device")


def _validate(weight: QuantizedMatrix, M: int, K: int, N: int, A, B, **others) -> int:
    """Shapes of a forward or backward call: codes [N][K], A [K][r], B [r][N] and every named
    operand in ``others`` (name -> (tensor, shape)). Returns r."""
    _check_codes(weight)
    if (A is None) != (B is None):
        raise ValueError("A and B must be given together")
    r = 0 if A is None else int(A.shape[-1])
    _check_shape(A, (K, r), "A ([K][r])")
    _check_shape(B, (r, N), "B ([r][N])")
    for name, (t, shape) in others.items():
        _check_shape(t, shape, name)
    return r


def _on_activation_device(weight: QuantizedMatrix, device) -> QuantizedMatrix:
    weight = _on_device(weight, device)
    if weight.values.device != device:
        raise ValueError(f"weight is on {weight.values.device}, the activations on {device}")
    if not (weight.values.is_contiguous() and weight.scales.is_contiguous()):
        weight = QuantizedMatrix(weight.values.contiguous(), weight.scales.contiguous(),
                                 weight.compute_dtype)
    return weight



def workspace_bytes(M: int, K: int, N: int, r: int, which: int,
                    dtype: torch.dtype = torch.bfloat16) -> int:
    """Workspace of reels_hip_i8lora_fwd / _bwd (the 16-bit entry points share one size) or,
    for float32, of reels_hip_i8lora_fwd_f32 / _bwd_f32."""
    L = _lib.lib()
    if dtype == torch.float32:
        return int(L.reels_hip_i8lora_workspace_bytes_f32(M, K, N, r, which))
    return int(L.reels_hip_i8lora_workspace_bytes(M, K, N, r, which))


def _on_device(weight: QuantizedMatrix, device) -> QuantizedMatrix:
    """An offloaded weight (codes in host memory, cpu_offload) is copied to the device for this
    call, as the reference's _materialize_weight does (quantization.jl:46-59)."""
    if weight.values.is_cuda:
        return weight
    from .offload import upload
    return upload(weight, device)


def i8lora_forward(x, weight: QuantizedMatrix, A=None, B=None, bias=None, lora_scale=1.0,
                   save_h: bool = False):
    """y = rnd(x deq(Wq)^T + lora_scale * rnd(x A) B + bias); returns (y, h or None).

    x [M][K] bfloat16, float16 or float32 (reels_hip_i8lora_fwd / _fwd_f16 / _fwd_f32; float32
    rounds nothing); A [K][r], B [r][N] and bias [N] of the same dtype (Julia A::(r,K),
    B::(N,r)); y and h come back in that dtype."""
    if x.dim() != 2:
        raise ValueError(f"x must be a [M][K] matrix, got shape {tuple(x.shape)}")
    M, K = x.shape
    N, Kw = weight.values.shape
    if Kw != K:
        raise ValueError("DimensionMismatch: LoRA input and weight dimensions differ")
    r = _validate(weight, M, K, N, A, B, bias=(bias, (N,)))
    dt = _act_dtype(x, "x")
    x = x.contiguous()
    weight = _on_activation_device(weight, x.device)
    A = _contig(A, dt, "A")
    B = _contig(B, dt, "B")
    bias = _contig(bias, dt, "bias")
    dev = x.device
    y = torch.empty((M, N), dtype=dt, device=dev)
    h = torch.empty((M, r), dtype=dt, device=dev) if (save_h and r) else None
    nbytes = workspace_bytes(M, K, N, r, _lib.WS_FWD, dt)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    fn = "reels_hip_i8lora_fwd" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(
        _ptr(x), _ptr(weight.values), _ptr(weight.scales), _ptr(A), _ptr(B), _ptr(bias),
        M, K, N, r, float(lora_scale), _ptr(y), _ptr(h), _ptr(ws), nbytes, _stream(dev)))
    return y, h


def i8lora_forward_gelu(x, weight: QuantizedMatrix, A=None, B=None, bias=None, lora_scale=1.0,
                        save_h: bool = False):
    """The FFN's first projection followed by gelu_tanh (transformer.jl:289-292): returns
    (y, g, h or None) with y as i8lora_forward returns it (the GELU's input, gx of
    i8lora_backward_gelu) and g = gelu_tanh(y) (reels_hip_i8lora_fwd_gelu*: in the forward GEMM's
    epilogue where that GEMM is unsplit, bit-identical to the two calls). float32 runs the two
    calls."""
    if x.dim() == 2 and x.dtype == torch.float32:
        y, h = i8lora_forward(x, weight, A, B, bias, lora_scale, save_h)
        return y, gelu_tanh(y), h
    if x.dim() != 2:
        raise ValueError(f"x must be a [M][K] matrix, got shape {tuple(x.shape)}")
    M, K = x.shape
    N, Kw = weight.values.shape
    if Kw != K:
        raise ValueError("DimensionMismatch: LoRA input and weight dimensions differ")
    r = _validate(weight, M, K, N, A, B, bias=(bias, (N,)))
    dt = _act_dtype(x, "x")
    x = x.contiguous()
    weight = _on_activation_device(weight, x.device)
    A = _contig(A, dt, "A")
    B = _contig(B, dt, "B")
    bias = _contig(bias, dt, "bias")
    dev = x.device
    y = torch.empty((M, N), dtype=dt, device=dev)
    g = torch.empty((M, N), dtype=dt, device=dev)
    h = torch.empty((M, r), dtype=dt, device=dev) if (save_h and r) else None
    nbytes = workspace_bytes(M, K, N, r, _lib.WS_FWD, dt)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    fn = "reels_hip_i8lora_fwd_gelu" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(
        _ptr(x), _ptr(weight.values), _ptr(weight.scales), _ptr(A), _ptr(B), _ptr(bias),
        M, K, N, r, float(lora_scale), _ptr(y), _ptr(g), _ptr(h), _ptr(ws), nbytes, _stream(dev)))
    return y, g, h


def i8lora_backward(dy, x, weight: QuantizedMatrix, A=None, B=None, lora_scale=1.0, h=None,
                    want_dx=True, want_dA=True, want_dB=True, want_dbias=False):
    """(dx [M][K], dA f32 [K][r], dB f32 [r][N]) of lora_backward (lora.jl:106-118). dy, x, h,
    A and B share one dtype, bfloat16, float16 or float32 (reels_hip_i8lora_bwd / _bwd_f16 /
    _bwd_f32); dx comes back in it. With want_dbias, a fourth result: the gradient of a trainable
    bias, dbias f32 [N] = sum over tokens of dy (reels_hip_i8lora_bwd_bias*), the pullback of the
    forward's mixed_add (linear.jl:7-13; lora.jl:37-38, 64-67)."""
    if dy.dim() != 2:
        raise ValueError(f"dy must be a [M][N] matrix, got shape {tuple(dy.shape)}")
    M, N = dy.shape
    Nw, K = weight.values.shape
    if Nw != N:
        raise ValueError("DimensionMismatch: dy and weight output dimensions differ")
    r = _validate(weight, M, K, N, A, B, **{"x ([M][K])": (x, (M, K))})
    _check_shape(h, (M, r), "h ([M][r])")
    if r and x is None and (want_dA or (want_dB and h is None)):
        raise ValueError("x is needed for dA and for recomputing h")
    dt = _act_dtype(dy, "dy")
    dy = dy.contiguous()
    weight = _on_activation_device(weight, dy.device)
    A = _contig(A, dt, "A")
    B = _contig(B, dt, "B")
    x = _contig(x, dt, "x") if x is not None else None
    h = _contig(h, dt, "h")
    dev = dy.device
    dx = torch.empty((M, K), dtype=dt, device=dev) if want_dx else None
    dA = torch.empty((K, r), dtype=torch.float32, device=dev) if (want_dA and r) else None
    dB = torch.empty((r, N), dtype=torch.float32, device=dev) if (want_dB and r) else None
    nbytes = workspace_bytes(M, K, N, r, _lib.WS_BWD, dt)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    if want_dbias:
        dbias = torch.empty((N,), dtype=torch.float32, device=dev)
        fn = "reels_hip_i8lora_bwd_bias" + _ACT_SUFFIX[dt]
        _lib.check(fn, getattr(_lib.lib(), fn)(
            _ptr(dy), _ptr(x), _ptr(h), _ptr(weight.values), _ptr(weight.scales), _ptr(A),
            _ptr(B), M, K, N, r, float(lora_scale), _ptr(dx), _ptr(dA), _ptr(dB), _ptr(dbias),
            _ptr(ws), nbytes, _stream(dev)))
        return dx, dA, dB, dbias
    fn = "reels_hip_i8lora_bwd" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(
        _ptr(dy), _ptr(x), _ptr(h), _ptr(weight.values), _ptr(weight.scales), _ptr(A), _ptr(B),
        M, K, N, r, float(lora_scale), _ptr(dx), _ptr(dA), _ptr(dB), _ptr(ws), nbytes,
        _stream(dev)))
    return dx, dA, dB


def i8lora_backward_gelu(dy, x, gx, weight: QuantizedMatrix, A=None, B=None, lora_scale=1.0,
                         h=None, want_dA=True, want_dB=True, want_dbias=False):
    """i8lora_backward of the projection after a GELU, with dx replaced by the GELU's pullback
    gelu_tanh_backward(gx, dx), gx [M][K] the GELU's input (reels_hip_i8lora_bwd_gelu*: in the
    dX GEMM's epilogue where that GEMM is unsplit, bit-identical to the two calls). Returns
    (dgx, dA, dB), and dbias with want_dbias. float32 runs the two calls."""
    if dy.dim() == 2 and dy.dtype == torch.float32:
        res = i8lora_backward(dy, x, weight, A, B, lora_scale, h, True, want_dA, want_dB, want_dbias)
        return (gelu_tanh_backward(gx, res[0]),) + tuple(res[1:])
    if dy.dim() != 2:
        raise ValueError(f"dy must be a [M][N] matrix, got shape {tuple(dy.shape)}")
    M, N = dy.shape
    Nw, K = weight.values.shape
    if Nw != N:
        raise ValueError("DimensionMismatch: dy and weight output dimensions differ")
    r = _validate(weight, M, K, N, A, B, **{"x ([M][K])": (x, (M, K))})
    _check_shape(h, (M, r), "h ([M][r])")
    _check_shape(gx, (M, K), "gx ([M][K])")
    if gx is None:
        raise ValueError("gx (the GELU's input) is required")
    if r and x is None and (want_dA or (want_dB and h is None)):
        raise ValueError("x is needed for dA and for recomputing h")
    dt = _act_dtype(dy, "dy")
    dy = dy.contiguous()
    weight = _on_activation_device(weight, dy.device)
    A, B, h, gx = _contig(A, dt, "A"), _contig(B, dt, "B"), _contig(h, dt, "h"), _contig(gx, dt, "gx")
    x = _contig(x, dt, "x") if x is not None else None
    dev = dy.device
    dx = torch.empty((M, K), dtype=dt, device=dev)
    dA = torch.empty((K, r), dtype=torch.float32, device=dev) if (want_dA and r) else None
    dB = torch.empty((r, N), dtype=torch.float32, device=dev) if (want_dB and r) else None
    dbias = torch.empty((N,), dtype=torch.float32, device=dev) if want_dbias else None
    nbytes = workspace_bytes(M, K, N, r, _lib.WS_BWD, dt)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    fn = "reels_hip_i8lora_bwd_gelu" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(
        _ptr(dy), _ptr(x), _ptr(h), _ptr(weight.values), _ptr(weight.scales), _ptr(A), _ptr(B),
        _ptr(gx), M, K, N, r, float(lora_scale), _ptr(dx), _ptr(dA), _ptr(dB), _ptr(dbias),
        _ptr(ws), nbytes, _stream(dev)))
    return (dx, dA, dB, dbias) if want_dbias else (dx, dA, dB)


# ---- reference-named layer API ----------------------------------------------------------------
def _weight_mul(weight: QuantizedMatrix, x: torch.Tensor) -> torch.Tensor:
    """_weight_mul (quantization.jl:73-74): x deq(W)^T (deq(W) lives only in the call's
    workspace, as the reference's _materialize_weight result lives only for the call)."""
    return i8lora_forward(x, weight)[0]


def _weight_transpose_mul(weight: QuantizedMatrix, dy: torch.Tensor) -> torch.Tensor:
    """_weight_transpose_mul (quantization.jl:75-76): dy deq(W) (the frozen-weight pullback of
    src/training/ad_rules.jl:70-80)."""
    return i8lora_backward(dy, None, weight, want_dA=False, want_dB=False)[0]


@dataclass
class DenseLayer:
    """DenseLayer (linear.jl:1-4) with a QuantizedMatrix weight."""

    weight: QuantizedMatrix
    bias: Optional[torch.Tensor] = None

    def __call__(self, x):
        return linear(self, x)


def _flatten(x: torch.Tensor, features: int):
    if x.shape[-1] != features:
        raise ValueError("DimensionMismatch: input and weight dimensions differ")
    return x.reshape(-1, features), x.shape[:-1]


def linear(layer: DenseLayer, x: torch.Tensor) -> torch.Tensor:
    """linear(layer, x) (linear.jl:38-46): x deq(W)^T + bias, trailing dims kept."""
    N, K = layer.weight.shape
    xf, lead = _flatten(x, K)
    y, _ = i8lora_forward(xf, layer.weight, bias=layer.bias)
    return y.reshape(*lead, N)


class LoRALinear:
    """LoRALinear (lora.jl:1-35) over a QuantizedMatrix base weight.

    A: [K][r] (Julia A::(r, K)), B: [r][N] (Julia B::(N, r)) on the device, in the weight's
    compute dtype (bfloat16, float16 or float32). The constructor initialises
    A ~ randn / sqrt(in) and B = 0 like the reference (lora.jl:22-24)."""

    def __init__(self, weight: QuantizedMatrix, rank: int, alpha: Optional[float] = None,
                 dropout: float = 0.0, bias: Optional[torch.Tensor] = None,
                 train_bias: bool = False, generator: Optional[torch.Generator] = None,
                 A: Optional[torch.Tensor] = None, B: Optional[torch.Tensor] = None):
        if rank <= 0:
            raise ValueError("rank must be positive")
        alpha = float(rank if alpha is None else alpha)
        if not (math.isfinite(alpha) and alpha > 0):
            raise ValueError("alpha must be finite and positive")
        if not (0 <= dropout < 1):
            raise ValueError("dropout must be in [0, 1)")
        if dropout > 0:
            raise NotImplementedError("LoRA dropout masks are not part of the int8 HIP path")
        if train_bias and bias is None:
            raise ValueError("cannot train a missing linear bias")
        out, inp = weight.shape
        dev = weight.values.device
        dt = weight.compute_dtype if weight.compute_dtype in _ACT_SUFFIX else torch.bfloat16
        if A is None:
            A = (torch.randn((inp, rank), generator=generator, dtype=torch.float32, device=dev)
                 * (1.0 / math.sqrt(inp))).to(dt)
        if B is None:
            B = torch.zeros((rank, out), dtype=dt, device=dev)
        self.weight, self.A, self.B = weight, A, B
        self.alpha, self.dropout = alpha, float(dropout)
        self.enabled, self.train_bias = True, train_bias
        self.base_bias = bias
        self.bias = bias.clone() if (train_bias and bias is not None) else bias

    @property
    def rank(self) -> int:
        return self.A.shape[1]

    @property
    def lora_scale(self) -> float:
        # layer.alpha / size(layer.A, 1) evaluated in Float32 (lora.jl:89, 111)
        return float(torch.tensor(self.alpha, dtype=torch.float32) /
                     torch.tensor(float(self.rank), dtype=torch.float32))

    def __call__(self, x, **kw):
        return lora_forward(self, x, **kw)


def set_adapter_enabled(layer: LoRALinear, enabled: bool) -> LoRALinear:
    """set_adapter_enabled! (lora.jl:39)."""
    layer.enabled = bool(enabled)
    return layer


def lora_parameters(layer: LoRALinear):
    """lora_parameters (lora.jl:37-38)."""
    p = {"A": layer.A, "B": layer.B}
    if layer.train_bias:
        p["bias"] = layer.bias
    return p


def lora_forward(layer: LoRALinear, x: torch.Tensor, training: bool = False,
                 save_h: bool = False, **_):
    """lora_forward (lora.jl:56-95): y = x deq(W)^T + bias + (alpha/r) (x A) B, one fused pass.

    x: [..., K] bfloat16 or float16 (the dtype of A and B). Returns y [..., N] (and h when
    save_h)."""
    N, K = layer.weight.shape
    xf, lead = _flatten(x, K)
    active_bias = layer.base_bias if (layer.train_bias and not layer.enabled) else layer.bias
    if not layer.enabled:
        y, h = i8lora_forward(xf, layer.weight, bias=active_bias)
    else:
        y, h = i8lora_forward(xf, layer.weight, layer.A, layer.B, active_bias,
                              layer.lora_scale, save_h=save_h)
    y = y.reshape(*lead, N)
    return (y, h) if save_h else y


def lora_backward(layer: LoRALinear, x: torch.Tensor, dy: torch.Tensor, h=None):
    """lora_backward (lora.jl:106-118): returns {"dx", "A", "B"} with dA [K][r] and dB [r][N]
    in float32 (Julia dA::(r, K), dB::(N, r))."""
    N, K = layer.weight.shape
    if tuple(x.shape[:-1]) != tuple(dy.shape[:-1]):
        raise ValueError("DimensionMismatch: LoRA input and output trailing dimensions differ")
    xf, lead = _flatten(x, K)
    dyf, _ = _flatten(dy, N)
    dx, dA, dB = i8lora_backward(dyf, xf, layer.weight, layer.A, layer.B, layer.lora_scale, h=h)
    return {"dx": dx.reshape(*lead, K), "A": dA, "B": dB}


def merged_weight(layer: LoRALinear) -> torch.Tensor:
    """merged_weight (lora.jl:120-122) as float32 [N][K]: deq(W) + (alpha/r) (A B)^T."""
    return (layer.weight.dequantize(torch.float32)
            + layer.lora_scale * (layer.A.float() @ layer.B.float()).t())


class I8LoRALinearFunction(torch.autograd.Function):
    """Autograd rule for lora_forward: the fused analogue of the reference's Zygote pullbacks
    (src/training/ad_rules.jl:53-80 for the frozen weight, Zygote's own rule for B*(A*z)).
    Returns no gradient for the frozen weight, like NoTangent()."""

    @staticmethod
    def forward(ctx, x, A, B, values, scales, bias, lora_scale):
        weight = QuantizedMatrix(values, scales)
        # f32 master parameters with 16-bit activations: the kernels take rounded copies, the
        # gradients come back in f32 (the reference's AdamW keeps f32 state, optimizer.jl:9-24)
        Ac = A if A.dtype == x.dtype else A.to(x.dtype)
        Bc = B if B.dtype == x.dtype else B.to(x.dtype)
        y, h = i8lora_forward(x, weight, Ac, Bc, bias, lora_scale, save_h=True)
        ctx.save_for_backward(x, Ac, Bc, values, scales, h)
        ctx.lora_scale = lora_scale
        ctx.param_dtypes = (A.dtype, B.dtype)
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, A, B, values, scales, h = ctx.saved_tensors
        weight = QuantizedMatrix(values, scales)
        dy = dy.contiguous()
        # a trainable bias (LoRALinear train_bias): the pullback of mixed_add (linear.jl:7-13)
        # sums dy over the tokens, in f32 inside the library (the dB pass's read of dy)
        want_bias = ctx.needs_input_grad[5]
        res = i8lora_backward(dy, x, weight, A, B, ctx.lora_scale, h=h,
                              want_dx=ctx.needs_input_grad[0],
                              want_dA=ctx.needs_input_grad[1],
                              want_dB=ctx.needs_input_grad[2], want_dbias=want_bias)
        dx, dA, dB = res[:3]
        dbias = res[3].to(ctx.bias_dtype) if want_bias else None
        # dA and dB keep the f32 of the kernels when the adapter parameters are f32 masters;
        # otherwise they take the parameter dtype
        ad, bd = ctx.param_dtypes
        return (dx, None if dA is None else dA.to(ad),
                None if dB is None else dB.to(bd), None, None, dbias, None)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """gelu_tanh (linear.jl:61-68), bfloat16, float16 or float32 in and out, f32 math."""
    dt = _act_dtype(x, "x")
    x = x.contiguous()
    y = torch.empty_like(x)
    fn = "reels_hip_gelu_tanh" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(_ptr(x), _ptr(y), x.numel(), _stream(x.device)))
    return y


def gelu_tanh_backward(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    dt = _act_dtype(x, "x")
    x = x.contiguous()
    dy = _contig(dy, dt, "dy")
    dx = torch.empty_like(x)
    fn = "reels_hip_gelu_tanh_bwd" + _ACT_SUFFIX[dt]
    _lib.check(fn, getattr(_lib.lib(), fn)(_ptr(x), _ptr(dy), _ptr(dx), x.numel(),
                                           _stream(x.device)))
    return dx


# ---- transfer policy --------------------------------------------------------------------------
@dataclass
class FrozenWeightTransfer:
    """FrozenWeightTransfer (quantization.jl:78-86)."""

    device: str
    precision: str
    quantization: str
    cpu_offload: bool


def frozen_weight_transfer(device: str, precision: str, quantization: str = "none",
                           cpu_offload: bool = False) -> FrozenWeightTransfer:
    """frozen_weight_transfer (quantization.jl:88-101).

    int8 with fp16 compute is the reference's own low-VRAM mode and runs on the f16 kernels;
    int8 with fp32 compute runs on the f32 kernels. The reference rejects int8 with bf16 compute
    because its backward runs through an fp32 shadow model; here bf16 is a compute precision of
    the HIP kernels, so that combination is accepted on the ROCm device too."""
    if quantization not in ("none", "int8"):
        raise ValueError("frozen weight quantization must be none or int8")
    if device not in ("cpu", "cuda", "hip"):
        raise ValueError("device must be cpu, cuda or hip")
    if cpu_offload and device == "cpu":
        raise ValueError("CPU weight offloading requires a GPU device")
    if cpu_offload and quantization != "int8":
        raise NotImplementedError("cpu_offload of dense (unquantized) weights is not part of the "
                                  "int8 HIP path")
    if quantization == "int8":
        if device == "cpu":
            raise ValueError("the int8 HIP path runs on the GPU only")
        if precision not in ("bf16", "fp16", "fp32"):
            raise ValueError(f"unknown compute precision {precision!r} (bf16, fp16 or fp32)")
    return FrozenWeightTransfer(device, precision, quantization, cpu_offload)


def move_weight(weight, transfer: FrozenWeightTransfer):
    """_move_weight (quantization.jl:111-144): quantize a frozen matrix on the device; an existing
    QuantizedMatrix keeps its codes and scales and takes the transfer's compute type."""
    compute = {"fp16": torch.float16, "fp32": torch.float32}.get(transfer.precision, torch.bfloat16)
    if isinstance(weight, QuantizedMatrix):
        if transfer.quantization == "int8":
            # the same codes, tagged with the transfer's compute type (lines 131-144)
            weight = QuantizedMatrix(weight.values, weight.scales, compute)
            if transfer.cpu_offload and weight.values.is_cuda:
                from .offload import offload_weight
                return offload_weight(weight)
            return weight
        return weight.dequantize(compute)
    if transfer.quantization == "int8":
        w = weight if weight.is_cuda else weight.to("cuda")
        qm = quantize_frozen_matrix(w, compute)
        if transfer.cpu_offload:  # codes and scales stay in pinned host memory (lines 117-119)
            from .offload import offload_weight
            return offload_weight(qm)
        return qm
    return weight.to("cuda" if transfer.device != "cpu" else "cpu")
