"""SafeTensors checkpoints of int8 frozen weights in the reference's portable layout.

`reels-umt5-int8-v1` (src/models/wan21/text_encoder.jl:296-353, 368-; docs/src/training/
low_vram.md:33-44):
- every quantized dense matrix keeps its ordinary key `<name>.weight` as an I8 tensor
  [out][in] (row major, the PyTorch layout);
- a sibling `<name>.weight.scale` holds its F32 per-output-channel scales [out];
- the file metadata holds format = "reels-umt5-int8-v1",
  quantization = "int8-per-output-channel" and the compute dtype;
- every other floating tensor is stored in the compute dtype.

The I8 layout is the kernels' code layout [N][K]. Loading therefore copies the file bytes into
device memory with no repacking, and writing stores what reels_hip_i8_pack produced.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, Optional, Tuple

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .layers import QuantizedMatrix, quantize_frozen_matrix

INT8_FORMAT = "reels-umt5-int8-v1"              # text_encoder.jl:296
INT8_QUANTIZATION = "int8-per-output-channel"   # text_encoder.jl:333

# compute dtypes of the file (the reference writes float16 or float32, text_encoder.jl:314-315;
# bfloat16 is this library's compute precision and is accepted as well)
_COMPUTE = {torch.float16: "float16", torch.float32: "float32", torch.bfloat16: "bfloat16"}
_COMPUTE_BY_NAME = {v: k for k, v in _COMPUTE.items()}


def umt5_dense_keys(layers: int) -> list:
    """_umt5_dense_keys (text_encoder.jl:298-309): the matrices an int8 UMT5 checkpoint stores
    as I8, per encoder block."""
    return [f"blocks.{b}.{k}.weight" for b in range(layers)
            for k in ("attn.q", "attn.k", "attn.v", "attn.o", "ffn.gate.0", "ffn.fc1", "ffn.fc2")]


@dataclass
class SafeTensorsHeader:
    """inspect_safetensors: the file's metadata and, per tensor, (dtype, shape)."""

    metadata: Dict[str, str]
    tensors: Dict[str, Tuple[str, Tuple[int, ...]]]


def inspect_safetensors(path: str) -> SafeTensorsHeader:
    """Reads only the header of a SafeTensors file: an 8-byte little-endian length, then JSON."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a SafeTensors file (short header)")
        (n,) = struct.unpack("<Q", raw)
        if n > 100_000_000:
            raise ValueError(f"{path}: SafeTensors header of {n} bytes is not plausible")
        header = json.loads(f.read(n).decode("utf-8"))
    meta = header.pop("__metadata__", {}) or {}
    tensors = {k: (v["dtype"], tuple(int(d) for d in v["shape"])) for k, v in header.items()}
    return SafeTensorsHeader(dict(meta), tensors)


def _check_compute(dtype) -> torch.dtype:
    if dtype not in _COMPUTE:
        raise ValueError("quantized checkpoint compute dtype must be float16, float32 or bfloat16")
    return dtype


def quantized_state_dict(state: Dict[str, object], dense_keys: Iterable[str],
                         compute_dtype: torch.dtype = torch.float16) -> Dict[str, torch.Tensor]:
    """quantized_umt5_state_dict (text_encoder.jl:312-327) for any set of dense keys.

    Each dense key's matrix is packed on the GPU by reels_hip_i8_pack, which is bit-exact with
    quantize_frozen_matrix. It is stored as its I8 codes plus a `<key>.scale` F32 vector. Every
    other floating tensor is cast to the compute dtype. A value that already is a
    QuantizedMatrix is stored as it is, without requantizing."""
    _check_compute(compute_dtype)
    keys = list(dense_keys)
    missing = [k for k in keys if k not in state]
    if missing:
        raise KeyError(f"dense keys missing from the state dict: {missing[:4]}")
    keyset = set(keys)
    out: Dict[str, torch.Tensor] = {}
    for k, v in state.items():
        if isinstance(v, QuantizedMatrix):
            out[k], out[k + ".scale"] = v.values, v.scales
        elif k in keyset:
            w = v if v.is_cuda else v.to("cuda")
            qm = quantize_frozen_matrix(w, compute_dtype)
            out[k], out[k + ".scale"] = qm.values, qm.scales
        elif torch.is_tensor(v) and torch.is_floating_point(v) and not k.endswith(".scale"):
            out[k] = v.to(compute_dtype)
        else:
            out[k] = v
    return out


def write_quantized(path: str, state: Dict[str, object], dense_keys: Iterable[str],
                    compute_dtype: torch.dtype = torch.float16,
                    metadata: Optional[Dict[str, str]] = None) -> str:
    """write_quantized_umt5 (text_encoder.jl:329-339): a reels-umt5-int8-v1 SafeTensors file,
    written to `path.tmp` and renamed into place like the reference's write_safetensors
    (src/checkpoints/safetensors.jl:102-133)."""
    info = {str(k): str(v) for k, v in (metadata or {}).items()}
    info["format"] = INT8_FORMAT
    info["quantization"] = INT8_QUANTIZATION
    info["compute_dtype"] = _COMPUTE[_check_compute(compute_dtype)]
    tensors, seen = {}, set()
    for k, v in quantized_state_dict(state, dense_keys, compute_dtype).items():
        t = v.detach().contiguous().cpu()
        if t.numel() and t.data_ptr() in seen:  # tied tensors: SafeTensors stores each once
            t = t.clone()
        seen.add(t.data_ptr())
        tensors[k] = t
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    tmp = path + ".tmp"
    save_file(tensors, tmp, metadata=info)
    os.replace(tmp, path)
    return path


def _device_string(device) -> str:
    d = torch.device(device)
    if d.type == "cuda":
        return f"cuda:{d.index if d.index is not None else 0}"
    return d.type


def load_quantized(path: str, device="cuda", compute_dtype: Optional[torch.dtype] = None,
                   dense_keys: Optional[Iterable[str]] = None) -> Dict[str, object]:
    """Loads a reels-umt5-int8-v1 file without requantizing (load_quantized_umt5_encoder and
    _load_quantized_t5_dense, text_encoder.jl:341-353, 368-).

    - Every `<k>.scale` F32 [out] pairs with `<k>` I8 [out][in] into a QuantizedMatrix whose
      codes come straight from the file into `device` memory.
    - ValueError (the reference's ArgumentError) for: a file of another format; an I8 tensor
      without its scale; a scale without its matrix; a scaled matrix not stored as I8; a
      scale of the wrong dtype or length; or one of `dense_keys` not stored quantized.
    - Other floating tensors are cast to the compute dtype. The compute dtype defaults to the
      one the file records."""
    hdr = inspect_safetensors(path)
    fmt = hdr.metadata.get("format")
    if fmt != INT8_FORMAT:
        raise ValueError(f"{path} is not a {INT8_FORMAT} checkpoint (format = {fmt!r})")
    if compute_dtype is None:
        name = hdr.metadata.get("compute_dtype", "float16")
        if name not in _COMPUTE_BY_NAME:
            raise ValueError(f"{path}: unknown compute_dtype {name!r}")
        compute_dtype = _COMPUTE_BY_NAME[name]
    _check_compute(compute_dtype)
    quantized = {k[: -len(".scale")] for k in hdr.tensors if k.endswith(".scale")}
    for base in sorted(quantized):
        if base not in hdr.tensors:
            raise ValueError(f"{base}.scale has no matrix {base}")
        dt, shape = hdr.tensors[base]
        sdt, sshape = hdr.tensors[base + ".scale"]
        if dt != "I8":
            raise ValueError(f"{base} must use SafeTensors I8 storage (found {dt})")
        if len(shape) != 2:
            raise ValueError(f"{base}: quantized matrix must be 2-D, found shape {shape}")
        if sdt != "F32" or sshape != (shape[0],):
            raise ValueError(f"{base}.scale must be F32 of shape ({shape[0]},), found {sdt} {sshape}")
    for k, (dt, _) in hdr.tensors.items():
        if dt == "I8" and k not in quantized:
            raise ValueError(f"{k}: I8 matrix without {k}.scale")
    for k in dense_keys or ():
        if k not in quantized:
            raise ValueError(f"{k} is missing or not stored as an int8 matrix")
    out: Dict[str, object] = {}
    with safe_open(path, framework="pt", device=_device_string(device)) as f:
        for k in hdr.tensors:
            if k.endswith(".scale") and k[: -len(".scale")] in quantized:
                continue
            if k in quantized:
                out[k] = QuantizedMatrix(f.get_tensor(k), f.get_tensor(k + ".scale"), compute_dtype)
            else:
                t = f.get_tensor(k)
                out[k] = t.to(compute_dtype) if torch.is_floating_point(t) else t
    return out
