"""CPU tests of the reels-umt5-int8-v1 SafeTensors layout (reels_amd/checkpoint.py;
src/models/wan21/text_encoder.jl:296-353, test/unit/wan_text_encoder.jl:50-57): header metadata
and dtypes as the reference's test checks them, bit-exact round trips of codes and scales of the
real Wan2.1 weights (golden codes of quantize_frozen_matrix), and the loader's validation."""
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from reels_amd import QuantizedMatrix
from reels_amd.checkpoint import (INT8_FORMAT, inspect_safetensors, load_quantized,
                                  umt5_dense_keys, write_quantized)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "wan21_block_tiny_int8.npz")
PROJ = [f"{a}_{p}" for a in ("self_attn", "cross_attn") for p in "qkvo"] + ["ffn_0", "ffn_2"]


def _key(name):
    a, p = name.rsplit("_", 1)
    return f"blocks.0.{a}.{p}.weight"


def _golden_state():
    g = np.load(GOLDEN)
    state, dense = {}, []
    for n in PROJ:
        k = _key(n)
        state[k] = QuantizedMatrix(torch.from_numpy(g[n + "_q"].copy()),
                                   torch.from_numpy(g[n + "_s"].copy()), torch.float32)
        state[k[: -len(".weight")] + ".bias"] = torch.from_numpy(g[n + "_b"].copy())
        dense.append(k)
    state["norm.weight"] = torch.linspace(0.5, 1.5, 24)
    state["token_ids"] = torch.arange(10, dtype=torch.int32)
    return g, state, dense


def test_dense_key_names_follow_the_reference():
    assert umt5_dense_keys(1) == [
        "blocks.0.attn.q.weight", "blocks.0.attn.k.weight", "blocks.0.attn.v.weight",
        "blocks.0.attn.o.weight", "blocks.0.ffn.gate.0.weight", "blocks.0.ffn.fc1.weight",
        "blocks.0.ffn.fc2.weight"]
    assert len(umt5_dense_keys(24)) == 24 * 7


@pytest.mark.parametrize("compute", [torch.float32, torch.float16, torch.bfloat16])
def test_round_trip_of_real_wan_codes(tmp_path, compute):
    g, state, dense = _golden_state()
    path = write_quantized(str(tmp_path / "wan-int8.safetensors"), state, dense, compute,
                           metadata={"source": "wan21_block_tiny"})
    hdr = inspect_safetensors(path)
    assert hdr.metadata["format"] == INT8_FORMAT == "reels-umt5-int8-v1"
    assert hdr.metadata["quantization"] == "int8-per-output-channel"
    assert hdr.metadata["compute_dtype"] == {torch.float32: "float32", torch.float16: "float16",
                                             torch.bfloat16: "bfloat16"}[compute]
    assert hdr.metadata["source"] == "wan21_block_tiny"
    q_key = "blocks.0.self_attn.q.weight"
    assert hdr.tensors[q_key] == ("I8", (24, 24))
    assert hdr.tensors[q_key + ".scale"] == ("F32", (24,))
    assert hdr.tensors["blocks.0.ffn.0.weight"] == ("I8", (32, 24))
    float_tag = {torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16"}[compute]
    assert hdr.tensors["blocks.0.self_attn.q.bias"][0] == float_tag
    assert hdr.tensors["token_ids"] == ("I32", (10,))
    assert not os.path.exists(path + ".tmp")

    loaded = load_quantized(path, device="cpu", dense_keys=dense)
    for n in PROJ:
        qm = loaded[_key(n)]
        assert isinstance(qm, QuantizedMatrix) and qm.compute_dtype == compute
        assert np.array_equal(qm.values.numpy(), g[n + "_q"])
        assert np.array_equal(qm.scales.numpy().view(np.uint32), g[n + "_s"].view(np.uint32))
        b = loaded[_key(n)[: -len(".weight")] + ".bias"]
        assert b.dtype == compute
        assert torch.equal(b, torch.from_numpy(g[n + "_b"]).to(compute))
    assert torch.equal(loaded["token_ids"], torch.arange(10, dtype=torch.int32))
    # the compute dtype recorded in the file is the default; an explicit one overrides it
    assert load_quantized(path, device="cpu", compute_dtype=torch.float32)[q_key].compute_dtype \
        == torch.float32


def test_file_bytes_are_the_kernel_layout(tmp_path):
    # the I8 payload is the [N][K] row-major code matrix itself (the ABI's q layout)
    g, state, dense = _golden_state()
    path = write_quantized(str(tmp_path / "f.safetensors"), state, dense, torch.float32)
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    import json
    hdr = json.loads(raw[8:8 + n])
    beg, end = hdr["blocks.0.ffn.2.weight"]["data_offsets"]
    codes = np.frombuffer(raw[8 + n + beg:8 + n + end], np.int8).reshape(24, 32)
    assert np.array_equal(codes, g["ffn_2_q"])


def _save(path, tensors, fmt=INT8_FORMAT):
    save_file(tensors, str(path), metadata={"format": fmt, "compute_dtype": "float32"})
    return str(path)


def test_loader_rejects_malformed_files(tmp_path):
    q = torch.zeros((4, 8), dtype=torch.int8)
    s = torch.ones(4)
    with pytest.raises(ValueError, match="not a reels-umt5-int8-v1"):
        load_quantized(_save(tmp_path / "a.st", {"w": q, "w.scale": s}, fmt="other"), "cpu")
    with pytest.raises(ValueError, match="has no matrix"):
        load_quantized(_save(tmp_path / "b.st", {"w.scale": s}), "cpu")
    with pytest.raises(ValueError, match="without w.scale"):
        load_quantized(_save(tmp_path / "c.st", {"w": q}), "cpu")
    with pytest.raises(ValueError, match="must use SafeTensors I8 storage"):
        load_quantized(_save(tmp_path / "d.st", {"w": q.float(), "w.scale": s}), "cpu")
    with pytest.raises(ValueError, match="must be F32 of shape"):
        load_quantized(_save(tmp_path / "e.st", {"w": q, "w.scale": torch.ones(5)}), "cpu")
    with pytest.raises(ValueError, match="must be F32 of shape"):
        load_quantized(_save(tmp_path / "f.st", {"w": q, "w.scale": s.half()}), "cpu")
    with pytest.raises(ValueError, match="not stored as an int8 matrix"):
        load_quantized(_save(tmp_path / "g.st", {"w": q, "w.scale": s, "v": s.clone()}), "cpu",
                       dense_keys=["v"])
    ok = load_quantized(_save(tmp_path / "h.st", {"w": q, "w.scale": s, "v": s.clone()}), "cpu")
    assert isinstance(ok["w"], QuantizedMatrix) and torch.equal(ok["v"], s)


def test_writer_handles_tensors_sharing_storage(tmp_path):
    # tied weights (one tensor under two keys) are written as two copies
    _, state, dense = _golden_state()
    state["tied.a"] = state["tied.b"] = torch.ones(3)
    loaded = load_quantized(write_quantized(str(tmp_path / "t.st"), state, dense, torch.float32), "cpu")
    assert torch.equal(loaded["tied.a"], loaded["tied.b"])


def test_writer_validation():
    _, state, dense = _golden_state()
    with pytest.raises(KeyError):
        write_quantized("/nonexistent/never.st", state, dense + ["blocks.9.attn.q.weight"])
    with pytest.raises(ValueError, match="compute dtype"):
        write_quantized("/nonexistent/never.st", state, dense, torch.float64)
