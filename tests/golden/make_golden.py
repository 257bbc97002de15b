"""Writes tests/golden/wan21_block_tiny_int8.npz: int8 packing goldens for the real Wan2.1 block
weights that the reference's parity fixture holds (test/fixtures/wan21_block_tiny.safetensors in
the Reels.jl repository: official Wan2.1-T2V-1.3B weights, fp32, PyTorch [out][in] layout).

For every projection weight W the fixture stores W itself (input data from the reference's own
test fixture), the codes and scales of quantize_frozen_matrix (src/layers/quantization.jl:35-44),
and the base linear output of the fixture's activations through the dequantized weight (f64).
Codes and scales come from the C oracle and are asserted equal to the independent numpy
restatement before writing. Reads the fixture with the safetensors loader (no pickle).

Run from the repo root: python tests/golden/make_golden.py [path/to/wan21_block_tiny.safetensors]
"""
import os
import sys

import numpy as np
from safetensors.numpy import load_file

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/test/fixtures/wan21_block_tiny.safetensors"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "wan21_block_tiny_int8.npz")

NAMES = [f"blocks.0.{a}.{p}" for a in ("self_attn", "cross_attn") for p in "qkvo"] + \
        ["blocks.0.ffn.0", "blocks.0.ffn.2"]


def main():
    d = load_file(SRC)
    x = d["fixture.x"].reshape(-1, d["fixture.x"].shape[-1]).astype(np.float32)  # [8][24]
    out = {"x": x}
    for name in NAMES:
        w = np.ascontiguousarray(d[name + ".weight"], dtype=np.float32)
        b = np.ascontiguousarray(d[name + ".bias"], dtype=np.float32)
        q, s, st = oracle.pack(w, "f32")
        q2, s2, st2 = oracle.numpy_pack(w)
        assert st == 0 and st2 == 0
        assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32)), name
        key = name.replace("blocks.0.", "").replace(".", "_")
        out[key + "_w"] = w
        out[key + "_b"] = b
        out[key + "_q"] = q
        out[key + "_s"] = s
        if w.shape[1] == x.shape[1]:
            deq = q.astype(np.float64) * s.astype(np.float64)[:, None]
            out[key + "_y"] = x.astype(np.float64) @ deq.T + b.astype(np.float64)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, "with", len(out), "arrays")


if __name__ == "__main__":
    main()
