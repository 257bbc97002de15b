"""GPU tests of the reels-umt5-int8-v1 checkpoint path (reels_amd/checkpoint.py): weights packed
on the GPU while writing carry exactly the codes of quantize_frozen_matrix
(src/layers/quantization.jl:35-44, the oracle's pack), and a loaded checkpoint gives forward
outputs bit-identical to quantizing the same weights in memory (the property the reference
documents for its prequantized UMT5 files, docs/src/training/low_vram.md:42-44)."""
import numpy as np
import pytest
import torch

import oracle
from reels_amd import QuantizedMatrix, i8lora_forward, quantize_frozen_matrix
from reels_amd.checkpoint import inspect_safetensors, load_quantized, write_quantized

pytestmark = pytest.mark.gpu

SHAPES = {"blocks.0.attn.q.weight": (512, 512), "blocks.0.ffn.fc1.weight": (1024, 512),
          "blocks.0.ffn.fc2.weight": (512, 1024)}


@pytest.mark.parametrize("src_dtype", ["bf16", "f32", "f16"])
def test_write_pack_load_forward(dev, tmp_path, src_dtype):
    print(f"[checkpoint] weights {src_dtype}", flush=True)
    state, ref = {}, {}
    for i, (k, (N, K)) in enumerate(SHAPES.items()):
        wb = oracle.normal_bf16(700 + i, (N, K), 0.02, outlier_rate=1e-3)
        if src_dtype == "bf16":
            w = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16)
            ref[k] = oracle.pack(wb, "bf16")
        else:
            wf = oracle.bf16_to_f32(wb) * np.float32(1.37)  # not bf16-representable
            if src_dtype == "f16":
                wf = wf.astype(np.float16)
            w = torch.from_numpy(np.ascontiguousarray(wf))
            ref[k] = oracle.pack(np.ascontiguousarray(wf, np.float32), "f32")
        assert ref[k][2] == 0
        state[k] = w.to(dev)
    state["blocks.0.norm1.weight"] = torch.linspace(0.5, 1.5, 512, device=dev)
    path = write_quantized(str(tmp_path / "m.safetensors"), state, list(SHAPES), torch.bfloat16)
    hdr = inspect_safetensors(path)
    assert all(hdr.tensors[k] == ("I8", SHAPES[k]) for k in SHAPES)
    loaded = load_quantized(path, device=dev, dense_keys=list(SHAPES))
    g = torch.Generator(device=dev).manual_seed(5)
    for k, (N, K) in SHAPES.items():
        qm = loaded[k]
        assert isinstance(qm, QuantizedMatrix) and qm.values.is_cuda
        q, s, _ = ref[k]
        assert np.array_equal(qm.values.cpu().numpy(), q), k
        assert np.array_equal(qm.scales.cpu().numpy().view(np.uint32), s.view(np.uint32)), k
        mem = quantize_frozen_matrix(state[k], torch.bfloat16)
        x = torch.randn((96, K), generator=g, device=dev).to(torch.bfloat16)
        A = (torch.randn((K, 16), generator=g, device=dev) * 0.01).to(torch.bfloat16)
        B = (torch.randn((16, N), generator=g, device=dev) * 0.01).to(torch.bfloat16)
        y1, _ = i8lora_forward(x, qm, A, B, lora_scale=0.5)
        y2, _ = i8lora_forward(x, mem, A, B, lora_scale=0.5)
        torch.cuda.synchronize(dev)
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), k
