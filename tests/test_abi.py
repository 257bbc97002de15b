"""CPU tests of the C ABI library (loads, exports every declared symbol, validates arguments
before touching the GPU) and of the host-side policy logic. No GPU compute is called here."""
import ctypes
import os
import re

import pytest

from reels_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "reels_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(reels_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_binding_table():
    assert declared_symbols() == sorted(_lib.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
    assert L.reels_hip_abi_version() == _lib.ABI_VERSION


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (REELS_HIP_\w+) \(?(-?\d+)\)?", text))
    assert int(consts["REELS_HIP_ABI_VERSION"]) == _lib.ABI_VERSION
    assert (int(consts["REELS_HIP_F32"]), int(consts["REELS_HIP_BF16"]),
            int(consts["REELS_HIP_F16"])) == (_lib.F32, _lib.BF16, _lib.F16)
    assert (int(consts["REELS_HIP_WS_FWD"]), int(consts["REELS_HIP_WS_BWD"]),
            int(consts["REELS_HIP_WS_FWD_NOALLOC"])) == (_lib.WS_FWD, _lib.WS_BWD,
                                                         _lib.WS_FWD_NOALLOC)


def test_workspace_sizes():
    L = _lib.lib()
    for (M, K, N, r) in [(32760, 5120, 5120, 32), (1024, 1536, 1536, 16), (77, 5120, 5120, 32),
                         (4, 5, 7, 3), (0, 16, 16, 0)]:
        for which in (0, 1):
            b = L.reels_hip_i8lora_workspace_bytes(M, K, N, r, which)
            assert b > 0 and b % 256 == 0
    # K and N multiples of 64: both directions hold the bf16 dequantized weight (N x K), the
    # backward also the h/u panels [M][r]
    for which in (0, 1):
        b = L.reels_hip_i8lora_workspace_bytes(32760, 5120, 13824, 32, which)
        assert b >= 13824 * 5120 * 2 + 32760 * 32 * 2 * (1 + which)
    # K a multiple of 16 but not of 64: the int8 GEMM path, whose backward holds dy*s [M][N] bf16
    assert L.reels_hip_i8lora_workspace_bytes(4096, 5136, 5120, 32, 1) >= 4096 * 5120 * 2
    assert L.reels_hip_i8lora_workspace_bytes(-1, 5, 5, 1, 0) == 0
    assert L.reels_hip_i8lora_workspace_bytes(4, 5, 5, 1, 7) == 0
    # the no-allocation forward's scratch: no dequantized weight copy, so far below the
    # workspace forward's on a Wan shape; the few-token kernel's partials, l and counters fit
    nw = L.reels_hip_i8lora_workspace_bytes(32760, 5120, 5120, 32, _lib.WS_FWD_NOALLOC)
    assert 0 < nw < L.reels_hip_i8lora_workspace_bytes(32760, 5120, 5120, 32, _lib.WS_FWD)
    assert nw >= 32760 * 32 * 2 and nw % 256 == 0
    few = L.reels_hip_i8lora_workspace_bytes(77, 5120, 5120, 32, _lib.WS_FWD_NOALLOC)
    assert 0 < few <= 32 << 20 and few >= 77 * 32 * 2 + 128
    # f32: the dequantized weight is N x K f32, h / u panels [M][r] f32, dA / dB partials
    for which in (0, 1):
        b = L.reels_hip_i8lora_workspace_bytes_f32(32760, 5120, 13824, 32, which)
        assert b % 256 == 0 and b >= 13824 * 5120 * 4 + 32760 * 32 * 4 * (1 + which)
    assert L.reels_hip_i8lora_workspace_bytes_f32(4, 5, 7, 3, 1) > 0
    assert L.reels_hip_i8lora_workspace_bytes_f32(-1, 5, 5, 1, 0) == 0
    assert L.reels_hip_i8lora_workspace_bytes_f32(4, 5, 5, 1, 7) == 0


def _err():
    return _lib.lib().reels_hip_last_error().decode()


def test_argument_errors_before_any_gpu_work():
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    # pack: empty rows (Julia's maximum over an empty collection throws), bad dtype
    assert L.reels_hip_i8_pack(fake, 1, 4, 0, 0, fake, fake, None, None) == -1
    assert "K > 0" in _err()
    assert L.reels_hip_i8_pack(fake, 7, 4, 4, 4, fake, fake, None, None) == -2
    assert L.reels_hip_i8_pack(fake, 1, 4, 8, 4, fake, fake, None, None) == -1  # ld < K
    assert L.reels_hip_i8_pack(None, 1, 4, 8, 8, fake, fake, None, None) == -1
    # forward / backward: workspace missing, bad shapes, NULL operands
    assert L.reels_hip_i8lora_fwd(fake, fake, fake, None, None, None, 8, 16, 16, 0, 1.0, fake,
                                  None, None, 0, None) == -3
    assert "workspace" in _err()
    assert L.reels_hip_i8lora_fwd(fake, fake, fake, None, None, None, 8, 0, 16, 0, 1.0, fake,
                                  None, fake, 1 << 20, None) == -1
    assert L.reels_hip_i8lora_fwd(fake, fake, fake, None, None, None, 8, 16, 16, 4, 1.0, fake,
                                  None, fake, 1 << 20, None) == -1  # r > 0 needs A and B
    assert L.reels_hip_i8lora_fwd(fake, fake, fake, None, None, None, 8, 16, 16, 0,
                                  float("nan"), fake, None, fake, 1 << 20, None) == -1
    assert L.reels_hip_i8lora_bwd(fake, fake, None, fake, fake, fake, fake, 8, 16, 16, 16, 1.0,
                                  fake, None, None, None, 0, None) == -3
    assert L.reels_hip_i8lora_bwd(None, fake, None, fake, fake, fake, fake, 8, 16, 16, 16, 1.0,
                                  fake, None, None, fake, 1 << 20, None) == -1
    # the f16 entry points validate the same way and name themselves in the message
    assert L.reels_hip_i8lora_fwd_f16(fake, fake, fake, None, None, None, 8, 16, 16, 0, 1.0, fake,
                                      None, None, 0, None) == -3
    assert "reels_hip_i8lora_fwd_f16" in _err()
    assert L.reels_hip_i8lora_bwd_f16(None, fake, None, fake, fake, fake, fake, 8, 16, 16, 16, 1.0,
                                      fake, None, None, fake, 1 << 20, None) == -1
    assert "reels_hip_i8lora_bwd_f16" in _err()
    assert L.reels_hip_gelu_tanh_f16(None, None, -1, None) == -1
    # ... and so do the f32 ones
    assert L.reels_hip_i8lora_fwd_f32(fake, fake, fake, None, None, None, 8, 16, 16, 0, 1.0, fake,
                                      None, None, 0, None) == -3
    assert "reels_hip_i8lora_fwd_f32" in _err() and "_workspace_bytes_f32" in _err()
    assert L.reels_hip_i8lora_fwd_f32(fake, fake, fake, None, None, None, 8, 0, 16, 0, 1.0, fake,
                                      None, fake, 1 << 20, None) == -1
    assert L.reels_hip_i8lora_fwd_f32(fake, fake, fake, None, None, None, 8, 16, 16, 4, 1.0, fake,
                                      None, fake, 1 << 20, None) == -1  # r > 0 needs A and B
    assert L.reels_hip_i8lora_fwd_f32(fake, fake, fake, None, None, None, 8, 16, 16, 0,
                                      float("nan"), fake, None, fake, 1 << 20, None) == -1
    assert L.reels_hip_i8lora_bwd_f32(fake, fake, None, fake, fake, fake, fake, 8, 16, 16, 16, 1.0,
                                      fake, None, None, None, 0, None) == -3
    assert L.reels_hip_i8lora_bwd_f32(None, fake, None, fake, fake, fake, fake, 8, 16, 16, 16, 1.0,
                                      fake, None, None, fake, 1 << 20, None) == -1
    assert "reels_hip_i8lora_bwd_f32" in _err()
    assert L.reels_hip_gelu_tanh_f32(None, None, -1, None) == -1
    assert L.reels_hip_gelu_tanh_bwd_f32(None, None, None, 5, None) == -1
    # a successful-looking call clears the message of the previous failure
    assert L.reels_hip_gelu_tanh(None, None, 0, None) == 0
    assert _err() == ""
    assert L.reels_hip_gelu_tanh(None, None, -1, None) == -1


def test_library_path_override(monkeypatch, tmp_path):
    monkeypatch.setenv("REELS_HIP_LIBRARY", str(tmp_path / "missing.so"))
    assert _lib.library_path() == str(tmp_path / "missing.so")


# ---- host policy logic (src/layers/quantization.jl:88-101, lora.jl:13-28) ------------------
def test_frozen_weight_transfer_policy():
    from reels_amd import frozen_weight_transfer
    t = frozen_weight_transfer("hip", "bf16", quantization="int8")
    assert t.quantization == "int8"
    with pytest.raises(ValueError):
        frozen_weight_transfer("hip", "bf16", quantization="int4")
    with pytest.raises(ValueError):
        frozen_weight_transfer("cpu", "fp32", cpu_offload=True)
    # int8 codes kept in pinned host memory, uploaded per use (quantization.jl:111-144)
    assert frozen_weight_transfer("hip", "bf16", quantization="int8", cpu_offload=True).cpu_offload
    with pytest.raises(NotImplementedError):
        frozen_weight_transfer("hip", "fp16", cpu_offload=True)  # dense offload: not this path
    with pytest.raises(ValueError):
        frozen_weight_transfer("cpu", "fp32", quantization="int8")
    # fp16 with int8 is the reference's own low-VRAM mode (quantization.jl:96-98 accepts it)
    assert frozen_weight_transfer("hip", "fp16", quantization="int8").precision == "fp16"
    # fp32 with int8 is the reference's Float32 path (quantization.jl:61-64): the f32 kernels
    assert frozen_weight_transfer("hip", "fp32", quantization="int8").precision == "fp32"
    with pytest.raises(ValueError):
        frozen_weight_transfer("hip", "fp8", quantization="int8")
    assert frozen_weight_transfer("cpu", "fp32").quantization == "none"


def test_lora_linear_constructor_validation():
    import torch
    from reels_amd import LoRALinear, QuantizedMatrix
    w = QuantizedMatrix(torch.zeros((3, 4), dtype=torch.int8), torch.ones(3))
    with pytest.raises(ValueError):
        LoRALinear(w, rank=0)
    with pytest.raises(ValueError):
        LoRALinear(w, rank=2, alpha=float("inf"))
    with pytest.raises(ValueError):
        LoRALinear(w, rank=2, alpha=-1.0)
    with pytest.raises(ValueError):
        LoRALinear(w, rank=2, dropout=1.0)
    with pytest.raises(ValueError):
        LoRALinear(w, rank=2, train_bias=True)
    layer = LoRALinear(w, rank=2, alpha=2)
    assert layer.A.shape == (4, 2) and layer.B.shape == (2, 3)
    assert float(layer.B.float().abs().sum()) == 0.0  # B = 0 at construction (lora.jl:24)
    assert layer.lora_scale == 1.0


def test_cpu_tensors_are_rejected_not_computed():
    import torch
    from reels_amd import quantize_frozen_matrix
    with pytest.raises(ValueError, match="ROCm device"):
        quantize_frozen_matrix(torch.zeros((4, 16)))


def test_mismatched_operands_raise_before_any_launch():
    """The C ABI sees only pointers: every shape, dtype and device mismatch must raise ValueError
    in the Python wrappers (checked before the device checks, so CPU tensors reach them)."""
    import torch
    from reels_amd import QuantizedMatrix, i8lora_backward, i8lora_forward
    bf = torch.bfloat16
    M, K, N, r = 6, 8, 5, 2
    W = QuantizedMatrix(torch.zeros((N, K), dtype=torch.int8), torch.ones(N))
    x, dy = torch.zeros((M, K), dtype=bf), torch.zeros((M, N), dtype=bf)
    A, B = torch.zeros((K, r), dtype=bf), torch.zeros((r, N), dtype=bf)
    h = torch.zeros((M, r), dtype=bf)
    bad_fwd = [
        dict(x=torch.zeros((M, K + 1), dtype=bf)),                 # K mismatch
        dict(x=torch.zeros((2, M, K), dtype=bf)),                  # not a matrix
        dict(A=torch.zeros((K + 1, r), dtype=bf)),                 # A [K][r]
        dict(A=torch.zeros((r, K), dtype=bf), B=torch.zeros((r, N), dtype=bf)),  # Julia order
        dict(B=torch.zeros((r, N + 1), dtype=bf)),                 # B [r][N]
        dict(B=torch.zeros((r + 1, N), dtype=bf)),                 # rank of B differs from A's
        dict(B=None),                                              # A without B
        dict(bias=torch.zeros((N + 1,), dtype=bf)),                # bias length
        dict(weight=QuantizedMatrix(torch.zeros((N, K), dtype=torch.int8), torch.ones(N + 1))),
        dict(weight=QuantizedMatrix(torch.zeros((N, K), dtype=torch.int8),
                                    torch.ones(N, dtype=torch.float64))),
        dict(weight=QuantizedMatrix(torch.zeros((N, K), dtype=torch.int16), torch.ones(N))),
    ]
    for case in bad_fwd:
        a = dict(x=x, weight=W, A=A, B=B, bias=None)
        a.update(case)
        with pytest.raises(ValueError):
            i8lora_forward(a["x"], a["weight"], a["A"], a["B"], a["bias"], 1.0)
    bad_bwd = [
        dict(dy=torch.zeros((M, N + 1), dtype=bf)),                # N mismatch
        dict(x=torch.zeros((M + 1, K), dtype=bf)),                 # x tokens differ from dy's
        dict(x=torch.zeros((M, K - 1), dtype=bf)),                 # x features
        dict(h=torch.zeros((M, r + 1), dtype=bf)),                 # h [M][r]
        dict(h=torch.zeros((M - 1, r), dtype=bf)),
        dict(A=torch.zeros((K, r + 1), dtype=bf)),                 # A and B ranks differ
        dict(x=None),                                              # dA needs x
        dict(weight=QuantizedMatrix(torch.zeros((N, K), dtype=torch.int8), torch.ones(N - 1))),
    ]
    for case in bad_bwd:
        a = dict(dy=dy, x=x, weight=W, A=A, B=B, h=h)
        a.update(case)
        with pytest.raises(ValueError):
            i8lora_backward(a["dy"], a["x"], a["weight"], a["A"], a["B"], 1.0, h=a["h"])
    # a well-formed call gets past the checks and stops at the device check
    with pytest.raises(ValueError, match="ROCm device"):
        i8lora_forward(x, W, A, B, None, 1.0)
    with pytest.raises(ValueError, match="ROCm device"):
        i8lora_backward(dy, x, W, A, B, 1.0, h=h)


def test_move_weight_tags_the_transfer_precision():
    """_move_weight(::QuantizedMatrix, transfer) keeps the codes and takes the transfer's compute
    type (quantization.jl:131-144)."""
    import torch
    from reels_amd import QuantizedMatrix, frozen_weight_transfer, move_weight
    W = QuantizedMatrix(torch.zeros((3, 4), dtype=torch.int8), torch.ones(3), torch.bfloat16)
    for prec, dt in (("fp16", torch.float16), ("fp32", torch.float32), ("bf16", torch.bfloat16)):
        moved = move_weight(W, frozen_weight_transfer("hip", prec, quantization="int8"))
        assert moved.compute_dtype == dt
        assert moved.values is W.values and moved.scales is W.scales


def test_dequant_argument_errors():
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    assert L.reels_hip_i8_dequant(fake, fake, 4, 8, 4, 0, 0, fake, None) == -1  # ld_q < K
    assert L.reels_hip_i8_dequant(fake, fake, -1, 8, 8, 0, 0, fake, None) == -1
    assert L.reels_hip_i8_dequant(fake, fake, 4, 8, 8, 9, 0, fake, None) == -2
    assert L.reels_hip_i8_dequant(fake, fake, 4, 8, 8, 0, 2, fake, None) == -1
    assert L.reels_hip_i8_dequant(None, fake, 4, 8, 8, 1, 0, fake, None) == -1
    assert "NULL" in _err()
    assert L.reels_hip_i8_dequant(None, None, 0, 8, 8, 1, 1, None, None) == 0  # empty: no work


def test_attention_argument_errors():
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    # head dim, dtype, sizes, NULL operands, workspace: all rejected before any GPU work
    for D in (0, 129, 256):
        assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, 1, 4, 4, 2, D, _lib.BF16, fake,
                                         None, None) == -1
        assert "head_dim" in _err()
    assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, 1, 4, 4, 2, 64, 7, fake,
                                     None, None) == -2
    # f32 counts 4 bytes an element in the 2 GiB bound: 2^23 x 2 x 32 x 4 = 2^31
    assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, 1, 1 << 23, 4, 2, 32, _lib.F32,
                                     fake, None, None) == -1
    assert "2 GiB" in _err()
    assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, -1, 4, 4, 2, 64, _lib.BF16, fake,
                                     None, None) == -1
    assert L.reels_hip_attention_fwd(None, fake, fake, None, 0, 1, 4, 4, 2, 64, _lib.BF16, fake,
                                     None, None) == -1
    assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, 1, 4, 4, 2, 64, _lib.BF16, None,
                                     None, None) == -1
    assert L.reels_hip_attention_fwd(ctypes.c_void_p(4098), fake, fake, None, 0, 1, 4, 4, 2, 64,
                                     _lib.BF16, fake, None, None) == -1  # unaligned
    assert L.reels_hip_attention_fwd(fake, fake, fake, None, 0, 1, 1 << 24, 4, 64, 128, _lib.BF16,
                                     fake, None, None) == -1  # one batch of q over 2 GiB
    assert L.reels_hip_attention_bwd(fake, fake, fake, fake, fake, fake, None, 0, 1, 4, 4, 2, 64,
                                     _lib.BF16, fake, fake, fake, None, 0, None) == -3
    assert "workspace" in _err()
    assert L.reels_hip_attention_bwd(fake, fake, fake, None, fake, fake, None, 0, 1, 4, 4, 2, 64,
                                     _lib.BF16, fake, fake, fake, fake, 1 << 20, None) == -1
    # nothing to compute: no queries in the forward
    assert L.reels_hip_attention_fwd(None, None, None, None, 0, 1, 0, 4, 2, 64, _lib.BF16, None,
                                     None, None) == 0
    assert L.reels_hip_attention_workspace_bytes(2, 100, 3) == 2560
    assert L.reels_hip_attention_workspace_bytes(-1, 1, 1) == 0
