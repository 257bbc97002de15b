"""reels_amd: MI355X (gfx950) HIP implementation of Reels.jl's int8 frozen-weight LoRA linear.

The compute lives in libreels_hip.so (C ABI: include/reels_hip.h); this package is the host-side
mirror of the reference layer API (src/layers/quantization.jl, lora.jl, linear.jl, attention.jl).
"""
from ._lib import ReelsHIPError, ReelsHIPUnavailable, library_path  # noqa: F401
from .attention import (  # noqa: F401
    TiledAttentionCache,
    memory_efficient_attention,
    memory_efficient_attention_backward,
)
from .layers import (  # noqa: F401
    DenseLayer,
    FrozenWeightTransfer,
    I8LoRALinearFunction,
    LoRALinear,
    QuantizedMatrix,
    _weight_mul,
    _weight_transpose_mul,
    frozen_weight_transfer,
    gelu_tanh,
    gelu_tanh_backward,
    i8lora_backward,
    i8lora_backward_gelu,
    i8lora_forward,
    i8lora_forward_gelu,
    linear,
    lora_backward,
    lora_forward,
    lora_parameters,
    merged_weight,
    move_weight,
    quantize_frozen_matrix,
    set_adapter_enabled,
    workspace_bytes,
)
