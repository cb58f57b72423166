"""MI355X-native (gfx950 HIP) MoE-LoRA expert layer behind ART's Megatron interfaces.

Submodules
----------
``art_amd.ops``                        tensor wrappers of the libart_moe C ABI
``art_amd.megatron.kernels.grouped_lora_hip``  drop-in for
                                       ``art.megatron.kernels.cute_grouped_lora_quack``
``art_amd.megatron.lora``              LoRA / expert FC1 / FC2 module mirrors
``art_amd.megatron.router``            top-k softmax router with routing replay
``art_amd.megatron.moe_layer``         the fused expert layer (router -> dispatch
                                       -> FC1+LoRA+SwiGLU -> FC2+LoRA -> combine)
"""
from ._lib import ArtMoeError, LIB_PATH, load  # noqa: F401

__version__ = "0.1.0"
