"""MI355X-native grouped MoE-LoRA operator: HIP kernels for gfx950 behind a C ABI (include/mlora.h),
with the Python interface of thinkube/meepsquared's `_grouped` and `_moe` modules.

    from meepsquared_amd import lora_linear, grouped_linear, tile_map, routed_forward, topk_softmax
"""

from meepsquared_amd._grouped import (BLOCK_M, RANK_MULTIPLE, Nf4Stack, grouped_linear, lora_linear, max_tiles,
                                      tile_map)
from meepsquared_amd._moe import Experts, routed_forward, sort_by_expert, topk_softmax
from meepsquared_amd import _experts as experts  # the Transformers ExpertsInterface implementation

__all__ = ["BLOCK_M", "RANK_MULTIPLE", "Nf4Stack", "grouped_linear", "lora_linear", "max_tiles", "tile_map",
           "Experts", "routed_forward", "sort_by_expert", "topk_softmax", "experts"]
