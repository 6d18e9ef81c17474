"""exl3mi: MI355X-native (gfx950) EXL3 trellis-quantized linear and grouped-MoE hot path.

Import with importlib (the directory name is not a Python identifier):
    exl3 = importlib.import_module("b70-inference_amd")
"""
from ._lib import ACT_GELU_TANH, ACT_SILU, Exl3Error, lib  # noqa: F401
from .linear import (BC_LinearEXL3, exl3_gemm, exl3_gemm_noalloc, exl3_mgemm, exl3_reconstruct,  # noqa: F401
                     fuse_linears, had_r_128, linear, mgemm_tables, reconstruct, reconstruct_had_slice,
                     reconstruct_slice)
from .moe import (BC_GatedMLP, BlockSparseMLP, ExpertTables, MixedEXL3, blob_unplanarize, gelu_mul,  # noqa: F401
                  moe_align, moe_forward, moe_forward_blobs, moe_forward_logits, moe_route, route_adjusted, route_block, route_fused, route_softmax_topk,
                  route_topk, router_logits, routing_ds3_nogroup, silu_mul)
from . import blob  # noqa: F401,E402
