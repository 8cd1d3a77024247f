"""ds_kernels — MI355X (gfx950) implementation of the DeepSeek-V2-Lite fused MoE
layer and MLA helper kernels, with the op surface of the reference pybind module
(src/kernels/bindings.cu:77-192). All compute runs in libdsk.so (hand-written
HIP); importing this package without the built library raises ImportError.
"""
from ._lib import LIB_PATH, DskError, lib  # noqa: F401  (loads libdsk.so or raises)
from .ops import (  # noqa: F401
    attn_softmax_,
    kv_upproj,
    linear,
    linear_batched,
    linear_rowscale,
    linear_rows,
    linear_rowsq,
    linear_split,
    mla_attn_pack,
    mla_decode_attention,
    moe_combine,
    moe_dispatch,
    moe_gemm1,
    moe_gemm1_swiglu,
    moe_gate,
    moe_gemm2,
    moe_routing,
    moe_scan,
    rms_norm,
    rope,
    swiglu,
)
from .expert_prepack import (  # noqa: F401
    pack_tensors,
    prepack_experts,
    prepack_with_shared,
    tile_weights,
    untile_weights,
    verify_prepack,
)
from .mla_cache import AbsorbedMLAWeights, LatentKVCache, mla_decode_forward  # noqa: F401
from .moe_fused import (  # noqa: F401
    FusedMoELayer,
    fused_moe_forward,
    moe_fused_forward_logits,
    moe_layer_forward,
    route_dispatch_combine,
)

__all__ = [
    "moe_gate", "moe_routing", "moe_scan", "moe_dispatch", "moe_combine", "swiglu", "moe_gemm1",
    "moe_gemm1_swiglu", "moe_gemm2", "rms_norm", "kv_upproj", "linear", "rope", "attn_softmax_",
    "linear_batched", "linear_rows", "linear_split", "linear_rowsq", "linear_rowscale", "mla_attn_pack", "mla_decode_attention", "LatentKVCache", "AbsorbedMLAWeights", "mla_decode_forward",
    "prepack_experts", "prepack_with_shared", "pack_tensors", "tile_weights", "untile_weights",
    "verify_prepack", "FusedMoELayer",
    "fused_moe_forward", "moe_fused_forward_logits", "moe_layer_forward",
    "route_dispatch_combine", "DskError",
]
