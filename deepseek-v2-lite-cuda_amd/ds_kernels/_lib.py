"""ctypes binding of libdsk.so (the C ABI declared in include/dsk.h).

torch is imported first on purpose: torch ships its own HIP runtime
(libamdhip64.so.7), and libdsk.so resolves its HIP dependency by that SONAME,
so both share one runtime instance and torch's stream handles are valid here.
There is no fallback: if the library is missing this module raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before libdsk.so, see above)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("DSK_LIB") or os.path.join(_HERE, "libdsk.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "dsk_last_error": (ctypes.c_char_p, []),
    "dsk_abi_version": (_I, []),
    "dsk_moe_gate_logits": (_I, [_P, _I64, _P, _P, _P, _I64, _I, _I, _I, _I, _P]),
    "dsk_moe_routing_workspace_size": (_SZ, [_I, _I]),
    "dsk_moe_routing": (_I, [_P, _I64, _P, _P, _P, _I, _I, _I, _P, _SZ, _P]),
    "dsk_moe_scan": (_I, [_P, _P, _I, _P]),
    "dsk_moe_dispatch_workspace_size": (_SZ, [_I, _I, _I]),
    "dsk_moe_dispatch": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P]),
    "dsk_moe_combine_workspace_size": (_SZ, [_I, _I]),
    "dsk_moe_combine": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _SZ, _P]),
    "dsk_swiglu": (_I, [_P, _P, _I, _I, _P]),
    "dsk_moe_gemm1": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "dsk_moe_gemm1_swiglu": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "dsk_moe_gemm2": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "dsk_linear": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _I, _P]),
    "dsk_kv_upproj": (_I, [_P, _I64, _P, _P, _I, _I, _I, _P]),
    "dsk_linear_ex": (_I, [_P, _I64, _P, _I, _P, _I64, _I, _I, _I, _P]),
    "dsk_linear_rowsq": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _I, _P, _I64, _I, _I, _P]),
    "dsk_linear_rowscale": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _I, _P, _I64, _I, _I, _F, _P]),
    "dsk_attn_softmax": (_I, [_P, _I64, _I64, _I, _I, _F, _I, _P]),
    "dsk_attn_softmax_masked": (_I, [_P, _I64, _I64, _I, _I, _I, _F, _I, _P, _I, _I64, _I64,
                                     _I64, _P]),
    "dsk_mla_attn_pack": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _P, _I, _I,
                               _I, _I, _I, _I, _P]),
    "dsk_mla_attn_pack_ex": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _P, _P, _P,
                                  _I, _I, _I, _I, _I, _I, _I, _P]),
    "dsk_linear_batched": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _I, _I, _I, _I, _P]),
    "dsk_linear_rows": (_I, [_P, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I, _I, _I,
                             _I, _I, _P]),
    "dsk_linear_split": (_I, [_P, _I64, _P, _P, _I64, _P, _I64, _I, _I, _I, _I, _P]),
    "dsk_mla_decode_workspace_size": (_SZ, [_I, _I, _I]),
    "dsk_mla_decode_attention": (_I, [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _I, _I64,
                                      _I64, _P, _P, _F, _F, _I, _I, _I, _P, _I64, _I64, _P, _SZ,
                                      _P]),
    "dsk_rms_norm": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _F, _P]),
    "dsk_rms_norm_f32": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _F, _P]),
    "dsk_rope": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I, _I, _I, _I, _P]),
    "dsk_rope_qk": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64,
                         _P, _P, _I, _I, _I, _I, _I, _P]),
    "dsk_moe_fused_workspace_size": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "dsk_moe_fused_forward": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P,
                                   _P, _P, _SZ, _P, _P]),
    "dsk_moe_layer_workspace_size": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "dsk_moe_layer_forward": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P,
                                   _P, _P, _SZ, _P, _P]),
    "dsk_moe_layer_forward_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                           _P, _P, _P, _P, _P]),
}


class DskError(RuntimeError):
    """Raised when a libdsk entry point returns a nonzero status."""


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libdsk.so not found at {LIB_PATH}; build it with "
            "`python deepseek-v2-lite-cuda_amd/csrc/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib.dsk_last_error().decode(errors="replace")
        raise DskError(f"{what} failed (status {rc}): {msg}")


def stream_handle(device: torch.device) -> int:
    """Handle of torch's current stream on `device` (kernels run there)."""
    return torch.cuda.current_stream(device).cuda_stream
