"""ctypes binding of libmoe_mi355x.so (include/moe_ops.h, moe_trace.h, moe_synth.h).

This is the binding a Python caller of the C ABI would add; it carries no torch types. Loading fails loudly
when the library has not been built: there is no CPU fallback for any operator.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libmoe_mi355x.so"

MOE_OK = 0
STATUS_NAMES = {
    0: "MOE_OK", 1: "MOE_ERR_NULL", 2: "MOE_ERR_RANK", 3: "MOE_ERR_SHAPE", 4: "MOE_ERR_ARG",
    5: "MOE_ERR_WORKSPACE", 6: "MOE_ERR_UNSUPPORTED", 7: "MOE_ERR_HIP",
}
DT_FLOAT16 = 1
DT_INT32 = 3


class MoeError(RuntimeError):
    """A C-ABI call returned a status other than MOE_OK."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class RoutingPlan(C.Structure):
    _fields_ = [("num_tokens", C.c_int64), ("hidden_size", C.c_int64), ("num_experts", C.c_int64),
                ("top_k", C.c_int64), ("tokens_per_block", C.c_int32), ("grid", C.c_int32),
                ("block", C.c_int32), ("lds_bytes", C.c_int32), ("workspace_bytes", C.c_size_t)]


class FfnPlan(C.Structure):
    _fields_ = [("num_tokens", C.c_int64), ("hidden_size", C.c_int64), ("num_experts", C.c_int64),
                ("top_k", C.c_int64), ("intermediate_size", C.c_int64), ("schedule", C.c_int32),
                ("permute_grid", C.c_int32), ("gateup_grid", C.c_int32), ("down_grid", C.c_int32),
                ("block", C.c_int32), ("rows_per_tile", C.c_int32), ("workspace_bytes", C.c_size_t)]


class CombinePlan(C.Structure):
    _fields_ = [("num_tokens", C.c_int64), ("hidden_size", C.c_int64), ("top_k", C.c_int64),
                ("grid", C.c_int32), ("block", C.c_int32), ("elems_per_thread", C.c_int32),
                ("workspace_bytes", C.c_size_t)]


_I64 = C.c_int64
_I32 = C.c_int32
_P = C.c_void_p
_I64P = C.POINTER(C.c_int64)

# name -> (restype, argtypes); every function declared in include/*.h
SIGNATURES = {
    "moe_status_string": (C.c_char_p, [_I32]),
    "moe_last_error": (C.c_char_p, []),
    "moe_version": (C.c_char_p, []),
    "moe_routing_topk_infer_shape": (_I32, [_I64P, _I32, _I64P, _I32, _I64, _I64P, _I64P]),
    "moe_routing_topk_infer_dtype": (_I32, [C.POINTER(_I32), C.POINTER(_I32)]),
    "moe_routing_topk_plan": (_I32, [_I64, _I64, _I64, _I64, C.POINTER(RoutingPlan)]),
    "moe_routing_topk": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "moe_expert_ffn_infer_shape": (_I32, [_I64P, _I32, _I64P, _I32, _I64P, _I32, _I64, _I64P, _I64P]),
    "moe_expert_ffn_infer_dtype": (_I32, [C.POINTER(_I32)]),
    "moe_expert_ffn_workspace_bytes": (C.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "moe_expert_ffn_plan": (_I32, [_I64, _I64, _I64, _I64, _I64, C.POINTER(FfnPlan)]),
    "moe_expert_ffn": (_I32, [_P, _P, _P, _P, _P, _P, C.c_size_t, _I64, _I64, _I64, _I64, _I64, _P]),
    "moe_expert_ffn_combine": (_I32, [_P, _P, _P, _P, _P, _P, _P, C.c_size_t, _I64, _I64, _I64, _I64, _I64, _P]),
    "moe_expert_ffn_no_alloc": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "moe_layer_workspace_bytes": (C.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "moe_layer": (_I32, [_P, _P, _P, _P, _P, _P, _P, _P, C.c_size_t, _I64, _I64, _I64, _I64, _I64, _P]),
    "moe_combine_infer_shape": (_I32, [_I64P, _I32, _I64P, _I32, _I64P]),
    "moe_combine_infer_dtype": (_I32, [C.POINTER(_I32)]),
    "moe_combine_plan_for": (_I32, [_I64, _I64, _I64, C.POINTER(CombinePlan)]),
    "moe_combine": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "moe_trace_enable": (_I32, [_I32]),
    "moe_trace_collect": (_I32, []),
    "moe_trace_get": (_I32, [_I32, C.POINTER(C.c_char_p), _I64P, C.POINTER(C.c_double)]),
    "moe_synth_normal_f16": (_I32, [_P, C.c_uint64, C.c_uint64, C.c_uint64, C.c_double, C.c_double,
                                    C.c_uint64, C.c_uint64, _P]),
    "moe_copy_bytes": (_I32, [_P, _P, C.c_uint64, _P]),
    "moe_stream_read_bytes": (_I32, [_P, C.c_uint64, _P]),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load the library once; raises RuntimeError if it was not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() (the MoE operators have no "
                    "CPU fallback)")
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def check(status: int) -> None:
    if status != MOE_OK:
        msg = load().moe_last_error().decode(errors="replace")
        raise MoeError(status, msg)


def dims(values) -> C.Array:
    arr = (C.c_int64 * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr
