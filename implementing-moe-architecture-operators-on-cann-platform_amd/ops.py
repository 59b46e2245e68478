"""Python mirror of the reference's three operators over the C ABI, with torch tensors as device memory.

Reference operator interface: op_host/moe_ops.cpp:537-679 (OpDef inputs/outputs/attrs) and the kernel
entries op_kernel/moe_routing.cpp:434, op_kernel/moe_expert_ffn.cpp:613, op_kernel/moe_combine.cpp:136.
Shapes and dtypes are inferred by the library (the InferShape/InferDataType replacements), and the launch is
queued on `stream` (torch's current stream when None). Outputs and any workspace the call allocates are
allocated while that stream is current, so torch's caching allocator ties them to the stream the kernels run
on: a workspace freed on return cannot be handed to other work before those kernels have finished with it.
Errors raise MoeError with the library's message, before anything is launched.
"""
from __future__ import annotations

import contextlib
import ctypes as C

import torch

from . import _lib
from ._lib import MoeError, check, dims

_TORCH_DT = {_lib.DT_FLOAT16: torch.float16, _lib.DT_INT32: torch.int32}


def _stream(stream) -> "torch.cuda.Stream":
    return stream if stream is not None else torch.cuda.current_stream()


def _stream_ptr(stream) -> int:
    return int(_stream(stream).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise MoeError(1, f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise MoeError(4, f"{name} must be a device tensor (got {t.device})")
    if t.dtype != dtype:
        raise MoeError(4, f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise MoeError(4, f"{name} must be contiguous (ND format)")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def infer_routing(x_shape, w_gate_shape, topK: int = 2):
    lib = _lib.load()
    ids, w = dims([0, 0]), dims([0, 0])
    check(lib.moe_routing_topk_infer_shape(dims(x_shape), len(x_shape), dims(w_gate_shape), len(w_gate_shape),
                                           topK, ids, w))
    t_ids, t_w = C.c_int32(), C.c_int32()
    check(lib.moe_routing_topk_infer_dtype(C.byref(t_ids), C.byref(t_w)))
    return (tuple(ids), _TORCH_DT[t_ids.value]), (tuple(w), _TORCH_DT[t_w.value])


def infer_expert_ffn(x_shape, ids_shape, ew_shape, intermediateSize: int = 0):
    lib = _lib.load()
    out, inter = dims([0, 0, 0]), C.c_int64()
    check(lib.moe_expert_ffn_infer_shape(dims(x_shape), len(x_shape), dims(ids_shape), len(ids_shape),
                                         dims(ew_shape), len(ew_shape), intermediateSize, out, C.byref(inter)))
    dt = C.c_int32()
    check(lib.moe_expert_ffn_infer_dtype(C.byref(dt)))
    return tuple(out), _TORCH_DT[dt.value], inter.value


def infer_combine(eo_shape, ids_shape=None):
    lib = _lib.load()
    y = dims([0, 0])
    ids_arr = dims(ids_shape) if ids_shape is not None else None
    check(lib.moe_combine_infer_shape(dims(eo_shape), len(eo_shape), ids_arr,
                                      len(ids_shape) if ids_shape is not None else 0, y))
    dt = C.c_int32()
    check(lib.moe_combine_infer_dtype(C.byref(dt)))
    return tuple(y), _TORCH_DT[dt.value]


def workspace_bytes(T: int, H: int, E: int, K: int, I: int) -> int:
    return int(_lib.load().moe_expert_ffn_workspace_bytes(T, H, E, K, I))


def layer_workspace_bytes(T: int, H: int, E: int, K: int, I: int) -> int:
    return int(_lib.load().moe_layer_workspace_bytes(T, H, E, K, I))


def MoeRoutingTopK(x: torch.Tensor, w_gate: torch.Tensor, topK: int = 2, stream=None):
    """x[T,H] fp16, w_gate[H,E] fp16 -> (expert_ids[T,K] int32, weights[T,K] fp16)."""
    _need(x, "x", torch.float16)
    _need(w_gate, "w_gate", torch.float16)
    (ids_shape, ids_dt), (w_shape, w_dt) = infer_routing(tuple(x.shape), tuple(w_gate.shape), topK)
    s = _stream(stream)
    with torch.cuda.stream(s):
        ids = torch.empty(ids_shape, dtype=ids_dt, device=x.device)
        w = torch.empty(w_shape, dtype=w_dt, device=x.device)
    T, H = x.shape
    check(_lib.load().moe_routing_topk(x.data_ptr(), w_gate.data_ptr(), ids.data_ptr(), w.data_ptr(), T, H,
                                       w_gate.shape[1], ids_shape[1], int(s.cuda_stream)))
    return ids, w


def MoeExpertFFN(x: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor, expert_weights: torch.Tensor,
                 intermediateSize: int = 0, workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """-> expert_out[T,K,H] fp16. `workspace` (uint8, >= workspace_bytes) is allocated when not given."""
    _need(x, "x", torch.float16)
    _need(expert_ids, "expert_ids", torch.int32)
    _need(weights, "weights", torch.float16)
    _need(expert_weights, "expert_weights", torch.float16)
    out_shape, out_dt, inter = infer_expert_ffn(tuple(x.shape), tuple(expert_ids.shape),
                                                tuple(expert_weights.shape), intermediateSize)
    T, H = x.shape
    E, K = expert_weights.shape[0], expert_ids.shape[1]
    need = workspace_bytes(T, H, E, K, inter)
    s = _stream(stream)
    with torch.cuda.stream(s):
        if workspace is None:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        expert_out = torch.empty(out_shape, dtype=out_dt, device=x.device)
    check(_lib.load().moe_expert_ffn(x.data_ptr(), expert_ids.data_ptr(), weights.data_ptr(),
                                     expert_weights.data_ptr(), expert_out.data_ptr(), workspace.data_ptr(),
                                     workspace.numel() * workspace.element_size(), T, H, E, K, inter,
                                     int(s.cuda_stream)))
    return expert_out


def MoeCombine(expert_out: torch.Tensor, expert_ids: torch.Tensor | None, weights: torch.Tensor, topK: int = 2,
               stream=None) -> torch.Tensor:
    """expert_out[T,K,H] fp16, weights[T,K] fp16 -> y[T,H] fp16. K comes from expert_out (the attr is kept
    for signature parity, as in the reference's TilingFunc, op_host/moe_ops.cpp:432)."""
    del topK
    _need(expert_out, "expert_out", torch.float16)
    _need(weights, "weights", torch.float16)
    if expert_ids is not None:
        _need(expert_ids, "expert_ids", torch.int32)
    y_shape, y_dt = infer_combine(tuple(expert_out.shape), tuple(expert_ids.shape) if expert_ids is not None else None)
    T, K, H = expert_out.shape
    if tuple(weights.shape) != (T, K):
        raise MoeError(3, f"weights shape {tuple(weights.shape)} != {(T, K)}")
    s = _stream(stream)
    with torch.cuda.stream(s):
        y = torch.empty(y_shape, dtype=y_dt, device=expert_out.device)
    check(_lib.load().moe_combine(expert_out.data_ptr(), _ptr(expert_ids), weights.data_ptr(), y.data_ptr(), T, H, K,
                                  int(s.cuda_stream)))
    return y


def MoeExpertFFNCombine(x: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor,
                        expert_weights: torch.Tensor, intermediateSize: int = 0,
                        workspace: torch.Tensor | None = None, stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """MoeExpertFFN then MoeCombine in one call (moe_expert_ffn_combine): -> (expert_out[T,K,H], y[T,H]), both
    fp16, expert_out as MoeExpertFFN returns it and y bit-identical to MoeCombine(expert_out, ...)."""
    _need(x, "x", torch.float16)
    _need(expert_ids, "expert_ids", torch.int32)
    _need(weights, "weights", torch.float16)
    _need(expert_weights, "expert_weights", torch.float16)
    out_shape, out_dt, inter = infer_expert_ffn(tuple(x.shape), tuple(expert_ids.shape),
                                                tuple(expert_weights.shape), intermediateSize)
    T, H = x.shape
    E, K = expert_weights.shape[0], expert_ids.shape[1]
    if tuple(weights.shape) != (T, K):
        raise MoeError(3, f"weights shape {tuple(weights.shape)} != {(T, K)}")
    need = workspace_bytes(T, H, E, K, inter)
    s = _stream(stream)
    with torch.cuda.stream(s):
        if workspace is None:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        expert_out = torch.empty(out_shape, dtype=out_dt, device=x.device)
        y = torch.empty((T, H), dtype=torch.float16, device=x.device)
    check(_lib.load().moe_expert_ffn_combine(x.data_ptr(), expert_ids.data_ptr(), weights.data_ptr(),
                                             expert_weights.data_ptr(), expert_out.data_ptr(), y.data_ptr(),
                                             workspace.data_ptr(), workspace.numel() * workspace.element_size(), T,
                                             H, E, K, inter, int(s.cuda_stream)))
    return expert_out, y


def moe_layer(x: torch.Tensor, w_gate: torch.Tensor, expert_weights: torch.Tensor, topK: int = 2,
              workspace: torch.Tensor | None = None, stream=None):
    """The three operators chained as the reference harness chains them (tests/test_moe.cpp:444-463).
    Returns (y, expert_ids, weights, expert_out)."""
    ids, w = MoeRoutingTopK(x, w_gate, topK, stream=stream)
    eo = MoeExpertFFN(x, ids, w, expert_weights, 0, workspace, stream=stream)
    y = MoeCombine(eo, ids, w, topK, stream=stream)
    return y, ids, w, eo


def moe_layer_fused(x: torch.Tensor, w_gate: torch.Tensor, expert_weights: torch.Tensor, topK: int = 2,
                    intermediateSize: int = 0, workspace: torch.Tensor | None = None, stream=None):
    """The whole layer in one library call (moe_layer): the routing kernel also ranks the slots for the FFN's
    permute. Returns (y, expert_ids, weights, expert_out), bit-identical to moe_layer's."""
    _need(x, "x", torch.float16)
    _need(w_gate, "w_gate", torch.float16)
    _need(expert_weights, "expert_weights", torch.float16)
    (ids_shape, ids_dt), (w_shape, w_dt) = infer_routing(tuple(x.shape), tuple(w_gate.shape), topK)
    out_shape, out_dt, inter = infer_expert_ffn(tuple(x.shape), ids_shape, tuple(expert_weights.shape),
                                                intermediateSize)
    T, H = x.shape
    E, K = expert_weights.shape[0], ids_shape[1]
    need = layer_workspace_bytes(T, H, E, K, inter)
    s = _stream(stream)
    with torch.cuda.stream(s):
        if workspace is None:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        ids = torch.empty(ids_shape, dtype=ids_dt, device=x.device)
        w = torch.empty(w_shape, dtype=w_dt, device=x.device)
        expert_out = torch.empty(out_shape, dtype=out_dt, device=x.device)
        y = torch.empty((T, H), dtype=torch.float16, device=x.device)
    check(_lib.load().moe_layer(x.data_ptr(), w_gate.data_ptr(), expert_weights.data_ptr(), ids.data_ptr(),
                                w.data_ptr(), expert_out.data_ptr(), y.data_ptr(), workspace.data_ptr(),
                                workspace.numel() * workspace.element_size(), T, H, E, K, inter,
                                int(s.cuda_stream)))
    return y, ids, w, expert_out


def synth_normal_f16_(out: torch.Tensor, seed: int, stream_id: int, sigma_a: float, sigma_b: float | None = None,
                      period: int = 0, split: int = 0, stream=None) -> torch.Tensor:
    """Fill an fp16 device tensor in place with the generator of synth.py (moe_synth_normal_f16)."""
    _need(out, "out", torch.float16)
    if sigma_b is None or period <= 0:
        sigma_b, period, split = sigma_a, 1, 1
    check(_lib.load().moe_synth_normal_f16(out.data_ptr(), out.numel(), seed, stream_id, sigma_a, sigma_b, period,
                                           split, _stream_ptr(stream)))
    return out


def copy_bytes_(dst: torch.Tensor, src: torch.Tensor, stream=None) -> None:
    n = src.numel() * src.element_size()
    check(_lib.load().moe_copy_bytes(dst.data_ptr(), src.data_ptr(), n, _stream_ptr(stream)))


def stream_read_(src: torch.Tensor, stream=None) -> None:
    """Read a device tensor (size a multiple of 16 KiB) with moe_stream_read_bytes: achievable HBM read rate."""
    n = src.numel() * src.element_size()
    check(_lib.load().moe_stream_read_bytes(src.data_ptr(), n, _stream_ptr(stream)))


@contextlib.contextmanager
def kernel_trace():
    """Record HIP events around every kernel the library launches; yields a dict filled on exit with
    {kernel_name: (launches, total_ms)}."""
    lib = _lib.load()
    result: dict[str, tuple[int, float]] = {}
    check(lib.moe_trace_enable(1))
    try:
        yield result
    finally:
        n = lib.moe_trace_collect()
        for i in range(n):
            name, launches, ms = C.c_char_p(), C.c_int64(), C.c_double()
            check(lib.moe_trace_get(i, C.byref(name), C.byref(launches), C.byref(ms)))
            result[name.value.decode()] = (launches.value, ms.value)
        check(lib.moe_trace_enable(0))
