"""TEST INFRASTRUCTURE, NOT PRODUCT CODE: ctypes access to the CPU oracle and to the reference simulator.

    liboracle.so            oracle/moe_oracle.cpp, the C++ restatement of tests/moe_cpu_sim.cpp (reference)
    _ref/libref_moe_sim.so  the reference's own tests/moe_cpu_sim.cpp, compiled from its source by
                            oracle/Makefile (present only where the reference checkout was available at build
                            time; it travels with the tree as a built file)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the
checker or the timed CPU baseline, never as the thing measured on the GPU.
All arrays are numpy; inputs are float32 (fp16 tensors are passed as their exact float32 upcasts).
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libref_moe_sim.so"

_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int32)
_D = C.POINTER(C.c_double)
_I64 = C.c_int64

_oracle = None
_ref = None


def build(reference_dir: str | None = "/root/reference") -> None:
    """Build liboracle.so, and _ref/ when the reference checkout exists."""
    targets = ["oracle"]
    if reference_dir and (pathlib.Path(reference_dir) / "tests" / "moe_cpu_sim.cpp").exists():
        targets.append("ref")
    cmd = ["make", "-s", "-B", "-C", str(HERE), *targets]
    if reference_dir:
        cmd.append(f"REF={reference_dir}")
    subprocess.run(cmd, check=True)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _ip(a: np.ndarray):
    return a.ctypes.data_as(_I)


def lib() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            raise RuntimeError(f"{ORACLE_LIB} missing: run oracle.build()")
        L = C.CDLL(str(ORACLE_LIB))
        L.oracle_routing.argtypes = [_F, _F, _I64, _I64, _I64, _I64, _I, _F, _F, _F]
        L.oracle_expert_ffn.argtypes = [_F, _I, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F]
        L.oracle_expert_ffn_tiled.argtypes = [_F, _I, _F, _I64, _I64, _I64, _I64, _I64, _F]
        L.oracle_combine.argtypes = [_F, _F, _I64, _I64, _I64, _F]
        L.oracle_moe_layer.argtypes = [_F, _F, _F, _I64, _I64, _I64, _I64, _I64, C.c_int, _I, _F, _F, _F]
        L.oracle_compare.argtypes = [_F, _F, _I64, _D]
        L.oracle_compare.restype = None
        for n in ("oracle_routing", "oracle_expert_ffn", "oracle_expert_ffn_tiled", "oracle_combine",
                  "oracle_moe_layer"):
            getattr(L, n).restype = C.c_int
        _oracle = L
    return _oracle


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"{what}: oracle rejected the arguments")


# ------------------------------------------------------------------------------------------------------------
# Oracle (restatement)
# ------------------------------------------------------------------------------------------------------------

def routing(x, w_gate, K: int):
    """-> (expert_ids [T,K] int32, weights [T,K] f32, probs [T,E] f32, logits [T,E] f32)."""
    x, w_gate = _f32(x), _f32(w_gate)
    T, H = x.shape
    E = w_gate.shape[1]
    ids = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    probs = np.empty((T, E), np.float32)
    logits = np.empty((T, E), np.float32)
    _ok(lib().oracle_routing(_fp(x), _fp(w_gate), T, H, E, K, _ip(ids), _fp(w), _fp(probs), _fp(logits)), "routing")
    return ids, w, probs, logits


def expert_ffn(x, expert_ids, expert_weights, I: int, t_begin: int = 0, t_end: int | None = None,
               tiled: bool = False) -> np.ndarray:
    """-> expert_out [T,K,H] f32 (rows outside [t_begin, t_end) are NaN for the naive schedule)."""
    x, ew = _f32(x), _f32(expert_weights)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    T, H = x.shape
    K = ids.shape[1]
    E = ew.shape[0]
    out = np.full((T, K, H), np.nan, np.float32)
    if tiled:
        _ok(lib().oracle_expert_ffn_tiled(_fp(x), _ip(ids), _fp(ew), T, H, E, K, I, _fp(out)), "expert_ffn_tiled")
    else:
        t_end = T if t_end is None else t_end
        _ok(lib().oracle_expert_ffn(_fp(x), _ip(ids), _fp(ew), T, H, E, K, I, t_begin, t_end, _fp(out)), "expert_ffn")
    return out


def combine(expert_out, weights) -> np.ndarray:
    eo, w = _f32(expert_out), _f32(weights)
    T, K, H = eo.shape
    y = np.empty((T, H), np.float32)
    _ok(lib().oracle_combine(_fp(eo), _fp(w), T, H, K, _fp(y)), "combine")
    return y


def moe_layer(x, w_gate, expert_weights, K: int, I: int, tiled: bool = False):
    """-> (y [T,H], expert_ids, weights, expert_out), all f32 except ids."""
    x, wg, ew = _f32(x), _f32(w_gate), _f32(expert_weights)
    T, H = x.shape
    E = wg.shape[1]
    ids = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    eo = np.empty((T, K, H), np.float32)
    y = np.empty((T, H), np.float32)
    _ok(lib().oracle_moe_layer(_fp(x), _fp(wg), _fp(ew), T, H, E, K, I, int(tiled), _ip(ids), _fp(w), _fp(eo),
                               _fp(y)), "moe_layer")
    return y, ids, w, eo


def compare(actual, expected) -> dict:
    """max abs, mean abs, cosine accumulated in double (tests/moe_cpu_sim.cpp:586-604 metric)."""
    a, b = _f32(actual).ravel(), _f32(expected).ravel()
    out = (C.c_double * 3)()
    lib().oracle_compare(_fp(a), _fp(b), a.size, out)
    return {"max_abs": out[0], "mean_abs": out[1], "cos": out[2]}


def topk_gaps(probs: np.ndarray, K: int):
    """Per token: (gap between the K-th and (K+1)-th probability, smallest gap between adjacent ranks within
    the top K). inf where undefined (K == E, or K == 1 for the within-top-K gap)."""
    p = -np.sort(-np.asarray(probs, dtype=np.float64), axis=1)
    E = p.shape[1]
    boundary = p[:, K - 1] - p[:, K] if K < E else np.full(p.shape[0], np.inf)
    inner = np.min(p[:, :K - 1] - p[:, 1:K], axis=1) if K > 1 else np.full(p.shape[0], np.inf)
    return boundary, inner


# ------------------------------------------------------------------------------------------------------------
# Reference simulator compiled from its own source
# ------------------------------------------------------------------------------------------------------------

def ref_available() -> bool:
    return REF_LIB.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise RuntimeError(f"{REF_LIB} missing (the reference checkout was not available at build time)")
        L = C.CDLL(str(REF_LIB))
        L.ref_gen_inputs.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint32, _F, _F, _F]
        L.ref_gen_inputs.restype = None
        L.ref_naive_moe.argtypes = [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F]
        L.ref_naive_moe.restype = None
        for n in ("ref_naive_moe_timed", "ref_tiled_moe_timed"):
            getattr(L, n).argtypes = [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F]
            getattr(L, n).restype = C.c_double
        L.ref_routing.argtypes = [_F, _F, C.c_int, C.c_int, C.c_int, C.c_int, _I, _F]
        L.ref_routing.restype = None
        L.ref_expert_ffn_tiled.argtypes = [_F, _F, _I, _F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F]
        L.ref_expert_ffn_tiled.restype = None
        L.ref_combine.argtypes = [_F, _I, _F, C.c_int, C.c_int, C.c_int, _F]
        L.ref_combine.restype = None
        L.ref_compare.argtypes = [_F, _F, _I64, _D]
        L.ref_compare.restype = None
        _ref = L
    return _ref


def ref_gen_inputs(T: int, H: int, E: int, I: int, seed: int):
    x = np.empty((T, H), np.float32)
    wg = np.empty((H, E), np.float32)
    ew = np.empty((E, 3 * I, H), np.float32)
    ref().ref_gen_inputs(T, H, E, I, seed, _fp(x), _fp(wg), _fp(ew))
    return x, wg, ew


def ref_naive_moe(x, w_gate, expert_weights, K: int, I: int) -> np.ndarray:
    x, wg, ew = _f32(x), _f32(w_gate), _f32(expert_weights)
    T, H = x.shape
    y = np.empty((T, H), np.float32)
    ref().ref_naive_moe(_fp(x), _fp(wg), _fp(ew), T, H, wg.shape[1], K, I, _fp(y))
    return y


def ref_moe_timed(x, w_gate, expert_weights, K: int, I: int, tiled: bool = False):
    """-> (y, milliseconds of the NaiveMoE / TiledMoE call alone)."""
    x, wg, ew = _f32(x), _f32(w_gate), _f32(expert_weights)
    T, H = x.shape
    y = np.empty((T, H), np.float32)
    fn = ref().ref_tiled_moe_timed if tiled else ref().ref_naive_moe_timed
    ms = fn(_fp(x), _fp(wg), _fp(ew), T, H, wg.shape[1], K, I, _fp(y))
    return y, ms


def ref_routing(x, w_gate, K: int):
    x, wg = _f32(x), _f32(w_gate)
    T, H = x.shape
    ids = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    ref().ref_routing(_fp(x), _fp(wg), T, H, wg.shape[1], K, _ip(ids), _fp(w))
    return ids, w


def ref_expert_ffn_tiled(x, expert_weights, expert_ids, weights, I: int) -> np.ndarray:
    x, ew, w = _f32(x), _f32(expert_weights), _f32(weights)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    T, H = x.shape
    K = ids.shape[1]
    out = np.empty((T, K, H), np.float32)
    ref().ref_expert_ffn_tiled(_fp(x), _fp(ew), _ip(ids), _fp(w), T, H, ew.shape[0], K, I, _fp(out))
    return out


def ref_combine(expert_out, expert_ids, weights) -> np.ndarray:
    eo, w = _f32(expert_out), _f32(weights)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    T, K, H = eo.shape
    y = np.empty((T, H), np.float32)
    ref().ref_combine(_fp(eo), _ip(ids), _fp(w), T, H, K, _fp(y))
    return y


def ref_compare(actual, expected) -> dict:
    a, b = _f32(actual).ravel(), _f32(expected).ravel()
    out = (C.c_double * 3)()
    ref().ref_compare(_fp(a), _fp(b), a.size, out)
    return {"max_abs": out[0], "mean_abs": out[1], "cos": out[2]}
