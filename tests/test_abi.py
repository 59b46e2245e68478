"""The C-ABI library on the CPU: it loads, exports every function include/*.h declares, and its host logic
(InferShape / InferDataType / planning / argument checks) behaves like the reference's op_host layer.
No kernel is launched here: every launch call below fails validation before reaching the GPU."""
from __future__ import annotations

import ctypes as C
import pathlib
import re

import pytest

from conftest import ROOT, package

pkg = package()
lib_mod = pkg._lib
MOE_OK, ERR_NULL, ERR_RANK, ERR_SHAPE, ERR_ARG, ERR_WS, ERR_UNSUP = 0, 1, 2, 3, 4, 5, 6


@pytest.fixture(scope="module")
def lib():
    return lib_mod.load()


def declared_functions() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"^[A-Za-z_][\w \*]*?\b(moe_\w+)\s*\(", text, flags=re.M))
    return names


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 20
    for n in sorted(names):
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    assert names == set(lib_mod.SIGNATURES), "ctypes binding and headers disagree"


def test_status_strings_and_version(lib):
    for code, name in lib_mod.STATUS_NAMES.items():
        assert lib.moe_status_string(code).decode() == name
    assert b"gfx950" in lib.moe_version()


def _routing_infer(lib, xd, wd, k):
    ids, w = lib_mod.dims([0, 0]), lib_mod.dims([0, 0])
    st = lib.moe_routing_topk_infer_shape(lib_mod.dims(xd), len(xd), lib_mod.dims(wd), len(wd), k, ids, w)
    return st, tuple(ids), tuple(w)


def test_routing_infer_shape(lib):
    assert _routing_infer(lib, [128, 2048], [2048, 16], 2) == (MOE_OK, (128, 2), (128, 2))
    assert _routing_infer(lib, [7, 64], [64, 4], 0) == (MOE_OK, (7, 2), (7, 2))  # attr default topK=2
    assert _routing_infer(lib, [7, 64], [64, 8], 6)[0] == MOE_OK
    assert _routing_infer(lib, [7, 64, 1], [64, 4], 2)[0] == ERR_RANK
    assert _routing_infer(lib, [7, 64], [32, 4], 2)[0] == ERR_SHAPE
    assert b"hiddenSize mismatch" in lib.moe_last_error()
    assert _routing_infer(lib, [7, 64], [64, 4], 5)[0] == ERR_ARG
    a, b = C.c_int32(), C.c_int32()
    assert lib.moe_routing_topk_infer_dtype(C.byref(a), C.byref(b)) == MOE_OK
    assert (a.value, b.value) == (lib_mod.DT_INT32, lib_mod.DT_FLOAT16)


def _ffn_infer(lib, xd, idd, ewd, attr=0):
    out, inter = lib_mod.dims([0, 0, 0]), C.c_int64()
    st = lib.moe_expert_ffn_infer_shape(lib_mod.dims(xd), len(xd), lib_mod.dims(idd), len(idd), lib_mod.dims(ewd),
                                        len(ewd), attr, out, C.byref(inter))
    return st, tuple(out), inter.value


def test_expert_ffn_infer_shape(lib):
    assert _ffn_infer(lib, [128, 2048], [128, 2], [16, 3 * 8192, 2048]) == (MOE_OK, (128, 2, 2048), 8192)
    assert _ffn_infer(lib, [128, 2048], [128, 2], [16, 3 * 8192, 2048], 8192)[0] == MOE_OK
    assert _ffn_infer(lib, [128, 2048], [128, 2], [16, 3 * 8192, 2048], 4096)[0] == ERR_SHAPE
    assert _ffn_infer(lib, [128, 2048], [128, 2], [16, 3 * 8192 + 1, 2048])[0] == ERR_SHAPE
    assert _ffn_infer(lib, [128, 2048], [128, 2], [16, 3 * 8192])[0] == ERR_RANK
    assert _ffn_infer(lib, [128, 2048], [128], [16, 3 * 8192, 2048])[0] == ERR_RANK
    assert _ffn_infer(lib, [128, 2048], [64, 2], [16, 3 * 8192, 2048])[0] == ERR_SHAPE
    assert _ffn_infer(lib, [128, 1024], [128, 2], [16, 3 * 8192, 2048])[0] == ERR_SHAPE
    dt = C.c_int32()
    assert lib.moe_expert_ffn_infer_dtype(C.byref(dt)) == MOE_OK and dt.value == lib_mod.DT_FLOAT16


def test_combine_infer_shape(lib):
    y = lib_mod.dims([0, 0])
    assert lib.moe_combine_infer_shape(lib_mod.dims([128, 2, 2048]), 3, lib_mod.dims([128, 2]), 2, y) == MOE_OK
    assert tuple(y) == (128, 2048)
    assert lib.moe_combine_infer_shape(lib_mod.dims([128, 2, 2048]), 3, None, 0, y) == MOE_OK
    assert lib.moe_combine_infer_shape(lib_mod.dims([128, 2048]), 2, None, 0, y) == ERR_RANK
    assert lib.moe_combine_infer_shape(lib_mod.dims([128, 2, 2048]), 3, lib_mod.dims([128, 3]), 2, y) == ERR_SHAPE
    assert lib.moe_combine_infer_shape(lib_mod.dims([128, 2, 2048]), 3, lib_mod.dims([128, 2, 1]), 3, y) == ERR_RANK


def test_plans(lib):
    rp = lib_mod.RoutingPlan()
    assert lib.moe_routing_topk_plan(128, 2048, 16, 2, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.workspace_bytes) == (8, 1024, 16, 0)
    # 16 waves x (16 tokens x 16 experts of fp32 partials + a w_gate stage of 32 rows x 16 fp16 experts)
    # 16 waves: partial logits (16 tokens x 16 experts fp32), a 32-row w_gate stage, a 2 KB x stage each
    assert rp.lds_bytes == 16 * (16 * 16 * 4 + 32 * 16 * 2 + 2048)
    # 32 < E <= 64: 4 waves per 16 tokens, or per 2 blocks of 16 when T keeps 256 workgroups busy
    assert lib.moe_routing_topk_plan(2048, 2048, 64, 6, C.byref(rp)) == MOE_OK
    # 4 waves x (16 tokens x 64 experts of fp32 partials + a w_gate stage of 32 rows x 64 fp16 experts)
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.lds_bytes) == (128, 256, 16, 4 * (16 * 64 * 4 + 32 * 64 * 2))
    # 32 < E <= 64 below 32768 tokens: the narrow kernel, at most 2 token blocks a workgroup, so two 48 KB
    # workgroups share a CU
    assert lib.moe_routing_topk_plan(16384, 2048, 64, 6, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.lds_bytes) == (512, 256, 32, 4 * (32 * 64 * 4 + 32 * 64 * 2))
    # from 32768 tokens (H = 1024 or 2048): the resident kernel, one 8-wave workgroup per CU over a run of
    # 16-token blocks (8 at T = 32768), an x ring of four 32 KB slots, the partials of 4 virtual waves and the
    # logits of 4 blocks awaiting selection
    assert lib.moe_routing_topk_plan(32768, 2048, 64, 6, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block) == (256, 512, 128)
    assert rp.lds_bytes == 4 * 32768 + 4 * 16 * 64 * 4 + 4 * 16 * 64 * 4 == 160 * 1024
    assert lib.moe_routing_topk_plan(32780, 2048, 64, 6, C.byref(rp)) == MOE_OK  # 2049 blocks: 9 a workgroup
    assert (rp.grid, rp.block, rp.tokens_per_block) == (228, 512, 144)
    assert lib.moe_routing_topk_plan(32768, 4096, 64, 6, C.byref(rp)) == MOE_OK  # H not 1024 or 2048: narrow
    assert (rp.grid, rp.block, rp.tokens_per_block) == (1024, 256, 32)
    # E <= 32: the narrow kernel at any T (16 waves, up to 4 token blocks a workgroup)
    assert lib.moe_routing_topk_plan(8192, 2048, 16, 2, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.lds_bytes) == (256, 1024, 32, 16 * (32 * 16 * 4 + 32 * 16 * 2))
    # E > 64: 64 tokens per workgroup; the rows kernel (4 waves of 16 tokens over all of H, four 16 KB w_gate
    # stages, each wave's x ring of 16 + 1 k-steps of 1 KB)
    assert lib.moe_routing_topk_plan(16384, 2048, 256, 8, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block) == (256, 256, 64)
    assert rp.lds_bytes == 4 * 16384 + 4 * (16 + 1) * 1024  # the rows kernel: 4 w_gate stages, x rings
    # E > 64 and T <= 8192: 16 tokens per workgroup; the quarters kernel (4 waves, each a quarter of H through two
    # 16 KB w_gate stages and two 1 KB x stages of its own)
    assert lib.moe_routing_topk_plan(128, 7168, 256, 8, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.lds_bytes) == (8, 256, 16, 4 * (2 * 16384 + 2 * 1024))
    assert lib.moe_routing_topk_plan(8192, 2048, 128, 8, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block, rp.lds_bytes) == (512, 256, 16, 4 * (2 * 16384 + 2 * 2 * 1024))
    # E % 8 != 0 (no 16-byte w_gate rows): the wide kernel, w_gate transposed through LDS
    assert lib.moe_routing_topk_plan(16384, 2048, 250, 8, C.byref(rp)) == MOE_OK
    assert (rp.grid, rp.block, rp.tokens_per_block) == (256, 256, 64)
    assert rp.lds_bytes == 2 * 256 * (2 * 32 + 8) * 2 + 64 * 256 * 4  # 2 stages of 64 h, fp32 logits
    assert lib.moe_routing_topk_plan(128, 2040, 16, 2, C.byref(rp)) == ERR_UNSUP
    assert lib.moe_routing_topk_plan(128, 2048, 300, 2, C.byref(rp)) == ERR_UNSUP
    fp = lib_mod.FfnPlan()
    assert lib.moe_expert_ffn_plan(128, 2048, 16, 2, 8192, C.byref(fp)) == MOE_OK
    ws = lib.moe_expert_ffn_workspace_bytes(128, 2048, 16, 2, 8192)
    assert fp.workspace_bytes == ws
    # offsets + sorted slots + the fp16 [T*K, I] intermediate + fp32 split-K partials of the down projection
    # (I = 8192 is split into 4 K-ranges of 2048) + the slot -> sorted-row map, each 256-byte aligned
    assert ws == 256 + 1024 + 128 * 2 * 8192 * 2 + 4 * 128 * 2 * 2048 * 4 + 1024
    assert fp.permute_grid == 0 and fp.gateup_grid > 0 and fp.down_grid > 0  # streaming: no permute kernels
    assert lib.moe_expert_ffn_plan(8192, 2048, 16, 2, 8192, C.byref(fp)) == MOE_OK
    assert fp.schedule == 1 and fp.permute_grid == 16  # 16384 slots in chunks of 1024
    assert lib.moe_expert_ffn_workspace_bytes(128, 2048, 16, 2, 8200) == 0  # I % 32 != 0
    assert lib.moe_expert_ffn_plan(16384, 2048, 64, 6, 1408, C.byref(fp)) == MOE_OK
    cp = lib_mod.CombinePlan()
    assert lib.moe_combine_plan_for(128, 2048, 2, C.byref(cp)) == MOE_OK
    assert cp.grid * cp.block * cp.elems_per_thread >= 128 * 2048 and cp.workspace_bytes == 0


def test_streaming_plan_grids(lib):
    """The weight-streaming schedule's launch grids as the plan reports them (units of 128 gate/up columns or 256
    down columns, times the K-ranges of the layout): with T*K <= E the K-ranges are halved until T*K experts would
    make 128 units, and the wide kernels (which never split H) take over from ~18-22 rows per expert, or from 4
    where the 32-row gate/up must split H."""
    from conftest import package

    lib_mod = package()._lib
    fp = lib_mod.FfnPlan()

    def grids(T, H, E, K, I):
        assert lib.moe_expert_ffn_plan(T, H, E, K, I, C.byref(fp)) == MOE_OK
        assert fp.schedule == 0
        return fp.gateup_grid, fp.down_grid

    # T = 1 at H = 2048, E = 64, K = 6, I = 1408: 6 slots x 11 column groups = 66 units -> H in 2 K-ranges (132);
    # down 6 x 8 = 48 -> I in 4 K-ranges of 352 (192)
    assert grids(1, 2048, 64, 6, 1408) == (64 * 11 * 2, 64 * 8 * 4)
    # T = 1 at H = 2048, E = 16, K = 2, I = 8192: gate/up 2 x 64 = 128 units, whole H; down 2 x 8 x 4 = 64 ->
    # I in 8 K-ranges of 1024
    assert grids(1, 2048, 16, 2, 8192) == (16 * 64, 16 * 8 * 8)
    # T*K > E: the layouts of a decode batch (down over 4 K-ranges of 2048)
    assert grids(128, 2048, 16, 2, 8192) == (16 * 64, 16 * 8 * 4)
    # DeepSeek-V3's experts at 4 rows per expert: the wide kernels (whole H) instead of 4 K-ranges of 1792
    assert grids(128, 7168, 256, 8, 2048) == (256 * 16, 256 * 28)
    # ... and at 2 rows per expert the 32-row kernels, H in 4 K-ranges
    assert grids(64, 7168, 256, 8, 2048)[0] == 256 * 16 * 4


def test_ffn_plan_at_the_32bit_bounds(lib):
    """Many rows per expert pick the LDS-tiled schedule also past 2 GiB of SwiGLU intermediate (hidden is
    addressed per tile); past its real 32-bit bounds (2 GiB of gathered x rows) the shape is rejected, never
    sent to the weight-streaming schedule, which would re-stream every expert's weights once per 32 rows."""
    fp = lib_mod.FfnPlan()
    assert lib.moe_expert_ffn_plan(65536, 2048, 16, 2, 8192, C.byref(fp)) == MOE_OK
    assert fp.schedule == 1
    assert fp.workspace_bytes >= 65536 * 2 * 8192 * 2  # hidden alone is 2 GiB
    assert lib.moe_expert_ffn_plan(65536, 256, 4, 2, 8192, C.byref(fp)) == MOE_OK and fp.schedule == 1
    # T*H*2 = 2 GiB of x: unsupported (explicitly), not the streaming schedule
    assert lib.moe_expert_ffn_plan(1 << 20, 1024, 16, 2, 1024, C.byref(fp)) == ERR_UNSUP
    assert b"32-bit" in lib.moe_last_error()
    assert lib.moe_expert_ffn_workspace_bytes(1 << 20, 1024, 16, 2, 1024) == 0
    # few rows per expert stay on the streaming schedule whatever their size
    assert lib.moe_expert_ffn_plan(128, 2048, 16, 2, 8192, C.byref(fp)) == MOE_OK and fp.schedule == 0


FAKE = 1 << 20  # non-null, 16-byte aligned, never dereferenced: every call below fails validation first


def test_launch_argument_errors_return_before_launch(lib):
    assert lib.moe_routing_topk(None, None, None, None, 4, 64, 4, 2, None) == ERR_NULL
    assert lib.moe_routing_topk(FAKE, FAKE, FAKE, FAKE, 4, 64, 4, 5, None) == ERR_ARG
    assert lib.moe_routing_topk(FAKE, FAKE, FAKE, FAKE, 4, 60, 4, 2, None) == ERR_UNSUP
    assert lib.moe_routing_topk(FAKE + 2, FAKE, FAKE, FAKE, 4, 64, 4, 2, None) == ERR_UNSUP  # misaligned x
    assert lib.moe_routing_topk(None, None, None, None, 0, 64, 4, 2, None) == MOE_OK  # T = 0: no-op
    need = lib.moe_expert_ffn_workspace_bytes(4, 64, 4, 2, 256)
    args = (4, 64, 4, 2, 256, None)
    assert lib.moe_expert_ffn(FAKE, FAKE, FAKE, FAKE, FAKE, None, need, *args) == ERR_WS
    assert lib.moe_expert_ffn(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need - 1, *args) == ERR_WS
    assert b"need" in lib.moe_last_error()
    assert lib.moe_expert_ffn(None, FAKE, FAKE, FAKE, FAKE, FAKE, need, *args) == ERR_NULL
    assert lib.moe_expert_ffn(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, 4, 64, 4, 5, 256, None) == ERR_ARG
    assert lib.moe_expert_ffn(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, 4, 64, 4, 2, 0, None) == ERR_ARG
    # the fused FFN + combine checks both operators' rules before any launch
    fused = lib.moe_expert_ffn_combine
    assert fused(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need - 1, *args) == ERR_WS
    assert fused(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, need, *args) == ERR_NULL  # y
    assert fused(FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE, need, *args) == ERR_NULL  # weights: used here
    assert fused(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE + 2, FAKE, need, *args) == ERR_UNSUP  # misaligned y
    assert fused(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, 4, 64, 4, 5, 256, None) == ERR_ARG
    assert fused(None, None, None, None, None, None, None, 0, 0, 64, 4, 2, 256, None) == MOE_OK  # T = 0
    # the whole layer checks the three operators' rules and its own workspace before any launch
    lneed = lib.moe_layer_workspace_bytes(4, 64, 4, 2, 256)
    assert lneed >= need
    layer = lib.moe_layer
    assert layer(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, lneed - 1, *args) == ERR_WS
    assert layer(FAKE, None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, lneed, *args) == ERR_NULL  # w_gate
    assert layer(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE + 2, FAKE, lneed, *args) == ERR_UNSUP  # misaligned y
    assert layer(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, lneed, 4, 64, 4, 5, 256, None) == ERR_ARG
    assert layer(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, lneed, 4, 60, 4, 2, 256, None) == ERR_UNSUP
    assert layer(None, None, None, None, None, None, None, None, 0, 0, 64, 4, 2, 256, None) == MOE_OK  # T = 0
    assert lib.moe_combine(None, None, None, None, 4, 64, 2, None) == ERR_NULL
    assert lib.moe_combine(FAKE, None, FAKE, FAKE, 4, 60, 2, None) == ERR_UNSUP
    assert lib.moe_combine(FAKE, None, FAKE, FAKE, 4, 64, 0, None) == ERR_ARG
    assert lib.moe_synth_normal_f16(None, 10, 0, 0, 1.0, 1.0, 1, 1, None) == ERR_NULL
    assert lib.moe_copy_bytes(FAKE, FAKE, 17, None) == ERR_ARG
    assert lib.moe_stream_read_bytes(None, 16384, None) == ERR_NULL
    assert lib.moe_stream_read_bytes(FAKE, 16000, None) == ERR_ARG


def test_layer_workspace_adds_the_routing_counts_on_the_tiled_schedule(lib):
    # streaming schedule (decode): the FFN's workspace as it is
    assert lib.moe_layer_workspace_bytes(128, 2048, 16, 2, 8192) == lib.moe_expert_ffn_workspace_bytes(128, 2048, 16, 2, 8192)
    # tiled schedule: + one row of counts_stride(E) int32 per 16 tokens (the most routing workgroups any routing
    # kernel runs), 256-byte aligned
    for T, E in ((16384, 64), (8192, 16), (3000, 130), (3001, 13)):
        ffn = lib.moe_expert_ffn_workspace_bytes(T, 2048, E, 6, 1408)
        extra = ((T + 15) // 16 * ((E + 3) // 4 * 4) * 4 + 255) // 256 * 256
        assert lib.moe_layer_workspace_bytes(T, 2048, E, 6, 1408) == ffn + extra, (T, E)
    assert lib.moe_layer_workspace_bytes(128, 2048, 16, 2, 8200) == 0  # I % 32 != 0


def test_top_k_up_to_the_expert_count(lib):
    rp = lib_mod.RoutingPlan()
    fp = lib_mod.FfnPlan()
    for E, K in ((64, 64), (256, 256), (48, 40)):
        assert lib.moe_routing_topk_plan(1000, 2048, E, K, C.byref(rp)) == MOE_OK, (E, K)
        assert lib.moe_expert_ffn_plan(1000, 2048, E, K, 1408, C.byref(fp)) == MOE_OK, (E, K)
        assert lib.moe_layer_workspace_bytes(1000, 2048, E, K, 1408) > 0
    assert lib.moe_routing_topk_plan(1000, 2048, 64, 65, C.byref(rp)) == ERR_ARG  # K > E


def test_last_error_is_cleared_on_success(lib):
    assert _routing_infer(lib, [7, 64], [32, 4], 2)[0] == ERR_SHAPE
    assert lib.moe_last_error() != b""
    assert _routing_infer(lib, [7, 64], [64, 4], 2)[0] == MOE_OK
    assert lib.moe_last_error() == b""


def test_trace_api_without_launches(lib):
    assert lib.moe_trace_enable(1) == MOE_OK
    assert lib.moe_trace_collect() == 0
    assert lib.moe_trace_get(0, None, None, None) == ERR_ARG
    assert lib.moe_trace_enable(0) == MOE_OK


def test_python_mirror_validates_before_launch():
    torch = pytest.importorskip("torch")
    ops = pkg.ops
    with pytest.raises(lib_mod.MoeError):
        ops.MoeRoutingTopK(torch.zeros(4, 64, dtype=torch.float16), torch.zeros(64, 4, dtype=torch.float16))  # CPU
    assert ops.infer_routing((9, 64), (64, 8), 3)[0] == ((9, 3), torch.int32)
    assert ops.infer_expert_ffn((9, 64), (9, 3), (8, 96, 64))[:2] == ((9, 3, 64), torch.float16)
    assert ops.infer_combine((9, 3, 64))[0] == (9, 64)
    with pytest.raises(lib_mod.MoeError) as err:
        ops.infer_expert_ffn((9, 64), (9, 3), (8, 96, 64), intermediateSize=64)
    assert err.value.status == ERR_SHAPE


def test_package_fails_loudly_without_library(tmp_path, monkeypatch):
    monkeypatch.setattr(lib_mod, "LIB_PATH", pathlib.Path(tmp_path) / "missing.so")
    monkeypatch.setattr(lib_mod, "_lib", None)
    with pytest.raises(RuntimeError, match="no\\s+CPU fallback"):
        lib_mod.load()
