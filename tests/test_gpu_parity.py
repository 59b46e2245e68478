"""Parity of the HIP path (libmoe_mi355x.so through its C ABI) with the oracle and the reference's vectors.

Bars (thresholds from tests/test_moe.cpp:486-490):
  expert_ids  bit-exact, except tokens whose K-th and (K+1)-th probabilities, or two adjacent ranks inside
              the top K, differ by less than 1e-3 (reported, not failed);
  weights, expert_out, y   max abs < 0.05, mean abs < 0.01, cosine > 0.99, plus the tighter fp16 bounds below;
  combine     bit-exact against the oracle's fp32 combine of the same fp16 inputs, rounded to fp16;
  permute     bit-exact against a stable sort of the slots by expert.
Tolerance sources: fp16 rounding of weights, the SwiGLU intermediate, expert_out and y (relative 2^-11
each) and fp32 summation order (MFMA accumulation vs the oracle's sequential sums, ~sqrt(n) * 2^-24 relative).
At the BASELINE sizes the oracle runs on a sample of tokens; everything else is checked in full.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import oracle
from conftest import GOLDEN_CASES, load_golden, synth_module

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
synth = synth_module()

NS = dict(max_abs=0.05, mean_abs=0.01, cos=0.99)  # north_star thresholds
TIE_GAP = 1e-3         # the near-tie rule: a K-th / (K+1)-th or consecutive-pick probability gap below it
TIE_GAP_STRICT = 2e-5  # ids must match wherever every gap is at least this


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: "torch.Tensor") -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def within(metrics: dict, max_abs: float = NS["max_abs"], mean_abs: float = NS["mean_abs"], cos: float = NS["cos"]):
    assert metrics["max_abs"] < max_abs, metrics
    assert metrics["mean_abs"] < mean_abs, metrics
    assert metrics["cos"] > cos, metrics


def check_routing(ids_g: np.ndarray, w_g: np.ndarray, x16, wg16, K: int, tag: str):
    ids_o, w_o, probs, _ = oracle.routing(f32(x16), f32(wg16), K)
    boundary, inner = oracle.topk_gaps(probs, K)
    near = (boundary < TIE_GAP) | (inner < TIE_GAP)
    differ = (ids_g != ids_o).any(axis=1)
    # logits summed in another order move a probability by ~1e-7, so ids must also match wherever every gap is
    # at least TIE_GAP_STRICT (this binds at many experts, where most gaps are below TIE_GAP)
    close = (boundary < TIE_GAP_STRICT) | (inner < TIE_GAP_STRICT)
    log(f"[{tag}] routing: {len(ids_g)} tokens, {int(near.sum())} near-tie (gap < {TIE_GAP}), "
        f"{int(close.sum())} with a gap < {TIE_GAP_STRICT}, {int(differ.sum())} with different ids, all of them "
        f"near-tie: {bool(not (differ & ~near).any())}, within {TIE_GAP_STRICT}: {bool(not (differ & ~close).any())}")
    assert not (differ & ~near).any(), np.nonzero(differ & ~near)[0][:10]
    assert not (differ & ~close).any(), np.nonzero(differ & ~close)[0][:10]
    w_g = f32(w_g)
    ok = ~near
    if ok.any():
        # fp16 weights in [0, 1]: one fp16 ulp is <= 2^-11; logits summed in another order move p by ~1e-7
        assert np.max(np.abs(w_g[ok] - w_o[ok])) <= 2.0**-10
    within(oracle.compare(w_g, w_o))
    np.testing.assert_allclose(w_g.astype(np.float64).sum(axis=1), 1.0, atol=K * 2.0**-11)
    return ids_o, w_o


def check_permute(ws: np.ndarray, ids: np.ndarray, E: int):
    S = ids.size
    off_bytes = ((4 * (E + 1) + 255) // 256) * 256
    offsets = ws[: 4 * (E + 1)].view(np.int32)
    sorted_slot = ws[off_bytes: off_bytes + 4 * S].view(np.int32)
    flat = ids.ravel()
    valid = (flat >= 0) & (flat < E)
    expect_sorted = np.nonzero(valid)[0][np.argsort(flat[valid], kind="stable")]
    expect_off = np.concatenate([[0], np.cumsum(np.bincount(flat[valid], minlength=E))]).astype(np.int32)
    assert np.array_equal(offsets, expect_off)
    assert np.array_equal(sorted_slot[: expect_sorted.size], expect_sorted.astype(np.int32))


def run_ffn(ops, x_d, ids_d, w_d, ew_d, I):
    T, H = x_d.shape
    E, K = ew_d.shape[0], ids_d.shape[1]
    ws = torch.empty(ops.workspace_bytes(T, H, E, K, I), dtype=torch.uint8, device="cuda")
    eo = ops.MoeExpertFFN(x_d, ids_d, w_d, ew_d, 0, ws)
    return eo, ws


# ------------------------------------------------------------------------------------------------------------
# golden vectors (reference outputs) and stage-wise parity at the small shapes
# ------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLDEN_CASES)
def test_layer_matches_reference_golden(ops, case):
    log(f"[golden {case}] start")
    g = load_golden(case)
    K, I, E = g["K"], g["I"], g["E"]
    x_d, wg_d, ew_d = dev(g["x"]), dev(g["w_gate"]), dev(g["expert_weights"])

    ids_d, w_d = ops.MoeRoutingTopK(x_d, wg_d, K)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, g["x"], g["w_gate"], K, case)
    near_free = np.array_equal(ids, g["expert_ids"])

    eo_d, ws = run_ffn(ops, x_d, ids_d, w_d, ew_d, I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    eo_o = oracle.expert_ffn(f32(g["x"]), ids, f32(g["expert_weights"]), I)
    m_eo = oracle.compare(eo, eo_o)
    log(f"[golden {case}] expert_out vs oracle: {m_eo}")
    within(m_eo, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    if near_free:
        within(oracle.compare(eo, g["expert_out_tiled"]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)

    y_d = ops.MoeCombine(eo_d, ids_d, w_d, K)
    y = host(y_d)
    y_o = oracle.combine(eo, f32(w)).astype(np.float16)
    assert np.array_equal(y.view(np.uint16), y_o.view(np.uint16)), "combine not bit-exact"
    m_y = oracle.compare(f32(y), g["y_naive"])
    log(f"[golden {case}] y vs reference NaiveMoE: {m_y}")
    within(m_y)
    within(m_y, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_moe_layer_chain_equals_stagewise(ops):
    g = load_golden("synth_mid_seed43")
    x_d, wg_d, ew_d = dev(g["x"]), dev(g["w_gate"]), dev(g["expert_weights"])
    y, ids, w, eo = ops.moe_layer(x_d, wg_d, ew_d, g["K"])
    ids2, w2 = ops.MoeRoutingTopK(x_d, wg_d, g["K"])
    eo2, _ = run_ffn(ops, x_d, ids2, w2, ew_d, g["I"])
    y2 = ops.MoeCombine(eo2, ids2, w2)
    for a, b in ((y, y2), (ids, ids2), (w, w2), (eo, eo2)):
        assert torch.equal(a, b)  # deterministic: no atomics anywhere on the path


def test_layer_empty_and_single_token(ops):
    # T = 0: every operator and the fused path return empty outputs and launch nothing
    H, E, K, I = 256, 8, 2, 512
    rng = np.random.default_rng(11)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    wg_d, ew_d = dev(wg), dev(ew)
    y0, ids0, w0, eo0 = ops.moe_layer(torch.empty(0, H, dtype=torch.float16, device="cuda"), wg_d, ew_d, K)
    assert ids0.shape == (0, K) and w0.shape == (0, K) and eo0.shape == (0, K, H) and y0.shape == (0, H)
    eo0f, y0f = ops.MoeExpertFFNCombine(torch.empty(0, H, dtype=torch.float16, device="cuda"), ids0, w0, ew_d)
    assert eo0f.shape == (0, K, H) and y0f.shape == (0, H)
    torch.cuda.synchronize()

    # T = 1: one token through the whole layer against the oracle
    x = rng.standard_normal((1, H)).astype(np.float16)
    y_d, ids_d, w_d, eo_d = ops.moe_layer(dev(x), wg_d, ew_d, K)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, x, wg, K, "T=1")
    eo = f32(host(eo_d))
    within(oracle.compare(eo, oracle.expert_ffn(f32(x), ids, f32(ew), I)), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    y_o = oracle.combine(eo, f32(w)).astype(np.float16)
    assert np.array_equal(host(y_d).view(np.uint16), y_o.view(np.uint16))


@pytest.mark.parametrize("T,H,E,K,I,schedule", [
    (64, 256, 8, 2, 512, 0),
    (512, 256, 4, 2, 512, 1),
    (2, 512, 64, 6, 1024, 0),  # T*K <= E: units dealt over the active experts, gate/up and down K-ranges halved
])
def test_layer_graph_replay_matches_eager(ops, T, H, E, K, I, schedule):
    """The layer's three C-ABI calls captured in one HIP graph: each replay, after eager work that changes x and
    clears the graph's outputs, equals an eager run on the same x bit for bit (ids, weights, expert_out, y), and
    the replay's own outputs pass the oracle checks (routing, the expert FFN, the combine bit for bit)."""
    lib = ops._lib.load()
    log(f"[graph] T={T} H={H} E={E} K={K} I={I} schedule={ffn_schedule(T, H, E, K, I)}")
    gen = torch.Generator(device="cpu").manual_seed(T + I)
    x = (torch.randn(T, H, generator=gen)).half().cuda()
    wg = (torch.randn(H, E, generator=gen) / math.sqrt(H)).half().cuda()
    ew = (torch.randn(E, 3 * I, H, generator=gen) / math.sqrt(H)).half().cuda()
    ws_bytes = ops.workspace_bytes(T, H, E, K, I)
    assert ffn_schedule(T, H, E, K, I) == schedule

    def buffers():
        return dict(ids=torch.empty(T, K, dtype=torch.int32, device="cuda"),
                    w=torch.empty(T, K, dtype=torch.float16, device="cuda"),
                    eo=torch.empty(T, K, H, dtype=torch.float16, device="cuda"),
                    y=torch.empty(T, H, dtype=torch.float16, device="cuda"),
                    ws=torch.empty(ws_bytes, dtype=torch.uint8, device="cuda"))

    def step(b, s):
        st = lib.moe_routing_topk(x.data_ptr(), wg.data_ptr(), b["ids"].data_ptr(), b["w"].data_ptr(), T, H, E, K, s)
        st |= lib.moe_expert_ffn(x.data_ptr(), b["ids"].data_ptr(), b["w"].data_ptr(), ew.data_ptr(),
                                 b["eo"].data_ptr(), b["ws"].data_ptr(), ws_bytes, T, H, E, K, I, s)
        st |= lib.moe_combine(b["eo"].data_ptr(), b["ids"].data_ptr(), b["w"].data_ptr(), b["y"].data_ptr(),
                              T, H, K, s)
        assert st == 0, lib.moe_last_error()

    gb, eb = buffers(), buffers()
    step(gb, torch.cuda.current_stream().cuda_stream)  # first launches set the kernels' LDS attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(gb, torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        x.copy_((torch.randn(T, H, generator=gen)).half())
        step(eb, torch.cuda.current_stream().cuda_stream)
        for t in gb.values():
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name in ("ids", "w", "eo", "y"):
            assert torch.equal(gb[name], eb[name]), (i, name)
        ids, w = host(gb["ids"]), host(gb["w"])
        xh = host(x)
        check_routing(ids, w, xh, host(wg), K, f"graph replay {i}")
        eo = f32(host(gb["eo"]))
        within(oracle.compare(eo, oracle.expert_ffn(f32(xh), ids, f32(host(ew)), I)), max_abs=1e-2, mean_abs=1e-3,
               cos=0.9999)
        y_o = oracle.combine(eo, f32(w)).astype(np.float16)
        assert np.array_equal(host(gb["y"]).view(np.uint16), y_o.view(np.uint16)), i
    del g


@pytest.mark.parametrize("T,H,E,K,I,schedule", [
    (64, 256, 8, 2, 512, 0),
    (1000, 128, 16, 2, 128, 1),
    (2, 512, 64, 6, 1024, 0),  # T*K <= E: units dealt over the active experts, gate/up and down K-ranges halved
])
def test_fused_layer_graph_replay(ops, T, H, E, K, I, schedule):
    """moe_layer (routing with the slot-ranking tail, one scatter launch, the FFN, the combine) captured in a HIP
    graph: every replay, after eager work that changes x and clears the outputs and the workspace, equals an eager
    moe_layer bit for bit, and its y is the oracle combine of its expert_out."""
    lib = ops._lib.load()
    log(f"[graph moe_layer] T={T} H={H} E={E} K={K} I={I} schedule={schedule}")
    assert ffn_schedule(T, H, E, K, I) == schedule
    gen = torch.Generator(device="cpu").manual_seed(T * 3 + I)
    x = torch.randn(T, H, generator=gen).half().cuda()
    wg = (torch.randn(H, E, generator=gen) / math.sqrt(H)).half().cuda()
    ew = (torch.randn(E, 3 * I, H, generator=gen) / math.sqrt(H)).half().cuda()
    ws_bytes = ops.layer_workspace_bytes(T, H, E, K, I)

    def buffers():
        return dict(ids=torch.empty(T, K, dtype=torch.int32, device="cuda"),
                    w=torch.empty(T, K, dtype=torch.float16, device="cuda"),
                    eo=torch.empty(T, K, H, dtype=torch.float16, device="cuda"),
                    y=torch.empty(T, H, dtype=torch.float16, device="cuda"),
                    ws=torch.empty(ws_bytes, dtype=torch.uint8, device="cuda"))

    def step(b, s):
        st = lib.moe_layer(x.data_ptr(), wg.data_ptr(), ew.data_ptr(), b["ids"].data_ptr(), b["w"].data_ptr(),
                           b["eo"].data_ptr(), b["y"].data_ptr(), b["ws"].data_ptr(), ws_bytes, T, H, E, K, I, s)
        assert st == 0, lib.moe_last_error()

    gb, eb = buffers(), buffers()
    step(gb, torch.cuda.current_stream().cuda_stream)  # first launches set the kernels' LDS attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(gb, torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        x.copy_(torch.randn(T, H, generator=gen).half())
        step(eb, torch.cuda.current_stream().cuda_stream)
        for t in gb.values():
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name in ("ids", "w", "eo", "y"):
            assert torch.equal(gb[name], eb[name]), (i, name)
        y_o = oracle.combine(f32(host(gb["eo"])), f32(host(gb["w"]))).astype(np.float16)
        assert np.array_equal(host(gb["y"]).view(np.uint16), y_o.view(np.uint16)), i
    del g


def test_combine_bit_exact_random(ops):
    rng = np.random.default_rng(0)
    for T, H, K in ((1, 8, 1), (37, 64, 2), (300, 2048, 6), (5, 4096, 32)):
        eo = (rng.standard_normal((T, K, H)) * 2).astype(np.float16)
        w = rng.random((T, K)).astype(np.float16)
        y = host(ops.MoeCombine(dev(eo), None, dev(w), K))
        y_o = oracle.combine(f32(eo), f32(w)).astype(np.float16)
        assert np.array_equal(y.view(np.uint16), y_o.view(np.uint16)), (T, H, K)


def test_combine_k1_is_copy_and_equal_weights_mean(ops):
    rng = np.random.default_rng(1)
    eo = rng.standard_normal((9, 1, 128)).astype(np.float16)
    y = host(ops.MoeCombine(dev(eo), None, dev(np.ones((9, 1), np.float16))))
    assert np.array_equal(y.view(np.uint16), eo[:, 0].view(np.uint16))


@pytest.mark.parametrize("T,H,E,K", [(37, 64, 4, 2), (16, 96, 8, 8), (200, 256, 64, 6), (5, 32, 256, 32),
                                     (1, 2048, 16, 2), (33, 128, 1, 1), (1000, 512, 130, 4),
                                     # two and four 16-token blocks per workgroup, T not a multiple of them
                                     (8200, 64, 20, 3), (16400, 96, 64, 6), (16384, 64, 8, 2),
                                     # K up to E, as the reference allows (tests/moe_cpu_sim.cpp:224-243)
                                     (40, 64, 64, 64), (7, 32, 256, 200), (300, 128, 48, 40)])
def test_routing_shapes(ops, T, H, E, K):
    rng = np.random.default_rng(T * 1000 + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ids_d, w_d = ops.MoeRoutingTopK(dev(x), dev(wg), K)
    check_routing(host(ids_d), host(w_d), x, wg, K, f"routing T{T} H{H} E{E} K{K}")


@pytest.mark.parametrize("E,K", [(16, 2), (64, 6), (40, 5)])
def test_routing_is_batch_invariant(ops, E, K):
    """A token's ids and weights do not depend on the batch it is routed in: 16400 tokens run several token
    blocks per workgroup (E <= 32) or the rows kernel (32 < E <= 64), their first 1000 alone run the narrow
    kernel with one block, and the rows agree bit for bit."""
    T, H = 16400, 512
    rng = np.random.default_rng(E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ids_all, w_all = ops.MoeRoutingTopK(dev(x), dev(wg), K)
    ids_few, w_few = ops.MoeRoutingTopK(dev(x[:1000]), dev(wg), K)
    assert np.array_equal(host(ids_all)[:1000], host(ids_few))
    assert np.array_equal(host(w_all)[:1000].view(np.uint16), host(w_few).view(np.uint16))


@pytest.mark.parametrize("T,H,E,K", [
    (32790, 2048, 64, 6),  # DeepSeek-V2-Lite's routing, T ragged: runs of 9 token blocks, 8 pairs a virtual wave,
                           # selection rounds of 4, 4 and 1 blocks
    (33000, 1024, 48, 5),  # one ring slot a token block, the last expert block padding
    (40000, 2048, 40, 4),  # runs of 10 blocks (250 workgroups), 24 padded experts
    (65536, 1024, 64, 8),  # 4 pairs a virtual wave, 16 blocks a run
])
def test_routing_resident_kernel_matches_narrow(ops, T, H, E, K):
    """32 < E <= 64 from 32768 tokens (H = 1024 or 2048): the resident kernel holds w_gate in registers and
    streams x through an LDS ring. It keeps the narrow kernel's summation order, so its ids and weights equal, bit
    for bit, those of the narrow kernel for the same tokens routed in a smaller batch (the first 1000, and the last
    600, which end in a partial token block), and every token is checked against the oracle."""
    log(f"[resident] T={T} H={H} E={E} K={K}")
    rng = np.random.default_rng(T + H + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    x_d, wg_d = dev(x), dev(wg)
    ids_all, w_all = ops.MoeRoutingTopK(x_d, wg_d, K)
    ids_all, w_all = host(ids_all), host(w_all)
    for lo, hi in ((0, 1000), (T - 600, T)):
        ids_few, w_few = ops.MoeRoutingTopK(x_d[lo:hi].contiguous(), wg_d, K)
        assert np.array_equal(ids_all[lo:hi], host(ids_few)), (lo, hi)
        assert np.array_equal(w_all[lo:hi].view(np.uint16), host(w_few).view(np.uint16)), (lo, hi)
    check_routing(ids_all, w_all, x, wg, K, f"resident T{T} H{H} E{E} K{K}")


@pytest.mark.parametrize("H,E,K", [
    (7168, 256, 8),  # DeepSeek-V3's routing: 224 stages, 56 a quarter
    (2048, 128, 6),  # two k-steps a stage (E = 128): 32 stages
    (160, 256, 4),   # 5 stages: quarters of 1, 1, 1 and 2 stages
    (128, 128, 2),   # 2 stages: quarters 0 and 2 empty
])
def test_routing_quarters_and_rows_kernels_agree(ops, H, E, K):
    """E > 64: up to 8192 tokens the quarters kernel routes (16 tokens a workgroup, a wave per quarter of H), above
    that the rows kernel (64 tokens a workgroup, the quarters one after the other in each wave). Both add a token's
    H in the same four quarter sums, so 8300 tokens routed together and their first 1000 routed alone agree bit for
    bit; the small batch is also checked against the oracle's routing."""
    T = 8300
    rng = np.random.default_rng(H + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ids_all, w_all = ops.MoeRoutingTopK(dev(x), dev(wg), K)
    ids_few, w_few = ops.MoeRoutingTopK(dev(x[:1000]), dev(wg), K)
    ids_few, w_few = host(ids_few), host(w_few)
    assert np.array_equal(host(ids_all)[:1000], ids_few)
    assert np.array_equal(host(w_all)[:1000].view(np.uint16), w_few.view(np.uint16))
    check_routing(ids_few, w_few, x[:1000], wg, K, f"quarters H{H} E{E} K{K}")


def test_routing_rows_kernel_past_2gib_of_x(ops):
    """E > 64 with x past 2 GiB (T = 2^19 + 80, H = 2048): the rows kernel addresses each workgroup's own x rows,
    so it still runs and a token's ids and weights are the same bits as when its workgroup's tokens are routed
    alone. The first and the last (partial) token blocks are also checked against the oracle."""
    T, H, E, K = (1 << 19) + 80, 2048, 128, 8
    assert T * H * 2 >= 1 << 31
    log(f"[rows past 2 GiB] T={T} H={H} E={E} K={K}")
    x = torch.empty((T, H), dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(x, 17, synth.STREAM_X, 1.0)
    rng = np.random.default_rng(17)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    wg_d = dev(wg)
    ids_all, w_all = ops.MoeRoutingTopK(x, wg_d, K)
    ids_all, w_all = host(ids_all), host(w_all)
    for lo, hi in ((0, 64), (T - 80, T)):
        ids_few, w_few = ops.MoeRoutingTopK(x[lo:hi].contiguous(), wg_d, K)
        assert np.array_equal(ids_all[lo:hi], host(ids_few))
        assert np.array_equal(w_all[lo:hi].view(np.uint16), host(w_few).view(np.uint16))
        check_routing(ids_all[lo:hi], w_all[lo:hi], host(x[lo:hi]), wg, K, f"rows past 2 GiB tokens {lo}-{hi}")
    del x
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,H,E,K", [(9000, 256, 64, 6), (8192, 128, 48, 8), (20000, 2048, 64, 6),
                                     (3000, 256, 72, 6), (2100, 64, 256, 8), (70, 128, 200, 40),
                                     # 55 MB of x (non-temporal x loads), H / 32 = 33 k-steps: a ragged last pair
                                     (26000, 1056, 16, 2)])
def test_routing_lds_weight_paths(ops, T, H, E, K):
    """w_gate through LDS: the narrow kernel's transposing-read path (E <= 64) and the rows kernel (E > 64, each
    wave 16 tokens over all of H). ids and weights against the oracle on every token; for E <= 64 also bit for bit
    against the 2-byte gathers, which run when w_gate is not 16-byte aligned (the same values one fp16 further
    into a larger buffer)."""
    log(f"[lds w_gate] T={T} H={H} E={E} K={K}")
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ids_d, w_d = ops.MoeRoutingTopK(dev(x), dev(wg), K)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, x, wg, K, f"rows T{T} H{H} E{E} K{K}")
    if E <= 64:
        buf = torch.empty(H * E + 8, dtype=torch.float16, device="cuda")
        wg_odd = buf[1: 1 + H * E].view(H, E)  # 2-byte aligned only: the narrow kernel's 2-byte gathers
        wg_odd.copy_(dev(wg))
        ids2, w2 = ops.MoeRoutingTopK(dev(x), wg_odd, K)
        assert np.array_equal(ids, host(ids2))
        assert np.array_equal(w.view(np.uint16), host(w2).view(np.uint16))


def test_routing_exact_ties_lowest_index_first(ops):
    # all-equal logits: the same SET as the reference (lowest K indices), listed in ascending order
    T, H, E, K = 4, 64, 8, 5
    ids, w = ops.MoeRoutingTopK(dev(np.zeros((T, H), np.float16)), dev(np.zeros((H, E), np.float16)), K)
    assert (host(ids) == np.arange(K)).all()
    assert (f32(host(w)) == np.float32(np.float16(0.2))).all()


def test_ffn_edge_routings(ops):
    # one expert takes every row (multi-pass over row tiles), others none; K=1; ids out of range -> zero rows
    rng = np.random.default_rng(2)
    T, H, E, K, I = 200, 64, 3, 2, 96
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.zeros((T, K), np.int32)
    ids[:, 1] = 2
    ids[5, 0] = -1
    ids[7, 1] = E
    w = np.full((T, K), 0.5, np.float16)
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    assert not eo[5, 0].any() and not eo[7, 1].any()
    ids_ok = ids.copy()
    ids_ok[5, 0] = 0
    ids_ok[7, 1] = 0
    eo_o = oracle.expert_ffn(f32(x), ids_ok, f32(ew), I)
    mask = np.ones((T, K), bool)
    mask[5, 0] = mask[7, 1] = False
    within(oracle.compare(eo[mask], eo_o[mask]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,schedule", [
    (50, 128, 8, 3, 128, 0),     # 32-row weight streaming
    (300, 256, 16, 2, 256, 0),   # wide weight streaming (~34 valid rows per expert)
    (3000, 128, 8, 3, 128, 1),   # tiled, several m-tiles per expert
    (700, 256, 32, 4, 192, 1),   # tiled, I = 6 x 32 (odd multiple of 32 on the down reduction)
])
def test_ffn_arbitrary_caller_ids(ops, T, H, E, K, I, schedule):
    """MoeExpertFFN takes expert_ids from its caller, not only from the routing operator: uniformly random ids in
    [-2, E + 2) put one token on the same expert twice, leave some slots without an expert and skew the experts'
    row counts. On every FFN schedule: offsets and sorted_slot equal a stable sort of the valid slots, the slots of
    ids outside [0, E) are zero rows, and every other slot matches the oracle FFN (tests/moe_cpu_sim.cpp:245-296)."""
    assert ffn_schedule(T, H, E, K, I) == schedule
    rng = np.random.default_rng(T * 7 + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = rng.integers(-2, E + 2, size=(T, K)).astype(np.int32)
    valid = (ids >= 0) & (ids < E)
    dup = int(sum(len(r) - len(set(r)) for r in np.where(valid, ids, -1 - np.arange(K)).tolist()))
    log(f"[caller ids] T={T} H={H} E={E} K={K} I={I} schedule={schedule}: {int((~valid).sum())} invalid slots, "
        f"{dup} repeated experts within a token")
    assert dup > 0 and (~valid).any()
    w = np.full((T, K), 0.25, np.float16)
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    assert not eo[~valid].any()
    eo_o = oracle_ffn_threads(f32(x), np.where(valid, ids, 0).astype(np.int32), f32(ew), I)
    within(oracle.compare(eo[valid], eo_o[valid]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,pattern", [
    (100, 64, 8, 2, 96, "skewed"),      # one expert 150 rows (5 passes of 32), one the rest, six empty
    (1000, 64, 16, 1, 64, "uniform"),   # S = 1000: each wave's id scan runs several unrolled rounds
    (37, 128, 64, 3, 160, "invalid"),   # mostly empty experts, ids outside [0, E), I tail (160 = 5 x 32)
    # ring depths of the whole-line weight stream (D k-steps = D/2 column blocks of 64 k):
    (64, 256, 8, 2, 512, "uniform"),    # gate/up D = 8, down D = 4 in one K-range (scatter epilogue)
    (48, 128, 8, 2, 384, "uniform"),    # gate/up D = 4, down D = 4 in one K-range
    (40, 512, 4, 2, 2560, "uniform"),   # down D = 4 over 2 K-ranges of 1280 (partials + reduce)
])
def test_ffn_streaming_schedule_edges(ops, T, H, E, K, I, pattern):
    """The weight-streaming schedule finds each expert's rows from expert_ids inside its gate/up kernel and
    writes offsets / sorted_slot for the down kernel: check both and expert_out against the oracle."""
    assert ffn_schedule(T, H, E, K, I) == 0
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    if pattern == "skewed":
        ids = np.full((T, K), 5, np.int32)
        ids.ravel()[:150] = 2
    elif pattern == "uniform":
        ids = rng.integers(0, E, (T, K)).astype(np.int32)
    else:
        ids = rng.integers(0, 4, (T, K)).astype(np.int32) * 7  # experts 0, 7, 14, 21
        ids[3, 1], ids[9, 0], ids[20, 2] = -1, E, 1000
    w = np.full((T, K), 0.5, np.float16)
    log(f"[stream edges] {pattern}: T={T} H={H} E={E} K={K} I={I}")
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    valid = (ids >= 0) & (ids < E)
    assert not eo[~valid].any()
    eo_o = oracle.expert_ffn(f32(x), np.where(valid, ids, 0), f32(ew), I)
    within(oracle.compare(eo[valid], eo_o[valid]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,pattern", [
    (256, 1024, 8, 2, 2048, "uniform"),  # 64 rows per expert: gate/up K in 2 chunks, down (one K-range) in 4
    (200, 512, 8, 2, 2560, "skewed"),    # 50 rows per expert: 64-row passes; one expert 150 rows (64 + 64 + 22),
                                         # down over 2 K-ranges (partials) staged in chunks of 256
    (384, 2048, 16, 2, 1024, "uniform"), # 48 rows per expert: 64-row passes, gate/up K in 2 chunks of 1024
    (140, 256, 4, 2, 512, "invalid"),    # 70 rows per expert, single chunks, ids outside [0, E)
    (160, 640, 8, 2, 1024, "uniform"),   # H = 640 (a multiple of 128, not of 256): gate/up ring depth 4
    (2048, 256, 64, 2, 512, "uniform"),  # E = 64, 64 rows per expert: the id scans over 4096 slots per expert
    (512, 256, 64, 6, 512, "zipf"),      # E = 64, K = 6, Zipf(1.1) experts, 48 rows per expert on average (64-row
                                         # passes): the head expert takes several passes
    (8192, 128, 256, 2, 256, "zipf"),    # E = 256, 64 rows per expert on average, head experts of thousands of rows
    (240, 256, 64, 6, 512, "uniform"),   # 22.5 rows per expert: wide at E = 64 (from ~19), though below 32
    (352, 512, 8, 2, 4096, "uniform"),   # 88 rows per expert, I >= 4096: still wide (to 96), experts above 128 rows
])
def test_ffn_wide_streaming_schedule(ops, T, H, E, K, I, pattern):
    """~18-22 to 72 rows per expert on average (96 when I >= 4096): the weight-streaming schedule with the wide kernels
    (up to 128 rows per pass; up to 56 rows per expert on average an expert's last pass of at most 64 rows runs with
    the deeper ring; the K-range staged in chunks). offsets / sorted_slot and expert_out against the oracle on every
    slot, so every expert's first and last sorted rows and every pass of the experts above 128 rows are checked."""
    assert ffn_schedule(T, H, E, K, I) == 0
    rng = np.random.default_rng(T + E + I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    if pattern == "zipf":  # K distinct experts per token drawn with p(e) ~ (e + 1)^-1.1 (Gumbel top-K)
        logp = -1.1 * np.log(np.arange(1, E + 1))
        ids = np.argsort(-(logp + rng.gumbel(size=(T, E))), axis=1)[:, :K].astype(np.int32)
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    if pattern == "skewed":
        ids[:150, 0] = 3
        ids[:150, 1] = rng.integers(4, E, 150)
    elif pattern == "invalid":
        ids[7, 1], ids[50, 0], ids[123, 1] = -1, E, 77
    w = np.full((T, K), 0.5, np.float16)
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    log(f"[wide stream] {pattern}: T={T} H={H} E={E} K={K} I={I}; rows per expert {counts.min()}..{counts.max()}, "
        f"{int((counts > 128).sum())} experts above 128 rows, {int((counts == 0).sum())} empty")
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    valid = (ids >= 0) & (ids < E)
    assert not eo[~valid].any()
    eo_o = oracle.expert_ffn(f32(x), np.where(valid, ids, 0), f32(ew), I)
    m = oracle.compare(eo[valid], eo_o[valid])
    log(f"[wide stream] expert_out vs oracle: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,pattern", [
    (1, 512, 256, 8, 256, "uniform"),   # one token: 8 active experts of 256
    (5, 1024, 64, 6, 512, "invalid"),   # 30 slots, ids outside [0, E) among them
    (2, 256, 32, 8, 256, "middle"),     # experts 10..19 only: empty experts before and after the active ones
    (3, 256, 64, 4, 384, "ends"),       # experts 0 and 63 active, one expert twice
    (2, 512, 16, 4, 4096, "uniform"),   # down projection split over I (fp32 partials) on the active experts
    (2, 256, 16, 4, 256, "none"),       # no valid id at all: every offset 0, expert_out all zero
    (1, 4096, 8, 2, 1024, "uniform"),   # H = 4096: the 16-row whole-H gate/up halved to 8 K-ranges of 512
    (1, 7168, 16, 4, 512, "uniform"),   # H = 7168: gate/up's 4 K-ranges of 1792 halved to 8 of 896 (ring of 4)
])
def test_ffn_streaming_dealt_over_active_experts(ops, T, H, E, K, I, pattern):
    """T*K <= E: the streaming kernels deal their units over the experts that have rows, so the few active
    experts' weights stream on the whole grid. Checked on a workspace filled with garbage first: offsets (written
    for the empty experts too) and sorted_slot against a stable sort, expert_out against the oracle on every valid
    slot and zero on the others."""
    assert T * K <= E and ffn_schedule(T, H, E, K, I) == 0
    rng = np.random.default_rng(T * 1000 + E + I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    if pattern == "middle":
        ids = np.stack([rng.permutation(10)[:K] + 10 for _ in range(T)]).astype(np.int32)
    elif pattern == "ends":
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
        ids[0, 0], ids[1, 0], ids[2, 1] = 0, E - 1, ids[1, 1]
    elif pattern == "none":
        ids = np.full((T, K), -1, np.int32)
        ids[1, 2] = E
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
        if pattern == "invalid":
            ids[0, 1], ids[2, 0], ids[4, 5] = -1, E, 999
    w = np.full((T, K), 0.5, np.float16)
    valid = (ids >= 0) & (ids < E)
    log(f"[dealt] {pattern}: T={T} H={H} E={E} K={K} I={I}; {len(np.unique(ids[valid]))} active experts")
    x_d, ids_d, w_d, ew_d = dev(x), dev(ids), dev(w), dev(ew)
    ws = torch.full((ops.workspace_bytes(T, H, E, K, I),), 0xAB, dtype=torch.uint8, device="cuda")
    eo = f32(host(ops.MoeExpertFFN(x_d, ids_d, w_d, ew_d, 0, ws)))
    check_permute(host(ws), ids, E)
    assert not eo[~valid].any()
    if valid.any():
        eo_o = oracle.expert_ffn(f32(x), np.where(valid, ids, 0), f32(ew), I)
        within(oracle.compare(eo[valid], eo_o[valid]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,pattern,nsplit", [
    (64, 4096, 8, 2, 256, "uniform", 2),   # 32-row kernel, H in two K-ranges of 2048 (16 rows per expert)
    (24, 4096, 8, 2, 256, "uniform", 1),   # 6 rows per expert: one 16-row pass over the whole H, no partial sums
    (40, 7168, 16, 4, 128, "invalid", 4),  # DeepSeek-V3's H in four K-ranges of 1792, ids outside [0, E)
    (100, 2816, 8, 2, 96, "skewed", 11),   # eleven K-ranges of 256; one expert 150 rows (5 passes), I tail
    (512, 7168, 16, 2, 128, "zipf", 1),    # wide kernel (64 rows per expert): all of H in 14 stages of 512
    (200, 5120, 8, 2, 128, "skewed", 1),   # wide kernel, 10 stages of 512; one expert 150 rows (two passes)
])
def test_ffn_streaming_large_hidden(ops, T, H, E, K, I, pattern, nsplit):
    """H too large for 32 rows of x to sit in LDS whole: the 32-row gate/up kernel splits H into nsplit
    K-ranges, each workgroup writes its range's fp32 gate and up partial sums, and a reduce kernel adds the ranges
    in order and applies SwiGLU; below 12 rows per expert an H that 16 rows fit (up to 4568) runs 16-row passes
    over the whole of it instead, and the wide kernel (from 32 rows per expert) stages all of H in chunks. The
    plan's gate/up grid shows the split (E x ceil(I / 128) column blocks x nsplit); offsets / sorted_slot and
    expert_out against the oracle on every slot."""
    import ctypes as C

    from conftest import package

    lib_mod = package()._lib
    plan = lib_mod.FfnPlan()
    assert lib_mod.load().moe_expert_ffn_plan(T, H, E, K, I, C.byref(plan)) == 0
    assert plan.schedule == 0
    assert plan.gateup_grid == E * ((I + 127) // 128) * nsplit
    rng = np.random.default_rng(T + H + I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    if pattern == "zipf":  # K distinct experts per token drawn with p(e) ~ (e + 1)^-1.1 (Gumbel top-K)
        logp = -1.1 * np.log(np.arange(1, E + 1))
        ids = np.argsort(-(logp + rng.gumbel(size=(T, E))), axis=1)[:, :K].astype(np.int32)
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    if pattern == "skewed":
        ids[:, :] = rng.integers(1, E, (T, K))
        ids.ravel()[:150] = 0
    elif pattern == "invalid":
        ids[3, 1], ids[9, 0], ids[20, 2] = -1, E, 1000
    w = np.full((T, K), 0.5, np.float16)
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    log(f"[large H] {pattern}: T={T} H={H} E={E} K={K} I={I} nsplit={nsplit}; rows per expert "
        f"{counts.min()}..{counts.max()}")
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    eo = f32(host(eo_d))
    check_permute(host(ws), ids, E)
    valid = (ids >= 0) & (ids < E)
    assert not eo[~valid].any()
    eo_o = oracle_ffn_threads(f32(x), np.where(valid, ids, 0), f32(ew), I)
    m = oracle.compare(eo[valid], eo_o[valid])
    log(f"[large H] expert_out vs oracle: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


@pytest.mark.parametrize("T,H,E,K,I,split", [
    (64, 256, 8, 2, 512, 1),       # weight streaming, down in one K-range: FFN then the combine kernel
    (40, 512, 4, 2, 2560, 2),      # weight streaming, down over 2 K-ranges: the split reduce also combines
    (37, 128, 64, 3, 160, 1),      # ids outside [0, E): zero expert_out rows enter y as zeros
    (300, 128, 4, 2, 128, 0),      # LDS-tiled schedule
])
def test_ffn_combine_fused_matches_separate(ops, T, H, E, K, I, split):
    """moe_expert_ffn_combine: expert_out bit-identical to MoeExpertFFN, y bit-identical to MoeCombine on it."""
    rng = np.random.default_rng(T * 7 + I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = rng.integers(0, E, (T, K)).astype(np.int32)
    if split == 1 and E == 64:
        ids[3, 1], ids[9, 0], ids[20, 2] = -1, E, 1000
    w = rng.uniform(0.05, 1.0, (T, K)).astype(np.float16)
    log(f"[ffn+combine] T={T} H={H} E={E} K={K} I={I} schedule={ffn_schedule(T, H, E, K, I)}")
    x_d, ids_d, w_d, ew_d = dev(x), dev(ids), dev(w), dev(ew)
    eo_ref, _ = run_ffn(ops, x_d, ids_d, w_d, ew_d, I)
    y_ref = ops.MoeCombine(eo_ref, ids_d, w_d, K)
    eo, y = ops.MoeExpertFFNCombine(x_d, ids_d, w_d, ew_d, I)
    torch.cuda.synchronize()
    assert np.array_equal(host(eo).view(np.uint16), host(eo_ref).view(np.uint16))
    assert np.array_equal(host(y).view(np.uint16), host(y_ref).view(np.uint16))
    # and y against the oracle's combine of that expert_out (fp32, k ascending), bit-exact
    y_o = oracle.combine(f32(host(eo)), f32(w)).astype(np.float16)
    assert np.array_equal(host(y).view(np.uint16), y_o.view(np.uint16))


def test_ffn_combine_fused_decode_shape(ops):
    """The decode layer's shape (down split over 4 K-ranges): fused y and expert_out equal the three-op path."""
    cfg = synth.CONFIGS["decode"]
    x_d, wg_d, ew_d = gpu_inputs(ops, cfg, 45)
    ids_d, w_d = ops.MoeRoutingTopK(x_d, wg_d, cfg.K)
    eo_ref, _ = run_ffn(ops, x_d, ids_d, w_d, ew_d, cfg.I)
    y_ref = ops.MoeCombine(eo_ref, ids_d, w_d, cfg.K)
    eo, y = ops.MoeExpertFFNCombine(x_d, ids_d, w_d, ew_d, cfg.I)
    torch.cuda.synchronize()
    assert torch.equal(eo.view(torch.int16), eo_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


def test_ffn_rejects_bad_workspace(ops):
    x = dev(np.zeros((4, 64), np.float16))
    ids = dev(np.zeros((4, 2), np.int32))
    w = dev(np.zeros((4, 2), np.float16))
    ew = dev(np.zeros((4, 3 * 32, 64), np.float16))
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(ops.MoeError) as err:
        ops.MoeExpertFFN(x, ids, w, ew, 0, small)
    assert err.value.status == 5


# ------------------------------------------------------------------------------------------------------------
# the GPU generator equals the numpy spec
# ------------------------------------------------------------------------------------------------------------

def test_gpu_synth_matches_numpy(ops):
    n = 1 << 20
    sa, sb, period, split = 0.02, 0.011, 3 * 96 * 64, 2 * 96 * 64
    t = torch.empty(n, dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(t, 44, 3, sa, sb, period, split)
    ref = synth.normal_f16(44, 3, n, sa, sb, period, split)
    assert np.array_equal(host(t).view(np.uint16), ref.view(np.uint16))
    t2 = torch.empty(4097, dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(t2, 5, 1, 1.0)
    assert np.array_equal(host(t2).view(np.uint16), synth.normal_f16(5, 1, 4097, 1.0).view(np.uint16))


# ------------------------------------------------------------------------------------------------------------
# BASELINE sizes: inputs generated on the GPU, oracle on a token sample
# ------------------------------------------------------------------------------------------------------------

def gpu_inputs(ops, cfg, seed: int):
    """x and expert_weights from the GPU generator, w_gate from numpy (it carries the Zipf scaling)."""
    x = torch.empty((cfg.T, cfg.H), dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(x, seed, synth.STREAM_X, 1.0)
    ew = torch.empty((cfg.E, 3 * cfg.I, cfg.H), dtype=torch.float16, device="cuda")
    sa, sb, period, split = synth.expert_weight_sigmas(cfg)
    ops.synth_normal_f16_(ew, seed, synth.STREAM_EXPERT_WEIGHTS, sa, sb, period, split)
    wg = dev(synth.gen_w_gate(cfg, seed))
    return x, wg, ew


def leftover_down_rows(offsets: np.ndarray, H: int, I: int, grid: int) -> list[int]:
    """Sorted rows, one per tile of the tiled down projection's leftover round (the tiles each XCD has left
    after its full rounds, which the kernel splits over k into partial tiles and a fix-up): the kernel's own
    schedule (tiles (expert, n-tile, m-tile), m fastest; XCD x owns a contiguous range, dealt round-robin to its
    grid / 8 workgroups), restated here to choose the sample."""
    bm, bn, xcds = 256, 256, 8
    ntn = (H + bn - 1) // bn
    counts = np.diff(offsets)
    mtiles = (counts + bm - 1) // bm
    prefix = np.concatenate([[0], np.cumsum(mtiles * ntn)])
    total = int(prefix[-1])
    nloc = grid // xcds
    per_xcd = (total + xcds - 1) // xcds
    rows = []
    for x in range(xcds):
        base = x * per_xcd
        n = max(0, min(per_xcd, total - base))
        R = n // nloc
        for t in range(base + R * nloc, base + n):
            e = int(np.searchsorted(prefix, t, side="right") - 1)
            mt = (t - prefix[e]) % mtiles[e]
            last = min(int(counts[e]), (mt + 1) * bm) - 1  # the tile's last row
            rows.append(int(offsets[e]) + last)
    return rows


@pytest.mark.parametrize("name", ["small", "decode", "prefill", "deepseek", "mixtral"])
def test_baseline_config_sampled(ops, name):
    """Each BASELINE config at full size on the GPU generator's inputs. Routing is checked on every token;
    expert_out and y against the oracle on a sample that holds every expert's first and last sorted row (its
    ragged last m-tile), a row of every leftover tile of the tiled down projection (split over k), and a spread
    of other tokens; y equals the combine of the full expert_out bit for bit on every token."""
    cfg = synth.CONFIGS[name]
    log(f"[{name}] T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K} I={cfg.I}: generating inputs on the GPU")
    x_d, wg_d, ew_d = gpu_inputs(ops, cfg, 44)
    # spot-check the device generator against numpy on slices of both weight blocks
    ew_flat = ew_d.view(-1)
    sa, sb, period, split = synth.expert_weight_sigmas(cfg)
    for start in (0, max(0, split - 1000), period * (cfg.E - 1) + split):
        n = min(2000, ew_flat.numel() - start)
        got = host(ew_flat[start:start + n])
        raw = synth.normal_f64(44, synth.STREAM_EXPERT_WEIGHTS, start, n)
        sig = np.where((np.arange(start, start + n) % period) < split, sa, sb)
        assert np.array_equal(got.view(np.uint16), (raw * sig).astype(np.float16).view(np.uint16))

    ids_d, w_d = ops.MoeRoutingTopK(x_d, wg_d, cfg.K)
    ids, w = host(ids_d), host(w_d)
    x16 = host(x_d)
    check_routing(ids, w, x16, host(wg_d), cfg.K, name)
    counts = np.bincount(ids.ravel(), minlength=cfg.E)
    log(f"[{name}] rows per expert: min {counts.min()} max {counts.max()}")

    eo_d, ws = run_ffn(ops, x_d, ids_d, w_d, ew_d, cfg.I)
    ws_head = host(ws[: 4 * (cfg.E + 1) + 256 + 4 * cfg.slots])
    check_permute(ws_head, ids, cfg.E)
    y_d = ops.MoeCombine(eo_d, ids_d, w_d, cfg.K)
    torch.cuda.synchronize()

    # the sample: first and last sorted row of every expert, one row of every (expert, m-tile) of the GEMMs, one
    # row per leftover down tile, a spread of tokens
    offsets = ws_head[: 4 * (cfg.E + 1)].view(np.int32)
    sorted_slot = ws_head[((4 * (cfg.E + 1) + 255) // 256) * 256:][: 4 * cfg.slots].view(np.int32)
    rows = set()
    bm = ffn_rows_per_tile(cfg)
    rng = np.random.default_rng(7)
    mtiles = 0
    for e in range(cfg.E):
        if counts[e]:
            rows.update((int(offsets[e]), int(offsets[e + 1]) - 1))
            for m0 in range(0, int(counts[e]), bm):  # a row inside every m-tile (interior rows of the tile)
                rows.add(int(offsets[e]) + int(rng.integers(m0, min(int(counts[e]), m0 + bm))))
                mtiles += 1
    leftover = []
    if ffn_schedule(cfg.T, cfg.H, cfg.E, cfg.K, cfg.I) == 1:
        grid = min(torch.cuda.get_device_properties(0).multi_processor_count,
                   tiled_down_grid(cfg)) // 8 * 8
        leftover = leftover_down_rows(offsets, cfg.H, cfg.I, grid)
        rows.update(leftover)
    tokens = {int(sorted_slot[r]) // cfg.K for r in rows}
    tokens.update(np.linspace(0, cfg.T - 1, min(cfg.T, 6)).astype(int).tolist())
    sample = np.array(sorted(tokens))
    covered = {int(e) for e in np.unique(ids[sample])}
    log(f"[{name}] oracle sample: {len(sample)} tokens; experts covered {len(covered)}/{int((counts > 0).sum())} "
        f"(first and last sorted row of each); m-tiles covered {mtiles} (one row each, {bm}-row tiles); leftover "
        f"down tiles covered {len(leftover)}")
    assert covered == {e for e in range(cfg.E) if counts[e]}

    ew_host = np.zeros((cfg.E, 3 * cfg.I, cfg.H), np.float32)
    for e in covered:
        ew_host[e] = f32(host(ew_d[int(e)]))
    eo_o = oracle_ffn_threads(f32(x16[sample]), ids[sample], ew_host, cfg.I)
    del ew_host
    eo_s = f32(host(eo_d))[sample]
    m_eo = oracle.compare(eo_s, eo_o)
    log(f"[{name}] expert_out on {len(sample)} sampled tokens: {m_eo}")
    within(m_eo, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    y_s = f32(host(y_d))[sample]
    y_o = oracle.combine(eo_o, f32(w[sample]))
    m_y = oracle.compare(y_s, y_o)
    log(f"[{name}] y on sampled tokens: {m_y}")
    within(m_y)
    within(m_y, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    # size-independent check over all tokens: y equals the combine of the full expert_out (bit-exact)
    y_all = host(y_d)
    y_chk = oracle.combine(f32(host(eo_d)), f32(w)).astype(np.float16)
    assert np.array_equal(y_all.view(np.uint16), y_chk.view(np.uint16))
    assert np.isfinite(f32(y_all)).all()


def oracle_ffn_threads(x: np.ndarray, ids: np.ndarray, ew: np.ndarray, I: int, workers: int = 8) -> np.ndarray:
    """oracle.expert_ffn over token chunks in parallel threads (the C oracle runs outside the GIL); each token's
    rows are the single-threaded oracle's, bit for bit."""
    import concurrent.futures

    T = x.shape[0]
    bounds = np.linspace(0, T, min(T, workers) + 1).astype(int)
    out = np.empty((T, ids.shape[1], x.shape[1]), np.float32)

    def part(i: int) -> None:
        b, e = int(bounds[i]), int(bounds[i + 1])
        out[b:e] = oracle.expert_ffn(x[b:e], ids[b:e], ew, I)

    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(part, range(len(bounds) - 1)))
    return out


def ffn_rows_per_tile(cfg) -> int:
    import ctypes as C

    from conftest import package

    lib_mod = package()._lib
    plan = lib_mod.FfnPlan()
    assert lib_mod.load().moe_expert_ffn_plan(cfg.T, cfg.H, cfg.E, cfg.K, cfg.I, C.byref(plan)) == 0
    return plan.rows_per_tile


def tiled_down_grid(cfg) -> int:
    import ctypes as C

    from conftest import package

    lib_mod = package()._lib
    plan = lib_mod.FfnPlan()
    assert lib_mod.load().moe_expert_ffn_plan(cfg.T, cfg.H, cfg.E, cfg.K, cfg.I, C.byref(plan)) == 0
    return plan.down_grid


@pytest.mark.parametrize("T", [
    2048,  # 64 rows per expert on average: the wide streaming kernels
    256,   # 8 rows: also the wide kernels (16 rows of H = 7168 do not fit the 32-row kernels' LDS)
])
def test_deepseek_v3_layer_shape_sampled(ops, T):
    """The DeepSeek-V3 layer's expert shape (H = 7168, E = 256, K = 8, I = 2048; 22.5 GB of fp16 expert
    weights) through moe_layer on T Zipf-routed tokens: routing on every token against the oracle, expert_out
    against the oracle on six tokens (the oracle gets only their experts' weights), y bit for bit the combine of
    expert_out, and the three operators' run bit for bit."""
    cfg = synth.MoeConfig(T, 7168, 256, 8, 2048, zipf=True, name="deepseek_v3_shape")
    log(f"[{cfg.name}] T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K} I={cfg.I}: generating inputs on the GPU")
    x_d, wg_d, ew_d = gpu_inputs(ops, cfg, 45)
    y_d, ids_d, w_d, eo_d = ops.moe_layer_fused(x_d, wg_d, ew_d, cfg.K)
    x, wg = host(x_d), host(wg_d)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, x, wg, cfg.K, cfg.name)
    sample = np.linspace(0, cfg.T - 1, 6).astype(np.int64)
    used = np.unique(ids[sample])  # the sampled tokens' experts, renumbered 0.. for the oracle
    ids_sub = np.searchsorted(used, ids[sample]).astype(np.int32)
    ew_sub = f32(host(ew_d[torch.from_numpy(used).cuda()]))
    eo_o = oracle.expert_ffn(f32(x[sample]), ids_sub, ew_sub, cfg.I)
    log(f"[{cfg.name}] oracle sample: {len(sample)} tokens, {len(used)} experts")
    within(oracle.compare(f32(host(eo_d))[sample], eo_o), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    y_o = oracle.combine(f32(host(eo_d)), f32(w)).astype(np.float16)
    assert np.array_equal(host(y_d).view(np.uint16), y_o.view(np.uint16))
    ref = ops.moe_layer(x_d, wg_d, ew_d, cfg.K)
    for name, a, b in zip(("y", "ids", "weights", "expert_out"), ref, (y_d, ids_d, w_d, eo_d)):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("T,H,E,K,I", [
    (64, 4096, 8, 2, 512),   # gate/up in two K-ranges of 2048, then the down projection and the combine
    (24, 7168, 16, 4, 256),  # DeepSeek-V3's H: four K-ranges of 1792
])
def test_layer_with_gateup_split(ops, T, H, E, K, I):
    """moe_layer at a long H on the streaming schedule (the gate/up kernel splits H, a reduce adds the K-ranges):
    routing against the oracle on every token, expert_out against the oracle FFN on every slot, y bit for bit
    the oracle combine of expert_out, and every output equal to the three operators' run bit for bit."""
    cfg = synth.MoeConfig(T, H, E, K, I, name="gateup_split_layer")
    log(f"[layer split] T={T} H={H} E={E} K={K} I={I}")
    x_d, wg_d, ew_d = gpu_inputs(ops, cfg, 46)
    y_d, ids_d, w_d, eo_d = ops.moe_layer_fused(x_d, wg_d, ew_d, K)
    ref = ops.moe_layer(x_d, wg_d, ew_d, K)
    for name, a, b in zip(("y", "ids", "weights", "expert_out"), ref, (y_d, ids_d, w_d, eo_d)):
        assert torch.equal(a, b), name
    x, ids, w = host(x_d), host(ids_d), host(w_d)
    check_routing(ids, w, x, host(wg_d), K, "layer split")
    eo_o = oracle_ffn_threads(f32(x), ids, f32(host(ew_d)), I)
    m = oracle.compare(f32(host(eo_d)), eo_o)
    log(f"[layer split] expert_out vs oracle on all {T} tokens: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)
    y_o = oracle.combine(f32(host(eo_d)), f32(w)).astype(np.float16)
    assert np.array_equal(host(y_d).view(np.uint16), y_o.view(np.uint16))


def test_reference_target_case_seed44(ops):
    """The reference's own target-size RunTest case (tests/moe_cpu_sim.cpp:862-864: T=128, H=2048, E=16, K=2,
    I=8192, seed 44) on its own generator's inputs rounded to fp16: ids bit-exact against the reference's
    routing, y against its NaiveMoE output on all 128 tokens."""
    g = load_golden("ref_target_seed44")
    K = g["K"]
    log("[ref seed 44] inputs regenerated and digest-checked; running the layer")
    x_d, wg_d, ew_d = dev(g["x"]), dev(g["w_gate"]), dev(g["expert_weights"])
    y_d, ids_d, w_d, _ = ops.moe_layer(x_d, wg_d, ew_d, K)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, g["x"], g["w_gate"], K, "ref seed 44")
    assert np.array_equal(ids, g["expert_ids"])
    m_y = oracle.compare(f32(host(y_d)), g["y_naive"])
    log(f"[ref seed 44] y vs reference NaiveMoE (all tokens): {m_y}")
    within(m_y)
    within(m_y, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_reference_harness_small_uniform_case(ops):
    """The NPU harness's own accuracy case (tests/test_moe.cpp:344-515, smallCfg T=8 H=64 E=4 K=2 I=256): inputs
    srand(42) / rand() uniform in [-1, 1], the three operators on their fp16 rounding, y compared with NaiveMoE.

    The harness compares against NaiveMoE on the unrounded fp32 inputs with absolute thresholds (max abs < 0.05,
    mean abs < 0.01, cos > 0.99; :486-490). Here |y| reaches ~156 (mean ~34), where one fp16 ulp is 0.125: the
    fp16 rounding of the inputs alone moves the reference's own y by 0.054 max / 0.0138 mean (pinned on the CPU by
    test_harness_small_uniform_fixture), so no fp16-input kernel can meet those two bars. Checked here:
      ids          bit-exact against the reference routing on the fp16 inputs;
      y vs NaiveMoE on the fp16 inputs (the kernels' own error): max abs < 2^-10 max|y| (two fp16 ulps of the
                   largest output: hidden, expert_out and y are each rounded to fp16, 2^-11 relative) and
                   mean abs < 2^-11 mean|y|, cos > 0.99999;
      y vs NaiveMoE on the fp32 inputs (the harness's comparison): cos > 0.99, the bar that rounding leaves
                   attainable; max and mean abs are logged."""
    from conftest import GOLDEN_DIR

    g = dict(np.load(GOLDEN_DIR / "harness_small_uniform.npz", allow_pickle=False))
    T, H, E, K, I = (int(v) for v in g["dims"])
    log(f"[harness uniform] T={T} H={H} E={E} K={K} I={I}")
    x_d, wg_d, ew_d = dev(g["x"]), dev(g["w_gate"]), dev(g["expert_weights"])
    ids_d, w_d = ops.MoeRoutingTopK(x_d, wg_d, K)
    eo_d, _ = run_ffn(ops, x_d, ids_d, w_d, ew_d, I)
    y = f32(host(ops.MoeCombine(eo_d, ids_d, w_d, K)))
    assert np.array_equal(host(ids_d), g["expert_ids"])
    ref16, ref32 = g["y_naive_fp16in"], g["y_naive"]
    m16, m32 = oracle.compare(y, ref16), oracle.compare(y, ref32)
    log(f"[harness uniform] |y| max {np.abs(ref32).max():.1f} mean {np.abs(ref32).mean():.2f}; y vs NaiveMoE on "
        f"fp16 inputs {m16}; vs NaiveMoE on fp32 inputs (harness) {m32}")
    assert m16["max_abs"] < 2.0**-10 * np.abs(ref16).max(), m16
    assert m16["mean_abs"] < 2.0**-11 * np.abs(ref16).mean(), m16
    assert m16["cos"] > 0.99999, m16
    assert m32["cos"] > NS["cos"], m32


def ffn_schedule(T, H, E, K, I) -> int:
    import ctypes as C

    from conftest import package

    lib_mod = package()._lib
    plan = lib_mod.FfnPlan()
    assert lib_mod.load().moe_expert_ffn_plan(T, H, E, K, I, C.byref(plan)) == 0
    return plan.schedule


@pytest.mark.parametrize("T,H,E,K,I", [
    (300, 128, 4, 2, 128),    # partial m-tiles (~150 rows per expert)
    (257, 320, 3, 2, 192),    # partial n-tiles in both GEMMs (I = 192 -> 2 x 128, H = 320 -> 2 x 256)
    (600, 128, 8, 3, 128),    # K = 3, two k-stages in both GEMMs (the shortest ring)
    (700, 192, 2, 1, 1408),   # >256 rows per expert (several m-tiles), DeepSeek's I, three k-stages
    (10300, 128, 256, 2, 128), # E = 256: the permute re-reads expert_ids instead of its LDS byte copy
    (900, 128, 8, 2, 128),    # ids outside [0, E) through the permute's LDS byte copy (sentinel 255)
    (600, 96, 4, 2, 160),     # H and I odd multiples of 32: both GEMMs end with a 32-column k-stage
    (700, 224, 3, 2, 192),    # gate/up's k-tail only (H = 3.5 stages)
    (1200, 352, 4, 2, 352),   # both k-tails, down's leftover round split over k (6 stages, the last piece's tail)
])
def test_ffn_tiled_schedule_full_oracle(ops, T, H, E, K, I):
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(T + H + I)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    valid = np.ones((T, K), bool)
    if T == 900:
        ids[5, 0], ids[77, 1], ids[600, 0], ids[899, 1] = -1, E, 255, 1 << 20
        valid = (ids >= 0) & (ids < E)
    w = np.full((T, K), 1.0 / K, np.float16)
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    check_permute(host(ws), ids, E)
    eo = f32(host(eo_d))
    assert not eo[~valid].any()
    eo_o = oracle.expert_ffn(f32(x), np.where(valid, ids, 0), f32(ew), I)
    m = oracle.compare(eo[valid], eo_o[valid])
    log(f"[tiled T{T} H{H} E{E} K{K} I{I}] expert_out vs oracle: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_ffn_tiled_unaligned_expert_ids(ops):
    """expert_ids 4-byte but not 16-byte aligned (rows 1.. of a [T + 1, K] buffer; the C ABI does not require
    more): expert_out equals the aligned call bit for bit and the permutation is stable."""
    T, H, E, K, I = 600, 128, 8, 3, 128
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(31)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = np.full((T, K), 1.0 / K, np.float16)
    buf = dev(np.concatenate([np.zeros((1, K), np.int32), ids]))
    ids_unaligned = buf[1:]
    assert ids_unaligned.is_contiguous() and ids_unaligned.data_ptr() % 16 != 0
    x_d, w_d, ew_d = dev(x), dev(w), dev(ew)
    eo_u, ws_u = run_ffn(ops, x_d, ids_unaligned, w_d, ew_d, I)
    eo_a, _ = run_ffn(ops, x_d, dev(ids), w_d, ew_d, I)
    check_permute(host(ws_u), ids, E)
    assert np.array_equal(host(eo_u).view(np.uint16), host(eo_a).view(np.uint16))


def test_ffn_tiled_invalid_ids_give_zero_rows(ops):
    """Tiled schedule, ids outside [0, E) of every kind (-2, -1, E, a large value): those expert_out rows are zero
    (written over a non-zero buffer), they take no place in the permutation, and every other row matches the
    oracle."""
    T, H, E, K, I = 600, 128, 8, 3, 128
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(37)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    bad = rng.choice(T * K, 40, replace=False)
    ids.ravel()[bad] = np.resize(np.array([-2, -1, E, 1 << 20], np.int32), bad.size)
    w = np.full((T, K), 1.0 / K, np.float16)
    x_d, w_d, ew_d = dev(x), dev(w), dev(ew)
    ws = torch.empty(ops.workspace_bytes(T, H, E, K, I), dtype=torch.uint8, device="cuda")
    eo_d = torch.full((T, K, H), 7.0, dtype=torch.float16, device="cuda")
    st = ops._lib.load().moe_expert_ffn(x_d.data_ptr(), dev(ids).data_ptr(), w_d.data_ptr(), ew_d.data_ptr(),
                                        eo_d.data_ptr(), ws.data_ptr(), ws.numel(), T, H, E, K, I,
                                        torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    eo = f32(host(eo_d)).reshape(T * K, H)
    assert not eo[bad].any()
    check_permute(host(ws), ids, E)
    good = np.setdiff1d(np.arange(T * K), bad)
    ids_valid = ids.copy()
    ids_valid.ravel()[bad] = 0  # the oracle takes valid ids only; each row depends on its own id alone
    eo_o = oracle.expert_ffn(f32(x), ids_valid, f32(ew), I).reshape(T * K, H)
    within(oracle.compare(eo[good], eo_o[good]), max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_ffn_tiled_several_tiles_per_workgroup(ops):
    """512 gate/up tiles on a grid of at most one workgroup per CU: each workgroup runs several tiles with the
    copy ring running on from one tile into the next (other experts, other n-tiles). Checked against the oracle
    on 256 sampled tokens, which touch every (expert, m-tile) row block."""
    T, H, E, K, I = 4096, 256, 4, 2, 2048
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = np.full((T, K), 1.0 / K, np.float16)
    eo_d, ws = run_ffn(ops, dev(x), dev(ids), dev(w), dev(ew), I)
    check_permute(host(ws), ids, E)
    eo = f32(host(eo_d))
    tok = np.sort(rng.choice(T, 256, replace=False))
    eo_o = oracle.expert_ffn(f32(x[tok]), ids[tok], f32(ew), I)
    m = oracle.compare(eo[tok], eo_o)
    log(f"[tiled multi-tile T{T} H{H} E{E} K{K} I{I}] expert_out vs oracle on 256 tokens: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_ffn_tiled_split_leftover_round(ops):
    """~560 down tiles on the persistent grid: two full rounds per workgroup, then each XCD's leftover tiles split
    over k into pieces (fp32 partial tiles) that the fix-up kernel adds in piece order. Checked against the oracle
    on 192 sampled tokens (every expert's rows, including the ragged last m-tiles), and bit-identical over two
    runs (the fix-up's order is fixed)."""
    T, H, E, K, I = 8192, 2048, 16, 2, 512
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(23)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / math.sqrt(H),
                         rng.standard_normal((E, I, H)) / math.sqrt(I)], axis=1).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = np.full((T, K), 1.0 / K, np.float16)
    x_d, ids_d, w_d, ew_d = dev(x), dev(ids), dev(w), dev(ew)
    with ops.kernel_trace() as launched:
        eo_d, ws = run_ffn(ops, x_d, ids_d, w_d, ew_d, I)
        torch.cuda.synchronize()
    log(f"[tiled split] kernels: {sorted(launched)}")
    assert launched.get("moe_ffn_down_fixup", (0, 0.0))[0] >= 1, "the split leftover round did not run"
    eo = host(eo_d)
    eo2_d, _ = run_ffn(ops, x_d, ids_d, w_d, ew_d, I)
    assert np.array_equal(eo.view(np.uint16), host(eo2_d).view(np.uint16)), "tiled FFN is not deterministic"
    check_permute(host(ws[: 4 * (E + 1) + 256 + 4 * T * K]), ids, E)
    # the last rows of each expert sit in its ragged m-tile; sample them and a spread of the rest
    tok = set(np.linspace(0, T - 1, 128).astype(int).tolist())
    for e in range(E):
        tok.update(np.nonzero((ids == e).any(axis=1))[0][-4:].tolist())
    tok = np.array(sorted(tok))
    eo_o = oracle.expert_ffn(f32(x[tok]), ids[tok], f32(ew), I)
    m = oracle.compare(f32(eo)[tok], eo_o)
    log(f"[tiled split T{T} H{H} E{E} K{K} I{I}] expert_out vs oracle on {len(tok)} tokens: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_ffn_tiled_past_2gib_hidden(ops):
    """T*K*I*2 = 2 GiB of SwiGLU intermediate (T=65536, K=2, I=8192): the tiled kernels address hidden per tile,
    so this shape stays on the tiled schedule. expert_out against the oracle on every expert's first and last
    rows and a spread of tokens (H is small to keep the oracle cheap)."""
    T, H, E, K, I = 65536, 256, 4, 2, 8192
    assert ffn_schedule(T, H, E, K, I) == 1
    rng = np.random.default_rng(65536)
    x_d = torch.empty((T, H), dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(x_d, 7, synth.STREAM_X, 1.0)
    ew_d = torch.empty((E, 3 * I, H), dtype=torch.float16, device="cuda")
    ops.synth_normal_f16_(ew_d, 7, synth.STREAM_EXPERT_WEIGHTS, 1.0 / math.sqrt(H), 1.0 / math.sqrt(I),
                          3 * I * H, 2 * I * H)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = np.full((T, K), 0.5, np.float16)
    log(f"[2 GiB hidden] T={T} H={H} E={E} K={K} I={I}: workspace {ops.workspace_bytes(T, H, E, K, I) >> 20} MiB")
    eo_d, ws = run_ffn(ops, x_d, dev(ids), dev(w), ew_d, I)
    torch.cuda.synchronize()
    check_permute(host(ws[: 4 * (E + 1) + 256 + 4 * T * K]), ids, E)
    tok = set(np.linspace(0, T - 1, 24).astype(int).tolist())
    for e in range(E):
        hit = np.nonzero((ids == e).any(axis=1))[0]
        tok.update((int(hit[0]), int(hit[-1])))
    tok = np.array(sorted(tok))
    eo_o = oracle.expert_ffn(f32(host(x_d[tok])), ids[tok], f32(host(ew_d)), I)
    m = oracle.compare(f32(host(eo_d))[tok], eo_o)
    log(f"[2 GiB hidden] expert_out vs oracle on {len(tok)} tokens: {m}")
    within(m, max_abs=1e-2, mean_abs=1e-3, cos=0.9999)


def test_layer_on_a_side_stream(ops):
    """The operators queued on a stream other than torch's current one (their outputs and workspace allocated on
    that stream): the results equal the current-stream run bit for bit, on both FFN schedules."""
    for T, H, E, K, I in ((64, 256, 8, 2, 512), (600, 128, 8, 3, 128)):
        gen = torch.Generator(device="cpu").manual_seed(T)
        x = torch.randn(T, H, generator=gen).half().cuda()
        wg = (torch.randn(H, E, generator=gen) / math.sqrt(H)).half().cuda()
        ew = (torch.randn(E, 3 * I, H, generator=gen) / math.sqrt(H)).half().cuda()
        ref = ops.moe_layer(x, wg, ew, K)
        eo_f, y_f = ops.MoeExpertFFNCombine(x, ref[1], ref[2], ew)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        got = ops.moe_layer(x, wg, ew, K, stream=side)
        eo_s, y_s = ops.MoeExpertFFNCombine(x, got[1], got[2], ew, stream=side)
        # churn the current stream's allocator while the side stream runs
        junk = [torch.empty(1 << 20, dtype=torch.uint8, device="cuda").fill_(7) for _ in range(8)]
        side.synchronize()
        del junk
        log(f"[side stream] T={T} H={H} E={E} K={K} I={I} schedule={ffn_schedule(T, H, E, K, I)}")
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        assert torch.equal(eo_f, eo_s) and torch.equal(y_f, y_s)


def test_concurrent_threads_and_streams(ops):
    """Two host threads, each queueing three layers on its own stream with no synchronisation in between, one on
    each FFN schedule, both through the three operators and through moe_layer. The calls are re-entrant: the
    kernel-attribute and occupancy caches are mutex-guarded, the last error is per thread and every buffer is the
    caller's. Every output equals a sequential run bit for bit."""
    import threading
    cases = ((64, 256, 8, 2, 512), (600, 128, 8, 3, 128))
    data, refs = [], []
    for T, H, E, K, I in cases:
        gen = torch.Generator(device="cpu").manual_seed(T + 7)
        x = torch.randn(T, H, generator=gen).half().cuda()
        wg = (torch.randn(H, E, generator=gen) / math.sqrt(H)).half().cuda()
        ew = (torch.randn(E, 3 * I, H, generator=gen) / math.sqrt(H)).half().cuda()
        data.append((x, wg, ew, K))
        refs.append((ops.moe_layer(x, wg, ew, K), ops.moe_layer_fused(x, wg, ew, K)))
    torch.cuda.synchronize()
    results, errors = [None] * len(cases), []

    def worker(c):
        try:
            x, wg, ew, K = data[c]
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(s):  # this thread's allocations belong to its stream
                outs = [(ops.moe_layer(x, wg, ew, K, stream=s), ops.moe_layer_fused(x, wg, ew, K, stream=s))
                        for _ in range(3)]
            s.synchronize()
            results[c] = outs
        except Exception as exc:  # re-raised in the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(c,)) for c in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if errors:
        raise errors[0]
    for c, (T, H, E, K, I) in enumerate(cases):
        log(f"[threads] T={T} H={H} E={E} K={K} I={I} schedule={ffn_schedule(T, H, E, K, I)}")
        for three_op, fused in results[c]:
            for got, ref in ((three_op, refs[c][0]), (fused, refs[c][1])):
                for a, b in zip(got, ref):
                    assert torch.equal(a, b)


@pytest.mark.parametrize("T,H,E,K,I,schedule", [
    (64, 256, 8, 2, 512, 0),       # weight streaming: routing, then the FFN with the combine in its reduce
    (1000, 128, 8, 2, 128, 1),     # tiled; routing 16-token blocks of 16 waves, w_gate through LDS
    (2100, 128, 20, 3, 128, 1),    # E % 8 != 0: w_gate by 2-byte loads; 32 experts' blocks
    (9000, 128, 64, 6, 128, 1),    # two 16-token blocks per workgroup, 192 slots per count chunk
    (17000, 128, 13, 2, 128, 1),   # four 16-token blocks; E % 4 != 0 pads the counts rows
    (3000, 128, 130, 4, 128, 1),   # E > 64: the wide routing kernel counts its 64 tokens
    (300, 128, 48, 40, 128, 1),    # K = 40: a block's 640 slots are ranked in two passes
    (1000, 128, 100, 64, 128, 1),  # wide kernel, K = 64: 4096 slots per block, two passes
    (4096, 256, 128, 8, 128, 1),   # E = 128, T <= 8192: the quarters kernel ranks its 16-token blocks
    (9000, 256, 128, 4, 128, 1),   # E = 128, T > 8192: the rows kernel ranks its 64-token blocks
    (32790, 1024, 64, 6, 128, 1),  # 32 < E <= 64, T >= 32768: the resident kernel ranks each workgroup's run of
                                   # 9 token blocks (144 tokens, 864 slots) in one pass
    (4, 2048, 256, 8, 128, 0),     # T <= 16, E > 64: split routing (32 workgroups of quarter sums, a selection)
    (16, 1024, 128, 8, 256, 0),    # E = 128: 16 workgroups of quarter sums
    (3, 1536, 160, 6, 128, 0),     # quarters of 12 k-steps (not a multiple of 8): the quarters kernel routes
])
def test_fused_layer_matches_oracle_and_operators(ops, T, H, E, K, I, schedule):
    """moe_layer (routing that also ranks its blocks' slots, one scatter launch, the FFN, the combine): ids and
    weights pass the oracle's routing check on every token; the workspace's offsets and sorted_slot equal a stable
    sort of those ids; expert_out matches the oracle FFN on a token sample and y is the oracle combine of it bit
    for bit; and every output equals the three operators' run bit for bit."""
    assert ffn_schedule(T, H, E, K, I) == schedule
    log(f"[fused layer] T={T} H={H} E={E} K={K} I={I} schedule={schedule}")
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = (rng.standard_normal((H, E)) / math.sqrt(H)).astype(np.float16)
    ew = (rng.standard_normal((E, 3 * I, H)) / math.sqrt(H)).astype(np.float16)
    x_d, wg_d, ew_d = dev(x), dev(wg), dev(ew)
    ws = torch.empty(ops.layer_workspace_bytes(T, H, E, K, I), dtype=torch.uint8, device="cuda")
    assert ws.numel() >= ops.workspace_bytes(T, H, E, K, I)
    ws.fill_(0xA5)  # the layer must write every byte it reads
    y_d, ids_d, w_d, eo_d = ops.moe_layer_fused(x_d, wg_d, ew_d, K, workspace=ws)
    ids, w = host(ids_d), host(w_d)
    check_routing(ids, w, x, wg, K, f"fused layer T{T} E{E}")
    if schedule == 1:
        check_permute(host(ws), ids, E)
    n = min(T, 48)
    eo = f32(host(eo_d))
    within(oracle.compare(eo[:n], oracle.expert_ffn(f32(x[:n]), ids[:n], f32(ew), I)), max_abs=1e-2, mean_abs=1e-3,
           cos=0.9999)
    y_o = oracle.combine(eo, f32(w)).astype(np.float16)
    assert np.array_equal(host(y_d).view(np.uint16), y_o.view(np.uint16))
    ref = ops.moe_layer(x_d, wg_d, ew_d, K)
    for name, a, b in zip(("y", "ids", "weights", "expert_out"), ref, (y_d, ids_d, w_d, eo_d)):
        assert torch.equal(a, b), name


def random_shapes(n: int, seed: int):
    """n seeded shapes inside the library's limits (H and I multiples of 32, K <= E, T <= 3000): every other one
    with E <= 8 so that experts get the many rows of the tiled schedule; sized so the oracle FFN over every token
    stays near 1e9 multiply-adds each."""
    rng = np.random.default_rng(seed)
    shapes = []
    while len(shapes) < n:
        H = 32 * int(rng.integers(1, 25))
        I = 32 * int(rng.integers(1, 25))
        E = int(rng.integers(1, 9)) if len(shapes) % 2 == 0 else int(rng.integers(1, 97))
        K = int(rng.integers(1, min(E, 8) + 1))
        t_cap = max(1, min(3000, int(1e9 // (3 * K * H * I))))
        T = int(rng.integers(1, t_cap + 1))
        shapes.append((T, H, E, K, I))
    return shapes


def run_shape_sweep(ops, shapes, tag):
    """Each shape through the three operators and through moe_layer, every token checked: ids and weights against
    the oracle's routing, expert_out against the oracle FFN of the same ids, y bit for bit against the oracle's
    combine of that expert_out, and moe_layer equal to the three operators bit for bit. Shapes the planner rejects
    must be rejected with MOE_ERR_UNSUPPORTED. Returns the number of shapes per FFN schedule and the number whose
    gate/up splits H over K-ranges (the plan's gate/up grid above E x ceil(I / 128) on the streaming schedule)."""
    import ctypes as C

    from conftest import package

    lib_mod = package()._lib
    lib = lib_mod.load()
    seen = {0: 0, 1: 0, "gateup_split": 0}
    for n, (T, H, E, K, I) in enumerate(shapes):
        plan = lib_mod.FfnPlan()
        st = lib.moe_expert_ffn_plan(T, H, E, K, I, C.byref(plan))
        if st != 0:
            assert lib_mod.STATUS_NAMES.get(st) == "MOE_ERR_UNSUPPORTED", (T, H, E, K, I, st)
            log(f"[{tag} {n}] T={T} H={H} E={E} K={K} I={I}: unsupported ({lib.moe_last_error().decode()})")
            continue
        seen[plan.schedule] += 1
        split = plan.schedule == 0 and plan.gateup_grid > E * ((I + 127) // 128)
        seen["gateup_split"] += int(split)
        rng = np.random.default_rng(n)
        x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
        wg = (rng.standard_normal((H, E), dtype=np.float32) / math.sqrt(H)).astype(np.float16)
        ew = np.concatenate([rng.standard_normal((E, 2 * I, H), dtype=np.float32) / math.sqrt(H),
                             rng.standard_normal((E, I, H), dtype=np.float32) / math.sqrt(I)], axis=1).astype(np.float16)
        x_d, wg_d, ew_d = dev(x), dev(wg), dev(ew)
        ids_d, w_d = ops.MoeRoutingTopK(x_d, wg_d, K)
        eo_d = ops.MoeExpertFFN(x_d, ids_d, w_d, ew_d)
        y_d = ops.MoeCombine(eo_d, ids_d, w_d, K)
        ids, w = host(ids_d), host(w_d)
        log(f"[{tag} {n}] T={T} H={H} E={E} K={K} I={I} schedule={plan.schedule} gate/up split={split}")
        check_routing(ids, w, x, wg, K, f"{tag} {n}")
        eo = f32(host(eo_d))
        within(oracle.compare(eo, oracle_ffn_threads(f32(x), ids, f32(ew), I)), max_abs=1e-2, mean_abs=1e-3,
               cos=0.9999)
        y_o = oracle.combine(eo, f32(w)).astype(np.float16)
        assert np.array_equal(host(y_d).view(np.uint16), y_o.view(np.uint16))
        layer = ops.moe_layer(x_d, wg_d, ew_d, K)
        for name, a, b in zip(("y", "ids", "weights", "expert_out"), layer, (y_d, ids_d, w_d, eo_d)):
            assert torch.equal(a, b), (name, n)
    log(f"[{tag}] shapes per schedule: {seen}")
    return seen


def test_random_shape_sweep(ops):
    """24 seeded random shapes (H, I <= 768) through run_shape_sweep; the sweep must reach both FFN schedules."""
    seen = run_shape_sweep(ops, random_shapes(24, 2026), "sweep")
    assert seen[0] >= 3 and seen[1] >= 3, seen


def random_long_hidden_shapes(n: int, seed: int):
    """n seeded shapes with H from 2304 to 8192 (multiples of 32; above 2272 the 32-row gate/up kernel splits H),
    E up to 256 (every routing kernel), expert weights up to 2e8 elements and the oracle FFN near 2e9 multiply-adds
    per shape, so T stays small and most shapes take the streaming schedule."""
    rng = np.random.default_rng(seed)
    shapes = []
    while len(shapes) < n:
        H = 32 * int(rng.integers(72, 257))
        I = 32 * int(rng.integers(1, 25))
        E = int(rng.integers(1, min(256, int(2e8 // (3 * I * H))) + 1))
        K = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.integers(1, max(1, min(600, int(2e9 // (3 * K * H * I)))) + 1))
        shapes.append((T, H, E, K, I))
    return shapes


def test_random_long_hidden_sweep(ops):
    """12 seeded random shapes with a long H through run_shape_sweep: the 32-row gate/up kernel's K-range split
    must be reached."""
    seen = run_shape_sweep(ops, random_long_hidden_shapes(12, 7168), "long-H sweep")
    assert seen["gateup_split"] >= 2, seen


def test_decode_uses_streaming_and_prefill_uses_tiled():
    assert ffn_schedule(128, 2048, 16, 2, 8192) == 0
    assert ffn_schedule(8192, 2048, 16, 2, 8192) == 1
    assert ffn_schedule(16384, 2048, 64, 6, 1408) == 1
    assert ffn_schedule(4096, 4096, 8, 2, 14336) == 1
