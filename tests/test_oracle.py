"""Pins the CPU oracle (oracle/moe_oracle.cpp) before it is trusted as the checker of the HIP path.

Three independent anchors:
  1. golden vectors written by the reference simulator itself (tests/golden/*.npz)   -> bit-exact
  2. the reference simulator compiled from its source (oracle/_ref), random shapes    -> bit-exact
  3. mathematics: brute-force fp64 evaluation of the layer from its definition, closed forms for one-hot
     inputs, softmax/renormalisation identities, K = 1 copies. Each is chosen so that a plausible slip in the
     oracle (transposed W_down, a swapped gate/up block, a dropped term, softmax over the wrong axis, an
     unsorted top-K) breaks it; test_brute_force_detects_planted_mistakes shows the checks have that power.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import GOLDEN_CASES, load_golden


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------------------------------------------------------
# 1. golden vectors from the reference
# ------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLDEN_CASES)
def test_oracle_matches_reference_golden_vectors(case):
    g = load_golden(case)
    x, wg, ew = (g[k].astype(np.float32) for k in ("x", "w_gate", "expert_weights"))
    K, I = g["K"], g["I"]
    ids, w, probs, _ = oracle.routing(x, wg, K)
    assert np.array_equal(ids, g["expert_ids"])
    assert np.array_equal(bits(w), bits(g["weights"]))
    y, _, _, _ = oracle.moe_layer(x, wg, ew, K, I)
    assert np.array_equal(bits(y), bits(g["y_naive"]))
    eo_t = oracle.expert_ffn(x, ids, ew, I, tiled=True)
    assert np.array_equal(bits(eo_t), bits(g["expert_out_tiled"]))
    y_t, _, _, _ = oracle.moe_layer(x, wg, ew, K, I, tiled=True)
    assert np.array_equal(bits(y_t), bits(g["y_tiled"]))
    # the reference's own pass criterion between its two schedules (tests/moe_cpu_sim.cpp:666)
    m = oracle.compare(g["y_tiled"], g["y_naive"])
    assert m["max_abs"] < 0.05 and m["cos"] > 0.999


# ------------------------------------------------------------------------------------------------------------
# 2. the reference simulator built from its source
# ------------------------------------------------------------------------------------------------------------

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference checkout)")


@needs_ref
@pytest.mark.parametrize("T,H,E,K,I,seed", [
    (8, 64, 4, 2, 256, 42),      # the reference's small test
    (32, 256, 8, 2, 1024, 43),   # the reference's medium test
    (5, 32, 3, 3, 64, 1),        # K == E
    (7, 64, 9, 1, 288, 2),       # K == 1, I = 256 + 32 tail
    (1, 128, 64, 6, 96, 3),      # one token, DeepSeek-like E/K
])
def test_oracle_matches_reference_build(T, H, E, K, I, seed):
    x, wg, ew = oracle.ref_gen_inputs(T, H, E, I, seed)
    ids_r, w_r = oracle.ref_routing(x, wg, K)
    ids, w, _, _ = oracle.routing(x, wg, K)
    assert np.array_equal(ids, ids_r) and np.array_equal(bits(w), bits(w_r))
    y, _, _, _ = oracle.moe_layer(x, wg, ew, K, I)
    assert np.array_equal(bits(y), bits(oracle.ref_naive_moe(x, wg, ew, K, I)))
    eo = oracle.expert_ffn(x, ids, ew, I, tiled=True)
    assert np.array_equal(bits(eo), bits(oracle.ref_expert_ffn_tiled(x, ew, ids_r, w_r, I)))
    assert np.array_equal(bits(oracle.combine(eo, w)), bits(oracle.ref_combine(eo, ids_r, w_r)))
    y_t, _, _, _ = oracle.moe_layer(x, wg, ew, K, I, tiled=True)
    y_tr, _ = oracle.ref_moe_timed(x, wg, ew, K, I, tiled=True)
    assert np.array_equal(bits(y_t), bits(y_tr))


@needs_ref
def test_routing_ties_match_reference():
    # exact ties resolve in the order std::partial_sort gives; the restatement calls the same routine
    rng = np.random.default_rng(0)
    for trial in range(40):
        E = int(rng.integers(2, 12))
        K = int(rng.integers(1, E + 1))
        levels = rng.integers(0, 3, size=E).astype(np.float32)  # few distinct logits -> many ties
        x = np.zeros((1, 32), np.float32)
        x[0, 0] = 1.0
        wg = np.zeros((32, E), np.float32)
        wg[0] = levels
        ids_r, w_r = oracle.ref_routing(x, wg, K)
        ids, w, _, _ = oracle.routing(x, wg, K)
        assert np.array_equal(ids, ids_r), (trial, levels, K)
        assert np.array_equal(bits(w), bits(w_r))


@needs_ref
def test_compare_metric_matches_reference():
    rng = np.random.default_rng(1)
    a = rng.standard_normal(5000).astype(np.float32)
    b = (a + 1e-3 * rng.standard_normal(5000)).astype(np.float32)
    mine, ref = oracle.compare(a, b), oracle.ref_compare(a, b)
    assert mine["max_abs"] == pytest.approx(ref["max_abs"], rel=1e-7)
    assert mine["cos"] == pytest.approx(ref["cos"], rel=1e-12)
    assert mine["mean_abs"] == pytest.approx(ref["mean_abs"], rel=1e-4)  # reference sums in float


# ------------------------------------------------------------------------------------------------------------
# 3. mathematics
# ------------------------------------------------------------------------------------------------------------

def brute_force_layer(x, wg, ew, K, I, down_layout="HI", swap_gate_up=False):
    """fp64 evaluation of the layer from its definition (independent of the oracle's code)."""
    x, wg, ew = (np.asarray(a, np.float64) for a in (x, wg, ew))
    T, H = x.shape
    logits = x @ wg
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :K]
    sel = np.take_along_axis(p, ids, axis=1)
    w = sel / sel.sum(axis=1, keepdims=True)
    eo = np.zeros((T, K, H))
    for t in range(T):
        for k in range(K):
            blk = ew[ids[t, k]]
            wgate, wup = blk[:I], blk[I:2 * I]
            if swap_gate_up:
                wgate, wup = wup, wgate
            wdown = blk[2 * I:].reshape(H, I) if down_layout == "HI" else blk[2 * I:].reshape(I, H).T
            g, u = wgate @ x[t], wup @ x[t]
            eo[t, k] = wdown @ (g / (1.0 + np.exp(-g)) * u)
    y = np.einsum("tk,tkh->th", w, eo)
    return y, ids, w, eo, p, logits


@pytest.mark.parametrize("T,H,E,K,I,seed", [(6, 32, 5, 2, 40, 0), (3, 48, 7, 3, 24, 1), (4, 16, 4, 4, 8, 2)])
def test_oracle_matches_fp64_brute_force(T, H, E, K, I, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    wg = (rng.standard_normal((H, E)) / np.sqrt(H)).astype(np.float32)
    # rows [2I, 3I) of each expert hold W_down [H, I] row-major, i.e. H*I values in that order
    down = rng.standard_normal((E, H * I)).reshape(E, I, H) / np.sqrt(I)
    ew = np.concatenate([rng.standard_normal((E, 2 * I, H)) / np.sqrt(H), down], axis=1).astype(np.float32)
    y, ids, w, eo = oracle.moe_layer(x, wg, ew, K, I)
    y64, ids64, w64, eo64, p64, l64 = brute_force_layer(x, wg, ew, K, I)
    assert np.array_equal(ids, ids64)
    np.testing.assert_allclose(w, w64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(eo, eo64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(y, y64, rtol=1e-4, atol=1e-5)
    _, _, probs, logits = oracle.routing(x, wg, K)
    np.testing.assert_allclose(logits, l64, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(probs.sum(axis=1), 1.0, atol=2e-6)


def test_brute_force_detects_planted_mistakes():
    """The fp64 check above distinguishes the plausible layout slips (planted in the checker's model)."""
    rng = np.random.default_rng(7)
    T, H, E, K, I = 4, 24, 5, 2, 16
    x = rng.standard_normal((T, H)).astype(np.float32)
    wg = rng.standard_normal((H, E)).astype(np.float32) / 5
    ew = (rng.standard_normal((E, 3 * I, H)) / 5).astype(np.float32)
    y, _, _, _ = oracle.moe_layer(x, wg, ew, K, I)
    good = brute_force_layer(x, wg, ew, K, I)[0]
    np.testing.assert_allclose(y, good, rtol=1e-4, atol=1e-5)
    for bad in (brute_force_layer(x, wg, ew, K, I, down_layout="IH")[0],
                brute_force_layer(x, wg, ew, K, I, swap_gate_up=True)[0]):
        assert np.max(np.abs(bad - y)) > 1e-2


def test_routing_closed_form_one_hot():
    # x = e_0 makes logits equal row 0 of w_gate exactly; weights have the closed form
    # w_k = exp(l_k - l_max) / sum_{j in topK} exp(l_j - l_max) (the softmax denominator cancels).
    E, K, H = 8, 3, 32
    levels = np.array([0.3, -1.0, 2.0, 0.7, 1.5, -0.2, 0.9, 0.1], np.float32)
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 1.0
    wg = np.zeros((H, E), np.float32)
    wg[0] = levels
    ids, w, probs, logits = oracle.routing(x, wg, K)
    assert np.array_equal(logits[0], levels)
    assert list(ids[0]) == [2, 4, 6]
    top = levels[[2, 4, 6]].astype(np.float64)
    closed = np.exp(top - top.max()) / np.exp(top - top.max()).sum()
    np.testing.assert_allclose(w[0], closed, rtol=3e-7)
    assert abs(float(w[0].astype(np.float64).sum()) - 1.0) < 3e-7


def test_routing_all_equal_logits_picks_lowest_indices():
    # std::partial_sort keeps the K lowest indices of an all-equal row as the selected SET, but lists them in
    # its heap order for K >= 4 (e.g. [1, 3, 0, 2]); the GPU kernel lists exact ties lowest index first.
    for K in (1, 2, 3, 4, 6):
        ids, w, _, _ = oracle.routing(np.zeros((3, 64), np.float32), np.zeros((64, 6), np.float32), K)
        assert all(sorted(row) == list(range(K)) for row in ids.tolist())
        assert np.all(w == np.float32(1.0 / K))
    ids, _, _, _ = oracle.routing(np.zeros((1, 64), np.float32), np.zeros((64, 6), np.float32), 4)
    assert ids[0].tolist() == [1, 3, 0, 2]


def test_ffn_closed_form_one_hot():
    # x_t = e_j, single expert: gate_i = Wg[i, j], up_i = Wu[i, j]; with W_down = [I_H | 0] (H <= I) the
    # output is out_h = silu(Wg[h, j]) * Wu[h, j].
    H, I, E, K = 8, 16, 1, 1
    rng = np.random.default_rng(3)
    ew = np.zeros((E, 3 * I, H), np.float32)
    ew[0, :I] = rng.standard_normal((I, H))
    ew[0, I:2 * I] = rng.standard_normal((I, H))
    wdown = np.zeros((H, I), np.float32)
    wdown[np.arange(H), np.arange(H)] = 1.0
    ew[0, 2 * I:] = wdown.reshape(I, H)
    for j in range(H):
        x = np.zeros((1, H), np.float32)
        x[0, j] = 1.0
        eo = oracle.expert_ffn(x, np.zeros((1, 1), np.int32), ew, I)
        g, u = ew[0, :H, j].astype(np.float64), ew[0, I:I + H, j].astype(np.float64)
        np.testing.assert_allclose(eo[0, 0], g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-7)


def test_silu_limits():
    # silu(0) = 0 and silu(g) -> g for large g, seen through a one-element FFN with unit weights
    ew = np.ones((1, 3, 1), np.float32)
    for g, expect in ((0.0, 0.0), (30.0, 30.0 * 30.0), (-30.0, 0.0)):
        eo = oracle.expert_ffn(np.array([[g]], np.float32), np.zeros((1, 1), np.int32), ew, 1)
        assert eo[0, 0, 0] == pytest.approx(expect, abs=1e-5)


def test_combine_identities():
    rng = np.random.default_rng(4)
    eo = rng.standard_normal((5, 1, 12)).astype(np.float32)
    assert np.array_equal(bits(oracle.combine(eo, np.ones((5, 1), np.float32))), bits(eo[:, 0]))  # K=1: copy
    eo2 = rng.standard_normal((5, 2, 12)).astype(np.float32)
    y = oracle.combine(eo2, np.full((5, 2), 0.5, np.float32))
    np.testing.assert_allclose(y, eo2.mean(axis=1), rtol=1e-6, atol=1e-7)


def test_naive_and_tiled_schedules_differ_only_in_down_chunking():
    x, wg, ew = oracle.ref_gen_inputs(6, 64, 4, 512, 11) if oracle.ref_available() else (
        np.random.default_rng(5).standard_normal((6, 64)).astype(np.float32) / 8,
        np.random.default_rng(6).standard_normal((64, 4)).astype(np.float32) / 8,
        np.random.default_rng(7).standard_normal((4, 1536, 64)).astype(np.float32) / 8)
    ids, _, _, _ = oracle.routing(x, wg, 2)
    naive = oracle.expert_ffn(x, ids, ew, 512)
    tiled = oracle.expert_ffn(x, ids, ew, 512, tiled=True)
    assert not np.array_equal(bits(naive), bits(tiled))  # I = 512: two chunks of 256 -> different rounding
    np.testing.assert_allclose(naive, tiled, rtol=1e-5, atol=1e-6)


def test_oracle_rejects_bad_arguments():
    with pytest.raises(ValueError):
        oracle.routing(np.zeros((2, 8), np.float32), np.zeros((8, 3), np.float32), 4)  # K > E
    with pytest.raises(ValueError):
        oracle.expert_ffn(np.zeros((1, 8), np.float32), np.array([[5]], np.int32), np.zeros((2, 3, 8), np.float32), 1)


# ------------------------------------------------------------------------------------------------------------
# the NPU harness's own accuracy case (uniform inputs, fp32 expectation)
# ------------------------------------------------------------------------------------------------------------

def test_harness_small_uniform_fixture():
    """tests/golden/harness_small_uniform.npz, the reference harness's smallCfg (tests/test_moe.cpp:344-515):
    the stored fp16 inputs are the C library's srand(42) / rand() stream as the harness draws it, rounded to
    fp16; the oracle restates NaiveMoE on those inputs bit for bit; and the fp16 rounding of the inputs alone
    moves y past the harness's max-abs and mean-abs thresholds (|y| reaches ~156, where one fp16 ulp is 0.125),
    which is why the GPU test holds this case to an fp16-ulp bound instead."""
    import sys

    from conftest import GOLDEN_DIR

    sys.path.insert(0, str(GOLDEN_DIR))
    from make_golden import harness_uniform_inputs, input_digest

    g = dict(np.load(GOLDEN_DIR / "harness_small_uniform.npz", allow_pickle=False))
    T, H, E, K, I = (int(v) for v in g["dims"])
    x, wg, ew = harness_uniform_inputs(T, H, E, I)
    assert np.array_equal(x.astype(np.float16), g["x"]) and np.array_equal(wg.astype(np.float16), g["w_gate"])
    assert np.array_equal(ew.astype(np.float16), g["expert_weights"])
    assert input_digest(g["x"], g["w_gate"], g["expert_weights"]) == str(g["digest"])
    x16, wg16, ew16 = (g[k].astype(np.float32) for k in ("x", "w_gate", "expert_weights"))
    y16, ids, w, _ = oracle.moe_layer(x16, wg16, ew16, K, I)
    assert np.array_equal(bits(y16), bits(g["y_naive_fp16in"]))
    assert np.array_equal(ids, g["expert_ids"]) and np.array_equal(bits(w), bits(g["weights"]))
    y32, _, _, _ = oracle.moe_layer(x, wg, ew, K, I)
    assert np.array_equal(bits(y32), bits(g["y_naive"]))
    m_in = oracle.compare(g["y_naive_fp16in"], g["y_naive"])
    assert m_in["max_abs"] > 0.05 and m_in["mean_abs"] > 0.01 and m_in["cos"] > 0.99, m_in
