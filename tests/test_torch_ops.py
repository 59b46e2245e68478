"""The torch.library registration of the three operators (the reference's empty framework adapter,
framework/CMakeLists.txt:1-9): shape/dtype rules on meta and fake tensors here, execution on the GPU below."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

from conftest import PKG_NAME, load_golden

torch = pytest.importorskip("torch")
tops = importlib.import_module(PKG_NAME + ".torch_ops")
op = torch.ops.moe_mi355x


def meta(*shape, dtype=torch.float16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def test_meta_shapes_follow_infer_rules():
    x, wg, ew = meta(7, 64), meta(64, 8), meta(8, 3 * 96, 64)
    ids, w = op.MoeRoutingTopK(x, wg, 3)
    assert (ids.shape, ids.dtype, w.shape, w.dtype) == ((7, 3), torch.int32, (7, 3), torch.float16)
    assert op.MoeRoutingTopK(x, wg, 0)[0].shape == (7, 2)  # attr default topK = 2
    eo = op.MoeExpertFFN(x, ids, w, ew, 0)
    assert (eo.shape, eo.dtype) == ((7, 3, 64), torch.float16)
    y = op.MoeCombine(eo, ids, w, 3)
    assert (y.shape, y.dtype) == ((7, 64), torch.float16)
    with pytest.raises(RuntimeError, match="hiddenSize mismatch"):
        op.MoeRoutingTopK(meta(7, 32), wg, 2)


def test_fake_tensor_mode_propagates_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x, wg, ew = torch.empty(5, 128, dtype=torch.float16), torch.empty(128, 16, dtype=torch.float16), \
            torch.empty(16, 3 * 256, 128, dtype=torch.float16)
        ids, w = op.MoeRoutingTopK(x, wg, 2)
        y = op.MoeCombine(op.MoeExpertFFN(x, ids, w, ew, 0), ids, w, 2)
        assert tuple(y.shape) == (5, 128)


def test_cpu_tensors_have_no_kernel():
    with pytest.raises(NotImplementedError):
        op.MoeRoutingTopK(torch.zeros(4, 64, dtype=torch.float16), torch.zeros(64, 4, dtype=torch.float16), 2)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["ref_small_seed42", "ref_mid_seed43", "synth_mid_seed43"])
def test_registered_ops_match_reference(ops, case):
    """torch.ops.moe_mi355x.* against the reference's own outputs stored in the golden fixture: expert_ids bit
    for bit (tokens whose K-th and (K+1)-th probabilities are within 1e-3 excepted), y against its NaiveMoE y at
    the reference's thresholds; and the same tensors as the direct C-ABI path."""
    import oracle

    g = load_golden(case)
    x, wg, ew = (torch.from_numpy(np.ascontiguousarray(g[k])).cuda() for k in ("x", "w_gate", "expert_weights"))
    K = int(g["K"])
    ids, w = op.MoeRoutingTopK(x, wg, K)
    eo = op.MoeExpertFFN(x, ids, w, ew, 0)
    y = op.MoeCombine(eo, ids, w, K)
    torch.cuda.synchronize()
    _, _, probs, _ = oracle.routing(g["x"].astype(np.float32), g["w_gate"].astype(np.float32), K)
    boundary, inner = oracle.topk_gaps(probs, K)
    settled = (boundary >= 1e-3) & (inner >= 1e-3)
    assert np.array_equal(ids.cpu().numpy()[settled], g["expert_ids"][settled])
    m = oracle.compare(y.float().cpu().numpy(), g["y_naive"])
    assert m["max_abs"] < 0.05 and m["mean_abs"] < 0.01 and m["cos"] > 0.99, m
    y2, ids2, w2, eo2 = ops.moe_layer(x, wg, ew, K)
    for a, b in ((y, y2), (ids, ids2), (w, w2), (eo, eo2)):
        assert torch.equal(a, b)
    assert torch.equal(tops.moe_layer(x, wg, ew, K), y)


@pytest.mark.gpu
def test_opcheck_and_fullgraph_compile(ops):
    g = load_golden("ref_small_seed42")
    x, wg, ew = (torch.from_numpy(np.ascontiguousarray(g[k])).cuda() for k in ("x", "w_gate", "expert_weights"))
    K = int(g["K"])
    ids, w = op.MoeRoutingTopK(x, wg, K)
    eo = op.MoeExpertFFN(x, ids, w, ew, 0)
    utils = ("test_schema", "test_faketensor")
    torch.library.opcheck(op.MoeRoutingTopK, (x, wg, K), test_utils=utils)
    torch.library.opcheck(op.MoeExpertFFN, (x, ids, w, ew, 0), test_utils=utils)
    torch.library.opcheck(op.MoeCombine, (eo, ids, w, K), test_utils=utils)
    compiled = torch.compile(tops.moe_layer, backend="aot_eager", fullgraph=True)
    assert torch.equal(compiled(x, wg, ew, K), tops.moe_layer(x, wg, ew, K))
