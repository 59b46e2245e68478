"""The header as a C call site sees it: include/moe_ops.h compiles as ISO C99 with every warning an error, links
against libmoe_mi355x.so, and the InferShape / workspace / argument-check path of the three operators behaves
as the reference's op_host layer does (op_host/moe_ops.cpp:71-90,181-226,241-258,340-349). The program launches
nothing: every launch call it makes fails its checks first, so it runs without a GPU."""
from __future__ import annotations

import shutil
import subprocess

import pytest

from conftest import ROOT, package

C_PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "moe_ops.h"

#define EXPECT(cond) do { if (!(cond)) { printf("FAIL line %d: %s (%s)\n", __LINE__, #cond, moe_last_error()); return 1; } } while (0)

int main(void) {
    const int64_t x_dims[2] = {128, 2048}, wg_dims[2] = {2048, 16}, ew_dims[3] = {16, 3 * 8192, 2048};
    int64_t ids_dims[2] = {0, 0}, w_dims[2] = {0, 0}, out_dims[3] = {0, 0, 0}, y_dims[2] = {0, 0}, inter = 0;
    moe_dtype t_ids, t_w, t_out;
    moe_ffn_plan plan;
    size_t ws;

    /* InferShape / InferDataType: [T, K] int32 + [T, K] fp16; [T, K, H] fp16 with I from expert_weights */
    EXPECT(moe_routing_topk_infer_shape(x_dims, 2, wg_dims, 2, 2, ids_dims, w_dims) == MOE_OK);
    EXPECT(ids_dims[0] == 128 && ids_dims[1] == 2 && w_dims[0] == 128 && w_dims[1] == 2);
    EXPECT(moe_routing_topk_infer_dtype(&t_ids, &t_w) == MOE_OK && t_ids == MOE_DT_INT32 && t_w == MOE_DT_FLOAT16);
    EXPECT(moe_expert_ffn_infer_shape(x_dims, 2, ids_dims, 2, ew_dims, 3, 0, out_dims, &inter) == MOE_OK);
    EXPECT(out_dims[0] == 128 && out_dims[1] == 2 && out_dims[2] == 2048 && inter == 8192);
    EXPECT(moe_expert_ffn_infer_dtype(&t_out) == MOE_OK && t_out == MOE_DT_FLOAT16);
    EXPECT(moe_combine_infer_shape(out_dims, 3, ids_dims, 2, y_dims) == MOE_OK && y_dims[0] == 128 && y_dims[1] == 2048);

    /* the reference's GRAPH_FAILED causes: null shape, wrong rank, hidden-size mismatch */
    EXPECT(moe_routing_topk_infer_shape(NULL, 2, wg_dims, 2, 2, ids_dims, w_dims) == MOE_ERR_NULL);
    EXPECT(moe_routing_topk_infer_shape(x_dims, 3, wg_dims, 2, 2, ids_dims, w_dims) == MOE_ERR_RANK);
    {
        const int64_t bad_wg[2] = {1024, 16};
        EXPECT(moe_routing_topk_infer_shape(x_dims, 2, bad_wg, 2, 2, ids_dims, w_dims) == MOE_ERR_SHAPE);
        EXPECT(strlen(moe_last_error()) > 0);
    }

    /* workspace: reported, never allocated; the plan agrees */
    ws = moe_expert_ffn_workspace_bytes(128, 2048, 16, 2, 8192);
    EXPECT(ws > 0);
    EXPECT(moe_expert_ffn_plan(128, 2048, 16, 2, 8192, &plan) == MOE_OK && plan.workspace_bytes == ws);

    /* launches fail their checks before anything is queued */
    EXPECT(moe_routing_topk(NULL, NULL, NULL, NULL, 128, 2048, 16, 2, NULL) == MOE_ERR_NULL);
    EXPECT(moe_expert_ffn(NULL, NULL, NULL, NULL, NULL, NULL, ws, 128, 2048, 16, 2, 8192, NULL) == MOE_ERR_NULL);
    EXPECT(moe_combine(NULL, NULL, NULL, NULL, 128, 2048, 2, NULL) == MOE_ERR_NULL);
    EXPECT(strcmp(moe_status_string(MOE_ERR_WORKSPACE), "MOE_ERR_WORKSPACE") == 0);
    printf("ok %s\n", moe_version());
    return 0;
}
"""


def test_header_compiles_as_c99_links_and_checks_arguments(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not installed")
    lib_path = package()._lib.LIB_PATH
    if not lib_path.exists():
        pytest.skip("libmoe_mi355x.so is not built")
    src = tmp_path / "callsite.c"
    src.write_text(C_PROGRAM)
    exe = tmp_path / "callsite"
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}", str(src),
           f"-L{lib_path.parent}", "-lmoe_mi355x", f"-Wl,-rpath,{lib_path.parent}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0 and run.stdout.startswith("ok "), run.stdout + run.stderr
