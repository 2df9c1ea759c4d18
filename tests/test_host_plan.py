"""The full Flux2 transformer recorded through the C++ host modules and
planned without a device (dit_cli --plan-only): graph size, the GEMM and
attention node counts, the parameter count of the 4B-shaped configuration,
and how many nodes each block type hands to fused kernels.

Per single-stream block 34 nodes are absorbed: adaLN 4 (NORM, MUL, and the
ADD and FILL of its 1 + scale, Tensor.hpp:233-236), each of
q and k 12 (RMS_NORM, MUL, 4 x (VIEW, ROPE), 2 inner CONCATs), q's root
CONCAT and its permuted VIEW into the attention's prologue 2, SwiGLU 2
(SIGMOID, MUL), gated residual 1 (MUL), GEMM accumulate 1 (MUL_MAT).  Per
double-stream block 56: 4 adaLNs x 4, q and k 15 each (two RMS_NORM + MUL
segments joined by the txt|img CONCAT, plus the RoPE tree), q's root and
view 2, 2 SwiGLUs x 2, 4 gated residuals x 1."""
import json
import os
import subprocess

import pytest

from conftest import PKG

CLI = os.path.join(PKG, "bin", "dit_cli")


def plan(**kw):
    if not os.path.exists(CLI):
        pytest.skip("dit_cli not built")
    args = [CLI, "Flux2Transformer2DModel", "--plan-only", "true"]
    for k, v in kw.items():
        args += ["--" + k, str(v)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_full_step_graph():
    p = plan()
    # 2 time-embedding + 3 modulation + 2 embedder Linears, 5 x 14 double-block
    # and 20 x 7 single-block projections, norm_out and proj_out
    assert p["mul_mat_nodes"] == 2 + 3 + 2 + 5 * 14 + 20 * 7 + 2 == 219
    assert p["attention_nodes"] == 25
    assert p["params"] == 3859815936
    assert p["arena_bytes"] < 1 << 30 and p["arena_bytes"] * 50 < p["naive_bytes"], p


def test_q8_0_weights_plan_like_bf16():
    """Q8_0 Linear weights (DT_TYPE_Q8_0_SPLIT) take the same MUL_MAT, GEMM
    accumulate and grouped-projection paths as BF16 ones: identical plan."""
    q, b = plan(**{"weight-format": "q8_0"}), plan(**{"weight-format": "bf16"})
    assert q == b


@pytest.mark.parametrize("kind,layers,nodes,fused,mm,grouped,deferred", [
    ("single", dict(num_layers=0), 58, 34, 7, 5, 1),
    ("double", dict(num_single_layers=0), 110, 56, 14, 8, 5),
])
def test_per_block_fusion(kind, layers, nodes, fused, mm, grouped, deferred):
    """A second block adds its nodes, fusions and GEMMs; `grouped` roots run
    in an earlier node's launch (single: k, v, gate, up with q's projection,
    and the SwiGLU with k's QK-RMSNorm+RoPE, q's being the attention's
    prologue; double:
    k, v and the three txt projections with q, up with gate on each stream,
    to_out with to_add_out), and `deferred` nodes run in a later launch:
    residuals written by the next adaLN's fused kernel (one per block
    boundary: single 1; double 2 inside the block and 2 at the boundary),
    and in a double block the image feed-forward's output projection, which
    joins the text stream's (192 + 24 tiles: one wave instead of two
    launches)."""
    key = "num_single_layers" if kind == "single" else "num_layers"
    a = plan(**layers, **{key: 1})
    b = plan(**layers, **{key: 2})
    assert b["nodes"] - a["nodes"] == nodes
    assert b["fused_nodes"] - a["fused_nodes"] == fused
    assert b["mul_mat_nodes"] - a["mul_mat_nodes"] == mm
    assert b["attention_nodes"] - a["attention_nodes"] == 1
    assert b["grouped_nodes"] - a["grouped_nodes"] == grouped
    assert b["deferred_nodes"] - a["deferred_nodes"] == deferred


def test_node_order_allocation_keeps_most_fusion():
    """The full step with node memory placed as ggml_gallocr places it (node
    order, in place where allowed; dit_cli --alloc node-order): the
    executor's address replay holds back the launches that would read
    memory another node took over, and keeps the rest fused."""
    p = plan(alloc="node-order")
    f = plan()
    assert f["launches_held"] == 0 and p["fused_nodes"] == f["fused_nodes"]
    assert 0 < p["launches_held"] < 100, p
    assert p["fused_nodes_checked"] > 0.7 * p["fused_nodes"], p


@pytest.mark.parametrize("path,rows,cols", [("transformer_blocks.0.attn.to_q.weight", 96, 256),
                                            ("single_transformer_blocks.19.attn.to_out.mlp.weight", 3, 9216),
                                            ("single_transformer_blocks.0.attn.norm_q.weight", 128, 0)])
def test_hash_weights_match_the_oracle(orc, tmp_path, path, rows, cols):
    """dit_cli --hash-weights draws its weights on the host by the rule the
    oracle restates (or_hash_q8_0 / or_hash_norm_weight): the Q8_0 blocks of
    a Linear weight and an RMSNorm weight's fp32 values are byte-identical,
    so a full-width model run on the GPU can be checked against the oracle
    on the same weights without shipping them."""
    if not os.path.exists(CLI):
        pytest.skip("dit_cli not built")
    out = tmp_path / "w.bin"
    args = [CLI, "HashWeights", "--seed", "11", "--path", path, "--rows", str(rows), "--out", str(out)]
    if cols:
        args += ["--cols", str(cols)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = out.read_bytes()
    want = orc.hash_q8_0(11, path, rows, cols) if cols else orc.hash_norm_weight(11, path, rows)
    assert got == want.tobytes()
