"""Recognition of the unfused self-attention subgraph that graph_execute runs as one
OP_MHA_FUSED node (graph_detect_mha; the reference's detect_and_fuse_mha,
src/application/engine/graph.c:347-665).  CPU only: these tests build graphs and inspect
the matches; the GPU execution of fused graphs is in test_fused_gpu.py."""

import numpy as np
import pytest

from helpers import (DT_F16, DT_F32, OP_INPUT, OP_OUTPUT, OP_RELU, FusedCase, Graph,
                     build_attention_subgraph)


def _graph(native, c, residual=True, **kw):
    import oracle as O
    dt = DT_F16 if c.f16 else DT_F32
    conv = (lambda a: O.to_f16(a)) if c.f16 else (lambda a: np.asarray(a, np.float32))
    g = Graph(native)
    tX, iX = g.tensor(conv(c.X), dt)
    iR = g.tensor(conv(c.R), dt)[1] if residual else None
    ids = build_attention_subgraph(g, c, iX, iR, **kw)
    native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
    native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids["out"]], []))
    assert native.graph_build(g.g) == 0
    return g, ids, iX, iR


@pytest.mark.parametrize("f16", [False, True])
def test_bert_pattern_is_detected(native, f16):
    import cudaforge_amd as cf
    c = FusedCase(2, 16, 4, 4, 8, seed=3, f16=f16, residual=True, bias_std=0.02)
    g, ids, iX, iR = _graph(native, c)
    try:
        m = cf.graph_detect_mha(g.g)
        assert len(m) == 1
        m = m[0]
        p = m.params
        assert (p.batch_size, p.seq_len, p.hidden_size, p.num_heads, p.num_kv_heads, p.head_dim) == (2, 16, 32, 4, 4, 8)
        assert p.has_residual and not p.causal
        assert abs(p.scale - 1 / np.sqrt(8)) < 1e-7
        assert m.input_tid == iX and m.residual_tid == iR and m.output_tid == ids["out"]
        assert m.out_node == ids["add_r"]
        pattern = {v for k, v in ids.items() if k != "out"}
        assert set(m.nodes[:m.num_nodes]) == pattern and m.num_nodes == 21
        assert all(m.weights[i] for i in range(8))
    finally:
        g.destroy()


def test_causal_gqa_and_scale_are_read_from_the_graph(native):
    import cudaforge_amd as cf
    c = FusedCase(1, 12, 4, 2, 8, seed=4, residual=False)
    g, ids, _, _ = _graph(native, c, residual=False, causal=True, scale=0.2, bias=False)
    try:
        (m,) = cf.graph_detect_mha(g.g)
        p = m.params
        assert p.causal and not p.has_residual and p.num_kv_heads == 2 and abs(p.scale - 0.2) < 1e-7
        assert m.residual_tid == -1 and m.out_node == ids["mm_o"]
        assert not any(m.weights[i] for i in (1, 3, 5, 7))       # no bias Adds
        assert m.num_nodes == 3 * 3 + 9                          # + CausalMask and its Add
        assert ids["mask"] in m.nodes[:m.num_nodes] and ids["add_mask"] in m.nodes[:m.num_nodes]
    finally:
        g.destroy()


def test_two_stacked_layers_are_both_detected(native):
    """The reference fused the first match only (graph.c:655); every layer is found here."""
    import cudaforge_amd as cf
    import oracle as O
    c = FusedCase(1, 8, 2, 2, 8, seed=5, residual=True)
    g = Graph(native)
    try:
        _, iX = g.tensor(np.asarray(c.X, np.float32))
        ids1 = build_attention_subgraph(g, c, iX, iX)
        ids2 = build_attention_subgraph(g, c, ids1["out"], ids1["out"])
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids2["out"]], []))
        assert native.graph_build(g.g) == 0
        ms = cf.graph_detect_mha(g.g)
        assert sorted(m.out_node for m in ms) == sorted([ids1["add_r"], ids2["add_r"]])
    finally:
        g.destroy()


@pytest.mark.parametrize("breakage", ["softmax_is_relu", "scores_read_twice", "weight_dtype", "no_mask_op"])
def test_broken_patterns_are_left_alone(native, breakage):
    import cudaforge_amd as cf
    c = FusedCase(1, 8, 2, 2, 8, seed=6, residual=True)
    kw = {"softmax_is_relu": dict(softmax_op=OP_RELU), "scores_read_twice": dict(extra_scores_reader=True),
          "weight_dtype": dict(wdtype=DT_F16), "no_mask_op": dict()}[breakage]
    g, ids, _, _ = _graph(native, c, **kw)
    try:
        ms = cf.graph_detect_mha(g.g)
        if breakage == "no_mask_op":
            assert len(ms) == 1 and not ms[0].params.causal
        else:
            assert ms == []
    finally:
        g.destroy()


def test_old_passthrough_mask_pattern_is_not_fused(native):
    """Mul -> CausalMask(scores) -> Softmax computes softmax(mask) op by op (CausalMask
    ignores its input, causal_mask.c:5-8), so running it as masked attention would change
    the result: it must stay unfused."""
    import cudaforge_amd as cf
    c = FusedCase(1, 12, 4, 2, 8, seed=4, residual=False)
    g, _, _, _ = _graph(native, c, residual=False, causal=True, mask_style="passthrough")
    try:
        assert cf.graph_detect_mha(g.g) == []
    finally:
        g.destroy()


def test_mask_of_another_length_is_not_fused(native):
    import cudaforge_amd as cf
    c = FusedCase(1, 12, 4, 2, 8, seed=4, residual=False)
    g, _, _, _ = _graph(native, c, residual=False, causal=True, mask_seq=11)
    try:
        assert cf.graph_detect_mha(g.g) == []
    finally:
        g.destroy()


def test_shared_mask_node_still_runs(native):
    """A mask that another node also reads is not swallowed by the match."""
    import cudaforge_amd as cf
    c = FusedCase(1, 12, 4, 2, 8, seed=4, residual=False)
    g, ids, _, _ = _graph(native, c, residual=False, causal=True, mask_style="add_shared")
    try:
        (m,) = cf.graph_detect_mha(g.g)
        nodes = set(m.nodes[:m.num_nodes])
        assert m.params.causal and ids["add_mask"] in nodes and ids["mask"] not in nodes
    finally:
        g.destroy()


@pytest.mark.parametrize("style,fused", [("weight", True), ("constant", False), ("produced", False),
                                         ("swapped", False)])
def test_scale_operand_rules(native, style, fused):
    """The scale is read on the host and becomes a kernel argument that a recorded replay
    keeps, so only a node weight counts (a graph tensor, even one no node writes, may be
    rewritten by the caller between executions), and the scores must be the Mul's first
    input."""
    import cudaforge_amd as cf
    c = FusedCase(1, 8, 2, 2, 8, seed=6, residual=True)
    g, _, _, _ = _graph(native, c, scale=0.3, scale_style=style)
    try:
        ms = cf.graph_detect_mha(g.g)
        if fused:
            assert len(ms) == 1 and abs(ms[0].params.scale - 0.3) < 1e-7
        else:
            assert ms == []
    finally:
        g.destroy()


def test_bias_from_a_graph_tensor_is_not_a_weight(native):
    """Bias Adds whose bias is only a graph tensor (no node weight) are not fused: the
    fused op uploads its weights once."""
    import cudaforge_amd as cf
    c = FusedCase(1, 8, 2, 2, 8, seed=6, residual=True)
    g, _, _, _ = _graph(native, c, bias_style="input")
    try:
        assert cf.graph_detect_mha(g.g) == []
    finally:
        g.destroy()


def test_single_token_residual_without_output_bias(native):
    """B*S == 1: the residual Add has D elements, like b_O; with no bias Add on W_O it is
    still the residual, because b_O only comes from a node weight."""
    import cudaforge_amd as cf
    c = FusedCase(1, 1, 2, 2, 8, seed=8, residual=True)
    g = Graph(native)
    try:
        _, iX = g.tensor(np.asarray(c.X, np.float32))
        _, iR = g.tensor(np.asarray(c.R, np.float32))
        ids = build_attention_subgraph(g, c, iX, iR, bias=False)
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids["out"]], []))
        assert native.graph_build(g.g) == 0
        (m,) = cf.graph_detect_mha(g.g)
        assert m.residual_tid == iR and m.params.has_residual and not m.weights[7]
        assert m.out_node == ids["add_r"]
    finally:
        g.destroy()
