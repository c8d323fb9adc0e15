"""MHA_Fused on the GPU through the C-ABI vs the CPU oracle.

FP32 path <= 1e-4 max abs error, FP16 path <= 2e-2 (fp32 accumulation).  Shapes: the
reference's own fused test (tests/test_bert_mha.c:36-40, LCG inputs, residual on), its
long-sequence test shape (S=128, H=12, d=64, X scaled by 1/D, :484-513), causal and GQA
variants, ragged tile edges, and BASELINE configs 3 and 5 at full size checked on
selected batch rows (rows are independent, so a row of the full-size run must equal the
oracle on that row alone).
"""

import ctypes

import numpy as np
import pytest

from helpers import FusedCase, dev, max_abs, run_fused_gpu

pytestmark = pytest.mark.gpu

TOL32 = 1e-4
TOL16 = 2e-2


@pytest.mark.parametrize("f16", [False, True])
def test_reference_bert_kat(gpu, f16):
    c = FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True, f16=f16)
    want = c.oracle()
    got = run_fused_gpu(c)
    assert max_abs(want, got) <= (TOL16 if f16 else TOL32)
    assert np.count_nonzero(np.abs(got) > 1e-6) > got.size // 2   # test_bert_mha.c:299-303


def f16_half_ulp(x):
    """Half the fp16 spacing at |x|: the rounding of an fp16 output alone."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -14)
    return 0.5 * 2.0 ** (np.floor(np.log2(ax)) - 10)


@pytest.mark.parametrize("f16", [False, True])
def test_reference_long_seq_shape(gpu, f16):
    """The reference's LCG data lie in [-1, 0), so outputs here are ~1e2 (residual and
    biases included) and the fp16 output grid alone is 0.0625 wide: the FP16 bound is
    2e-2 on top of half an fp16 ulp of the exact value."""
    c = FusedCase(1, 128, 12, 12, 64, fill="lcg", residual=True, f16=f16, x_scale=1.0 / 768)
    want = c.oracle()
    got = run_fused_gpu(c)
    if f16:
        assert np.all(np.abs(want.astype(np.float64) - got) <= TOL16 + f16_half_ulp(want))
    else:
        assert max_abs(want, got) <= TOL32


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("B,S,H,H_kv,d,causal", [(2, 200, 4, 4, 64, True), (1, 96, 8, 2, 64, False),
                                                  (2, 77, 4, 4, 64, False), (1, 130, 2, 2, 128, True),
                                                  (2, 33, 3, 3, 16, True)])
def test_fused_vs_oracle(gpu, f16, B, S, H, H_kv, d, causal):
    c = FusedCase(B, S, H, H_kv, d, seed=S + d, f16=f16, causal=causal, residual=(S % 2 == 0), bias_std=0.02)
    want = c.oracle()
    got = run_fused_gpu(c)
    assert max_abs(want, got) <= (TOL16 if f16 else TOL32)


@pytest.mark.parametrize("B,S,H,H_kv,d,causal,residual", [(2, 64, 4, 4, 64, False, True), (1, 130, 8, 2, 64, True, False),
                                                         (2, 33, 3, 3, 16, False, True), (8, 512, 12, 12, 64, False, False)])
def test_fused_f16_entry_takes_float_buffers(gpu, B, S, H, H_kv, d, causal, residual):
    """mha_fused_f16_cuda keeps the reference's contract (mha_fused_f16_cuda.cu:209-244,
    registered "f32", called with float buffers by tests/bench_bert_mha.c:233-266): FP32
    inputs and output, fp16 arithmetic inside.  Its result is bit for bit the fp16-I/O
    op's (mha_fused_f16io_cuda) on the inputs rounded to fp16, widened to fp32, and within
    the fp16 tolerance of the oracle on those rounded inputs."""
    import cudaforge_amd as cf
    c32 = FusedCase(B, S, H, H_kv, d, seed=40 + S, f16=False, causal=causal, residual=residual, bias_std=0.02)
    c16 = FusedCase(B, S, H, H_kv, d, seed=40 + S, f16=True, causal=causal, residual=residual, bias_std=0.02)
    bufs = [None if a is None else dev(a, False) for a in c32.arrays()]
    Y = cf.DeviceBuffer.empty((B, S, H * d), np.float32)
    assert cf.call_op("mha_fused_f16_cuda", bufs, [Y], c32.params(cf.MhaFusedParams)) == 0
    got = Y.download()
    assert got.dtype == np.float32
    assert np.array_equal(got, run_fused_gpu(c16))
    assert max_abs(c16.oracle(), got) <= TOL16


def test_config3_bert_base_full_size(gpu):
    """B=8, S=512, D=768, 12x64, fp16, no mask.  Every row of the
    full-size run against a float64 evaluation of the same math, and batch rows 0 and 7
    against the oracle on those rows alone."""
    from helpers import fused_ref64
    c = FusedCase(8, 512, 12, 12, 64, seed=3, f16=True)
    got = run_fused_gpu(c)
    per_row = np.abs(fused_ref64(c) - got).max(axis=2)
    assert (per_row <= TOL16).all(), per_row.max()
    for b in (0, 7):
        sub = FusedCase(1, 512, 12, 12, 64, seed=3, f16=True)
        for n in ("X", "WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO"):
            setattr(sub, n, getattr(c, n))
        sub.X = c.X[b:b + 1]
        assert max_abs(sub.oracle(), got[b:b + 1]) <= TOL16
    assert np.isfinite(got).all()


def test_config5_causal_full_size_row(gpu):
    """BASELINE config 5 shape (B=4, S=1024, D=1024, 16x64, causal, fp16): every row
    against a float64 evaluation of the same math, and batch row 2 against the oracle."""
    from helpers import fused_ref64
    c = FusedCase(4, 1024, 16, 16, 64, seed=5, f16=True, causal=True)
    got = run_fused_gpu(c)
    per_row = np.abs(fused_ref64(c) - got).max(axis=2)
    assert (per_row <= TOL16).all(), per_row.max()
    sub = FusedCase(1, 1024, 16, 16, 64, seed=5, f16=True, causal=True)
    for n in ("WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO"):
        setattr(sub, n, getattr(c, n))
    sub.X = c.X[2:3]
    assert max_abs(sub.oracle(), got[2:3]) <= TOL16


@pytest.mark.parametrize("B,S,H,d,causal", [(8, 512, 12, 64, False), (4, 1024, 16, 64, True)])
def test_fp32_full_size_configs(gpu, B, S, H, d, causal):
    """Configs 3 and 5's shapes through the FP32 entry (fp32 MFMA GEMMs and attention;
    the second shape takes the attention kernel's 32-query waves): every row against a
    float64 evaluation of the same math, within the FP32 bound."""
    from helpers import fused_ref64
    c = FusedCase(B, S, H, H, d, seed=70 + S, f16=False, causal=causal, residual=True, bias_std=0.02)
    got = run_fused_gpu(c)
    per_row = np.abs(fused_ref64(c) - got).max(axis=2)
    assert (per_row <= TOL32).all(), per_row.max()


def test_residual_flag_with_null_residual(gpu):
    """has_residual with a NULL residual slot adds nothing (the reference's `R != NULL`
    guard, mha_fused.c:165-170)."""
    c = FusedCase(2, 64, 4, 4, 64, seed=9, f16=True, residual=False, bias_std=0.02)
    want = c.oracle()
    c.residual = True          # flag on, slot 1 stays NULL
    got = run_fused_gpu(c)
    assert max_abs(want, got) <= TOL16


@pytest.mark.parametrize("f16", [False, True])
def test_graph_fused_on_gpu(gpu, native, f16):
    """graph_execute(use_cuda) over one OP_MHA_FUSED node (the reference's GPU graph test,
    tests/test_bert_mha.c:167-306): F32 tensors resolve to mha_fused_f32_cuda, F16 tensors
    to the fp16-I/O mha_fused_f16io_cuda."""
    from helpers import DT_F16, DT_F32, OP_INPUT, OP_MHA_FUSED, OP_OUTPUT, Graph
    import oracle as O
    c = FusedCase(2, 48, 4, 2, 32, seed=17, f16=f16, residual=True, causal=True, bias_std=0.02)
    dt, npdt = (DT_F16, np.float16) if f16 else (DT_F32, np.float32)
    conv = (lambda a: O.to_f16(a)) if f16 else (lambda a: np.asarray(a, np.float32))
    g = Graph(native)
    try:
        tX, iX = g.tensor(conv(c.X), dt)
        tR, iR = g.tensor(conv(c.R), dt)
        tY, iY = g.tensor(conv(np.zeros_like(c.X)), dt)
        ws = [g.tensor(conv(w), dt)[0] for w in (c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO)]
        p = O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, True, True)
        nid = g.node(OP_MHA_FUSED, [iX, iR], [iY], ws, p)
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
        assert native.graph_build(g.g) == 0
        buf = ctypes.create_string_buffer(64)
        assert native.graph_resolve_op(g.g, nid, True, buf, 64)
        assert buf.value == (b"mha_fused_f16io_cuda" if f16 else b"mha_fused_f32_cuda")
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(g.g, ins, outs, True) == 0
        got = g.read(tY, c.X.shape, npdt)
        assert max_abs(c.oracle(), got) <= (TOL16 if f16 else TOL32)
    finally:
        g.destroy()


@pytest.mark.parametrize("causal", [False, True])
def test_flash_kernel_variants_agree(gpu, native, causal):
    """The fp16 d = 64 attention kernels (register staged; DMA ring with 32 or 16 queries
    per wave) on a GQA shape whose length is a multiple of 8 but not of the 64-key
    block: each within the FP16 bound of the oracle and close to the others."""
    c = FusedCase(2, 264, 8, 2, 64, seed=71, f16=True, causal=causal, residual=True, bias_std=0.02)
    want = c.oracle()
    outs = []
    try:
        for mode in (0, 1, 2, 3):
            native.cf_flash_set_mode(mode)
            outs.append(run_fused_gpu(c))
    finally:
        native.cf_flash_set_mode(3)
    for o in outs:
        assert max_abs(want, o) <= TOL16
        assert max_abs(outs[0], o) <= 1e-2


@pytest.mark.parametrize("B,S,H,H_kv,mode", [(2, 264, 8, 2, 2), (2, 264, 8, 2, 1), (1, 1024, 16, 16, 2), (3, 72, 4, 4, 2)])
def test_causal_attention_schedules_bit_identical(gpu, native, B, S, H, H_kv, mode):
    """Causal DMA attention with each query block paired with its mirror in one
    workgroup (cf_flash_set_causal_pairs(1)) and with one block per workgroup, heaviest
    first (0, the default): the same per-block arithmetic, so the same bits, at 16- and
    32-query waves, an odd block count and a length inside a block."""
    c = FusedCase(B, S, H, H_kv, 64, seed=S + 5, f16=True, causal=True, residual=False, bias_std=0.02)
    outs = []
    try:
        native.cf_flash_set_mode(mode)
        for pairs in (1, 0):
            native.cf_flash_set_causal_pairs(pairs)
            outs.append(run_fused_gpu(c))
    finally:
        native.cf_flash_set_causal_pairs(0)
        native.cf_flash_set_mode(3)
    assert max_abs(c.oracle(), outs[0]) <= TOL16
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("B,S,H,H_kv,causal", [(16, 200, 8, 2, False), (16, 200, 8, 2, True), (1, 384, 6, 6, True),
                                              (2, 512, 12, 12, False)])
def test_prefill_row_concatenated_qkv(gpu, native, B, S, H, H_kv, causal):
    """fp16 prefill with the QKV product written as one row-major (B*S, (H + 2 H_kv) d)
    matrix that attention reads directly (K and V rows as they are, V transposed on its
    way out of LDS), against the oracle and against the head-major q / k / v^T scatter:
    GQA, a length that ends inside a 64-key block, causal and not, and both query widths
    of the attention kernel."""
    c = FusedCase(B, S, H, H_kv, 64, seed=S + H, f16=True, causal=causal, residual=True, bias_std=0.02)
    want = c.oracle()
    outs = []
    try:
        for rowcat, mode in ((1, 2), (1, 1), (0, 3)):
            native.mha_fused_set_rowcat(rowcat)
            native.cf_flash_set_mode(mode)
            outs.append(run_fused_gpu(c))
    finally:
        native.mha_fused_set_rowcat(1)
        native.cf_flash_set_mode(3)
    for o in outs:
        assert max_abs(want, o) <= TOL16
    assert max_abs(outs[0], outs[1]) <= 1e-2
    assert max_abs(outs[0], outs[2]) <= 1e-2


WS_SHAPES = [(256, 192), (256, 144), (256, 128), (256, 96), (256, 64), (256, 48), (128, 192), (128, 128),
             (128, 96), (128, 64)]


@pytest.mark.parametrize("H,H_kv", [(6, 6), (6, 2), (7, 1)])
def test_gemm_wave_specialised_shapes_agree(gpu, native, H, H_kv):
    """The wave-specialised fp16 projection GEMM at each of its tiles (a tile that does not
    fit a product leaves that product to the cost model's choice).  D = 384, M = 256: the
    QKV product's 144-column tiles straddle the Q|K and K|V boundaries; WO carries a bias
    and a residual (fp32 staging); H_kv = 2 gives K and V segments narrower than Q, and
    H = 7, H_kv = 1 a 192-column tile over the end of Q and all of K and V (the loaders'
    three-way segment choice; the other tiles take the one- and two-segment ones).  Every
    run within the FP16 bound of the oracle and bit-identical to the others (each output
    element sums the same 32-k MFMA steps in the same order), and within a few fp16 ulps
    of the kernels it replaces and of the default choice (the QKV product keeps the
    pipelined kernel unless a tile is forced)."""
    c = FusedCase(2, 128, H, H_kv, 64, seed=95, f16=True, causal=True, residual=True, bias_std=0.02)
    want = c.oracle()
    outs = []
    try:
        for bm, bn in WS_SHAPES:
            native.cf_gemm_set_ws_shape(bm, bn)
            outs.append(run_fused_gpu(c))
        native.cf_gemm_set_ws_shape(0, 0)
        auto = run_fused_gpu(c)
        native.cf_gemm_set_ws(1)
        native.cf_gemm_set_ksplit(1)
        old = run_fused_gpu(c)
    finally:
        native.cf_gemm_set_ws_shape(0, 0)
        native.cf_gemm_set_ws(0)
        native.cf_gemm_set_ksplit(0)
    for o in outs + [auto, old]:
        assert max_abs(want, o) <= TOL16
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)
    assert max_abs(outs[0], old) <= 1e-2
    assert max_abs(outs[0], auto) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
def test_gemm_tile_widths_agree(gpu, native, causal):
    """The fp16 projection GEMM with 128-, 96- and 192-column tiles on a shape all fit
    (D = 384 = 3 x 128 = 4 x 96 = 2 x 192; QKV with head-major and V^T scatter, WO with
    bias and residual): each within the FP16 bound of the oracle, and bit-identical to
    each other (every output element sums the same k-steps in the same order)."""
    c = FusedCase(2, 128, 6, 6, 64, seed=96, f16=True, causal=causal, residual=True, bias_std=0.02)
    want = c.oracle()
    outs = []
    try:
        native.cf_gemm_set_ws(1)       # the kernels this test is about
        native.cf_gemm_set_ksplit(1)   # one k group everywhere, so the sums match bit for bit
        for bn in (128, 96, 192, 0):
            native.cf_gemm_set_bn(bn)
            outs.append(run_fused_gpu(c))
    finally:
        native.cf_gemm_set_ws(0)
        native.cf_gemm_set_bn(0)
        native.cf_gemm_set_ksplit(0)
    for o in outs:
        assert max_abs(want, o) <= TOL16
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


def test_gemm_stage_depths_agree(gpu, native):
    """The fp16 projection GEMM's ring as 3 or 4 stages of 32 k and as 2 stages of 64 k
    (K = 384, both QKV with its head-major and V^T scatter and WO with bias and residual):
    within the FP16 bound of the oracle, and bit-identical to each other (every output
    element sums the same 32-k MFMA steps in the same order)."""
    c = FusedCase(2, 128, 6, 6, 64, seed=97, f16=True, causal=False, residual=True, bias_std=0.02)
    want = c.oracle()
    outs = []
    try:
        native.cf_gemm_set_ws(1)       # the kernels this test is about
        native.cf_gemm_set_ksplit(1)
        for bk, stages in ((32, 3), (32, 4), (64, 0), (0, 0)):
            native.cf_gemm_set_bk(bk)
            native.cf_gemm_set_stages(stages)
            outs.append(run_fused_gpu(c))
    finally:
        native.cf_gemm_set_ws(0)
        native.cf_gemm_set_bk(0)
        native.cf_gemm_set_stages(0)
        native.cf_gemm_set_ksplit(0)
    for o in outs:
        assert max_abs(want, o) <= TOL16
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


@pytest.mark.parametrize("bn", [128, 96])
def test_gemm_two_k_groups(gpu, native, bn):
    """The fp16 projection GEMM with each tile's k-loop split between two groups of 4
    waves (K = 384 and 768; QKV with its scatter, WO with bias and residual): within the
    FP16 bound of the oracle, and within a few fp16 ulps of the one-group kernel (the two
    halves of K are summed separately in fp32 and then added, so roundings differ)."""
    for case in (FusedCase(2, 128, 6, 6, 64, seed=98, f16=True, residual=True, bias_std=0.02),
                 FusedCase(1, 256, 12, 12, 64, seed=99, f16=True, causal=True, residual=True, bias_std=0.02)):
        want = case.oracle()
        outs = []
        try:
            native.cf_gemm_set_ws(1)
            native.cf_gemm_set_bn(bn)
            for ks in (1, 2):
                native.cf_gemm_set_ksplit(ks)
                outs.append(run_fused_gpu(case))
        finally:
            native.cf_gemm_set_ws(0)
            native.cf_gemm_set_ksplit(0)
            native.cf_gemm_set_bn(0)
        for o in outs:
            assert max_abs(want, o) <= TOL16
        assert max_abs(outs[0], outs[1]) <= 1e-2


@pytest.mark.parametrize("f16,causal", [(False, False), (True, False), (True, True)])
def test_graph_runs_unfused_attention_as_one_fused_op(gpu, native, f16, causal):
    """An unfused self-attention block (MatMul/Add/Reshape/Transpose/Mul/[CausalMask]/
    Softmax nodes, the reference fusion pass's pattern, graph.c:347-665) executed with
    use_cuda: graph_execute runs it as one OP_MHA_FUSED (no Softmax or Reshape operator is
    registered, and the MatMul nodes carry no params, so any node that ran unfused would
    fail the execution) and the output matches the oracle."""
    from helpers import DT_F16, DT_F32, OP_INPUT, OP_OUTPUT, Graph, build_attention_subgraph
    import oracle as O
    c = FusedCase(2, 40, 4, 2, 32, seed=23, f16=f16, residual=True, causal=causal, bias_std=0.02)
    dt, npdt = (DT_F16, np.float16) if f16 else (DT_F32, np.float32)
    conv = (lambda a: O.to_f16(a)) if f16 else (lambda a: np.asarray(a, np.float32))
    g = Graph(native)
    try:
        tX, iX = g.tensor(conv(c.X), dt)
        tR, iR = g.tensor(conv(c.R), dt)
        ids = build_attention_subgraph(g, c, iX, iR, causal=causal)
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids["out"]], []))
        assert native.graph_build(g.g) == 0
        tY = g.tensor(np.zeros(c.X.shape, npdt), dt)[0]
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(g.g, ins, outs, True) == 0
        got = g.read(tY, c.X.shape, npdt)
        assert max_abs(c.oracle(), got) <= (TOL16 if f16 else TOL32)
        # A second execution (fusion is decided per execution, the graph is unchanged).
        assert native.graph_execute(g.g, ins, outs, True) == 0
        assert max_abs(c.oracle(), g.read(tY, c.X.shape, npdt)) <= (TOL16 if f16 else TOL32)
    finally:
        g.destroy()


@pytest.mark.parametrize("f16", [False, True])
def test_graph_replay_matches_eager(gpu, native, f16):
    """GPU executions of an unchanged graph are recorded into a HIP graph on the second
    run and replayed after it.  Five executions with a new input each, with eager work
    (a direct operator call on the legacy stream) and synchronisations between them: every
    replayed result equals, bit for bit, the same graph run with replay off, and is
    within the bound of the oracle.  Changing the graph discards the recording."""
    import cudaforge_amd as cf
    from helpers import DT_F16, DT_F32, OP_INPUT, OP_OUTPUT, Graph, build_attention_subgraph
    import oracle as O
    c = FusedCase(2, 64, 4, 4, 32, seed=41, f16=f16, residual=True, bias_std=0.02)
    dt, npdt = (DT_F16, np.float16) if f16 else (DT_F32, np.float32)
    conv = (lambda a: O.to_f16(a)) if f16 else (lambda a: np.asarray(a, np.float32))
    graphs = []
    try:
        for replay in (1, 0):
            g = Graph(native)
            graphs.append(g)
            tX, iX = g.tensor(conv(c.X), dt)
            tR, iR = g.tensor(conv(c.R), dt)
            ids = build_attention_subgraph(g, c, iX, iR)
            native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
            native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids["out"]], []))
            assert native.graph_build(g.g) == 0
            native.graph_set_replay(g.g, replay)
            g.tX = tX
            g.tY = g.tensor(np.zeros(c.X.shape, npdt), dt)[0]
        side_in = cf.DeviceBuffer.from_numpy(np.ones(4096, np.float32))
        side_out = cf.DeviceBuffer.empty((64, 64), np.float32)
        states = []
        for it in range(5):
            X = conv(O.normal(c.X.shape, 900 + it))
            outs = []
            for g in graphs:
                g.write(g.tX, X)
                ins, os_ = (ctypes.c_void_p * 1)(g.tX), (ctypes.c_void_p * 1)(g.tY)
                assert native.graph_execute(g.g, ins, os_, True) == 0
                outs.append(g.read(g.tY, c.X.shape, npdt).astype(np.float32))
            states.append(native.graph_replay_state(graphs[0].g))
            assert np.array_equal(outs[0], outs[1]), f"execution {it}"
            want = O.mha_fused(np.asarray(X, np.float32), c.R, c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO,
                               O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, True, False))
            assert max_abs(want, outs[0]) <= (TOL16 if f16 else TOL32)
            # Eager work on the legacy stream between replays.
            assert cf.call_op("causal_mask_f32_cuda", [side_in], [side_out], cf.CausalMaskParams(64)) == 0
            native.gpu_stream_synchronize(None)
        assert states == [1, 2, 2, 2, 2]
        assert native.graph_replay_state(graphs[1].g) == 0
        graphs[0].tensor(np.zeros(4, npdt), dt)          # changing the graph drops the recording
        assert native.graph_replay_state(graphs[0].g) == 0
    finally:
        for g in graphs:
            g.destroy()


def test_graph_fuses_every_layer(gpu, native):
    """Two stacked attention blocks, each with the residual from its own input (BERT's
    wiring): both run fused; the reference fused only the first (graph.c:655)."""
    from helpers import DT_F32, OP_INPUT, OP_OUTPUT, Graph, build_attention_subgraph
    import oracle as O
    c = FusedCase(1, 24, 4, 4, 16, seed=29, residual=True, bias_std=0.02)
    g = Graph(native)
    try:
        tX, iX = g.tensor(np.asarray(c.X, np.float32))
        ids1 = build_attention_subgraph(g, c, iX, iX)
        ids2 = build_attention_subgraph(g, c, ids1["out"], ids1["out"])
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids2["out"]], []))
        assert native.graph_build(g.g) == 0
        tY = g.tensor(np.zeros_like(c.X, dtype=np.float32), DT_F32)[0]
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(g.g, ins, outs, True) == 0
        p = O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, True, False)
        w = [c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO]
        y1 = O.mha_fused(c.X, c.X, *w, p)
        y2 = O.mha_fused(y1, y1, *w, p)
        assert max_abs(y2, g.read(tY, c.X.shape)) <= 2 * TOL32
    finally:
        g.destroy()


@pytest.mark.parametrize("replay", [1, 0])
def test_graph_permanent_fusion_rewrites_once(gpu, native, replay):
    """graph_set_permanent_fusion (graph.c:151-153, :810-815): the first GPU execution
    rewrites each attention block of a two-layer stack into one OP_MHA_FUSED node (the
    block's last node, which then resolves to mha_fused_f32_cuda) and the pattern is no
    longer found; later executions, with new inputs, run the rewritten graph and match
    the oracle, recorded and replayed or eager."""
    import cudaforge_amd as cf
    from helpers import DT_F32, OP_INPUT, OP_OUTPUT, Graph, build_attention_subgraph
    import oracle as O
    c = FusedCase(1, 24, 4, 4, 16, seed=33, residual=True, bias_std=0.02)
    g = Graph(native)
    try:
        tX, iX = g.tensor(np.asarray(c.X, np.float32))
        ids1 = build_attention_subgraph(g, c, iX, iX)
        ids2 = build_attention_subgraph(g, c, ids1["out"], ids1["out"])
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids2["out"]], []))
        assert native.graph_build(g.g) == 0
        native.graph_set_replay(g.g, replay)
        native.graph_set_permanent_fusion(g.g, 1)
        last = [m.out_node for m in cf.graph_detect_mha(g.g)]
        assert len(last) == 2
        tY = g.tensor(np.zeros_like(c.X, dtype=np.float32), DT_F32)[0]
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        p = O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, True, False)
        w = [c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO]
        buf = ctypes.create_string_buffer(64)
        for it in range(4):
            X = O.normal(c.X.shape, 600 + it)
            g.write(tX, X)
            assert native.graph_execute(g.g, ins, outs, True) == 0, f"execution {it}"
            y1 = O.mha_fused(X, X, *w, p)
            assert max_abs(O.mha_fused(y1, y1, *w, p), g.read(tY, c.X.shape)) <= 2 * TOL32, f"execution {it}"
            assert cf.graph_detect_mha(g.g) == []
            for nid in last:
                assert native.graph_resolve_op(g.g, nid, True, buf, 64) and buf.value == b"mha_fused_f32_cuda"
        native.graph_set_permanent_fusion(g.g, 0)       # does not undo the rewrite
        assert cf.graph_detect_mha(g.g) == []
        assert native.graph_execute(g.g, ins, outs, True) == 0
    finally:
        g.destroy()


def test_graph_broken_attention_pattern_is_not_fused(gpu, native):
    """Softmax replaced by ReLU: nothing is fused, so the nodes run as themselves and the
    execution fails at the first one that cannot (its MatMul nodes carry no params here,
    which matmul_f32_cuda rejects with -1; ops that do not exist give -2)."""
    import cudaforge_amd as cf
    from helpers import DT_F32, OP_INPUT, OP_OUTPUT, OP_RELU, Graph, build_attention_subgraph
    c = FusedCase(1, 8, 2, 2, 8, seed=31, residual=True)
    g = Graph(native)
    try:
        tX, iX = g.tensor(np.asarray(c.X, np.float32))
        ids = build_attention_subgraph(g, c, iX, iX, softmax_op=OP_RELU)
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [ids["out"]], []))
        assert native.graph_build(g.g) == 0
        tY = g.tensor(np.zeros_like(c.X, dtype=np.float32), DT_F32)[0]
        assert cf.graph_detect_mha(g.g) == []
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(g.g, ins, outs, True) in (-1, -2)
    finally:
        g.destroy()
