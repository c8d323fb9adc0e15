"""RoPE: the oracle against the reference's rope.c (CPU), and the HIP operators
rope_{f32,f16}_cuda and mha_decode_rope_{f32,f16}_cuda against the oracle (GPU).

Reference test: tests/test_rope.c (S=4, H=2, d=4, srand(42) fill, base 10000; CPU vs
reference < 1e-5, magnitude preserved, in place == out of place, CUDA vs CPU).  Here the
RoPE operators are compared bit for bit: the angle table is the reference formula
evaluated with the same libm, and the rotation is fp32 without contraction.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import DecodeCase, dev, max_abs

TOL32, TOL16 = 1e-4, 2e-2


# ------------------------------------------------------------------ oracle (CPU) ---

@pytest.mark.skipif(not O.ref_available(), reason="reference build not available")
def test_oracle_rope_matches_reference_kat():
    """tests/test_rope.c:71-120: srand(42) fill of (4, 2, 4), base 10000."""
    x = O.glibc_rand((4, 2, 4), 42)
    got = O.rope(x)
    assert np.array_equal(got, O.rope(x, use_ref=True))
    mag_in = np.hypot(x[..., 0::2], x[..., 1::2])
    mag_out = np.hypot(got[..., 0::2], got[..., 1::2])
    assert np.max(np.abs(mag_in - mag_out)) < 1e-5                     # test_rope.c:105-116
    assert np.array_equal(got[0], x[0])                                  # position 0: identity


@pytest.mark.skipif(not O.ref_available(), reason="reference build not available")
@pytest.mark.parametrize("S,H,d,base", [(300, 8, 64, 10000.0), (2048, 2, 128, 500000.0), (33, 3, 2, 10.0)])
def test_oracle_rope_matches_reference_build(S, H, d, base):
    x = O.normal((S, H, d), S + d)
    assert np.array_equal(O.rope(x, base), O.rope(x, base, use_ref=True))


def test_oracle_rope_in_place_equals_out_of_place():
    """tests/test_rope.c:127-165."""
    x = O.glibc_rand((4, 2, 4), 42)
    y = x.copy()
    assert O.lib().oracle_rope_f32(O._fp(y), O._fp(y), 4, 2, 4, 10000.0) == 0
    assert np.array_equal(y, O.rope(x))


def _unit_rotation(pos, d, base):
    """(cos, sin) per pair at position pos, read off the rope oracle on unit vectors."""
    e = np.zeros((pos + 1, 1, d), np.float32)
    e[pos, 0, 0::2] = 1.0
    r = O.rope(e, base)[pos, 0]
    return r[0::2].astype(np.float64), r[1::2].astype(np.float64)


def _rotate_columns(W, H, d, c, s):
    """Rotate output-column pairs (2i, 2i+1) of every head of W (..., H*d)."""
    W = np.asarray(W, np.float64).copy()
    lead = W.shape[:-1]
    v = W.reshape(lead + (H, d // 2, 2))
    x0, x1 = v[..., 0].copy(), v[..., 1].copy()
    v[..., 0] = x0 * c - x1 * s
    v[..., 1] = x0 * s + x1 * c
    return v.reshape(lead + (H * d,)).astype(np.float32)


def test_oracle_decode_rope_at_position_zero_is_decode():
    c = DecodeCase(2, 4, 2, 8, 6, cache_len=0, seed=8, wstd=0.3)
    p = O.decode_params(2, c.D, 4, 2, 8, 0, 6)
    plain = O.mha_decode(*c.arrays(), p)
    roped = O.mha_decode_rope(*c.arrays(), p, 10000.0)
    for a, b in zip(plain, roped):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("ragged", [False, True])
def test_oracle_decode_rope_equals_rotated_projection_weights(ragged):
    """Rotating Q and K_new at position p equals projecting with W_Q, b_Q, W_K, b_K whose
    output columns are rotated by the same angles (R·(xW + b) = x(W R^T) + R b)."""
    B, H, H_kv, d, max_seq, base = 2, 4, 2, 8, 12, 10000.0
    lens = [7, 7] if not ragged else None
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=7 if not ragged else None,
                   seq_lens=None if not ragged else [7, 10], seed=9, wstd=0.3)
    p = O.decode_params(B, c.D, H, H_kv, d, -1 if ragged else 7, max_seq)
    got = O.mha_decode_rope(*c.arrays(), p, base, seq_lens=c.seq_lens)
    positions = c.seq_lens if ragged else lens
    for b, pos in enumerate(positions):
        co, si = _unit_rotation(int(pos), d, base)
        arrs = c.arrays()
        arrs[0] = c.X[b:b + 1]
        arrs[1] = c.Kc[b:b + 1]
        arrs[2] = c.Vc[b:b + 1]
        arrs[3] = _rotate_columns(c.WQ, H, d, co, si)
        arrs[4] = _rotate_columns(c.bQ, H, d, co, si)
        arrs[5] = _rotate_columns(c.WK, H_kv, d, co, si)
        arrs[6] = _rotate_columns(c.bK, H_kv, d, co, si)
        pb = O.decode_params(1, c.D, H, H_kv, d, int(pos), max_seq)
        want = O.mha_decode(*arrs, pb)
        assert max_abs(want[0], got[0][b:b + 1]) < 1e-5
        assert max_abs(want[1], got[1][b:b + 1]) < 1e-5


# ------------------------------------------------------------------ HIP (GPU) ---

def _rope_gpu(x, base, f16=False, in_place=False):
    import cudaforge_amd as cf
    S, H, d = x.shape
    xin = dev(x, f16)
    out = xin if in_place else cf.DeviceBuffer.empty(x.shape, np.float16 if f16 else np.float32)
    p = cf.RopeParams(S, d, H, base)
    rc = cf.call_op("rope_f16_cuda" if f16 else "rope_f32_cuda", [xin], [out], p)
    assert rc == 0
    return out.download().astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,base", [((4, 2, 4), 10000.0), ((300, 8, 64), 10000.0), ((4096, 8, 128), 500000.0)])
def test_rope_f32_cuda_is_bit_exact(gpu, shape, base):
    x = O.glibc_rand(shape, 42) if shape == (4, 2, 4) else O.normal(shape, 77)
    want = O.rope(x, base)
    assert np.array_equal(_rope_gpu(x, base), want)
    assert np.array_equal(_rope_gpu(x, base, in_place=True), want)       # test_rope.c:127-165


@pytest.mark.gpu
def test_rope_f16_cuda_rounds_once(gpu):
    x = O.round_f16(O.normal((512, 4, 64), 78))
    want = O.round_f16(O.rope(x, 10000.0))
    assert np.array_equal(_rope_gpu(x, 10000.0, f16=True), want)


@pytest.mark.gpu
def test_rope_rejects_odd_head_dim_and_bad_base(gpu):
    import cudaforge_amd as cf
    x = dev(np.zeros((2, 1, 3), np.float32))
    assert cf.call_op("rope_f32_cuda", [x], [x], cf.RopeParams(2, 3, 1, 10000.0)) == -1
    x = dev(np.zeros((2, 1, 4), np.float32))
    assert cf.call_op("rope_f32_cuda", [x], [x], cf.RopeParams(2, 4, 1, 0.0)) == -1


@pytest.mark.gpu
def test_graph_rope_node_runs_on_gpu(gpu, native):
    """OP_ROPE resolves to rope_f32_cuda (graph.c name rule) and runs in a graph."""
    from helpers import DT_F32, OP_INPUT, OP_OUTPUT, Graph
    OP_ROPE = 31
    x = O.normal((64, 4, 32), 79)
    g = Graph(native)
    try:
        tX, iX = g.tensor(x)
        tY, iY = g.tensor(np.zeros_like(x))
        p = O.RopeParams(64, 32, 4, 10000.0)
        nid = g.node(OP_ROPE, [iX], [iY], (), p)
        native.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
        native.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
        assert native.graph_build(g.g) == 0
        buf = ctypes.create_string_buffer(64)
        assert native.graph_resolve_op(g.g, nid, True, buf, 64) and buf.value == b"rope_f32_cuda"
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(g.g, ins, outs, True) == 0
        assert np.array_equal(g.read(tY, x.shape), O.rope(x))
    finally:
        g.destroy()


def _decode_rope_gpu(c: DecodeCase, base):
    import cudaforge_amd as cf
    bufs = [dev(a, c.f16) for a in c.arrays()]
    extra = [dev(c.seq_lens)] if c.seq_lens is not None else []
    dt = np.float16 if c.f16 else np.float32
    Y = cf.DeviceBuffer.empty((c.B, 1, c.D), dt)
    p = cf.MhaDecodeRopeParams(c.params(cf.MhaDecodeParams), base, 0)
    name = "mha_decode_rope_f16_cuda" if c.f16 else "mha_decode_rope_f32_cuda"
    assert cf.call_op(name, bufs, [Y, bufs[1], bufs[2]], p, extra_inputs=extra) == 0
    return Y.download().astype(np.float32), bufs[1].download().astype(np.float32)


def _decode_rope_oracle(c: DecodeCase, base):
    p = O.decode_params(c.B, c.D, c.H, c.H_kv, c.d, -1 if c.seq_lens is not None else c.cache_len, c.max_seq)
    return O.mha_decode_rope(*c.arrays(), p, base, seq_lens=c.seq_lens)


@pytest.mark.gpu
@pytest.mark.parametrize("f16,ragged", [(False, False), (False, True), (True, False), (True, True)])
def test_mha_decode_rope_matches_oracle(gpu, f16, ragged):
    c = DecodeCase(3, 8, 2, 64, 300, cache_len=None if ragged else 257, seq_lens=[5, 299, 128] if ragged else None,
                   seed=11, f16=f16)
    Y, K = _decode_rope_gpu(c, 10000.0)
    want = _decode_rope_oracle(c, 10000.0)
    tol = TOL16 if f16 else TOL32
    assert max_abs(want[0], Y) <= tol
    assert max_abs(want[1], K) <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("small", [0, 2])
def test_mha_decode_rope_fused_and_separate_rotation(gpu, native, f16, small):
    """The rotation done in the projection's K-chunk sum (where the projection splits K),
    by the separate rotation kernel after a single-chunk projection, and in the one-pass
    small projection kernel: each within the bound of the oracle.  small = 0 keeps the
    split-K kernels (fp16: K split forced to one chunk, then automatic; fp32: hidden size
    16 plans one chunk, 512 several); small = 2 runs the same cases on the one-pass kernel."""
    tol = TOL16 if f16 else TOL32
    if f16:
        cases = [(DecodeCase(3, 8, 2, 64, 300, cache_len=257, seed=14, f16=True), ks) for ks in (1, 0)]
    else:
        cases = [(DecodeCase(2, 1, 1, 16, 100, cache_len=77, seed=15), 0),
                 (DecodeCase(2, 8, 8, 64, 100, cache_len=77, seed=16), 0)]
    try:
        native.cf_gemv_set_small(small)
        for c, ks in cases:
            native.cf_gemv_set_dma_ksplit(ks)
            Y, K = _decode_rope_gpu(c, 10000.0)
            want = _decode_rope_oracle(c, 10000.0)
            assert max_abs(want[0], Y) <= tol
            assert max_abs(want[1], K) <= tol
    finally:
        native.cf_gemv_set_dma_ksplit(0)
        native.cf_gemv_set_small(1)


@pytest.mark.gpu
def test_mha_decode_rope_long_context_gqa_f16(gpu):
    """Llama-3 shape per head (32/8 heads, d = 128, base 500000) at the last position of a
    4096 cache, where the angles are largest."""
    c = DecodeCase(2, 32, 8, 128, 4096, cache_len=4095, seed=12, f16=True)
    Y, K = _decode_rope_gpu(c, 500000.0)
    want = _decode_rope_oracle(c, 500000.0)
    assert max_abs(want[0], Y) <= TOL16
    assert max_abs(want[1][:, 4095], K[:, 4095]) <= TOL16


@pytest.mark.gpu
def test_mha_decode_rope_config2_full_size(gpu):
    """Config 2 (B 16, 32/8 heads, d 128, KV 4096, fp16) with RoPE at base 500000, the
    Llama-3 step: every output row and the appended (rotated) K row of every sequence
    against the oracle; the rest of the K cache unchanged."""
    c = DecodeCase(16, 32, 8, 128, 4096, cache_len=4095, seed=17, f16=True)
    want = _decode_rope_oracle(c, 500000.0)
    Y, K = _decode_rope_gpu(c, 500000.0)
    assert max_abs(want[0], Y) <= TOL16
    assert max_abs(want[1][:, 4095], K[:, 4095]) <= TOL16
    assert np.array_equal(K[:, :4095], c.Kc[:, :4095])


@pytest.mark.gpu
def test_mha_decode_rope_at_position_zero_equals_decode(gpu):
    from helpers import run_decode_gpu
    c = DecodeCase(2, 4, 4, 32, 16, cache_len=0, seed=13)
    Y, K = _decode_rope_gpu(c, 10000.0)
    c2 = DecodeCase(2, 4, 4, 32, 16, cache_len=0, seed=13)
    Yp, Kp, _ = run_decode_gpu(c2)
    assert np.array_equal(Y, Yp) and np.array_equal(K, Kp)
