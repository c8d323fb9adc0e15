"""MHA_Decode on the GPU through the C-ABI vs the CPU oracle.

Tolerances: FP32 max abs error <= 1e-4; FP16 with fp32
accumulation <= 2e-2.  Shapes cover the reference's own decode test
(tests/test_mha_decode.c:35-39, glibc-rand inputs, cache_len 0 then 1), BASELINE
configs 1, 2 and 4 (full size through size-independent checks where the oracle would be
slow), GQA group sizes 1..8, head sizes on the fast (64, 128) and generic paths, ragged
lengths, split-count invariance and non-aliased output caches.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import DecodeCase, max_abs, run_decode_attn_gpu, run_decode_gpu

pytestmark = pytest.mark.gpu

TOL32 = 1e-4
TOL16 = 2e-2


def attn_ref64(Q, K, V, attend, H_kv, scale):
    """float64 attention core (numpy), used for full-size checks of selected rows."""
    B, H, d = Q.shape
    G = H // H_kv
    out = np.zeros((B, H, d))
    for b in range(B):
        T = attend[b]
        for h in range(H):
            k = K[b, :T, h // G, :].astype(np.float64)
            v = V[b, :T, h // G, :].astype(np.float64)
            s = k @ Q[b, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ v
    return out


def test_reference_kat_two_steps_f32(gpu):
    """tests/test_mha_decode.c:145-248 inputs (srand seeds 42, 100..107, 200), B=1 H=2 d=4."""
    TB, TH, Td, TMAX = 1, 2, 4, 8
    TD = TH * Td
    c = DecodeCase(TB, TH, TH, Td, TMAX, cache_len=0)
    c.X = O.glibc_rand((TB, 1, TD), 42)
    c.WQ, c.bQ = O.glibc_rand((TD, TD), 100), O.glibc_rand((TD,), 101)
    c.WK, c.bK = O.glibc_rand((TD, TD), 102), O.glibc_rand((TD,), 103)
    c.WV, c.bV = O.glibc_rand((TD, TD), 104), O.glibc_rand((TD,), 105)
    c.WO, c.bO = O.glibc_rand((TD, TD), 106), O.glibc_rand((TD,), 107)
    c.Kc = np.zeros((TB, TMAX, TH, Td), np.float32)
    c.Vc = np.zeros_like(c.Kc)
    want = c.oracle()
    got = run_decode_gpu(c)
    for w, g in zip(want, got):
        assert max_abs(w, g) <= TOL32
    # step 2 on the updated cache (test_mha_decode.c:217-242)
    c.Kc, c.Vc = want[1], want[2]
    c.X = O.glibc_rand((TB, 1, TD), 200)
    c.cache_len = 1
    want2 = c.oracle()
    got2 = run_decode_gpu(c)
    for w, g in zip(want2, got2):
        assert max_abs(w, g) <= TOL32


def test_config1_gpt2_small_f32(gpu):
    """B=1, H=12=H_kv, d=64, KV length 1024 (cache_len 1023)."""
    c = DecodeCase(1, 12, 12, 64, 1024, cache_len=1023, seed=11)
    want = c.oracle()
    got = run_decode_gpu(c)
    assert max_abs(want[0], got[0]) <= TOL32
    assert max_abs(want[1], got[1]) <= TOL32
    assert max_abs(want[2], got[2]) <= TOL32


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("H,H_kv,d,T", [(8, 8, 64, 333), (8, 4, 128, 700), (16, 4, 128, 1030),
                                         (16, 2, 64, 129), (8, 1, 128, 64), (6, 2, 32, 250), (4, 4, 80, 90),
                                         (4, 4, 80, 1000), (4, 2, 96, 777), (4, 4, 48, 600)])
def test_attn_core_vs_oracle(gpu, f16, H, H_kv, d, T):
    """Head sizes off the MFMA path (80, 96, 48) with 10-16 splits take the row merge
    with 12, 10 and 21 thread groups: its LDS tree must fold a group count that is not a
    power of two (a tree that halved 12 groups as 6, 3, 1 dropped group 2's splits)."""
    B, max_seq = 3, T + 5
    Q = O.normal((B, H, d), 7 + d)
    K = O.normal((B, max_seq, H_kv, d), 8 + H)
    V = O.normal((B, max_seq, H_kv, d), 9 + T)
    if f16:
        Q, K, V = O.round_f16(Q), O.round_f16(K), O.round_f16(V)
    scale = float(1.0 / np.sqrt(d))
    want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), scale, H_kv)
    got = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, f16)
    assert max_abs(want, got) <= (TOL16 if f16 else TOL32)


@pytest.mark.parametrize("B,H,H_kv,d,max_seq,cl", [(4, 8, 2, 64, 300, 257), (2, 32, 8, 128, 520, 511),
                                                   (20, 4, 4, 64, 70, 0), (3, 12, 12, 64, 600, 599),
                                                   (2, 6, 2, 16, 50, 33), (17, 4, 4, 32, 64, 63)])
def test_full_decode_f16(gpu, B, H, H_kv, d, max_seq, cl):
    """Full op in fp16.  The last two shapes have projection widths that are not
    multiples of 64 (register-transposing projection kernel), a head size off the MFMA
    split path (generic split kernel) and more than 16 batch rows (two M tiles)."""
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=cl, seed=B + H, f16=True)
    want = c.oracle()
    got = run_decode_gpu(c)
    assert max_abs(want[0], got[0]) <= TOL16
    assert max_abs(want[1], got[1]) <= TOL16
    assert max_abs(want[2], got[2]) <= TOL16


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("B,H,H_kv,d,max_seq,cl", [(1, 12, 12, 64, 1024, 1023), (4, 8, 2, 64, 200, 150),
                                                   (3, 2, 1, 16, 40, 0), (4, 16, 4, 64, 64, 31)])
def test_full_decode_small_projection_paths(gpu, native, f16, B, H, H_kv, d, max_seq, cl):
    """The one-pass projection kernel for small weights (batch rows <= 4) and the split-K
    kernels with their reduce on the same op: both within the bound of the oracle for
    the output and the appended cache rows, at config 1's shape (batch 1, 12 heads,
    d 64), a GQA shape with batch 4, projection widths of 32 and 16 columns, and batch
    4 x hidden 1024, where X fills the kernel's 4096-float LDS stage exactly."""
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=cl, seed=B + 7 * H, f16=f16)
    want = c.oracle()
    tol = TOL16 if f16 else TOL32
    outs = []
    try:
        for small in (0, 2):
            native.cf_gemv_set_small(small)
            outs.append(run_decode_gpu(c))
    finally:
        native.cf_gemv_set_small(1)
    for got in outs:
        for w, g in zip(want, got):
            assert max_abs(w, g) <= tol


@pytest.mark.parametrize("B,H,H_kv,d,max_seq,cl", [(2, 8, 2, 64, 200, 150), (17, 4, 2, 32, 40, 39)])
def test_full_decode_f32(gpu, B, H, H_kv, d, max_seq, cl):
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=cl, seed=5)
    want = c.oracle()
    got = run_decode_gpu(c)
    for w, g in zip(want, got):
        assert max_abs(w, g) <= TOL32


def test_not_inplace_outputs(gpu):
    """Non-aliased output caches equal the input caches with row cache_len replaced."""
    c = DecodeCase(2, 4, 2, 64, 64, cache_len=40, seed=3)
    want = c.oracle()
    got = run_decode_gpu(c, inplace=False)
    for w, g in zip(want, got):
        assert max_abs(w, g) <= TOL32
    mask = np.ones(c.max_seq, bool)
    mask[40] = False
    assert np.array_equal(got[1][:, mask], c.Kc[:, mask])


@pytest.mark.parametrize("f16", [True, False])
def test_ragged_lengths(gpu, f16):
    """Config 4 semantics (per-sequence lengths) at a reduced capacity."""
    B, H, H_kv, d, max_seq = 4, 8, 2, 128, 2048
    lens = O.uniform_int(B, 99, 1, max_seq - 1)
    c = DecodeCase(B, H, H_kv, d, max_seq, seq_lens=lens, seed=21, f16=f16)
    want = c.oracle()
    got = run_decode_gpu(c)
    tol = TOL16 if f16 else TOL32
    for w, g in zip(want, got):
        assert max_abs(w, g) <= tol
    # core entry with the same lengths
    Q = O.normal((B, H, d), 5)
    Q = O.round_f16(Q) if f16 else Q
    core = run_decode_attn_gpu(Q, c.Kc, c.Vc, None, H_kv, f16, seq_lens=lens)
    ref = O.decode_attn(Q, c.Kc, c.Vc, lens + 1, float(1 / np.sqrt(d)), H_kv)
    assert max_abs(ref, core) <= tol


@pytest.mark.parametrize("f16", [True, False])
def test_device_held_uniform_length_modes(gpu, f16):
    """cache_len -2 and -3 (one length for the whole batch, held in a device array in
    slot 11) give the host-length result; -3 also adds one to every device length after
    the step and -2 leaves them; the attention-only entry rejects -3."""
    import cudaforge_amd as cf
    from helpers import dev
    B, H, H_kv, d, max_seq, L = 3, 8, 2, 64, 640, 517
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=L, seed=31, f16=f16)
    want = c.oracle()
    tol = TOL16 if f16 else TOL32
    dt = np.float16 if f16 else np.float32
    name = "mha_decode_f16_cuda" if f16 else "mha_decode_f32_cuda"
    for mode, step in ((-2, 0), (-3, 1)):
        bufs = [dev(a, f16) for a in c.arrays()]
        lens = dev(np.full(B, L, np.int32))
        Y = cf.DeviceBuffer.empty((B, 1, c.D), dt)
        p = cf.MhaDecodeParams(B, c.D, H, H_kv, d, float(1 / np.sqrt(d)), mode, max_seq)
        assert cf.call_op(name, bufs, [Y, bufs[1], bufs[2]], p, None, extra_inputs=[lens]) == 0
        got = [Y.download(), bufs[1].download(), bufs[2].download()]
        for w, g in zip(want, got):
            assert max_abs(w, g.astype(np.float32)) <= tol
        assert np.array_equal(lens.download(), np.full(B, L + step, np.int32))
    Q = dev(O.normal((B, H, d), 5), f16)
    out = cf.DeviceBuffer.empty((B, H, d), dt)
    p = cf.MhaDecodeParams(B, c.D, H, H_kv, d, float(1 / np.sqrt(d)), -3, max_seq)
    core = "mha_decode_attn_f16_cuda" if f16 else "mha_decode_attn_f32_cuda"
    assert cf.call_op(core, [Q, bufs[1], bufs[2]], [out], p, None, extra_inputs=[lens]) == -1


def test_split_count_invariance(gpu, native):
    """The result must not depend on how positions are split across workgroups."""
    B, H, H_kv, d, T = 2, 16, 4, 128, 3000
    Q, K, V = (O.round_f16(O.normal(s, i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    outs = []
    try:
        for chunk in (0, 64, 256, 1024):
            native.mha_decode_set_split_chunk(chunk)
            outs.append(run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True))
    finally:
        native.mha_decode_set_split_chunk(0)
    ref = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
    for o in outs:
        assert max_abs(o, ref) <= TOL16
        assert max_abs(o, outs[0]) <= 2e-3


def test_config2_full_size_core(gpu):
    """BASELINE config 2 at full size (B=16, 32/8 heads, d=128, KV 4096, fp16): every
    output row of every batch row against a float64 reference, and batch rows 0 and 15
    also against the scalar float64 loop."""
    from helpers import attn_ref64_all
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    Q = O.round_f16(O.normal((B, H, d), 1))
    K = O.round_f16(O.normal((B, T, H_kv, d), 2))
    V = O.round_f16(O.normal((B, T, H_kv, d), 3))
    got = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True)
    scale = float(1 / np.sqrt(d))
    ref = attn_ref64_all(Q, K, V, [T] * B, H_kv, scale)
    per_row = np.abs(ref - got).reshape(B, -1).max(axis=1)
    assert (per_row <= TOL16).all(), per_row
    rows = [0, B - 1]
    assert max_abs(attn_ref64(Q[rows], K[rows], V[rows], [T, T], H_kv, scale), got[rows]) <= TOL16


def test_full_decode_config2_full_size(gpu):
    """Config 2 (B 16, D 4096, 32/8 heads, d 128, KV 4096, fp16) through the plain full op
    (mha_decode_f16_cuda: projections, append, attention, output projection), the
    reference's CUDA-against-CPU op check (tests/test_mha_decode.c:263-414) at the
    headline shape: every output row and the appended K and V row of every sequence
    against the oracle, and the rest of both caches unchanged."""
    c = DecodeCase(16, 32, 8, 128, 4096, cache_len=4095, seed=19, f16=True)
    want = c.oracle()
    got = run_decode_gpu(c)
    assert max_abs(want[0], got[0]) <= TOL16
    for i, cache in ((1, c.Kc), (2, c.Vc)):
        assert max_abs(want[i][:, 4095], got[i][:, 4095]) <= TOL16
        assert np.array_equal(got[i][:, :4095], cache[:, :4095])


@pytest.mark.parametrize("L", [40, 41, -1])
def test_device_length_outside_the_cache(gpu, L):
    """A device-held uniform length (cache_len -2) the host cannot check: at max_seq or
    beyond, nothing is appended and all max_seq positions are attended; a negative one
    appends nothing and attends position 0.  Q is projected either way (its store has no
    position), so Y is the float64 result of X.WQ+bQ attending the unchanged cache, then
    the output projection."""
    import cudaforge_amd as cf
    from helpers import dev
    B, H, H_kv, d, max_seq = 2, 4, 2, 64, 40
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=0, seed=37)
    bufs = [dev(a) for a in c.arrays()]
    lens = dev(np.full(B, L, np.int32))
    Y = cf.DeviceBuffer.empty((B, 1, c.D), np.float32)
    p = cf.MhaDecodeParams(B, c.D, H, H_kv, d, float(1 / np.sqrt(d)), -2, max_seq)
    assert cf.call_op("mha_decode_f32_cuda", bufs, [Y, bufs[1], bufs[2]], p, None, extra_inputs=[lens]) == 0
    q = (c.X[:, 0].astype(np.float64) @ c.WQ + c.bQ).reshape(B, H, d)
    att = np.full(B, max_seq if L >= max_seq else 1)
    o = attn_ref64(q, c.Kc, c.Vc, att, H_kv, 1 / np.sqrt(d))
    want = o.reshape(B, c.D) @ c.WO.astype(np.float64) + c.bO
    assert max_abs(want, Y.download()[:, 0]) <= TOL32
    assert np.array_equal(bufs[1].download(), c.Kc) and np.array_equal(bufs[2].download(), c.Vc)


def test_cache_len_zero_is_value_row(gpu):
    """T = 1: softmax is 1, so the core returns the single V row (closed form)."""
    B, H, H_kv, d = 2, 8, 2, 128
    Q = O.normal((B, H, d), 1)
    K = O.normal((B, 4, H_kv, d), 2)
    V = O.normal((B, 4, H_kv, d), 3)
    got = run_decode_attn_gpu(Q, K, V, 0, H_kv, False)
    want = np.repeat(V[:, 0], H // H_kv, axis=1)
    assert max_abs(want, got) <= 1e-6


def test_config4_ragged_full_size(gpu):
    """BASELINE config 4 at full size: B=4, 32/8 heads, d=128, capacity 32768, lengths
    L_b ~ U[1024, 32768] (attended positions; cache_len_b = L_b - 1), fp16.  Every output
    row against a float64 reference."""
    B, H, H_kv, d, max_seq = 4, 32, 8, 128, 32768
    L = O.uniform_int(B, 4, 1024, max_seq)
    Q = O.round_f16(O.normal((B, H, d), 41))
    K = O.round_f16(O.normal((B, max_seq, H_kv, d), 42))
    V = O.round_f16(O.normal((B, max_seq, H_kv, d), 43))
    got = run_decode_attn_gpu(Q, K, V, None, H_kv, True, seq_lens=L - 1)
    ref = attn_ref64(Q, K, V, L, H_kv, float(1 / np.sqrt(d)))
    assert max_abs(ref, got) <= TOL16


@pytest.mark.parametrize("lens", [[1], [1, 1, 1], [4096, 1, 17, 2999], [33] * 64, [1] * 63 + [5000],
                                  [16, 4080, 16, 4080], [257, 4095, 1000, 3]])
def test_balanced_ragged_partition(gpu, native, lens):
    """Ragged fp16 lengths on the grouped kernel split the batch's attended positions
    about evenly over one round of workgroups, each one range of one sequence: ranges
    that start anywhere (inside a 16-position block too), one workgroup for each of many
    short sequences, length-1 sequences and totals smaller than one position per
    workgroup.  Every row against float64, and against the one-wave kernel (chunked
    splits over the capacity)."""
    from helpers import attn_ref64_all
    B, H_kv, G, d, cap = len(lens), 2, 4, 128, 4096
    H = H_kv * G
    L = np.asarray(lens, np.int32)
    Q, K, V = (O.round_f16(O.normal(s, 510 + i)) for i, s in enumerate([(B, H, d), (B, cap, H_kv, d), (B, cap, H_kv, d)]))
    got = run_decode_attn_gpu(Q, K, V, None, H_kv, True, seq_lens=L - 1)
    ref = attn_ref64_all(Q, K, V, L, H_kv, float(1 / np.sqrt(d)))
    per_row = np.abs(ref - got).reshape(B, -1).max(axis=1)
    assert (per_row <= TOL16).all(), per_row
    try:
        native.cf_decode_attn_set_wide(0)
        one_wave = run_decode_attn_gpu(Q, K, V, None, H_kv, True, seq_lens=L - 1)
    finally:
        native.cf_decode_attn_set_wide(1)
    assert max_abs(one_wave, got) <= TOL16


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("chunk", [0, 256])
def test_ragged_edge_lengths(gpu, native, f16, chunk):
    """Per-sequence lengths at the split boundaries: one position, one short of a chunk,
    exactly a chunk, one past it, a full cache."""
    B, H, H_kv, d, max_seq = 8, 8, 2, 128, 1024
    cl = np.array([0, 254, 255, 256, 511, 31, 32, max_seq - 1], np.int32)
    Q = O.normal((B, H, d), 61)
    K = O.normal((B, max_seq, H_kv, d), 62)
    V = O.normal((B, max_seq, H_kv, d), 63)
    if f16:
        Q, K, V = O.round_f16(Q), O.round_f16(K), O.round_f16(V)
    try:
        native.mha_decode_set_split_chunk(chunk)
        got = run_decode_attn_gpu(Q, K, V, None, H_kv, f16, seq_lens=cl)
    finally:
        native.mha_decode_set_split_chunk(0)
    want = O.decode_attn(Q, K, V, cl + 1, float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, got) <= (TOL16 if f16 else TOL32)


def test_split_cap_1024(gpu, native):
    """A requested chunk that would need more than 1024 splits is widened, not refused."""
    B, H, H_kv, d, T = 1, 8, 2, 128, 40000
    Q, K, V = (O.round_f16(O.normal(s, 70 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    try:
        native.mha_decode_set_split_chunk(32)
        got = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True)
    finally:
        native.mha_decode_set_split_chunk(0)
    want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, got) <= TOL16


def test_config2_kv_permutation_invariance(gpu):
    """Attention over a set of positions does not depend on their order: permuting K and V
    rows together at full config-2 size changes only the summation order."""
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    Q = O.round_f16(O.normal((B, H, d), 81))
    K = O.round_f16(O.normal((B, T, H_kv, d), 82))
    V = O.round_f16(O.normal((B, T, H_kv, d), 83))
    perm = np.random.default_rng(84).permutation(T)
    a = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True)
    b = run_decode_attn_gpu(Q, np.ascontiguousarray(K[:, perm]), np.ascontiguousarray(V[:, perm]), T - 1, H_kv, True)
    assert max_abs(a, b) <= 2e-3


@pytest.mark.parametrize("f16", [True, False])
def test_config2_linear_in_v(gpu, f16):
    """Output is linear in V; scaling V by 2 is exact in binary floating point, so the
    output must double bit for bit (any lost or double-counted term would break it).
    Exception: fp16 outputs up to 2^-14 are subnormal or may have rounded up from the
    subnormal range, where round-to-nearest on a fixed 2^-24 grid is not scale-invariant;
    there the two may differ by one 2^-24 step."""
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    Q = O.round_f16(O.normal((B, H, d), 91))
    K = O.round_f16(O.normal((B, T, H_kv, d), 92))
    V = O.round_f16(O.normal((B, T, H_kv, d), 93))
    a = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, f16)
    b = run_decode_attn_gpu(Q, K, V * np.float32(2), T - 1, H_kv, f16)
    normal = np.abs(a) > 2.0 ** -14 if f16 else np.ones(a.shape, bool)
    assert np.array_equal(2 * a[normal], b[normal])
    assert np.all(np.abs(2 * a[~normal] - b[~normal]) <= 2.0 ** -24)
    assert normal.mean() > 0.99


def test_decode_on_created_stream_matches_default(gpu):
    """Ops enqueue on the caller's stream: a created (non-default) stream gives the same bits."""
    import cudaforge_amd as cf
    c = DecodeCase(4, 32, 8, 128, 600, cache_len=555, seed=12, f16=True)
    a = run_decode_gpu(c)
    s = cf.Stream()
    b = run_decode_gpu(c, stream=s)
    s.synchronize()
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("f16", [False, True])
def test_graph_decode_two_steps_on_gpu(gpu, native, f16):
    """graph_execute(use_cuda) over an OP_MHA_DECODE node with device-resident in-place
    caches: step 1 at cache_len 5, then graph_update_cache_len(6) with a new token."""
    from helpers import build_decode_graph
    c = DecodeCase(2, 8, 2, 64, 16, cache_len=5, seed=31, f16=f16, wstd=0.1)
    g, t = build_decode_graph(native, c)
    dt = np.float16 if f16 else np.float32
    tol = TOL16 if f16 else TOL32
    ins, outs = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
    try:
        assert native.graph_execute(g.g, ins, outs, True) == 0
        want = c.oracle()
        assert max_abs(want[0], g.read(t["Y"], c.X.shape, dt)) <= tol
        c2 = DecodeCase(2, 8, 2, 64, 16, cache_len=6, seed=31, f16=f16, wstd=0.1)
        c2.Kc, c2.Vc = want[1], want[2]
        c2.X = O.normal(c.X.shape, 32)
        if f16:
            c2.X = O.round_f16(c2.X)
        g.write(t["X"], O.to_f16(c2.X) if f16 else c2.X)
        native.graph_update_cache_len(g.g, 6)
        assert native.graph_execute(g.g, ins, outs, True) == 0
        want2 = c2.oracle()
        assert max_abs(want2[0], g.read(t["Y"], c.X.shape, dt)) <= tol
    finally:
        g.destroy()


@pytest.mark.parametrize("d,G,H_kv,T", [(128, 4, 8, 3000), (64, 2, 4, 777), (128, 8, 2, 1500), (64, 1, 8, 64),
                                         (128, 1, 1, 33)])
def test_grouped_and_one_wave_split_kernels_agree(gpu, native, d, G, H_kv, T):
    """Uniform lengths take the grouped fp16 split kernel (a workgroup per (split, b), a
    wave per KV head, 16-position blocks); cf_decode_attn_set_wide(0) forces the one-wave
    kernel (32-position blocks).  Both within the FP16 bound of the oracle and close to
    each other, including lengths that end inside a block and a single split."""
    B = 3
    H = H_kv * G
    Q, K, V = (O.round_f16(O.normal(s, 170 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
    outs = []
    try:
        for wide in (1, 0):
            native.cf_decode_attn_set_wide(wide)
            outs.append(run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True))
    finally:
        native.cf_decode_attn_set_wide(1)
    for got in outs:
        assert max_abs(want, got) <= TOL16
    assert max_abs(outs[0], outs[1]) <= TOL16


@pytest.mark.parametrize("G,H_kv", [(4, 8), (1, 2), (2, 4), (8, 2)])
@pytest.mark.parametrize("chunk", [0, 32, 96, 128, 160, 256])
def test_grouped_kernel_k_in_registers_matches_lds_ring(gpu, native, G, H_kv, chunk):
    """The grouped kernel at d = 128 loads K straight into registers (seven 16-position
    blocks ahead, eight register sets) and keeps only V in its LDS ring;
    cf_decode_attn_set_kreg(0) selects the kernel with K in the ring too.  Same MFMA
    operands in the same order, so bit-identical outputs: uniform lengths cut into
    splits of fewer, exactly and more than eight blocks (the unrolled group), lengths
    that end inside a block, and ragged lengths on the balanced partition."""
    assert native.cf_decode_attn_kreg_ok(G) == 1
    B, d, T = 3, 128, 1000
    H = H_kv * G
    Q, K, V = (O.round_f16(O.normal(s, 530 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    lens = np.array([T - 1, 17, 513], np.int32)
    outs = []
    try:
        native.mha_decode_set_split_chunk(chunk)
        for kreg in (1, 0):
            native.cf_decode_attn_set_kreg(kreg)
            outs.append((run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True),
                         run_decode_attn_gpu(Q, K, V, None, H_kv, True, seq_lens=lens - 1)))
    finally:
        native.cf_decode_attn_set_kreg(1)
        native.mha_decode_set_split_chunk(0)
    want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, outs[0][0]) <= TOL16
    want = O.decode_attn(Q, K, V, lens, float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, outs[0][1]) <= TOL16
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("f16", [False, True])
def test_graph_decode_replay(gpu, native, f16):
    """A decode graph executed repeatedly at one cache_len (each execution rewrites row
    cache_len) is recorded on its second execution and replayed after; the length lives
    on the device, so a length change keeps the recording.  Every execution equals, bit
    for bit, the same graph with replay off, and the oracle."""
    from helpers import build_decode_graph
    dt = np.float16 if f16 else np.float32
    tol = TOL16 if f16 else TOL32
    c = DecodeCase(2, 8, 2, 64, 16, cache_len=5, seed=61, f16=f16, wstd=0.1)
    graphs = [build_decode_graph(native, c) for _ in range(2)]
    native.graph_set_replay(graphs[1][0].g, 0)
    try:
        states = []
        for it, cl in enumerate([5, 5, 5, 5, 6, 6, 6]):
            X = O.normal(c.X.shape, 700 + it)
            if f16:
                X = O.round_f16(X)
            outs = []
            for g, t in graphs:
                g.write(t["X"], O.to_f16(X) if f16 else X)
                native.graph_update_cache_len(g.g, cl)
                ins, os_ = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
                assert native.graph_execute(g.g, ins, os_, True) == 0
                outs.append(g.read(t["Y"], c.X.shape, dt).astype(np.float32))
            states.append(native.graph_replay_state(graphs[0][0].g))
            assert np.array_equal(outs[0], outs[1]), f"execution {it}"
            # Each execution rewrites row cl and attends rows 0..cl: rows below 5 are the
            # initial history, row 5 (for cl = 6) holds the last execution at cl = 5.
            want_case = DecodeCase(2, 8, 2, 64, 16, cache_len=cl, seed=61, f16=f16, wstd=0.1)
            want_case.X = X
            if cl == 5:
                last_x5 = X
            else:
                prev = DecodeCase(2, 8, 2, 64, 16, cache_len=5, seed=61, f16=f16, wstd=0.1)
                prev.X = last_x5
                _, want_case.Kc, want_case.Vc = prev.oracle()
            assert max_abs(want_case.oracle()[0], outs[0]) <= tol
        assert states == [1, 2, 2, 2, 2, 2, 2]
    finally:
        for g, _ in graphs:
            g.destroy()


@pytest.mark.parametrize("f16", [False, True])
def test_graph_decode_replay_advancing_length(gpu, native, f16):
    """A token-by-token decode loop (execute, then graph_update_cache_len(L + 1)) over
    seven tokens: from the third execution on, every step replays the one recording
    (state 2), each output equals the replay-off graph bit for bit and the oracle run
    step by step on its own caches.  Then a buffer-generation bump (a workspace or table
    that a recording may point at was freed) makes the next execution re-record."""
    from helpers import build_decode_graph
    dt = np.float16 if f16 else np.float32
    tol = TOL16 if f16 else TOL32
    L0, n_tok = 5, 7
    c = DecodeCase(2, 8, 2, 64, 16, cache_len=L0, seed=81, f16=f16, wstd=0.1)
    graphs = [build_decode_graph(native, c) for _ in range(2)]
    native.graph_set_replay(graphs[1][0].g, 0)
    Kc, Vc = c.Kc, c.Vc
    try:
        states = []
        for step in range(n_tok):
            L = L0 + step
            X = O.normal(c.X.shape, 900 + step)
            if f16:
                X = O.round_f16(X)
            outs = []
            for g, t in graphs:
                g.write(t["X"], O.to_f16(X) if f16 else X)
                ins, os_ = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
                assert native.graph_execute(g.g, ins, os_, True) == 0
                outs.append(g.read(t["Y"], c.X.shape, dt).astype(np.float32))
                native.graph_update_cache_len(g.g, L + 1)
            states.append(native.graph_replay_state(graphs[0][0].g))
            assert np.array_equal(outs[0], outs[1]), f"step {step}"
            ref = DecodeCase(2, 8, 2, 64, 16, cache_len=L, seed=81, f16=f16, wstd=0.1)
            ref.X, ref.Kc, ref.Vc = X, Kc, Vc
            want = ref.oracle()
            assert max_abs(want[0], outs[0]) <= tol, f"step {step}"
            Kc, Vc = want[1], want[2]
        assert states == [1, 2, 2, 2, 2, 2, 2]
        # Caches on the device hold every appended token.
        g0, t0 = graphs[0]
        assert native.tensor_copy_to_host(t0["K"]) == 0
        K_dev = g0.read(t0["K"], c.Kc.shape, dt).astype(np.float32)
        assert max_abs(Kc[:, :L0 + n_tok], K_dev[:, :L0 + n_tok]) <= tol
        # Re-record after a generation bump.
        native.gpu_buffer_generation_bump()
        for g, t in graphs:
            ins, os_ = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
            assert native.graph_execute(g.g, ins, os_, True) == 0
        assert native.graph_replay_state(graphs[0][0].g) == 1
        ins, os_ = (ctypes.c_void_p * 1)(t0["X"]), (ctypes.c_void_p * 1)(t0["Y"])
        assert native.graph_execute(g0.g, ins, os_, True) == 0
        assert native.graph_replay_state(g0.g) == 2
    finally:
        for g, _ in graphs:
            g.destroy()


@pytest.mark.parametrize("f16", [False, True])
def test_graph_decode_uniform_then_ragged_with_lengths_weight(gpu, native, f16):
    """A decode node that carries per-sequence lengths as its 9th weight runs uniform
    steps (device-held length, replayed), then ragged steps whose host lengths change
    between executions, then uniform again; every output against the oracle run step by
    step on its own caches.  The uniform steps neither read nor advance the lengths
    weight (its device copy, read back, still holds what the caller wrote), and each
    ragged step uses the lengths the caller wrote for it."""
    from helpers import build_decode_graph
    dt = np.float16 if f16 else np.float32
    tol = TOL16 if f16 else TOL32
    B, H, H_kv, d, max_seq = 3, 8, 2, 64, 48
    lens0 = np.array([30, 12, 41], np.int32)
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=5, seed=91, f16=f16, wstd=0.1)
    g, t = build_decode_graph(native, c, lens=lens0)
    Kc, Vc = c.Kc, c.Vc
    ins, os_ = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
    # (cache_len, lengths written to the weight before the step)
    plan = [(5, None), (6, None), (7, None), (-1, lens0), (-1, lens0 + 1), (-1, np.array([3, 47, 0], np.int32)),
            (9, None)]
    try:
        for step, (cl, lens) in enumerate(plan):
            X = O.normal(c.X.shape, 700 + step)
            if f16:
                X = O.round_f16(X)
            g.write(t["X"], O.to_f16(X) if f16 else X)
            if lens is not None:
                g.write(t["L"], lens)
            native.graph_update_cache_len(g.g, cl)
            assert native.graph_execute(g.g, ins, os_, True) == 0, f"step {step}"
            got = g.read(t["Y"], c.X.shape, dt).astype(np.float32)
            ref = DecodeCase(B, H, H_kv, d, max_seq, cache_len=None if cl < 0 else cl,
                             seq_lens=None if cl >= 0 else lens, seed=91, f16=f16, wstd=0.1)
            ref.X, ref.Kc, ref.Vc = X, Kc, Vc
            want = ref.oracle()
            assert max_abs(want[0], got) <= tol, f"step {step}"
            Kc, Vc = want[1], want[2]
            if step == 2:
                assert native.tensor_copy_to_host(t["L"]) == 0
                assert np.array_equal(g.read(t["L"], (B,), np.int32), lens0)
        assert native.tensor_copy_to_host(t["K"]) == 0
        assert max_abs(Kc, g.read(t["K"], c.Kc.shape, dt).astype(np.float32)) <= tol
    finally:
        g.destroy()


def test_graph_decode_rejects_length_past_capacity(gpu, native):
    """cache_len >= max_seq returns -1 from graph_execute (the reference op's check,
    mha_decode.c:14-16), eager or recorded."""
    from helpers import build_decode_graph
    c = DecodeCase(1, 4, 2, 64, 8, cache_len=6, seed=83, f16=True, wstd=0.1)
    g, t = build_decode_graph(native, c)
    ins, os_ = (ctypes.c_void_p * 1)(t["X"]), (ctypes.c_void_p * 1)(t["Y"])
    try:
        for L in (6, 7):
            native.graph_update_cache_len(g.g, L)
            assert native.graph_execute(g.g, ins, os_, True) == 0
        native.graph_update_cache_len(g.g, 8)
        assert native.graph_execute(g.g, ins, os_, True) == -1
    finally:
        g.destroy()


@pytest.mark.parametrize("bn", [64, 128, 256])
def test_projection_tile_widths(gpu, native, bn):
    """The fp16 projection kernel at each column-tile width (64/128/256) gives the same
    decode result within tolerance (full op, config-2 head layout at reduced sizes)."""
    c = DecodeCase(5, 8, 2, 128, 300, cache_len=299, seed=50 + bn, f16=True)
    want = c.oracle()
    try:
        native.cf_gemv_set_dma_tile(bn)
        got = run_decode_gpu(c)
    finally:
        native.cf_gemv_set_dma_tile(0)
    for w, g in zip(want, got):
        assert max_abs(w, g) <= TOL16


@pytest.mark.parametrize("ks", [2, 3, 8, 13, 32])
def test_projection_k_splits(gpu, native, ks):
    """The fp16 projections with K split into 2..32 chunks, which the partial reduce sums
    with each of its chunk bounds (4, 8, 16, 32; the surplus loads clamped to the last
    chunk), give the decode result within tolerance of the oracle."""
    c = DecodeCase(5, 8, 2, 128, 300, cache_len=299, seed=70 + ks, f16=True)
    want = c.oracle()
    try:
        native.cf_gemv_set_dma_ksplit(ks)
        got = run_decode_gpu(c)
    finally:
        native.cf_gemv_set_dma_ksplit(0)
    for w, g in zip(want, got):
        assert max_abs(w, g) <= TOL16


@pytest.mark.parametrize("stages", [2, 3, 4])
def test_split_ring_depths(gpu, native, stages):
    """The fp16 split kernel at each LDS ring depth (2/3/4 stages), with ragged lengths that
    end inside, at, and one past a 32-position block."""
    B, H, H_kv, d, max_seq = 4, 16, 4, 128, 1200
    lens = np.array([1199, 31, 32, 700], np.int32)     # cache_len_b; attended = +1
    Q, K, V = (O.round_f16(O.normal(s, 90 + i)) for i, s in
               enumerate([(B, H, d), (B, max_seq, H_kv, d), (B, max_seq, H_kv, d)]))
    try:
        native.cf_decode_attn_set_stages(stages)
        got = run_decode_attn_gpu(Q, K, V, None, H_kv, True, seq_lens=lens)
    finally:
        native.cf_decode_attn_set_stages(0)
    want = O.decode_attn(Q, K, V, lens + 1, float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, got) <= TOL16


def test_concurrent_streams_have_separate_scratch(gpu):
    """Two decode cores on two streams at once (each splits its KV and merges through
    scratch memory) give the same bits as the same calls one after the other."""
    import cudaforge_amd as cf
    from helpers import dev
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    sets = []
    for i in range(2):
        Q = O.round_f16(O.normal((B, H, d), 500 + i))
        K = O.round_f16(O.normal((B, T, H_kv, d), 510 + i))
        V = O.round_f16(O.normal((B, T, H_kv, d), 520 + i))
        sets.append([dev(Q, True), dev(K, True), dev(V, True)])
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1 / np.sqrt(d)), T - 1, T)
    seq = []
    for ins in sets:
        out = cf.DeviceBuffer.empty((B, H, d), np.float16)
        assert cf.call_op("mha_decode_attn_f16_cuda", ins, [out], p) == 0
        seq.append(out.download())
    streams = [cf.Stream(), cf.Stream()]
    outs = [cf.DeviceBuffer.empty((B, H, d), np.float16) for _ in range(2)]
    for _ in range(3):
        for ins, out, st in zip(sets, outs, streams):
            assert cf.call_op("mha_decode_attn_f16_cuda", ins, [out], p, st) == 0
    for st in streams:
        st.synchronize()
    for out, want in zip(outs, seq):
        assert np.array_equal(out.download(), want)


def test_split_chunks_longer_than_4096(gpu, native):
    """The fp16 split kernel takes chunks beyond 4096 positions (its LDS use does not
    grow with the chunk), which long caches need once the 1024-split cap binds."""
    B, H, H_kv, d, T = 1, 8, 2, 128, 20000
    Q, K, V = (O.round_f16(O.normal(s, 120 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    try:
        native.mha_decode_set_split_chunk(8192)
        got = run_decode_attn_gpu(Q, K, V, T - 1, H_kv, True)
    finally:
        native.mha_decode_set_split_chunk(0)
    want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
    assert max_abs(want, got) <= TOL16


@pytest.mark.parametrize("f16,d", [(True, 128), (True, 64), (False, 128)])
def test_merge_many_splits(gpu, native, f16, d):
    """Uniform lengths cut into 32-position splits, 157 and 94 splits per row (the row
    merge), against the oracle, and the row merge forced the same way."""
    B, H_kv, G = 2, 2, 4
    H = H_kv * G
    r = O.round_f16 if f16 else (lambda a: a)
    for T in (5000, 3000):
        Q, K, V = (r(O.normal(s, 150 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
        want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
        outs = []
        try:
            native.mha_decode_set_split_chunk(32)
            for rows in (0, 1):
                native.cf_decode_attn_set_merge_rows(rows)
                outs.append(run_decode_attn_gpu(Q, K, V, T - 1, H_kv, f16))
        finally:
            native.cf_decode_attn_set_merge_rows(0)
            native.mha_decode_set_split_chunk(0)
        tol = TOL16 if f16 else TOL32
        for got in outs:
            assert max_abs(want, got) <= tol
        assert max_abs(outs[0], outs[1]) <= tol


@pytest.mark.parametrize("f16,d,G", [(True, 128, 4), (True, 64, 2), (True, 64, 8), (True, 128, 1),
                                     (False, 64, 1), (False, 128, 8)])
def test_merge_kernels_agree(gpu, native, f16, d, G):
    """The one-wave merge (d = 64 / 128, up to 16 splits) and the row merge on the same
    partials: both within the bound of the oracle, and close to each other.  The one-wave
    merge gives the same bits with 1, 2 or 4 rows per workgroup; the row merge with 1, 2
    or 4 workgroups per row (each a different summation tree) stays within the bound."""
    B, H_kv, T = 3, 2, 3000
    H = H_kv * G
    r = O.round_f16 if f16 else (lambda a: a)
    Q, K, V = (r(O.normal(s, 140 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    lens = [2999, 17, 1500]
    want = O.decode_attn(Q, K, V, np.asarray([l + 1 for l in lens], np.int32), float(1 / np.sqrt(d)), H_kv)
    outs = []
    try:
        native.mha_decode_set_split_chunk(256)         # <= 12 splits: the one-wave merge applies
        for rows in (0, 1):
            native.cf_decode_attn_set_merge_rows(rows)
            outs.append(run_decode_attn_gpu(Q, K, V, None, H_kv, f16, seq_lens=lens))
        for ds in (1, 2, 4):
            native.cf_decode_attn_set_merge_rows_split(ds)
            outs.append(run_decode_attn_gpu(Q, K, V, None, H_kv, f16, seq_lens=lens))
        native.cf_decode_attn_set_merge_rows_split(0)
        native.cf_decode_attn_set_merge_rows(0)
        per_wg = []
        for per in (1, 4):
            native.cf_decode_attn_set_merge_wave_wg(per)
            per_wg.append(run_decode_attn_gpu(Q, K, V, None, H_kv, f16, seq_lens=lens))
    finally:
        native.cf_decode_attn_set_merge_wave_wg(2)
        native.cf_decode_attn_set_merge_rows_split(0)
        native.cf_decode_attn_set_merge_rows(0)
        native.mha_decode_set_split_chunk(0)
    for got in per_wg:
        assert np.array_equal(got, outs[0])
    tol = TOL16 if f16 else TOL32
    for got in outs:
        assert max_abs(want, got) <= tol
    for got in outs[1:]:
        assert max_abs(outs[0], got) <= tol
