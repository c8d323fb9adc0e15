"""The allocation-free decode entry (mha_decode_attn_f16_noalloc) through the C-ABI.

It must give the same bits as mha_decode_attn_f16_cuda (same plan, same kernels, its
split partials in the library's fixed per-GPU scratch instead of the stream
workspace), on two calls in a row with the second smaller, leave the workspace
untouched, and reject a plan whose partials exceed the scratch with -1.
"""

import numpy as np
import pytest

import cudaforge_amd as cf
from helpers import dev

pytestmark = pytest.mark.gpu


def _inputs(rng, B, H, H_kv, d, max_seq):
    q = rng.standard_normal((B, H, d)).astype(np.float16)
    k = rng.standard_normal((B, max_seq, H_kv, d)).astype(np.float16)
    v = rng.standard_normal((B, max_seq, H_kv, d)).astype(np.float16)
    return q, k, v


def _both(B, H, H_kv, d, max_seq, cache_len, seq_lens=None):
    """Run the existing entry and the allocation-free one on the same device inputs."""
    rng = np.random.default_rng(1000 + B * 7 + max_seq)
    q, k, v = _inputs(rng, B, H, H_kv, d, max_seq)
    bufs = [dev(q), dev(k), dev(v)]
    if seq_lens is not None:
        bufs.append(dev(np.asarray(seq_lens, np.int32)))
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1.0 / np.sqrt(d)),
                           -1 if seq_lens is not None else cache_len, max_seq)
    o_ref = cf.DeviceBuffer.empty((B, H, d), np.float16)
    o_na = cf.DeviceBuffer.empty((B, H, d), np.float16)
    assert cf.call_op("mha_decode_attn_f16_cuda", bufs, [o_ref], p) == 0
    ref = o_ref.download()
    ws_before = cf.lib.gpu_workspace_size()
    assert cf.call_entry("mha_decode_attn_f16_noalloc", bufs, [o_na], p) == 0
    got = o_na.download()
    assert cf.lib.gpu_workspace_size() == ws_before, "the allocation-free entry touched the workspace"
    return ref, got


def test_noalloc_matches_workspace_entry_uniform(gpu):
    """BASELINE config 2 (B16, 32/8 heads, d128, KV 4096), then a smaller call."""
    ref, got = _both(16, 32, 8, 128, 4096, 4095)
    assert np.isfinite(got.astype(np.float32)).all()
    assert np.array_equal(ref.view(np.uint16), got.view(np.uint16))
    ref2, got2 = _both(3, 8, 2, 64, 800, 777)
    assert np.array_equal(ref2.view(np.uint16), got2.view(np.uint16))


def test_noalloc_matches_workspace_entry_ragged(gpu):
    """Ragged lengths (config 4's shape at a smaller capacity), then a smaller call."""
    ref, got = _both(4, 32, 8, 128, 8192, 0, seq_lens=[8191, 10, 4000, 6001])
    assert np.array_equal(ref.view(np.uint16), got.view(np.uint16))
    ref2, got2 = _both(2, 16, 4, 128, 1000, 0, seq_lens=[0, 999])
    assert np.array_equal(ref2.view(np.uint16), got2.view(np.uint16))


def test_noalloc_rejects_partials_beyond_scratch(gpu):
    """32-position splits over 4096 positions need ~34 MB of partials: -1, no launch."""
    cap = cf.lib.cf_decode_attn_scratch_bytes()
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    assert B * H * (T // 32) * (d + 4) * 4 > cap
    rng = np.random.default_rng(5)
    q, k, v = _inputs(rng, B, H, H_kv, d, T)
    bufs = [dev(q), dev(k), dev(v)]
    out = cf.DeviceBuffer.empty((B, H, d), np.float16)
    out.fill_zero()
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1.0 / np.sqrt(d)), T - 1, T)
    cf.lib.mha_decode_set_split_chunk(32)
    try:
        rc = cf.call_entry("mha_decode_attn_f16_noalloc", bufs, [out], p)
    finally:
        cf.lib.mha_decode_set_split_chunk(0)
    assert rc == -1
    assert not out.download().any(), "a rejected call must not write its output"
