"""The session entry on the GPU and the operators' allocation-failure path.

inference_session_run(..., use_cuda=1) (the reference's inference_engine.c:31-37 runs
graph_execute on the session's graph) through the C-ABI against the oracle, for a fused
prefill graph and a decode graph; and gpu_inject_alloc_failures: an operator whose
workspace allocation fails returns -1 without launching, and works on the next call.
"""

import ctypes
from ctypes import c_void_p

import numpy as np
import pytest

from helpers import DecodeCase, FusedCase, build_decode_graph, build_fused_graph, dev, max_abs

pytestmark = pytest.mark.gpu


def test_session_run_fused_on_gpu(gpu, native):
    """tests/test_bert_mha.c:167-306's graph (one MHA_Fused node) through a session, GPU."""
    c = FusedCase(2, 48, 4, 4, 16, seed=12, residual=True, bias_std=0.02)
    g, _, tX, tY = build_fused_graph(native, c)
    s = native.inference_session_from_graph(g.g, 1, 1)
    assert s
    ins, outs = (c_void_p * 1)(tX), (c_void_p * 1)(tY)
    try:
        for _ in range(3):                       # eager, recorded, replayed
            assert native.inference_session_run(s, ins, outs, 1) == 0
            assert max_abs(c.oracle(), g.read(tY, c.X.shape)) <= 1e-4
    finally:
        native.inference_session_destroy(s)      # owns and destroys the graph


def test_session_run_decode_on_gpu(gpu, native):
    c = DecodeCase(2, 8, 2, 64, 32, cache_len=9, seed=13, f16=True, wstd=0.1)
    g, t = build_decode_graph(native, c)
    s = native.inference_session_from_graph(g.g, 1, 1)
    assert s
    ins, outs = (c_void_p * 1)(t["X"]), (c_void_p * 1)(t["Y"])
    try:
        assert native.inference_session_run(s, ins, outs, 1) == 0
        assert max_abs(c.oracle()[0], g.read(t["Y"], c.X.shape, np.float16).astype(np.float32)) <= 2e-2
    finally:
        native.inference_session_destroy(s)


def test_workspace_allocation_failure_returns_minus_one(gpu, native):
    """With every workspace released, the decode core's first call must allocate: with
    that allocation made to fail it returns -1 and writes nothing; the next call
    allocates and succeeds."""
    import cudaforge_amd as cf
    import oracle as O
    B, H, H_kv, d, T = 2, 8, 2, 128, 600
    Q, K, V = (O.round_f16(O.normal(s, 300 + i)) for i, s in enumerate([(B, H, d), (B, T, H_kv, d), (B, T, H_kv, d)]))
    bufs = [dev(Q, True), dev(K, True), dev(V, True)]
    out = cf.DeviceBuffer.empty((B, H, d), np.float16)
    out.fill_zero()
    native.gpu_device_synchronize()
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1 / np.sqrt(d)), T - 1, T)
    st = cf.Stream()
    native.gpu_workspace_release()
    try:
        native.gpu_inject_alloc_failures(1)
        try:
            rc = cf.call_op("mha_decode_attn_f16_cuda", bufs, [out], p, st)
        finally:
            native.gpu_inject_alloc_failures(0)
        assert rc == -1
        st.synchronize()
        assert not out.download(st).any()
        assert cf.call_op("mha_decode_attn_f16_cuda", bufs, [out], p, st) == 0
        want = O.decode_attn(Q, K, V, np.full(B, T, np.int32), float(1 / np.sqrt(d)), H_kv)
        assert max_abs(want, out.download(st).astype(np.float32)) <= 2e-2
    finally:
        st.close()
