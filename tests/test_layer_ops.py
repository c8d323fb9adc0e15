"""LayerNorm, Cast and MatMul: the oracle against the reference's own C files (CPU), and
the HIP operators against the oracle (GPU), including an FP16 chain through the graph
(Cast -> LayerNorm -> MatMul + bias -> Cast) that stays on the device.

Tolerances: FP32 <= 1e-4 absolute (LayerNorm outputs are O(1); MatMul sums are scaled so
the outputs are O(1)), FP16 <= 2e-2 with fp32 accumulation; Cast is exact.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import dev, max_abs

TOL32, TOL16 = 1e-4, 2e-2
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference build not available")


def _ln_inputs(N, D, seed):
    x = O.normal((N, D), seed)
    g = O.normal((D,), seed + 1, 1.0, 0.1)
    b = O.normal((D,), seed + 2, 0.0, 0.1)
    return x, g, b


# ------------------------------------------------------------------ oracle (CPU) ---

@needs_ref
@pytest.mark.parametrize("N,D", [(33, 768), (5, 1000), (2, 1), (3, 4098)])
def test_oracle_layernorm_matches_reference_build(N, D):
    x, g, b = _ln_inputs(N, D, N + D)
    assert np.array_equal(O.layernorm(x, g, b, 1e-5), O.layernorm(x, g, b, 1e-5, use_ref=True))


def test_oracle_layernorm_constant_rows_give_beta():
    x = np.full((3, 64), 2.5, np.float32)
    g = O.normal((64,), 5)
    b = O.normal((64,), 6)
    assert np.array_equal(O.layernorm(x, g, b), np.broadcast_to(b, x.shape))


@needs_ref
@pytest.mark.parametrize("ta,tb,batch,bias", [(False, False, 1, True), (True, False, 1, False), (False, True, 3, True),
                                              (True, True, 2, True)])
def test_oracle_matmul_matches_reference_build(ta, tb, batch, bias):
    M, N, K = 7, 5, 9
    A = O.normal((batch, M * K), 1)
    B = O.normal((batch, K * N), 2)
    bb = O.normal((N,), 3) if bias else None
    kw = dict(transpose_a=ta, transpose_b=tb, batch=batch, stride_a=M * K, stride_b=K * N, stride_c=M * N)
    assert np.array_equal(O.matmul(A, B, bb, M, N, K, **kw), O.matmul(A, B, bb, M, N, K, use_ref=True, **kw))


def test_oracle_matmul_identity():
    A = O.normal((6, 6), 4)
    assert np.array_equal(O.matmul(A, np.eye(6, dtype=np.float32), None, 6, 6, 6).reshape(6, 6), A)


@needs_ref
def test_reference_cast_agrees_with_ieee_where_its_cuda_op_does():
    """cast.c's FLOAT16 -> FLOAT and INT64 <-> FLOAT match IEEE conversions (numpy); its
    FLOAT -> FLOAT16 truncates (cast.c:8-16), which only agrees with the CUDA op's
    round-to-nearest on exactly representable values."""
    h = O.to_f16(O.normal((1000,), 7))
    assert np.array_equal(O.cast_ref(h, O.ONNX_FLOAT16, O.ONNX_FLOAT), h.astype(np.float32))
    i = np.arange(-500, 500, dtype=np.int64) * 12345
    assert np.array_equal(O.cast_ref(i, O.ONNX_INT64, O.ONNX_FLOAT), i.astype(np.float32))
    f = O.normal((1000,), 8) * 1000
    assert np.array_equal(O.cast_ref(f, O.ONNX_FLOAT, O.ONNX_INT64), f.astype(np.int64))
    exact = h.astype(np.float32)
    assert np.array_equal(O.cast_ref(exact, O.ONNX_FLOAT, O.ONNX_FLOAT16), h)


# ------------------------------------------------------------------ HIP (GPU) ---

def _ln_gpu(x, g, b, eps, f16, in_place=False):
    import cudaforge_amd as cf
    N, D = x.shape
    bx, bg, bb = dev(x, f16), dev(g, f16), dev(b, f16)
    out = bx if in_place else cf.DeviceBuffer.empty(x.shape, np.float16 if f16 else np.float32)
    p = O.LayerNormParams(N, D, eps)
    assert cf.call_op("layernorm_f16_cuda" if f16 else "layernorm_f32_cuda", [bx, bg, bb], [out], p) == 0
    return out.download().astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("N,D,eps", [(4096, 768, 1e-12), (7, 1000, 1e-5), (3, 4098, 1e-5), (2, 8192, 1e-5),
                                     (5, 64, 1e-5)])
def test_layernorm_f32_cuda(gpu, N, D, eps):
    x, g, b = _ln_inputs(N, D, N * 7 + D)
    assert max_abs(O.layernorm(x, g, b, eps), _ln_gpu(x, g, b, eps, False)) <= TOL32


@pytest.mark.gpu
@pytest.mark.parametrize("N,D", [(4096, 768), (9, 1024), (3, 4098)])
def test_layernorm_f16_cuda(gpu, N, D):
    x, g, b = (O.round_f16(a) for a in _ln_inputs(N, D, N + 3 * D))
    want = O.layernorm(x, g, b, 1e-5)
    assert max_abs(want, _ln_gpu(x, g, b, 1e-5, True)) <= TOL16
    assert max_abs(want, _ln_gpu(x, g, b, 1e-5, True, in_place=True)) <= TOL16


@pytest.mark.gpu
def test_cast_f32_cuda_all_pairs(gpu):
    import cudaforge_amd as cf

    def run(arr, src, dst, out_dtype):
        i = cf.DeviceBuffer.from_numpy(np.ascontiguousarray(arr))
        o = cf.DeviceBuffer.empty(arr.shape, out_dtype)
        assert cf.call_op("cast_f32_cuda", [i], [o], O.CastParams(src, dst, arr.size)) == 0
        return o.download()

    f = np.concatenate([O.normal((5000,), 9) * 100, np.float32([0.0, -0.0, 1e-7, -3e-6, 65504.0, 70000.0, 6.1e-5])])
    with np.errstate(over="ignore"):                                         # 70000 -> inf on purpose
        want16 = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(run(f, O.ONNX_FLOAT, O.ONNX_FLOAT16, np.float16).view(np.uint16),
                          want16)                                            # RNE, subnormals, overflow
    h = O.to_f16(O.normal((5000,), 10))
    assert np.array_equal(run(h, O.ONNX_FLOAT16, O.ONNX_FLOAT, np.float32), h.astype(np.float32))
    i = (np.arange(-2500, 2500, dtype=np.int64) * 987654321)
    assert np.array_equal(run(i, O.ONNX_INT64, O.ONNX_FLOAT, np.float32), i.astype(np.float32))
    g = O.normal((5000,), 11) * 1e6
    assert np.array_equal(run(g, O.ONNX_FLOAT, O.ONNX_INT64, np.int64), g.astype(np.int64))
    assert np.array_equal(run(g, O.ONNX_FLOAT, O.ONNX_FLOAT, np.float32), g)    # other pairs copy


def _mm_gpu(A, B, bias, M, N, K, f16, **kw):
    import cudaforge_amd as cf
    dt = np.float16 if f16 else np.float32
    batch = kw.get("batch", 1)
    C = cf.DeviceBuffer.empty(((batch - 1) * kw.get("stride_c", 0) + M * N,), dt)
    p = O.MatmulParams(M, N, K, kw.get("transpose_a", False), kw.get("transpose_b", False), batch,
                       kw.get("stride_a", 0), kw.get("stride_b", 0), kw.get("stride_c", 0), 0)
    slots = [dev(A, f16), dev(B, f16), None if bias is None else dev(bias, f16)]
    name = "matmul_f16_cuda" if f16 else "matmul_f32_cuda"
    assert cf.call_op(name, slots, [C], p) == 0
    return C.download().astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("M,N,K", [(33, 70, 17), (128, 256, 64), (256, 3072, 768)])
def test_matmul_cuda(gpu, f16, M, N, K):
    r = O.round_f16 if f16 else (lambda a: a)
    A = r(O.normal((M, K), M + N))
    B = r(O.normal((K, N), K + 1, 0.0, 1.0 / np.sqrt(K)))
    bias = r(O.normal((N,), 5, 0.0, 0.1))
    want = A.astype(np.float64) @ B.astype(np.float64) + bias
    if M * N * K <= 1 << 20:
        want = O.matmul(A, B, bias, M, N, K).reshape(M, N)
    got = _mm_gpu(A, B, bias, M, N, K, f16).reshape(M, N)
    assert max_abs(want, got) <= (TOL16 if f16 else TOL32)


@pytest.mark.gpu
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_matmul_cuda_transposed_batched(gpu, f16, ta, tb):
    r = O.round_f16 if f16 else (lambda a: a)
    M, N, K, batch = 40, 72, 48, 3
    sa, sb, sc = M * K + 5, K * N + 3, M * N + 7          # padded slices: strides are honoured
    A = r(O.normal(((batch - 1) * sa + M * K,), 21))
    B = r(O.normal(((batch - 1) * sb + K * N,), 22, 0.0, 0.2))
    bias = r(O.normal((N,), 23))
    kw = dict(transpose_a=ta, transpose_b=tb, batch=batch, stride_a=sa, stride_b=sb, stride_c=sc)
    want = O.matmul(A, B, bias, M, N, K, **kw)
    got = _mm_gpu(A, B, bias, M, N, K, f16, **kw)
    for bi in range(batch):
        sl = slice(bi * sc, bi * sc + M * N)
        assert max_abs(want[sl], got[sl]) <= (TOL16 if f16 else TOL32)


@pytest.mark.gpu
def test_fp16_layer_chain_through_the_graph(gpu, native):
    """X (F32) -> Cast -> F16 -> LayerNorm -> MatMul (+ bias, slot 2) -> Cast -> F32, every
    node resolved to a HIP operator by the graph's name rule and run on the device."""
    from helpers import DT_F16, DT_F32, OP_INPUT, OP_OUTPUT, Graph
    OP_MATMUL, OP_LAYERNORM, OP_CAST = 3, 21, 26
    S, D, F = 64, 256, 512
    x = O.normal((S, D), 31)
    g16, b16 = O.to_f16(O.normal((D,), 32, 1.0, 0.1)), O.to_f16(O.normal((D,), 33, 0.0, 0.1))
    W16 = O.to_f16(O.normal((D, F), 34, 0.0, 1.0 / np.sqrt(D)))
    bias16 = O.to_f16(O.normal((F,), 35, 0.0, 0.1))
    gr = Graph(native)
    try:
        tX, iX = gr.tensor(x)
        _, iXh = gr.tensor(np.zeros((S, D), np.float16), DT_F16)
        _, iL = gr.tensor(np.zeros((S, D), np.float16), DT_F16)
        _, iM = gr.tensor(np.zeros((S, F), np.float16), DT_F16)
        tY, iY = gr.tensor(np.zeros((S, F), np.float32))
        tg = gr.tensor(g16, DT_F16)[0]
        tb = gr.tensor(b16, DT_F16)[0]
        tW = gr.tensor(W16, DT_F16)[0]
        tbias = gr.tensor(bias16, DT_F16)[0]
        names = []
        buf = ctypes.create_string_buffer(64)
        n1 = gr.node(OP_CAST, [iX], [iXh], (), O.CastParams(O.ONNX_FLOAT, O.ONNX_FLOAT16, S * D))
        n2 = gr.node(OP_LAYERNORM, [iXh], [iL], (tg, tb), O.LayerNormParams(S, D, 1e-5))
        n3 = gr.node(OP_MATMUL, [iL], [iM], (tW, tbias), O.MatmulParams(S, F, D, False, False, 1, 0, 0, 0, 0))
        n4 = gr.node(OP_CAST, [iM], [iY], (), O.CastParams(O.ONNX_FLOAT16, O.ONNX_FLOAT, S * F))
        native.graph_set_input(gr.g, gr.node(OP_INPUT, [], [iX]))
        native.graph_set_output(gr.g, gr.node(OP_OUTPUT, [iY], []))
        assert native.graph_build(gr.g) == 0
        for n in (n1, n2, n3, n4):
            assert native.graph_resolve_op(gr.g, n, True, buf, 64)
            names.append(buf.value)
        assert names == [b"cast_f32_cuda", b"layernorm_f16_cuda", b"matmul_f16_cuda", b"cast_f32_cuda"]
        ins, outs = (ctypes.c_void_p * 1)(tX), (ctypes.c_void_p * 1)(tY)
        assert native.graph_execute(gr.g, ins, outs, True) == 0
        got = gr.read(tY, (S, F))
        xh = O.round_f16(x)
        ln = O.round_f16(O.layernorm(xh, g16.astype(np.float32), b16.astype(np.float32), 1e-5))
        want = O.matmul(ln, W16.astype(np.float32), bias16.astype(np.float32), S, F, D).reshape(S, F)
        assert max_abs(want, got) <= TOL16
    finally:
        gr.destroy()
