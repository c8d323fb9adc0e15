"""Shared builders for the parity tests: seeded inputs, GPU calls through the C-ABI,
and error metrics.  Inputs are drawn by the oracle's generators (splitmix64 +
Box-Muller, or the reference tests' own glibc-rand / LCG fills)."""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_int, c_int64, c_void_p

import numpy as np

import oracle as O

# op_type_t values (include/graph.h, the reference's enum order) and data_type_t values.
OP_MHA_FUSED, OP_MHA_DECODE, OP_CAUSAL_MASK, OP_RELU, OP_INPUT, OP_OUTPUT = 28, 29, 30, 0, 36, 37
DT_F32, DT_F16 = 0, 1


def max_abs(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


class DecodeCase:
    """Inputs of one MHA_Decode call (fp32 arrays holding fp16-exact values if f16)."""

    def __init__(self, B, H, H_kv, d, max_seq, cache_len=None, seq_lens=None, seed=1, f16=False,
                 wstd=0.02, fill="normal", kv_std=1.0):
        self.B, self.H, self.H_kv, self.d, self.max_seq = B, H, H_kv, d, max_seq
        self.D = H * d
        self.kvd = H_kv * d
        self.f16 = f16
        self.cache_len = cache_len
        self.seq_lens = None if seq_lens is None else np.asarray(seq_lens, np.int32)
        D, kvd = self.D, self.kvd
        g = (lambda shape, s, std=1.0: O.normal(shape, seed * 1000 + s, 0.0, std))
        self.X = g((B, 1, D), 1)
        self.Kc = g((B, max_seq, H_kv, d), 2, kv_std)
        self.Vc = g((B, max_seq, H_kv, d), 3, kv_std)
        self.WQ = g((D, D), 4, wstd)
        self.bQ = g((D,), 5, wstd)
        self.WK = g((D, kvd), 6, wstd)
        self.bK = g((kvd,), 7, wstd)
        self.WV = g((D, kvd), 8, wstd)
        self.bV = g((kvd,), 9, wstd)
        self.WO = g((D, D), 10, wstd)
        self.bO = g((D,), 11, wstd)
        if f16:
            for n in ("X", "Kc", "Vc", "WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO"):
                setattr(self, n, O.round_f16(getattr(self, n)))

    def arrays(self):
        return [self.X, self.Kc, self.Vc, self.WQ, self.bQ, self.WK, self.bK, self.WV, self.bV, self.WO, self.bO]

    def params(self, api_params_cls):
        cl = -1 if self.seq_lens is not None else self.cache_len
        return api_params_cls(self.B, self.D, self.H, self.H_kv, self.d, float(1.0 / np.sqrt(self.d)), cl,
                              self.max_seq)

    def oracle(self):
        p = O.decode_params(self.B, self.D, self.H, self.H_kv, self.d,
                            -1 if self.seq_lens is not None else self.cache_len, self.max_seq)
        return O.mha_decode(*self.arrays(), p, seq_lens=self.seq_lens)


def dev(arr, f16=False):
    from cudaforge_amd import DeviceBuffer
    a = np.ascontiguousarray(arr)
    if f16 and a.dtype != np.float16:
        a = O.to_f16(a)
    return DeviceBuffer.from_numpy(a)


def run_decode_gpu(case: DecodeCase, inplace=True, stream=None):
    """Run mha_decode_{f16,f32}_cuda; returns (Y, K_out, V_out) as float32 arrays."""
    import cudaforge_amd as cf
    f16 = case.f16
    bufs = [dev(a, f16) for a in case.arrays()]
    extra = []
    if case.seq_lens is not None:
        extra = [dev(case.seq_lens)]
    dt = np.float16 if f16 else np.float32
    Y = cf.DeviceBuffer.empty((case.B, 1, case.D), dt)
    if inplace:
        Ko, Vo = bufs[1], bufs[2]
    else:
        Ko = cf.DeviceBuffer.empty(case.Kc.shape, dt)
        Vo = cf.DeviceBuffer.empty(case.Vc.shape, dt)
    p = case.params(cf.MhaDecodeParams)
    name = "mha_decode_f16_cuda" if f16 else "mha_decode_f32_cuda"
    rc = cf.call_op(name, bufs, [Y, Ko, Vo], p, stream, extra_inputs=extra)
    assert rc == 0, f"{name} returned {rc}"
    out = [Y.download(stream), Ko.download(stream), Vo.download(stream)]
    return [o.astype(np.float32) for o in out]


def run_decode_attn_gpu(Q, K, V, cache_len, H_kv, f16, seq_lens=None, scale=None, stream=None):
    import cudaforge_amd as cf
    B, H, d = Q.shape
    max_seq = K.shape[1]
    dt = np.float16 if f16 else np.float32
    bq, bk, bv = dev(Q, f16), dev(K, f16), dev(V, f16)
    out = cf.DeviceBuffer.empty((B, H, d), dt)
    extra = [dev(np.asarray(seq_lens, np.int32))] if seq_lens is not None else []
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1.0 / np.sqrt(d)) if scale is None else scale,
                           -1 if seq_lens is not None else cache_len, max_seq)
    name = "mha_decode_attn_f16_cuda" if f16 else "mha_decode_attn_f32_cuda"
    rc = cf.call_op(name, [bq, bk, bv], [out], p, stream, extra_inputs=extra)
    assert rc == 0, f"{name} returned {rc}"
    return out.download(stream).astype(np.float32)


class FusedCase:
    def __init__(self, B, S, H, H_kv, d, seed=1, f16=False, residual=False, causal=False, wstd=0.02,
                 bias_std=0.0, fill="normal", x_scale=1.0):
        self.B, self.S, self.H, self.H_kv, self.d = B, S, H, H_kv, d
        self.D = H * d
        self.kvd = H_kv * d
        self.f16, self.residual, self.causal = f16, residual, causal
        D, kvd = self.D, self.kvd
        if fill == "lcg":
            g = (lambda shape, s, std=1.0: O.lcg(shape, s))
            seeds = [42, 99, 123, 456, 789, 234, 567, 890, 345, 678]
        else:
            g = (lambda shape, s, std=1.0: O.normal(shape, seed * 1000 + s, 0.0, std))
            seeds = list(range(1, 11))
        self.X = g((B, S, D), seeds[0]) * np.float32(x_scale)
        self.R = g((B, S, D), seeds[1]) if residual else None
        self.WQ = g((D, D), seeds[2], wstd)
        self.bQ = g((D,), seeds[3], bias_std) if (bias_std or fill == "lcg") else np.zeros(D, np.float32)
        self.WK = g((D, kvd), seeds[4], wstd)
        self.bK = g((kvd,), seeds[5], bias_std) if (bias_std or fill == "lcg") else np.zeros(kvd, np.float32)
        self.WV = g((D, kvd), seeds[6], wstd)
        self.bV = g((kvd,), seeds[7], bias_std) if (bias_std or fill == "lcg") else np.zeros(kvd, np.float32)
        self.WO = g((D, D), seeds[8], wstd)
        self.bO = g((D,), seeds[9], bias_std) if (bias_std or fill == "lcg") else np.zeros(D, np.float32)
        if f16:
            for n in ("X", "R", "WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO"):
                v = getattr(self, n)
                if v is not None:
                    setattr(self, n, O.round_f16(v))

    def arrays(self):
        return [self.X, self.R, self.WQ, self.bQ, self.WK, self.bK, self.WV, self.bV, self.WO, self.bO]

    def params(self, cls):
        return cls(self.B, self.S, self.D, self.H, self.H_kv, self.d, float(1.0 / np.sqrt(self.d)),
                   self.residual, self.causal)

    def oracle(self):
        p = O.fused_params(self.B, self.S, self.D, self.H, self.H_kv, self.d, self.residual, self.causal)
        return O.mha_fused(*self.arrays(), p)


def run_fused_gpu(case: FusedCase, stream=None):
    import cudaforge_amd as cf
    bufs = [None if a is None else dev(a, case.f16) for a in case.arrays()]
    dt = np.float16 if case.f16 else np.float32
    Y = cf.DeviceBuffer.empty((case.B, case.S, case.D), dt)
    p = case.params(cf.MhaFusedParams)
    name = "mha_fused_f16io_cuda" if case.f16 else "mha_fused_f32_cuda"
    rc = cf.call_op(name, bufs, [Y], p, stream)
    assert rc == 0, f"{name} returned {rc}"
    return Y.download(stream).astype(np.float32)


# ----------------------------------------------------------------------- graph ---

class Graph:
    """Small wrapper over the graph C-ABI; tensors are owned by the graph once added."""

    def __init__(self, lib):
        self.lib = lib
        self.g = lib.graph_create()
        assert self.g

    @staticmethod
    def _tensor(t):
        import cudaforge_amd as cf
        return ctypes.cast(t, POINTER(cf.TensorT)).contents

    def tensor(self, arr, dtype=DT_F32):
        arr = np.ascontiguousarray(arr)
        assert arr.itemsize == (2 if dtype == DT_F16 else 4), "host array must match the tensor's element size"
        shape = (c_int64 * max(arr.ndim, 1))(*arr.shape)
        t = self.lib.tensor_create(dtype, arr.ndim, shape)
        assert t
        ctypes.memmove(self._tensor(t).data, arr.ctypes.data, arr.nbytes)
        return t, self.lib.graph_add_tensor(self.g, t)

    def write(self, t, arr):
        """Overwrite a tensor's host data (same element count and size)."""
        arr = np.ascontiguousarray(arr)
        tt = self._tensor(t)
        assert arr.size == tt.numel
        ctypes.memmove(tt.data, arr.ctypes.data, arr.nbytes)

    def node(self, op, ins, outs, weights=(), params=None):
        ia = (c_int * max(len(ins), 1))(*ins)
        oa = (c_int * max(len(outs), 1))(*outs)
        wa = (c_void_p * max(len(weights), 1))(*weights)
        pp = ctypes.addressof(params) if params is not None else None
        ps = ctypes.sizeof(params) if params is not None else 0
        return self.lib.graph_add_node(self.g, op, len(ins), ia, len(outs), oa, len(weights), wa, pp, ps)

    def read(self, t, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        ctypes.memmove(out.ctypes.data, self._tensor(t).data, out.nbytes)
        return out

    def destroy(self):
        self.lib.graph_destroy(self.g)


DT_I32 = 3


def build_decode_graph(lib, c: DecodeCase, lens=None):
    """One OP_MHA_DECODE node with in-place KV caches registered through graph_set_kv_cache
    (the reference's decode-session wiring, graph.c:133-153).  f16 cases use F16 tensors,
    so the executor resolves mha_decode_f16_cuda.  `lens` (int32, B entries) adds the
    per-sequence lengths as the node's 9th weight, read when cache_len < 0.  Returns
    (graph, {name: tensor})."""
    dt = DT_F16 if c.f16 else DT_F32
    conv = (lambda a: O.to_f16(a)) if c.f16 else (lambda a: np.asarray(a, np.float32))
    g = Graph(lib)
    tX, iX = g.tensor(conv(c.X), dt)
    tK, iK = g.tensor(conv(c.Kc), dt)
    tV, iV = g.tensor(conv(c.Vc), dt)
    tY, iY = g.tensor(conv(np.zeros_like(c.X)), dt)
    ws = [g.tensor(conv(w), dt)[0] for w in (c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO)]
    tL = None
    if lens is not None:
        tL = g.tensor(np.asarray(lens, np.int32), DT_I32)[0]
        ws.append(tL)
    p = O.decode_params(c.B, c.D, c.H, c.H_kv, c.d, c.cache_len, c.max_seq)
    g.node(OP_MHA_DECODE, [iX, iK, iV], [iY, iK, iV], ws, p)
    lib.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
    lib.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
    lib.graph_set_kv_cache(g.g, iK, iV)
    assert lib.graph_build(g.g) == 0
    return g, {"X": tX, "K": tK, "V": tV, "Y": tY, "L": tL}


# op_type_t values of the unfused attention pattern (include/graph.h enum order).
OP_MATMUL, OP_ADD, OP_RESHAPE, OP_SOFTMAX, OP_MUL, OP_TRANSPOSE = 3, 8, 9, 11, 13, 16


def build_attention_subgraph(g: Graph, c: FusedCase, x_id, r_id=None, *, bias=True, causal=False,
                             scale=None, softmax_op=None, extra_scores_reader=False, wdtype=None,
                             mask_style="add", mask_seq=None, scale_style="weight", bias_style="weight"):
    """Appends the unfused self-attention block the reference's fusion pass recognises
    (graph.c:347-358, the ONNX BERT export's node pattern) reading tensor x_id:
      X -> 3 x [MatMul -> Add(bias) -> Reshape -> Transpose] -> Q, K, V;
      MatMul(Q, K^T) -> Mul(scale) [-> Add(CausalMask output)] -> Softmax -> MatMul(., V)
      -> Transpose -> Reshape -> MatMul(W_O) -> Add(b_O) [-> Add(residual r_id)].
    Intermediate tensors get their real shapes (never computed: the pattern runs fused).
    Bias Adds take the bias as their second input and as their weight, as the
    reference's Add nodes do.  Variants for the matcher's tests:
      mask_style "add" (CausalMask output added to the scores), "add_shared" (the mask is
        also read by another node), "passthrough" (CausalMask reading the scores, a
        pattern whose op-by-op meaning is not masked attention); mask_seq overrides the
        CausalMask node's seq_len;
      scale_style "weight", "constant" (second input, no producer), "produced" (second
        input written by a node), "swapped" (scores as the Mul's second input);
      bias_style "weight", or "input" (bias Adds read the bias as a graph tensor only).
    Returns {name: id} for the nodes and tensors."""
    B, S, D, H, H_kv, d = c.B, c.S, c.D, c.H, c.H_kv, c.d
    dt = DT_F16 if c.f16 else DT_F32
    npdt = np.float16 if c.f16 else np.float32
    conv = (lambda a: O.to_f16(a)) if c.f16 else (lambda a: np.asarray(a, np.float32))
    wdt = dt if wdtype is None else wdtype
    wconv = (lambda a: O.to_f16(a)) if wdt == DT_F16 else (lambda a: np.asarray(a, np.float32))

    def t(shape):
        return g.tensor(np.zeros(shape, npdt), dt)

    ids = {}
    chains = {}
    for name, W, bvec, heads, kt in (("q", c.WQ, c.bQ, H, False), ("k", c.WK, c.bK, H_kv, True),
                                     ("v", c.WV, c.bV, H_kv, False)):
        width = heads * d
        w_t, _ = g.tensor(wconv(W), wdt)
        _, mm_out = t((B, S, width))
        ids["mm_" + name] = g.node(OP_MATMUL, [x_id], [mm_out], [w_t])
        cur = mm_out
        if bias:
            b_t, b_id = g.tensor(wconv(bvec), wdt)
            _, add_out = t((B, S, width))
            ids["add_" + name] = g.node(OP_ADD, [cur, b_id], [add_out], [b_t] if bias_style == "weight" else [])
            cur = add_out
        _, rs = t((B, S, heads, d))
        ids["rs_" + name] = g.node(OP_RESHAPE, [cur], [rs])
        _, tr = t((B, heads, d, S) if kt else (B, heads, S, d))
        ids["tr_" + name] = g.node(OP_TRANSPOSE, [rs], [tr])
        chains[name] = tr
    _, scores = t((B, H, S, S))
    ids["attn"] = g.node(OP_MATMUL, [chains["q"], chains["k"]], [scores])
    if extra_scores_reader:
        _, spare = t((B, H, S, S))
        ids["spare"] = g.node(OP_RELU, [scores], [spare])
    s_t, s_id = g.tensor(np.full((1,), 1.0 / np.sqrt(d) if scale is None else scale, np.float32))
    _, scaled = t((B, H, S, S))
    if scale_style == "weight":
        ids["mul"] = g.node(OP_MUL, [scores], [scaled], [s_t])
    elif scale_style == "constant":
        ids["mul"] = g.node(OP_MUL, [scores, s_id], [scaled])
    elif scale_style == "swapped":
        ids["mul"] = g.node(OP_MUL, [s_id, scores], [scaled])
    else:
        _, s_src = g.tensor(np.ones((1,), np.float32))
        ids["scale_src"] = g.node(OP_RELU, [s_src], [s_id])
        ids["mul"] = g.node(OP_MUL, [scores, s_id], [scaled])
    cur = scaled
    if causal:
        import cudaforge_amd as cf
        _, masked = t((B, H, S, S))
        if mask_style == "passthrough":
            ids["mask"] = g.node(OP_CAUSAL_MASK, [cur], [masked], params=cf.CausalMaskParams(S))
        else:
            # The causal pattern as graphs hold it: CausalMask writes an (S, S) 0 / -inf
            # mask (its input is a placeholder, causal_mask.c:5-8) that an Add puts on
            # the scaled scores.
            _, mask = g.tensor(np.zeros((S, S), np.float32), DT_F32)
            ms = S if mask_seq is None else mask_seq
            ids["mask"] = g.node(OP_CAUSAL_MASK, [x_id], [mask], params=cf.CausalMaskParams(ms))
            ids["add_mask"] = g.node(OP_ADD, [cur, mask], [masked])
            if mask_style == "add_shared":
                _, mask2 = g.tensor(np.zeros((S, S), np.float32), DT_F32)
                ids["mask_reader"] = g.node(OP_RELU, [mask], [mask2])
        cur = masked
    _, probs = t((B, H, S, S))
    ids["softmax"] = g.node(OP_SOFTMAX if softmax_op is None else softmax_op, [cur], [probs])
    _, ctx = t((B, H, S, d))
    ids["pv"] = g.node(OP_MATMUL, [probs, chains["v"]], [ctx])
    _, ctx_t = t((B, S, H, d))
    ids["tr_o"] = g.node(OP_TRANSPOSE, [ctx], [ctx_t])
    _, merged = t((B, S, D))
    ids["rs_o"] = g.node(OP_RESHAPE, [ctx_t], [merged])
    wo_t, _ = g.tensor(wconv(c.WO), wdt)
    _, proj = t((B, S, D))
    ids["mm_o"] = g.node(OP_MATMUL, [merged], [proj], [wo_t])
    cur = proj
    if bias:
        bo_t, bo_id = g.tensor(wconv(c.bO), wdt)
        _, projb = t((B, S, D))
        ids["add_o"] = g.node(OP_ADD, [cur, bo_id], [projb], [bo_t] if bias_style == "weight" else [])
        cur = projb
    if r_id is not None:
        _, out = t((B, S, D))
        ids["add_r"] = g.node(OP_ADD, [cur, r_id], [out])
        cur = out
    ids["out"] = cur
    return ids


def build_fused_graph(lib, c: FusedCase, f16_out=False):
    """One OP_MHA_FUSED node with INPUT/OUTPUT wrappers (tests/test_bert_mha.c:167-306);
    F32 tensors, or an F16 output tensor.  Returns (graph, node id, X tensor, Y tensor)."""
    g = Graph(lib)
    tX, iX = g.tensor(c.X)
    tR, iR = g.tensor(c.R if c.R is not None else np.zeros_like(c.X))
    tY, iY = (g.tensor(np.zeros(c.X.shape, np.float16), DT_F16) if f16_out
              else g.tensor(np.zeros_like(c.X), DT_F32))
    ws = [g.tensor(w)[0] for w in (c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO)]
    p = O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, c.residual, c.causal)
    nid = g.node(OP_MHA_FUSED, [iX, iR], [iY], ws, p)
    g.lib.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
    g.lib.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
    assert lib.graph_build(g.g) == 0
    return g, nid, tX, tY


def fused_ref64(c: FusedCase):
    """MHA_Fused in float64 (numpy) on the case's exact inputs: projections, scaled
    scores with the causal rule j <= i, softmax, P.V, W_O, bias, residual
    (mha_fused.c:67-172 in exact arithmetic).  Returns (B, S, D) float64."""
    f = lambda a: np.asarray(a, np.float64)
    B, S, D, H, H_kv, d = c.B, c.S, c.D, c.H, c.H_kv, c.d
    G = H // H_kv
    X = f(c.X).reshape(B * S, D)
    q = (X @ f(c.WQ) + f(c.bQ)).reshape(B, S, H, d).transpose(0, 2, 1, 3)
    k = (X @ f(c.WK) + f(c.bK)).reshape(B, S, H_kv, d).transpose(0, 2, 1, 3)
    v = (X @ f(c.WV) + f(c.bV)).reshape(B, S, H_kv, d).transpose(0, 2, 1, 3)
    k = np.repeat(k, G, axis=1)
    v = np.repeat(v, G, axis=1)
    s = np.matmul(q, k.transpose(0, 1, 3, 2)) * float(np.float32(1.0 / np.sqrt(d)))
    if c.causal:
        s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, v).transpose(0, 2, 1, 3).reshape(B * S, D)
    y = o @ f(c.WO) + f(c.bO)
    if c.residual and c.R is not None:
        y = y + f(c.R).reshape(B * S, D)
    return y.reshape(B, S, D)


def attn_ref64_all(Q, K, V, attend, H_kv, scale):
    """Decode attention core in float64 for every (b, head), vectorised over heads."""
    B, H, d = Q.shape
    G = H // H_kv
    out = np.zeros((B, H, d))
    for b in range(B):
        T = int(attend[b])
        k = K[b, :T].astype(np.float64)                      # (T, H_kv, d)
        v = V[b, :T].astype(np.float64)
        q = Q[b].astype(np.float64).reshape(H_kv, G, d)
        s = np.einsum("tkd,kgd->kgt", k, q) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("kgt,tkd->kgd", p, v).reshape(H, d)
    return out
