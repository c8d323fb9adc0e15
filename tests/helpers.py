"""Shared builders for the parity tests: seeded inputs, GPU calls through the C-ABI,
and error metrics.  Inputs are drawn by the oracle's generators (splitmix64 +
Box-Muller, or the reference tests' own glibc-rand / LCG fills)."""

from __future__ import annotations

import numpy as np

import oracle as O


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
    name = "mha_fused_f16_cuda" if case.f16 else "mha_fused_f32_cuda"
    rc = cf.call_op(name, bufs, [Y], p, stream)
    assert rc == 0, f"{name} returned {rc}"
    return Y.download(stream).astype(np.float32)
