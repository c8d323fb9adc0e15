"""CPU parity oracle — TEST INFRASTRUCTURE ONLY.

ctypes bindings for ``oracle/_build/liboracle.so`` (this repo's C restatement of the
reference fallbacks, oracle.c) and, where it was built, ``oracle/_ref/libcfref.so`` (the
reference's own C fallback compiled from /root/reference).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker; the product library never calls it.

Pinning status of each oracle function (see tests/test_oracle.py):
  oracle_mha_decode_f32   pinned: bit-exact vs the reference build and its golden vectors
                          (d <= 64, T <= 512), closed forms (T = 1), invariants.
  oracle_decode_attn_f32  pinned: vs the decode op (Q-given inner loop), float64 brute
                          force, KV permutation / split / GQA invariants, identical-key and
                          one-hot closed forms.
  oracle_mha_fused_f32    pinned: bit-exact vs the reference build (non-causal, H_kv = H)
                          and golden vectors; causal via the prefix invariant (row i of a
                          causal run == last row of a non-causal run over i+1 tokens),
                          GQA via repeated-KV equivalence.
  oracle_causal_mask_f32  pinned: vs the reference build (exact).
  oracle_layernorm_f32    pinned: bit-exact vs the reference build (layernorm.c, scalar
                          path); constant rows give beta.
  oracle_matmul_f32       pinned: bit-exact vs the reference build (matmul.c) with
                          transposes, batches and bias; identity matrices.
  oracle_rope_f32         pinned: bit-exact vs the reference build (rope.c) on the
                          tests/test_rope.c known-answer inputs and on larger seeded ones;
                          norm preservation; position 0 = identity.
  oracle_mha_decode_rope_f32  pinned: position 0 == plain decode (bit-exact); rotating the
                          Q/K projection weights' output columns instead of Q and K_new
                          gives the same result (fp32 rounding apart).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint, c_uint16, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_SO may name the sanitizer build (tests/sanitize.sh).
ORACLE_SO = os.environ.get("CUDAFORGE_ORACLE_SO") or os.path.join(HERE, "_build", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libcfref.so")

_lib = None
_ref = None


class DecodeParams(ctypes.Structure):
    _fields_ = [("batch_size", c_int64), ("hidden_size", c_int64), ("num_heads", c_int64),
                ("num_kv_heads", c_int64), ("head_dim", c_int64), ("scale", c_float),
                ("cache_len", c_int64), ("max_seq", c_int64)]


class FusedParams(ctypes.Structure):
    _fields_ = [("batch_size", c_int64), ("seq_len", c_int64), ("hidden_size", c_int64),
                ("num_heads", c_int64), ("num_kv_heads", c_int64), ("head_dim", c_int64),
                ("scale", c_float), ("has_residual", ctypes.c_bool), ("causal", ctypes.c_bool)]


class LayerNormParams(ctypes.Structure):
    """layernorm_params_t (src/operator/nn/layernorm_int.h:6-10)."""
    _fields_ = [("N", c_int64), ("normalized_size", c_int64), ("epsilon", c_float)]


class MatmulParams(ctypes.Structure):
    """matmul_params_t (src/operator/blas/matmul_int.h:7-17)."""
    _fields_ = [("M", c_int64), ("N", c_int64), ("K", c_int64), ("transpose_a", ctypes.c_bool),
                ("transpose_b", ctypes.c_bool), ("batch_size", c_int64), ("stride_a", c_int64),
                ("stride_b", c_int64), ("stride_c", c_int64), ("tuning_config", c_int)]


class CastParams(ctypes.Structure):
    """cast_params_t (src/operator/nn/cast_int.h:12-16); dtypes are ONNX codes."""
    _fields_ = [("src_dtype", c_int), ("dst_dtype", c_int), ("numel", c_int64)]


ONNX_FLOAT, ONNX_FLOAT16, ONNX_INT64 = 1, 10, 7


class RopeParams(ctypes.Structure):
    """rope_params_t (src/operator/nn/rope_int.h:6-11)."""
    _fields_ = [("seq_len", c_int64), ("head_dim", c_int64), ("num_heads", c_int64), ("base", c_float)]


def _build_if_missing(target: str, path: str) -> None:
    if not os.path.exists(path):
        subprocess.run(["make", "-C", HERE, target], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        _build_if_missing("oracle", ORACLE_SO)
        L = ctypes.CDLL(ORACLE_SO)
        F = POINTER(c_float)
        L.oracle_mha_decode_f32.argtypes = [POINTER(c_void_p), POINTER(c_void_p), c_void_p]
        L.oracle_decode_attn_f32.argtypes = [F, F, F, F, c_int64, c_int64, c_int64, c_int64, c_int64,
                                             POINTER(c_int32), c_float]
        L.oracle_mha_fused_f32.argtypes = [POINTER(c_void_p), POINTER(c_void_p), c_void_p]
        L.oracle_rope_f32.argtypes = [F, F, c_int64, c_int64, c_int64, c_float]
        L.oracle_layernorm_f32.argtypes = [F, F, F, F, c_int64, c_int64, c_float]
        L.oracle_matmul_f32.argtypes = [F, F, F, F, c_int64, c_int64, c_int64, c_int, c_int, c_int64, c_int64,
                                        c_int64, c_int64]
        L.oracle_mha_decode_rope_f32.argtypes = [POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_float]
        L.oracle_causal_mask_f32.argtypes = [F, c_int64]
        L.oracle_causal_mask_f32.restype = None
        L.oracle_fill_normal.argtypes = [F, c_size_t, c_uint64, c_float, c_float]
        L.oracle_fill_normal.restype = None
        L.oracle_fill_uniform_int.argtypes = [POINTER(c_int32), c_size_t, c_uint64, c_int32, c_int32]
        L.oracle_fill_uniform_int.restype = None
        L.oracle_fill_glibc_rand.argtypes = [F, c_size_t, c_int]
        L.oracle_fill_glibc_rand.restype = None
        L.oracle_fill_lcg.argtypes = [F, c_size_t, c_uint]
        L.oracle_fill_lcg.restype = None
        L.oracle_f32_to_f16_array.argtypes = [F, POINTER(c_uint16), c_size_t]
        L.oracle_f32_to_f16_array.restype = None
        L.oracle_f16_to_f32_array.argtypes = [POINTER(c_uint16), F, c_size_t]
        L.oracle_f16_to_f32_array.restype = None
        L.oracle_now.restype = c_double
        _lib = L
    return _lib


def ref_available() -> bool:
    if not os.path.exists(REF_SO) and os.path.isdir("/root/reference"):
        try:
            _build_if_missing("ref", REF_SO)
        except Exception:
            return False
    return os.path.exists(REF_SO)


def ref():
    """The reference's own C fallback (mha_decode_f32, mha_fused_f32, causal_mask_f32)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(REF_SO)
        L = ctypes.CDLL(REF_SO)
        for n in ("mha_decode_f32", "mha_fused_f32", "causal_mask_f32", "rope_f32", "layernorm_f32", "cast_f32",
                  "matmul_f32"):
            getattr(L, n).argtypes = [POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p]
            getattr(L, n).restype = c_int
        _ref = L
    return _ref


def _fp(a):
    return a.ctypes.data_as(POINTER(c_float))


def _slots(arrs):
    return (c_void_p * len(arrs))(*[None if a is None else a.ctypes.data for a in arrs])


# ---------------------------------------------------------------- generators ---

def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().oracle_fill_normal(_fp(out), n, seed, mean, std)
    return out.reshape(shape)


def uniform_int(n: int, seed: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().oracle_fill_uniform_int(out.ctypes.data_as(POINTER(c_int32)), n, seed, lo, hi)
    return out


def glibc_rand(shape, seed: int) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().oracle_fill_glibc_rand(_fp(out), n, seed)
    return out.reshape(shape)


def lcg(shape, seed: int) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().oracle_fill_lcg(_fp(out), n, seed)
    return out.reshape(shape)


def to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_fp(a), out.ctypes.data_as(POINTER(c_uint16)), a.size)
    return out.view(np.float16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h).view(np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(h.ctypes.data_as(POINTER(c_uint16)), _fp(out), h.size)
    return out


def round_f16(a: np.ndarray) -> np.ndarray:
    """fp32 values that are exactly representable in fp16 (RNE)."""
    return f16_to_f32(to_f16(a))


def now() -> float:
    return lib().oracle_now()


# ---------------------------------------------------------------- operators ---

def decode_params(B, D, H, H_kv, d, cache_len, max_seq, scale=None) -> DecodeParams:
    return DecodeParams(B, D, H, H_kv, d, float(1.0 / np.sqrt(d)) if scale is None else scale, cache_len, max_seq)


def fused_params(B, S, D, H, H_kv, d, has_residual=False, causal=False, scale=None) -> FusedParams:
    return FusedParams(B, S, D, H, H_kv, d, float(1.0 / np.sqrt(d)) if scale is None else scale,
                       has_residual, causal)


def mha_decode(X, Kc, Vc, WQ, bQ, WK, bK, WV, bV, WO, bO, p: DecodeParams, seq_lens=None, use_ref=False):
    """Run the decode op on the CPU; returns (Y, K_out, V_out)."""
    arrs = [np.ascontiguousarray(a, np.float32) for a in (X, Kc, Vc, WQ, bQ, WK, bK, WV, bV, WO, bO)]
    if seq_lens is not None:
        arrs.append(np.ascontiguousarray(seq_lens, np.int32))
    Y = np.zeros((p.batch_size, 1, p.hidden_size), np.float32)
    Ko = np.zeros_like(arrs[1])
    Vo = np.zeros_like(arrs[2])
    ins, outs = _slots(arrs), _slots([Y, Ko, Vo])
    if use_ref:
        rc = ref().mha_decode_f32(ins, outs, ctypes.addressof(p), None)
    else:
        rc = lib().oracle_mha_decode_f32(ins, outs, ctypes.addressof(p))
    if rc != 0:
        raise ValueError(f"decode oracle returned {rc}")
    return Y, Ko, Vo


def decode_attn(Q, K, V, attend, scale, H_kv):
    """Attention core with Q given: Q (B,H,d), K/V (B,max_seq,H_kv,d), attend (B,) positions."""
    Q = np.ascontiguousarray(Q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    B, H, d = Q.shape
    max_seq = K.shape[1]
    O = np.zeros_like(Q)
    att = np.ascontiguousarray(attend, np.int32)
    rc = lib().oracle_decode_attn_f32(_fp(Q), _fp(K), _fp(V), _fp(O), B, H, H_kv, d, max_seq,
                                      att.ctypes.data_as(POINTER(c_int32)), scale)
    if rc != 0:
        raise ValueError(f"decode_attn oracle returned {rc}")
    return O


def mha_fused(X, R, WQ, bQ, WK, bK, WV, bV, WO, bO, p: FusedParams, use_ref=False):
    arrs = [None if a is None else np.ascontiguousarray(a, np.float32) for a in (X, R, WQ, bQ, WK, bK, WV, bV, WO, bO)]
    Y = np.zeros((p.batch_size, p.seq_len, p.hidden_size), np.float32)
    ins, outs = _slots(arrs), _slots([Y])
    if use_ref:
        rc = ref().mha_fused_f32(ins, outs, ctypes.addressof(p), None)
    else:
        rc = lib().oracle_mha_fused_f32(ins, outs, ctypes.addressof(p))
    if rc != 0:
        raise ValueError(f"fused oracle returned {rc}")
    return Y


def layernorm(x, gamma, beta, eps=1e-5, use_ref=False) -> np.ndarray:
    """LayerNorm over the last axis of x (layernorm.c, scalar path)."""
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    b = np.ascontiguousarray(beta, np.float32)
    D = x.shape[-1]
    N = x.size // D
    y = np.zeros_like(x)
    if use_ref:
        p = LayerNormParams(N, D, eps)
        rc = ref().layernorm_f32(_slots([x, g, b]), _slots([y]), ctypes.addressof(p), None)
    else:
        rc = lib().oracle_layernorm_f32(_fp(x), _fp(g), _fp(b), _fp(y), N, D, eps)
    if rc != 0:
        raise ValueError(f"layernorm returned {rc}")
    return y


def matmul(A, B, bias=None, M=None, N=None, K=None, transpose_a=False, transpose_b=False, batch=1,
           stride_a=0, stride_b=0, stride_c=0, use_ref=False) -> np.ndarray:
    """matmul.c: C = A·B (+ bias) per batch slice; A, B flat or shaped, sizes explicit."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    C = np.zeros(max(batch, 1) * M * N if batch > 1 else M * N, np.float32)
    if batch > 1:
        C = np.zeros((batch - 1) * stride_c + M * N, np.float32)
    if use_ref:
        p = MatmulParams(M, N, K, transpose_a, transpose_b, batch, stride_a, stride_b, stride_c, 0)
        rc = ref().matmul_f32(_slots([A, B, bb]), _slots([C]), ctypes.addressof(p), None)
    else:
        rc = lib().oracle_matmul_f32(_fp(A), _fp(B), None if bb is None else _fp(bb), _fp(C), M, N, K,
                                     int(transpose_a), int(transpose_b), batch, stride_a, stride_b, stride_c)
    if rc != 0:
        raise ValueError(f"matmul returned {rc}")
    return C


def cast_ref(x, src_dtype: int, dst_dtype: int) -> np.ndarray:
    """The reference's CPU cast (cast.c), for the conversions it shares with its CUDA op."""
    x = np.ascontiguousarray(x)
    out_dt = {ONNX_FLOAT: np.float32, ONNX_FLOAT16: np.uint16, ONNX_INT64: np.int64}[dst_dtype]
    out = np.zeros(x.size, out_dt)
    p = CastParams(src_dtype, dst_dtype, x.size)
    rc = ref().cast_f32(_slots([x]), _slots([out]), ctypes.addressof(p), None)
    if rc != 0:
        raise ValueError(rc)
    return out.view(np.float16) if dst_dtype == ONNX_FLOAT16 else out


def rope(x, base: float = 10000.0, use_ref=False) -> np.ndarray:
    """RoPE op on x (S, H, d): row pos rotated by position pos (rope.c)."""
    x = np.ascontiguousarray(x, np.float32)
    S, H, d = x.shape
    out = np.zeros_like(x)
    if use_ref:
        p = RopeParams(S, d, H, base)
        rc = ref().rope_f32(_slots([x]), _slots([out]), ctypes.addressof(p), None)
    else:
        rc = lib().oracle_rope_f32(_fp(x), _fp(out), S, H, d, base)
    if rc != 0:
        raise ValueError(f"rope returned {rc}")
    return out


def mha_decode_rope(X, Kc, Vc, WQ, bQ, WK, bK, WV, bV, WO, bO, p: DecodeParams, rope_base: float,
                    seq_lens=None):
    """Decode op with RoPE on Q and K_new at the token's position; returns (Y, K_out, V_out)."""
    arrs = [np.ascontiguousarray(a, np.float32) for a in (X, Kc, Vc, WQ, bQ, WK, bK, WV, bV, WO, bO)]
    if seq_lens is not None:
        arrs.append(np.ascontiguousarray(seq_lens, np.int32))
    Y = np.zeros((p.batch_size, 1, p.hidden_size), np.float32)
    Ko = np.zeros_like(arrs[1])
    Vo = np.zeros_like(arrs[2])
    rc = lib().oracle_mha_decode_rope_f32(_slots(arrs), _slots([Y, Ko, Vo]), ctypes.addressof(p), rope_base)
    if rc != 0:
        raise ValueError(f"decode rope oracle returned {rc}")
    return Y, Ko, Vo


def causal_mask(S: int, use_ref=False) -> np.ndarray:
    m = np.zeros((S, S), np.float32)
    if use_ref:
        p = c_int64(S)
        outs = _slots([m])
        rc = ref().causal_mask_f32(_slots([m]), outs, ctypes.addressof(p), None)
        if rc != 0:
            raise ValueError(rc)
    else:
        lib().oracle_causal_mask_f32(_fp(m), S)
    return m


def cpu_op_pointer(name: str):
    """Address of an oracle operator-signature wrapper, for registering CPU ops in the
    product registry during graph tests."""
    return ctypes.cast(getattr(lib(), name), c_void_p).value
