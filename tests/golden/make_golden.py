#!/usr/bin/env python3
"""Writes the golden vectors in this directory from the REFERENCE'S OWN C fallback
(src/operator/nn/mha_decode.c, mha_fused.c, causal_mask.c compiled unmodified from
/root/reference into oracle/_ref/libcfref.so by oracle/Makefile).

Each .npz holds inputs and the reference's outputs; tests compare the oracle (CPU) and
the HIP operators (GPU) against them.  Inputs use the reference tests' own generators
(glibc rand for tests/test_mha_decode.c, the LCG of tests/test_bert_mha.c) or the
oracle's seeded normal generator.  Run from the repo root:
    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
from helpers import DecodeCase, FusedCase  # noqa: E402


def save_decode(name, c: DecodeCase, note):
    p = O.decode_params(c.B, c.D, c.H, c.H_kv, c.d, c.cache_len, c.max_seq)
    Y, K, V = O.mha_decode(*c.arrays(), p, use_ref=True)
    np.savez_compressed(os.path.join(HERE, name), kind="decode", note=note,
                        params=np.array([c.B, c.D, c.H, c.H_kv, c.d, c.cache_len, c.max_seq], np.int64),
                        scale=np.float32(p.scale), X=c.X, Kc=c.Kc, Vc=c.Vc, WQ=c.WQ, bQ=c.bQ, WK=c.WK, bK=c.bK,
                        WV=c.WV, bV=c.bV, WO=c.WO, bO=c.bO, Y=Y,
                        K_row=K[:, c.cache_len], V_row=V[:, c.cache_len])
    return Y, K, V


def save_fused(name, c: FusedCase, note):
    p = O.fused_params(c.B, c.S, c.D, c.H, c.H_kv, c.d, c.residual, False)
    Y = O.mha_fused(*c.arrays(), p, use_ref=True)
    R = c.R if c.R is not None else np.zeros(1, np.float32)
    np.savez_compressed(os.path.join(HERE, name), kind="fused", note=note,
                        params=np.array([c.B, c.S, c.D, c.H, c.H_kv, c.d, int(c.residual)], np.int64),
                        scale=np.float32(p.scale), X=c.X, R=R, WQ=c.WQ, bQ=c.bQ, WK=c.WK, bK=c.bK,
                        WV=c.WV, bV=c.bV, WO=c.WO, bO=c.bO, Y=Y)


def main():
    if not O.ref_available():
        sys.exit("needs oracle/_ref/libcfref.so (built from /root/reference by `make -C oracle ref`)")
    # tests/test_mha_decode.c:145-248: B=1, H=2, d=4, max_seq=8, glibc rand seeds.
    TD = 8
    c = DecodeCase(1, 2, 2, 4, 8, cache_len=0)
    c.X = O.glibc_rand((1, 1, TD), 42)
    c.WQ, c.bQ = O.glibc_rand((TD, TD), 100), O.glibc_rand((TD,), 101)
    c.WK, c.bK = O.glibc_rand((TD, TD), 102), O.glibc_rand((TD,), 103)
    c.WV, c.bV = O.glibc_rand((TD, TD), 104), O.glibc_rand((TD,), 105)
    c.WO, c.bO = O.glibc_rand((TD, TD), 106), O.glibc_rand((TD,), 107)
    c.Kc = np.zeros((1, 8, 2, 4), np.float32)
    c.Vc = np.zeros_like(c.Kc)
    Y, K, V = save_decode("decode_ref_kat_step1.npz", c, "test_mha_decode.c step 1 (cache_len=0)")
    c.Kc, c.Vc, c.X, c.cache_len = K, V, O.glibc_rand((1, 1, TD), 200), 1
    save_decode("decode_ref_kat_step2.npz", c, "test_mha_decode.c step 2 (cache_len=1, chained cache)")
    # GQA decode inside the reference's fixed-array limits (d <= 64, T <= 512).
    save_decode("decode_gqa_b1_h4x2_d32_t300.npz", DecodeCase(1, 4, 2, 32, 300, cache_len=299, seed=31),
                "GQA 4/2 heads, d=32, 300 attended positions, N(0,1) caches, N(0,0.02) weights")
    save_decode("decode_mha_b1_h4_d16_t512.npz", DecodeCase(1, 4, 4, 16, 512, cache_len=511, seed=32),
                "MHA 4 heads, d=16, 512 attended positions (the reference's scores[512] limit)")
    # tests/test_bert_mha.c:36-40,205-216: B=1, S=4, H=2, d=8, LCG seeds, residual on.
    save_fused("fused_ref_bert_kat.npz", FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True),
               "test_bert_mha.c CPU test inputs (LCG seeds 42,99,123,...), residual")
    save_fused("fused_b2_s24_h3_d16.npz", FusedCase(2, 24, 3, 3, 16, seed=33, bias_std=0.05),
               "B=2, S=24, H=3, d=16, N(0,1) X, N(0,0.02) weights, N(0,0.05) biases, no residual")
    m = O.causal_mask(6, use_ref=True)
    np.savez_compressed(os.path.join(HERE, "causal_mask_s6.npz"), kind="causal_mask", S=np.int64(6), mask=m,
                        note="causal_mask.c S=6")
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
