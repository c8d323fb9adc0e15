"""Pinning the CPU oracle (oracle/oracle.c) before it is trusted as the parity checker.

1. Against the reference's own C fallback, compiled from /root/reference into oracle/_ref
   (skipped where that checkout is absent, e.g. on the GPU box): bit-exact at the
   reference tests' shapes and seeds and at random shapes inside its fixed-array limits.
2. Against golden vectors written by that build (tests/golden/, travels with the repo).
3. Closed forms and invariants that a dropped term, wrong index or transposed operand
   would break, and a float64 brute force.
"""

import os

import numpy as np
import pytest

import oracle as O
from helpers import DecodeCase, FusedCase

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference checkout not present (GPU box)")


def decode_kat_case():
    """tests/test_mha_decode.c:145-173 inputs (glibc srand/rand)."""
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
    return c


def decode_pair(c, seq_lens=None):
    p = O.decode_params(c.B, c.D, c.H, c.H_kv, c.d, c.cache_len, c.max_seq)
    a = O.mha_decode(*c.arrays(), p)
    b = O.mha_decode(*c.arrays(), p, use_ref=True)
    return a, b


# ----------------------------------------------------------------- vs reference ---

@needs_ref
def test_decode_reference_kat_bit_exact():
    c = decode_kat_case()
    a, b = decode_pair(c)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    # second step on the updated cache (test_mha_decode.c:217-242)
    c.Kc, c.Vc, c.X, c.cache_len = a[1], a[2], O.glibc_rand((1, 1, 8), 200), 1
    a2, b2 = decode_pair(c)
    for x, y in zip(a2, b2):
        assert np.array_equal(x, y)


@needs_ref
@pytest.mark.parametrize("B,H,H_kv,d,max_seq,cl", [(2, 4, 2, 16, 64, 37), (1, 12, 12, 64, 512, 511),
                                                   (3, 8, 1, 32, 100, 0), (2, 6, 3, 8, 300, 299)])
def test_decode_matches_reference_build(B, H, H_kv, d, max_seq, cl):
    c = DecodeCase(B, H, H_kv, d, max_seq, cache_len=cl, seed=B * 7 + d)
    a, b = decode_pair(c)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@needs_ref
@pytest.mark.parametrize("B,S,H,d,res", [(1, 4, 2, 8, True), (2, 16, 4, 16, False), (1, 33, 3, 8, True)])
def test_fused_matches_reference_build(B, S, H, d, res):
    c = FusedCase(B, S, H, H, d, seed=S, residual=res, bias_std=0.1)
    p = O.fused_params(B, S, H * d, H, H, d, res, False)
    a = O.mha_fused(*c.arrays(), p)
    b = O.mha_fused(*c.arrays(), p, use_ref=True)
    assert np.array_equal(a, b)


@needs_ref
def test_fused_reference_bert_kat_bit_exact():
    c = FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True)
    p = O.fused_params(1, 4, 16, 2, 2, 8, True, False)
    assert np.array_equal(O.mha_fused(*c.arrays(), p), O.mha_fused(*c.arrays(), p, use_ref=True))


@needs_ref
def test_causal_mask_matches_reference_build():
    for S in (1, 4, 17):
        assert np.array_equal(O.causal_mask(S), O.causal_mask(S, use_ref=True))


# ----------------------------------------------------------------- golden vectors ---

def _golden_files():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")) if os.path.isdir(GOLDEN) else []


def test_golden_fixtures_present():
    assert len(_golden_files()) >= 4


@pytest.mark.parametrize("fname", _golden_files())
def test_oracle_vs_golden(fname):
    z = np.load(os.path.join(GOLDEN, fname))
    kind = str(z["kind"])
    if kind == "decode":
        pv = z["params"]
        p = O.decode_params(*[int(v) for v in pv[:5]], int(pv[5]), int(pv[6]), float(z["scale"]))
        ins = [z[k] for k in ("X", "Kc", "Vc", "WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO")]
        Y, K, V = O.mha_decode(*ins, p)
        cl = int(pv[5])
        assert np.array_equal(Y, z["Y"])
        assert np.array_equal(K[:, cl], z["K_row"]) and np.array_equal(V[:, cl], z["V_row"])
        keep = np.arange(K.shape[1]) != cl
        assert np.array_equal(K[:, keep], z["Kc"][:, keep]) and np.array_equal(V[:, keep], z["Vc"][:, keep])
    elif kind == "fused":
        pv = z["params"]
        p = O.fused_params(*[int(v) for v in pv[:6]], bool(pv[6]), False, float(z["scale"]))
        R = z["R"] if bool(pv[6]) else None
        ins = [z["X"], R] + [z[k] for k in ("WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO")]
        assert np.array_equal(O.mha_fused(*ins, p), z["Y"])
    elif kind == "causal_mask":
        assert np.array_equal(O.causal_mask(int(z["S"])), z["mask"])
    else:
        pytest.fail(f"unknown fixture kind {kind}")


# ----------------------------------------------------------------- closed forms ---

def test_decode_t1_closed_form():
    """cache_len = 0: softmax over one position is 1, so Y = (x·WV + bV)·WO + bO."""
    c = DecodeCase(2, 4, 2, 8, 4, cache_len=0, seed=3, wstd=0.3)
    Y, K, V = c.oracle()
    x = c.X[:, 0].astype(np.float64)
    v = x @ c.WV.astype(np.float64) + c.bV
    merged = np.repeat(v.reshape(2, 2, 8), 2, axis=1).reshape(2, 32)
    want = merged @ c.WO.astype(np.float64) + c.bO
    assert np.max(np.abs(Y[:, 0] - want)) < 1e-5
    k = x @ c.WK.astype(np.float64) + c.bK
    assert np.max(np.abs(K[:, 0].reshape(2, 16) - k)) < 1e-5


def test_attn_identical_keys_give_mean_of_values():
    B, H, H_kv, d, T = 2, 4, 2, 16, 50
    Q = O.normal((B, H, d), 1)
    K = np.repeat(O.normal((B, 1, H_kv, d), 2), T, axis=1)
    V = O.normal((B, T, H_kv, d), 3)
    got = O.decode_attn(Q, K, V, np.full(B, T, np.int32), 0.25, H_kv)
    want = np.repeat(V.astype(np.float64).mean(axis=1), 2, axis=1)
    assert np.max(np.abs(got - want)) < 1e-5


def test_attn_one_hot_scores_select_value_row():
    B, H, d, T = 1, 2, 8, 20
    K = np.zeros((B, T, H, d), np.float32)
    K[0, 7, :, 0] = 100.0
    Q = np.zeros((B, H, d), np.float32)
    Q[..., 0] = 1.0
    V = O.normal((B, T, H, d), 4)
    got = O.decode_attn(Q, K, V, np.array([T], np.int32), 1.0, H)
    assert np.max(np.abs(got[0] - V[0, 7])) < 1e-6


def test_attn_float64_brute_force():
    B, H, H_kv, d, T = 2, 6, 3, 32, 97
    Q, K, V = O.normal((B, H, d), 5), O.normal((B, T + 3, H_kv, d), 6), O.normal((B, T + 3, H_kv, d), 7)
    scale = 1 / np.sqrt(d)
    got = O.decode_attn(Q, K, V, np.array([T, 40], np.int32), scale, H_kv)
    for b, Tb in ((0, T), (1, 40)):
        for h in range(H):
            s = K[b, :Tb, h // 2].astype(np.float64) @ Q[b, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            want = (p / p.sum()) @ V[b, :Tb, h // 2].astype(np.float64)
            assert np.max(np.abs(got[b, h] - want)) < 2e-6


# ----------------------------------------------------------------- invariants ---

def test_attn_kv_permutation_invariance():
    B, H, d, T = 1, 4, 16, 64
    Q, K, V = O.normal((B, H, d), 8), O.normal((B, T, H, d), 9), O.normal((B, T, H, d), 10)
    perm = np.random.default_rng(0).permutation(T)
    a = O.decode_attn(Q, K, V, np.array([T], np.int32), 0.25, H)
    b = O.decode_attn(Q, K[:, perm], V[:, perm], np.array([T], np.int32), 0.25, H)
    assert np.max(np.abs(a - b)) < 1e-5


def test_gqa_equals_repeated_kv_mha():
    B, H, H_kv, d, T = 2, 8, 2, 16, 30
    Q, K, V = O.normal((B, H, d), 11), O.normal((B, T, H_kv, d), 12), O.normal((B, T, H_kv, d), 13)
    g = O.decode_attn(Q, K, V, np.full(B, T, np.int32), 0.25, H_kv)
    m = O.decode_attn(Q, np.repeat(K, 4, axis=2), np.repeat(V, 4, axis=2), np.full(B, T, np.int32), 0.25, H)
    assert np.array_equal(g, m)


def test_ragged_equal_lengths_equals_uniform():
    c = DecodeCase(3, 4, 2, 16, 40, cache_len=25, seed=14)
    u = c.oracle()
    c2 = DecodeCase(3, 4, 2, 16, 40, seq_lens=[25, 25, 25], seed=14)
    r = c2.oracle()
    for x, y in zip(u, r):
        assert np.array_equal(x, y)


def test_ragged_rows_equal_per_row_uniform_runs():
    lens = [3, 17, 39]
    c = DecodeCase(3, 4, 2, 16, 40, seq_lens=lens, seed=15)
    Y, K, V = c.oracle()
    for b, L in enumerate(lens):
        cb = DecodeCase(3, 4, 2, 16, 40, cache_len=L, seed=15)
        Yb, Kb, Vb = cb.oracle()
        assert np.array_equal(Y[b], Yb[b]) and np.array_equal(K[b], Kb[b])


def test_causal_row_equals_prefix_attention():
    """Row i of a causal run equals the last row of a non-causal run over tokens 0..i."""
    c = FusedCase(1, 12, 2, 2, 8, seed=16, causal=True, bias_std=0.1, wstd=0.3)
    Yc = c.oracle()
    for i in (0, 5, 11):
        sub = FusedCase(1, i + 1, 2, 2, 8, seed=16, causal=False, bias_std=0.1, wstd=0.3)
        for n in ("WQ", "bQ", "WK", "bK", "WV", "bV", "WO", "bO"):
            setattr(sub, n, getattr(c, n))
        sub.X = c.X[:, : i + 1]
        Yp = sub.oracle()
        assert np.max(np.abs(Yc[0, i] - Yp[0, i])) < 1e-6


def test_fused_gqa_equals_repeated_weights():
    """H_kv < H with WK/WV (D, H_kv*d) equals H_kv = H with the KV head columns repeated."""
    c = FusedCase(1, 10, 4, 2, 8, seed=17, bias_std=0.1, wstd=0.3)
    Yg = c.oracle()
    rep = lambda w: np.repeat(w.reshape(w.shape[:-1] + (2, 8)), 2, axis=-2).reshape(w.shape[:-1] + (32,))
    m = FusedCase(1, 10, 4, 4, 8, seed=17)
    for n in ("X", "WQ", "bQ", "WO", "bO"):
        setattr(m, n, getattr(c, n))
    m.WK, m.bK, m.WV, m.bV = rep(c.WK), rep(c.bK), rep(c.WV), rep(c.bV)
    assert np.max(np.abs(Yg - m.oracle())) < 1e-6


def test_fused_s1_equals_decode_t1():
    """MHA_Fused with S = 1 equals MHA_Decode at cache_len = 0 (same weights and token)."""
    d, H = 8, 2
    c = DecodeCase(1, H, H, d, 2, cache_len=0, seed=18, wstd=0.3)
    Yd, _, _ = c.oracle()
    p = O.fused_params(1, 1, H * d, H, H, d)
    Yf = O.mha_fused(c.X, None, c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO, p)
    assert np.max(np.abs(Yd - Yf)) < 1e-6


def test_value_scaling_linearity():
    B, H, d, T = 1, 2, 8, 33
    Q, K, V = O.normal((B, H, d), 19), O.normal((B, T, H, d), 20), O.normal((B, T, H, d), 21)
    a = O.decode_attn(Q, K, V, np.array([T], np.int32), 0.3, H)
    b = O.decode_attn(Q, K, V * 4.0, np.array([T], np.int32), 0.3, H)
    assert np.max(np.abs(4.0 * a - b)) < 1e-5


def test_invalid_arguments_rejected():
    c = DecodeCase(1, 4, 3, 8, 8, cache_len=0)   # 4 % 3 != 0
    with pytest.raises(ValueError):
        c.oracle()
    c = DecodeCase(1, 4, 2, 8, 8, cache_len=8)   # cache_len >= max_seq
    with pytest.raises(ValueError):
        c.oracle()


# ----------------------------------------------------------------- conversions ---

def test_f16_conversion_matches_ieee_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000) * s for s in (1e-8, 1e-5, 1e-3, 1, 100, 7e4)]).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, 65504, 65520, -65520, 6.1e-5, 5.96e-8, 2.98e-8, np.inf, -np.inf],
                                    np.float32)])
    with np.errstate(over="ignore"):
        ref16 = x.astype(np.float16)
    assert np.array_equal(O.to_f16(x).view(np.uint16), ref16.view(np.uint16))
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    ok = np.isnan(ref) | (f.view(np.uint32) == ref.view(np.uint32))
    assert ok.all()


def test_generators_are_seeded_and_shaped():
    a = O.normal((1000,), 5)
    assert np.array_equal(a, O.normal((1000,), 5))
    assert abs(a.mean()) < 0.1 and abs(a.std() - 1) < 0.1
    L = O.uniform_int(1000, 3, 1024, 32768)
    assert L.min() >= 1024 and L.max() <= 32768
