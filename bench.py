#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path; prints ONE JSON line.

Headline (`value`): split-KV decode attention at BASELINE config 2 (MHA_Decode GQA,
Llama-3-8B shape: B=16, 32 query / 8 KV heads, d=128, KV length 4096, fp16 cache,
fp32 softmax/accumulate), as achieved HBM GB/s = algorithmic bytes / time per step.
One step = one call of the mha_decode_attn_f16_cuda operator (split kernel + merge
kernel).  The steps rotate over independent KV sets whose total is beyond the 256 MB
Infinity Cache, so each step reads its cache from HBM.  `roofline` is the split kernel
alone, timed with HIP events around its launches on the op's stream (cross-checked by
the rocprofv3 summaries in profiles/).

Also reported (`extra`): the full MHA_Decode op at config 2 (projections + append +
attention + output projection), decode config 1 (FP32, GPT-2 small), config 4 (ragged
long context), and fused prefill configs 3 (BERT-base) and 5 (causal GPT-2 medium) in
TFLOP/s against the fp16 MFMA peak.  `cpu_baseline` times the CPU oracle (a C port of the
reference fallback, single thread) on a bounded sample of the same decode workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "split-KV decode µs/step + HBM GB/s; fused MHA prefill TFLOP/s (fp16)"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_op(cf, name, inputs, outputs, params, stream, steps, warmup, extra=()):
    """Average ms per call over `steps` back-to-back calls on `stream`, timed by HIP
    events in the library's C loop (operator_time), after `warmup` untimed calls."""
    from cudaforge_amd.api import time_op as _t
    return _t(name, inputs, outputs, params, stream, warmup, steps, extra_inputs=extra)


def dnormal(cf, shape, seed, std=1.0, f16=True):
    """Seeded N(0, std) synthetic data made on the device: splitmix64 + Box-Muller
    (synthetic_fill_normal), the generator the CPU baseline's oracle inputs come from, so
    a seed names the same values in both legs.  The GPU legs never call the oracle."""
    return cf.DeviceBuffer.normal(shape, np.float16 if f16 else np.float32, seed, std)


def splitmix_uniform_int(n, seed, lo, hi):
    """n integers lo + (splitmix64 output % (hi - lo + 1)) from one sequence seeded with
    `seed` (the oracle's oracle_fill_uniform_int, restated so the GPU legs need no oracle)."""
    mask = (1 << 64) - 1
    st, out = seed & mask, []
    for _ in range(n):
        st = (st + 0x9E3779B97F4A7C15) & mask
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        out.append(lo + z % (hi - lo + 1))
    return np.array(out, np.int64)


# Seeds of every synthetic tensor, written into the JSON line.
SEEDS = {
    "config2_core": "set i (0..2): Q 101+10i, K 102+10i, V 103+10i",
    "config2_full_op": "set i: base 200+100i; X base+1, K base+2, V base+3, WQ base+4, WK base+6, WV base+8, "
                       "WO base+10 (weights std 0.02, biases 0)",
    "config1_full_op_f32": "base 200: as config2_full_op, set 0 only",
    "config4_ragged": "lengths splitmix64 seed 404 uniform in [1024, 32768]; set i: Q 401+10i, K 402+10i, V 403+10i",
    "config3_prefill": "base 300: X base+1, WQ/WK/WV/WO base+2..5 (std 0.02), biases 0",
    "config5_prefill": "base 500: as config3_prefill",
    "layer_neighbours": "base 900",
    "generator": "splitmix64 + Box-Muller (both outputs), fp16 by round-to-nearest-even from fp32",
}


# Independent input sets the decode legs rotate over: 3 x 268 MB of KV cache (plus the
# weights, for the full op) is far beyond MI355X's 256 MB Infinity Cache, so every step
# reads its KV cache from HBM, as it does in a model whose other layers run in between.
# (Timing one set in a loop lets part of it be served from that cache: ~15 % faster.)
KV_SETS = 3


STAT_REPS = 9   # extra timed loops of K steps behind the median / min figures


def step_stats(cf, name, sets, out_sets, p, stream, steps):
    """Median and min of the per-step mean over STAT_REPS further timed loops of `steps`
    back-to-back steps each (events around each loop, no per-step events, which would
    add their own gaps between launches)."""
    from cudaforge_amd.api import time_op_sets
    v = sorted(time_op_sets(name, sets, out_sets, p, stream, 1, steps) for _ in range(STAT_REPS))
    return v[len(v) // 2], v[0]


def bench_decode_core(cf, stream, steps, warmup):
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    sets = [[dnormal(cf, (B, H, d), 101 + 10 * i), dnormal(cf, (B, T, H_kv, d), 102 + 10 * i),
             dnormal(cf, (B, T, H_kv, d), 103 + 10 * i)] for i in range(KV_SETS)]
    O_ = cf.DeviceBuffer.empty((B, H, d), np.float16)
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1 / np.sqrt(d)), T - 1, T)
    from cudaforge_amd.api import time_op_sets
    ms = time_op_sets("mha_decode_attn_f16_cuda", sets, [[O_]] * KV_SETS, p, stream, warmup, steps)
    med, mn = step_stats(cf, "mha_decode_attn_f16_cuda", sets, [[O_]] * KV_SETS, p, stream, steps)
    ms_split, ms_merge = kernel_times(cf, sets, [O_], p, stream, min(steps, 1000), warmup)
    kv_bytes = 2 * B * T * H_kv * d * 2
    alg_bytes = kv_bytes + 2 * B * H * d * 2
    chunk, n_split = plan(cf, p)
    return ms, (med, mn), ms_split, ms_merge, alg_bytes, dict(B=B, H_q=H, H_kv=H_kv, d=d, kv_len=T, chunk=chunk,
                                                              n_split=n_split, kv_sets=KV_SETS)


def kernel_times(cf, input_sets, outputs, params, stream, iters, warmup, f16=True):
    """Mean duration of the split kernel and of the merge kernel (HIP events around
    each launch, on the stream they run on), rotating over the input sets."""
    import ctypes
    from ctypes import POINTER, c_float, c_void_p
    from cudaforge_amd.api import _ptr
    lib = cf.load_library()
    flat = [_ptr(x) for s in input_sets for x in s]
    ins = (c_void_p * len(flat))(*flat)
    outs = (c_void_p * len(outputs))(*[_ptr(x) for x in outputs])
    a, b = c_float(0), c_float(0)
    rc = lib.mha_decode_attn_kernel_times(ctypes.cast(ins, POINTER(c_void_p)), len(input_sets[0]), len(input_sets),
                                          ctypes.cast(outs, POINTER(c_void_p)), ctypes.addressof(params),
                                          stream.stream_t(), 1 if f16 else 0, warmup, iters,
                                          ctypes.byref(a), ctypes.byref(b))
    if rc != 0:
        raise RuntimeError(f"mha_decode_attn_kernel_times returned {rc}")
    return a.value, b.value


def plan(cf, params, f16=True):
    import ctypes
    lib = cf.load_library()
    c, n = ctypes.c_int64(0), ctypes.c_int64(0)
    lib.mha_decode_plan(ctypes.addressof(params), 1 if f16 else 0, ctypes.byref(c), ctypes.byref(n))
    return int(c.value), int(n.value)


def bench_decode_full(cf, stream, steps, warmup, f16=True, B=16, H=32, H_kv=8, d=128, T=4096, seed=200, n_sets=1,
                      rope_base=None):
    D, kvd = H * d, H_kv * d
    dt = np.float16 if f16 else np.float32

    def mk(shape, s, std=1.0):
        return dnormal(cf, shape, s, std, f16)

    input_sets, output_sets = [], []
    for i in range(n_sets):
        b = seed + 100 * i
        ins = [mk((B, 1, D), b + 1), mk((B, T, H_kv, d), b + 2), mk((B, T, H_kv, d), b + 3),
               mk((D, D), b + 4, 0.02), cf.DeviceBuffer.from_numpy(np.zeros(D, dt)),
               mk((D, kvd), b + 6, 0.02), cf.DeviceBuffer.from_numpy(np.zeros(kvd, dt)),
               mk((D, kvd), b + 8, 0.02), cf.DeviceBuffer.from_numpy(np.zeros(kvd, dt)),
               mk((D, D), b + 10, 0.02), cf.DeviceBuffer.from_numpy(np.zeros(D, dt))]
        input_sets.append(ins)
        # In-place cache update (outputs alias the input caches), the decode-loop use.
        output_sets.append([cf.DeviceBuffer.empty((B, 1, D), dt), ins[1], ins[2]])
    p = cf.MhaDecodeParams(B, D, H, H_kv, d, float(1 / np.sqrt(d)), T - 1, T)
    name = "mha_decode_f16_cuda" if f16 else "mha_decode_f32_cuda"
    if rope_base is not None:
        p = cf.MhaDecodeRopeParams(p, rope_base, 0)
        name = name.replace("mha_decode_", "mha_decode_rope_")
    from cudaforge_amd.api import time_op_sets
    ms = time_op_sets(name, input_sets, output_sets, p, stream, warmup, steps)
    med, mn = step_stats(cf, name, input_sets, output_sets, p, stream, steps)
    esz = 2 if f16 else 4
    alg = (2 * B * T * kvd + (D * D * 2 + 2 * D * kvd) + 2 * D + 2 * kvd + 2 * B * D + 2 * B * kvd) * esz
    return ms, alg, (med, mn)


def bench_decode_ragged(cf, stream, steps, warmup):
    B, H, H_kv, d, cap = 4, 32, 8, 128, 32768
    # Attended lengths L_b ~ U[1024, 32768] from a seed; cache_len_b = L_b - 1.
    lens = (ragged_lengths(B, cap) - 1).astype(np.int32)
    L = cf.DeviceBuffer.from_numpy(lens)
    sets = [[dnormal(cf, (B, H, d), 401 + 10 * i), dnormal(cf, (B, cap, H_kv, d), 402 + 10 * i),
             dnormal(cf, (B, cap, H_kv, d), 403 + 10 * i), L] for i in range(KV_SETS)]
    O_ = cf.DeviceBuffer.empty((B, H, d), np.float16)
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, float(1 / np.sqrt(d)), -1, cap)
    from cudaforge_amd.api import time_op_sets
    ms = time_op_sets("mha_decode_attn_f16_cuda", sets, [[O_]] * KV_SETS, p, stream, warmup, steps)
    med, mn = step_stats(cf, "mha_decode_attn_f16_cuda", sets, [[O_]] * KV_SETS, p, stream, steps)
    ms_split, ms_merge = kernel_times(cf, sets, [O_], p, stream, min(steps, 1000), warmup)
    alg = int(4096 * int((lens.astype(np.int64) + 1).sum()) + 2 * B * H * d * 2)
    return ms, alg, [int(x) + 1 for x in lens], ms_split, ms_merge, (med, mn)


def ragged_lengths(B=4, cap=32768):
    """Config 4's attended lengths: splitmix64 seed 404, uniform in [1024, cap]."""
    return splitmix_uniform_int(B, 404, 1024, cap)


def bench_decode_graph(cf, steps, warmup, B=16, H=32, H_kv=8, d=128, T=4096, seed=700, replay=True):
    """Config-2 decode through the graph executor, the host-buffer boundary: each step
    copies X_new host->device, runs the MHA_Decode node against device-resident in-place
    KV caches (graph_set_kv_cache), synchronises and copies Y back (graph.c:670-1115 is
    the reference executor).  Host wall-clock per step, PCIe transfers included."""
    import ctypes
    from ctypes import POINTER, c_int, c_int64, c_void_p
    lib = cf.load_library()
    D, kvd = H * d, H_kv * d
    g = lib.graph_create()

    def tensor(arr):
        arr = np.ascontiguousarray(arr)
        shape = (c_int64 * arr.ndim)(*arr.shape)
        t = lib.tensor_create(1, arr.ndim, shape)                 # DTYPE_F16
        tt = ctypes.cast(t, POINTER(cf.TensorT)).contents
        ctypes.memmove(tt.data, arr.ctypes.data, arr.nbytes)
        return t, lib.graph_add_tensor(g, t)

    mk = (lambda shape, s, std=1.0: dnormal(cf, shape, seed + s, std).download())
    tX, iX = tensor(mk((B, 1, D), 1))
    _, iK = tensor(mk((B, T, H_kv, d), 2))
    _, iV = tensor(mk((B, T, H_kv, d), 3))
    tY, iY = tensor(np.zeros((B, 1, D), np.float16))
    ws = [tensor(w)[0] for w in (mk((D, D), 4, 0.02), np.zeros(D, np.float16), mk((D, kvd), 6, 0.02),
                                 np.zeros(kvd, np.float16), mk((D, kvd), 8, 0.02), np.zeros(kvd, np.float16),
                                 mk((D, D), 10, 0.02), np.zeros(D, np.float16))]
    cl0 = T - 1 - (warmup + steps)
    p = cf.MhaDecodeParams(B, D, H, H_kv, d, float(1 / np.sqrt(d)), cl0, T)
    node = lib.graph_add_node(g, 29, 3, (c_int * 3)(iX, iK, iV), 3, (c_int * 3)(iY, iK, iV), 8,
                              (c_void_p * 8)(*ws), ctypes.addressof(p), ctypes.sizeof(p))
    if node < 0:
        raise RuntimeError("graph_add_node failed")
    lib.graph_set_input(g, lib.graph_add_node(g, 36, 0, None, 1, (c_int * 1)(iX), 0, None, None, 0))
    lib.graph_set_output(g, lib.graph_add_node(g, 37, 1, (c_int * 1)(iY), 0, None, 0, None, None, 0))
    lib.graph_set_kv_cache(g, iK, iV)
    if lib.graph_build(g) != 0:
        raise RuntimeError("graph_build failed")
    if not replay:
        lib.graph_set_replay(g, 0)
    ins, outs = (c_void_p * 1)(tX), (c_void_p * 1)(tY)
    t_start, cl = None, cl0
    for i in range(warmup + steps):
        if i == warmup:
            t_start = time.perf_counter()
        lib.graph_update_cache_len(g, cl)
        if lib.graph_execute(g, ins, outs, True) != 0:
            raise RuntimeError("graph_execute failed")
        cl += 1
    ms = (time.perf_counter() - t_start) * 1e3 / steps
    lib.graph_destroy(g)
    return ms


def bench_layer_neighbours(cf, stream, steps, warmup, rows=4096, D=768, F=3072, seed=900):
    """LayerNorm (F16, BERT-base rows) and the FFN MatMul (F16, rows x D -> F with bias)."""
    x = dnormal(cf, (rows, D), seed)
    g = dnormal(cf, (D,), seed + 1, 0.1)
    b = dnormal(cf, (D,), seed + 2, 0.1)
    y = cf.DeviceBuffer.empty((rows, D), np.float16)
    ms_ln = time_op(cf, "layernorm_f16_cuda", [x, g, b], [y], cf.LayerNormParams(rows, D, 1e-12), stream, steps, warmup)
    W = dnormal(cf, (D, F), seed + 3, 0.02)
    bias = dnormal(cf, (F,), seed + 4, 0.02)
    C = cf.DeviceBuffer.empty((rows, F), np.float16)
    p = cf.MatmulParams(rows, F, D, False, False, 1, 0, 0, 0, 0)
    ms_mm = time_op(cf, "matmul_f16_cuda", [x, W, bias], [C], p, stream, steps, warmup)
    return ms_ln, 2 * rows * D * 2 + 2 * D * 2, ms_mm, 2 * rows * D * F


def fused_kernel_times(cf, ins, outs, params, stream, f16, iters, warmup):
    """Mean time per launch of the fused op's three kernels (QKV GEMM, attention, WO
    GEMM), each launched back to back between HIP events on the op's stream."""
    import ctypes
    from ctypes import POINTER, c_float, c_void_p
    from cudaforge_amd.api import _ptr
    lib = cf.load_library()
    ia = (c_void_p * len(ins))(*[_ptr(x) for x in ins])
    oa = (c_void_p * len(outs))(*[_ptr(x) for x in outs])
    ms = (c_float * 3)()
    rc = lib.mha_fused_kernel_times(ctypes.cast(ia, POINTER(c_void_p)), ctypes.cast(oa, POINTER(c_void_p)),
                                    ctypes.addressof(params), stream.stream_t(), 1 if f16 else 0, warmup, iters, ms)
    if rc != 0:
        raise RuntimeError(f"mha_fused_kernel_times returned {rc}")
    return [ms[0], ms[1], ms[2]]


def bench_fused(cf, stream, steps, warmup, B, S, H, d, causal, seed, f16=True):
    """The fused op at one shape: ms per call, the algorithmic FLOPs, and per kernel
    (QKV GEMM, attention, WO GEMM) its time and algorithmic FLOPs."""
    D = H * d
    dt = np.float16 if f16 else np.float32
    mk = (lambda shape, s, std=1.0: dnormal(cf, shape, seed + s, std, f16))
    zero = (lambda n: cf.DeviceBuffer.from_numpy(np.zeros(n, dt)))
    ins = [mk((B, S, D), 1), None, mk((D, D), 2, 0.02), zero(D), mk((D, D), 3, 0.02), zero(D),
           mk((D, D), 4, 0.02), zero(D), mk((D, D), 5, 0.02), zero(D)]
    Y = cf.DeviceBuffer.empty((B, S, D), dt)
    p = cf.MhaFusedParams(B, S, D, H, H, d, float(1 / np.sqrt(d)), False, causal)
    name = "mha_fused_f16io_cuda" if f16 else "mha_fused_f32_cuda"
    ms = time_op(cf, name, ins, [Y], p, stream, steps, warmup)
    st = sorted(time_op(cf, name, ins, [Y], p, stream, steps, 1) for _ in range(STAT_REPS))
    kms = fused_kernel_times(cf, ins, [Y], p, stream, f16, steps, warmup)
    pairs = B * H * (S * (S + 1) // 2 if causal else S * S)
    kfl = [2 * B * S * D * 3 * D, 4 * pairs * d, 2 * B * S * D * D]
    return ms, sum(kfl), kms, kfl, (st[len(st) // 2], st[0])


def cpu_baseline_decode(budget_s: float):
    """Oracle (C port of mha_decode.c's attention loop, single thread) on config-2 inputs,
    on as many batch rows as fit the time budget; scaled to the full step."""
    import oracle as O
    B, H, H_kv, d, T = 16, 32, 8, 128, 4096
    rows = 1
    Q = O.round_f16(O.normal((rows, H, d), 101))
    K = O.round_f16(O.normal((rows, T, H_kv, d), 102))
    V = O.round_f16(O.normal((rows, T, H_kv, d), 103))
    att = np.full(rows, T, np.int32)
    scale = float(1 / np.sqrt(d))
    t0 = O.now()
    n = 0
    while True:
        O.decode_attn(Q, K, V, att, scale, H_kv)
        n += 1
        if O.now() - t0 >= budget_s:
            break
    per_row = (O.now() - t0) / n
    step_s = per_row * B
    alg_bytes = 2 * B * T * H_kv * d * 2 + 2 * B * H * d * 2
    return {
        "value": round(alg_bytes / step_s / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(step_s * 1e6, 1),
        "cores": 1,
        "kind": "port",
        "sample": f"{n} x 1 of 16 batch rows of config 2 (32/8 heads, d=128, KV 4096), fp16 values as fp32, "
                  f"scaled x16 to one step; oracle/oracle.c decode_attn, -O3, 1 thread "
                  f"(host has {os.cpu_count()} logical CPUs)",
    }


def _cpu_time(fn, budget_s, min_runs=1):
    """Seconds per call of fn, repeated until budget_s has passed (at least min_runs)."""
    import oracle as O
    t0 = O.now()
    n = 0
    while n < min_runs or O.now() - t0 < budget_s:
        fn()
        n += 1
    return (O.now() - t0) / n, n


def cpu_baseline_configs(budget_s: float) -> dict:
    """The CPU oracle (C port of the reference fallbacks, -O3, one thread) on configs 1,
    3, 4 and 5, each on a bounded sample scaled to one step, beside the GPU figures."""
    import oracle as O
    out = {}
    cores = os.cpu_count()
    # Config 1: the full MHA_Decode FP32 op (mha_decode.c:11-125 restated), whole step.
    B, H, d, T = 1, 12, 64, 1024
    D = H * d
    args = [O.normal((B, 1, D), 201), O.normal((B, T, H, d), 202), O.normal((B, T, H, d), 203),
            O.normal((D, D), 204, 0, 0.02), np.zeros(D, np.float32), O.normal((D, D), 206, 0, 0.02),
            np.zeros(D, np.float32), O.normal((D, D), 208, 0, 0.02), np.zeros(D, np.float32),
            O.normal((D, D), 210, 0, 0.02), np.zeros(D, np.float32)]
    p = O.decode_params(B, D, H, H, d, T - 1, T)
    sec, n = _cpu_time(lambda: O.mha_decode(*args, p), budget_s / 4, 3)
    alg = (2 * B * T * H * d + 4 * D * D + 4 * D + 2 * B * D + 2 * B * H * d) * 4
    out["config1_decode_full_op_f32"] = {"us_per_step": round(sec * 1e6, 1), "GB_s": round(alg / sec / 1e9, 3),
                                         "cores": 1, "kind": "port",
                                         "sample": f"{n} whole steps (includes the reference's per-call cache copy)"}
    # Config 4: ragged core, one batch row (length 10639 of the seed-404 draw), scaled by
    # the total attended length.
    lens = ragged_lengths()
    L = int(lens[1])
    Q = O.round_f16(O.normal((1, 32, 128), 401))
    K = O.round_f16(O.normal((1, L, 8, 128), 402))
    V = O.round_f16(O.normal((1, L, 8, 128), 403))
    sec, n = _cpu_time(lambda: O.decode_attn(Q, K, V, np.array([L], np.int32), float(1 / np.sqrt(128)), 8),
                       budget_s / 4, 1)
    step = sec * float(lens.sum()) / L
    alg = 4096 * int(lens.sum()) + 2 * 4 * 32 * 128 * 2
    out["config4_decode_core_ragged"] = {"us_per_step": round(step * 1e6, 1), "GB_s": round(alg / step / 1e9, 3),
                                         "cores": 1, "kind": "port",
                                         "sample": f"{n} x batch row 1 (L={L}) of 4, scaled by sum(L)/L = "
                                                   f"{float(lens.sum()) / L:.3f}"}
    # Configs 3 and 5: the fused op on one batch row, scaled by B.
    for key, (Bc, S, H, d, causal, base) in {"config3_prefill_bert_base": (8, 512, 12, 64, False, 300),
                                             "config5_prefill_causal_gpt2_medium": (4, 1024, 16, 64, True, 500)}.items():
        D = H * d
        X = O.round_f16(O.normal((1, S, D), base + 1))
        Ws = [O.round_f16(O.normal((D, D), base + 2 + i, 0, 0.02)) for i in range(4)]
        z = np.zeros(D, np.float32)
        pf = O.fused_params(1, S, D, H, H, d, False, causal)
        sec, n = _cpu_time(lambda: O.mha_fused(X, None, Ws[0], z, Ws[1], z, Ws[2], z, Ws[3], z, pf), 0.0, 1)
        step = sec * Bc
        pairs = Bc * H * (S * (S + 1) // 2 if causal else S * S)
        fl = 2 * Bc * S * D * D * 4 + 4 * pairs * d
        out[key] = {"us_per_step": round(step * 1e6, 1), "GFLOP_s": round(fl / step / 1e9, 3), "cores": 1,
                    "kind": "port", "sample": f"{n} x 1 of {Bc} batch rows, scaled x{Bc}; fp16 values as fp32"}
    for v in out.values():
        v["host_logical_cpus"] = cores
    return out


def read_traffic(kernel_prefix: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(ROOT, "profiles", f"{kernel_prefix}_decode_config2_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            d = json.load(f)
        return d.get("hbm_bytes_per_launch")
    except Exception:
        return None


def vendor_comparison(reps: int = 50) -> dict:
    """The same prefill shapes through the vendor libraries, for context only (not the
    product path): torch.matmul on fp16 (hipBLASLt on ROCm) for the plain projection
    products, and torch's scaled_dot_product_attention for the attention.  Events on
    torch's current stream."""
    import torch
    import torch.nn.functional as F
    dev = "cuda"
    out = {}

    def timed(fn, n):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    g = torch.Generator(device=dev).manual_seed(0)
    for name, (M, K, N) in {"config3_qkv": (4096, 768, 2304), "config3_wo": (4096, 768, 768),
                            "config5_qkv": (4096, 1024, 3072), "config5_wo": (4096, 1024, 1024)}.items():
        a = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
        w = torch.randn(K, N, device=dev, dtype=torch.float16, generator=g)
        us = timed(lambda: a @ w, reps)
        out[f"matmul_{name}"] = {"M": M, "K": K, "N": N, "us": round(us, 2),
                                 "TFLOP_s": round(2 * M * N * K / us / 1e6, 1)}
    for name, (B, H, S, d, causal) in {"config3": (8, 12, 512, 64, False),
                                       "config5": (4, 16, 1024, 64, True)}.items():
        q, k, v = (torch.randn(B, H, S, d, device=dev, dtype=torch.float16, generator=g) for _ in range(3))
        us = timed(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal), 20)
        pairs = B * H * (S * (S + 1) // 2 if causal else S * S)
        out[f"sdpa_{name}"] = {"B": B, "H": H, "S": S, "d": d, "causal": causal, "us": round(us, 2),
                               "TFLOP_s": round(4 * pairs * d / us / 1e6, 1)}
    return out


def bench_prefill(cf, stream, steps, warmup, fp32=True) -> dict:
    """Configs 3 and 5 through mha_fused_f16io_cuda (fp16 buffers), and config 3's shape through the FP32
    entry (mha_fused_f32_cuda, fp32 MFMA): TFLOP/s over the algorithmic FLOPs, with a
    roofline block per config (the whole op and each of its three kernels, timed in this
    run) against the dense MFMA peak of the arithmetic type."""
    out = {}
    legs = {"prefill_config3_bert_base_f16": (8, 512, 12, 64, False, 300, True),
            "prefill_config5_causal_gpt2_medium_f16": (4, 1024, 16, 64, True, 500, True)}
    if fp32:
        legs["prefill_config3_bert_base_f32"] = (8, 512, 12, 64, False, 300, False)
    for key, (B, S, H, d, causal, seed, f16) in legs.items():
        log(key)
        n = max(steps, 10) if f16 else max(steps // 20, 5)
        ms_p, fl, kms, kfl, (med, mn) = bench_fused(cf, stream, n, max(warmup // 2, 3), B, S, H, d, causal, seed, f16)
        peak = FP16_PEAK_TFLOPS if f16 else FP32_PEAK_TFLOPS
        tf = fl / (ms_p * 1e-3) / 1e12
        kernels = {}
        for kname, kt, kf in zip(("qkv_gemm", "attention", "wo_gemm"), kms, kfl):
            ktf = kf / (kt * 1e-3) / 1e12
            kernels[kname] = {"us": round(kt * 1e3, 2), "alg_flop": kf, "TFLOP_s": round(ktf, 1),
                              "frac": round(ktf / peak, 4)}
        out[key] = {"us_per_step": round(ms_p * 1e3, 2), "us_per_step_median": round(med * 1e3, 2),
                    "us_per_step_min": round(mn * 1e3, 2), "TFLOP_s": round(tf, 1), "alg_flop": fl,
                    "mfma_frac": round(tf / peak, 4),
                    "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": peak, "unit": "TFLOP/s",
                                 "frac": round(tf / peak, 4), "dtype": "f16" if f16 else "f32",
                                 "kernel_sum_us": round(sum(kms) * 1e3, 2), "kernels": kernels}}
        log(f"  {ms_p * 1e3:.1f} us/step (median {med * 1e3:.1f}, min {mn * 1e3:.1f}) {tf:.1f} TFLOP/s; kernels " +
            ", ".join(f"{k} {v['us']} us ({v['frac']:.3f})" for k, v in kernels.items()))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU oracle timing")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-core", action="store_true", help="time only the headline kernel (for profiling)")
    ap.add_argument("--only-prefill", action="store_true",
                    help="time only the two prefill configs and print their figures (for counter runs)")
    ap.add_argument("--vendor", action="store_true",
                    help="only time the prefill shapes through torch (hipBLASLt matmul, SDPA) for comparison")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 5 device-to-device copies of 256 MiB: the known-size reference that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one MI355X only; multi-GPU runs are out of scope "
                                   "(--gpus must be 1)", "n_gpus": args.gpus}))
        return 2

    if args.vendor:
        print(json.dumps({"vendor_comparison": vendor_comparison()}), flush=True)
        return 0

    import cudaforge_amd as cf
    cf.init_gpu(0)
    caps = cf.device_caps(0)
    log(f"device {caps.name.decode()} {caps.arch.decode()} CUs={caps.cu_count}")
    stream = cf.Stream()
    steps, warmup = args.steps, args.warmup
    if args.copy_calibration:
        lib = cf.load_library()
        n = 256 << 20
        src, dst = cf.DeviceBuffer(n), cf.DeviceBuffer(n)
        src.fill_zero(stream)
        for _ in range(5):
            if lib.gpu_memcpy_d2d(dst.ptr, src.ptr, n, stream.handle) != 0:
                raise RuntimeError("calibration copy failed")
        stream.synchronize()
        log(f"calibration: 5 copies of {n} bytes")

    if args.only_prefill:
        print(json.dumps({"prefill": bench_prefill(cf, stream, steps, warmup)}), flush=True)
        return 0

    log("decode core, config 2")
    ms, (ms_med, ms_min), ms_split, ms_merge, alg_bytes, cfg = bench_decode_core(cf, stream, steps, warmup)
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    gbs_split = alg_bytes / (ms_split * 1e-3) / 1e9
    log(f"  {ms * 1e3:.2f} us/step (median {ms_med * 1e3:.2f}, min {ms_min * 1e3:.2f})  {gbs:.0f} GB/s; "
        f"split kernel {ms_split * 1e3:.2f} us ({gbs_split:.0f} GB/s), merge kernel {ms_merge * 1e3:.2f} us")
    extra = {}
    if not args.only_core:
        log("decode full op, config 2")
        ms_f, alg_f, st_f = bench_decode_full(cf, stream, steps, warmup, n_sets=KV_SETS)
        extra["decode_full_op_config2_f16"] = {"us_per_step": round(ms_f * 1e3, 2),
                                               "us_per_step_median": round(st_f[0] * 1e3, 2),
                                               "us_per_step_min": round(st_f[1] * 1e3, 2),
                                               "GB_s": round(alg_f / (ms_f * 1e-3) / 1e9, 1),
                                               "hbm_frac": round(alg_f / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                               "alg_bytes": alg_f}
        log(f"  {ms_f * 1e3:.2f} us/step")
        log("decode full op with RoPE (base 500000), config 2")
        ms_fr, _, st_fr = bench_decode_full(cf, stream, steps, warmup, n_sets=KV_SETS, rope_base=500000.0)
        extra["decode_full_op_config2_f16_rope"] = {"us_per_step": round(ms_fr * 1e3, 2),
                                                    "us_per_step_median": round(st_fr[0] * 1e3, 2),
                                                    "us_per_step_min": round(st_fr[1] * 1e3, 2),
                                                    "GB_s": round(alg_f / (ms_fr * 1e-3) / 1e9, 1),
                                                    "hbm_frac": round(alg_f / (ms_fr * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                                    "alg_bytes": alg_f}
        log(f"  {ms_fr * 1e3:.2f} us/step")
        log("decode through graph_execute, config 2 (host X/Y)")
        ms_g = bench_decode_graph(cf, 50, 5)
        extra["decode_graph_config2_f16"] = {"us_per_step": round(ms_g * 1e3, 2),
                                             "note": "graph_execute per step: X_new H2D + op + sync + Y D2H, "
                                                     "host wall-clock, KV caches device-resident"}
        log(f"  {ms_g * 1e3:.2f} us/step")
        log("decode full op, config 1 (fp32)")
        ms_1, alg_1, st_1 = bench_decode_full(cf, stream, steps, warmup, f16=False, B=1, H=12, H_kv=12, d=64,
                                              T=1024)
        extra["decode_full_op_config1_f32"] = {"us_per_step": round(ms_1 * 1e3, 2),
                                               "us_per_step_median": round(st_1[0] * 1e3, 2),
                                               "us_per_step_min": round(st_1[1] * 1e3, 2),
                                               "GB_s": round(alg_1 / (ms_1 * 1e-3) / 1e9, 1),
                                               "alg_bytes": alg_1}
        log("decode ragged, config 4")
        ms_r, alg_r, lens, ms_rs, ms_rm, st_r = bench_decode_ragged(cf, stream, steps, warmup)
        extra["decode_core_config4_ragged"] = {"us_per_step": round(ms_r * 1e3, 2),
                                               "us_per_step_median": round(st_r[0] * 1e3, 2),
                                               "us_per_step_min": round(st_r[1] * 1e3, 2),
                                               "GB_s": round(alg_r / (ms_r * 1e-3) / 1e9, 1),
                                               "alg_bytes": alg_r, "lengths": lens,
                                               "hbm_frac": round(alg_r / (ms_r * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                               "split_kernel_us": round(ms_rs * 1e3, 2),
                                               "merge_kernel_us": round(ms_rm * 1e3, 2)}
        log(f"  config 4: {ms_r * 1e3:.2f} us/step; split {ms_rs * 1e3:.2f} us, merge {ms_rm * 1e3:.2f} us")
        extra.update(bench_prefill(cf, stream, steps, warmup))
        log("layer neighbours: LayerNorm F16 (4096 x 768), FFN MatMul F16 (4096 x 768 -> 3072)")
        ms_ln, by_ln, ms_mm, fl_mm = bench_layer_neighbours(cf, stream, max(steps // 4, 10), max(warmup // 2, 3))
        extra["layernorm_f16_4096x768"] = {"us_per_step": round(ms_ln * 1e3, 2),
                                           "GB_s": round(by_ln / (ms_ln * 1e-3) / 1e9, 1), "alg_bytes": by_ln}
        extra["matmul_f16_ffn_4096x768x3072"] = {"us_per_step": round(ms_mm * 1e3, 2),
                                                 "TFLOP_s": round(fl_mm / (ms_mm * 1e-3) / 1e12, 1), "alg_flop": fl_mm}
        log(f"  LayerNorm {ms_ln * 1e3:.2f} us, MatMul {ms_mm * 1e3:.2f} us")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline_decode(args.cpu_budget)
        if not args.only_core:
            log("cpu baseline, configs 1, 3, 4, 5")
            extra["cpu_baseline_configs"] = cpu_baseline_configs(args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "us_per_step_median": round(ms_med * 1e3, 2),
        "us_per_step_min": round(ms_min * 1e3, 2),
        "step_stats": f"median and min of the per-step mean over {STAT_REPS} further timed loops of "
                      f"{steps} back-to-back steps",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": f"synthetic (seeded N(0,1) fp16 Q/K/V made on the device by splitmix64 + Box-Muller, seeds "
                f"in `seeds`; resident in HBM; {KV_SETS} independent KV sets rotated per step, beyond the 256 MB "
                "Infinity Cache)",
        "config": {"workload": "MHA_Decode GQA Llama-3-8B attention core (config 2): split-KV + LSE merge "
                               "(split kernel + merge kernel per step)", **cfg},
        "roofline": {"bound": "hbm", "achieved": round(gbs_split, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_split / HBM_PEAK_GBS, 4), "traffic": read_traffic("split_f16_kv"),
                     "kernel": "split_f16_kv<128,4> (decode_attn.hip; a workgroup per (split, batch row), a wave per KV "
                               "head, K loaded into registers, V through a 4-stage LDS ring)",
                     "alg_bytes_per_launch": alg_bytes,
                     "kernel_us": round(ms_split * 1e3, 2), "merge_kernel_us": round(ms_merge * 1e3, 2),
                     "step": {"what": "the whole step (split + merge launches), as `value`",
                              "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "us": round(ms * 1e3, 2)}},
        "cpu_baseline": cpu,
        "seeds": SEEDS,
        "extra": extra,
        "device": {"name": caps.name.decode(), "arch": caps.arch.decode(), "cu_count": caps.cu_count},
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
