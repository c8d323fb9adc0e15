"""CPU tests of the C-ABI boundary and the host logic (no GPU work is launched).

- every function declared in include/*.h is exported by libcudaforge_amd.so;
- struct layouts match the reference interface sizes;
- the registry holds exactly the HIP operators, under the reference's names;
- argument validation returns -1 before touching the device (mha_decode.c:14-16,
  mha_fused_cuda.cu:940-941 error contract);
- the graph: topological build, cycle detection, the reference's name-resolution rule
  (graph.c:836-884), and execution through graph_execute / inference_session_run with the
  oracle registered as the CPU ops (the reference's CPU-vs-reference graph tests,
  tests/test_bert_mha.c:167-306, in a CPU-only process).
"""

import ctypes
import os
import re
import subprocess
from ctypes import POINTER, c_int, c_int64, c_void_p

import numpy as np
import pytest

import oracle as O
from helpers import (DT_F16, DT_F32, OP_CAUSAL_MASK, OP_INPUT, OP_MHA_DECODE, OP_MHA_FUSED, OP_OUTPUT,
                     OP_RELU, DecodeCase, FusedCase, Graph, build_fused_graph)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")

def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(INCLUDE, fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"^\s*#[^\n]*", "", src, flags=re.M)
        depth, stmt = 0, ""
        for ch in src:
            if ch == "{":
                depth += 1
                stmt = ""
                continue
            if ch == "}":
                depth -= 1
                stmt = ""
                continue
            if depth > 0 and not stmt.lstrip().startswith("extern"):
                # inside extern "C" { ... } blocks depth is 1: treat that as top level
                pass
            stmt += ch
            if ch == ";":
                s = " ".join(stmt.split())
                stmt = ""
                if s.startswith("typedef") or "(" not in s or "(*" in s:
                    continue
                m = re.match(r"^(?:extern\s+)?[\w\s\*]+?\b(\w+)\s*\(", s)
                if m:
                    names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported(native):
    names = declared_functions()
    assert len(names) > 60
    out = subprocess.run(["nm", "-D", "--defined-only", native._name], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(n for n in names if n not in exported)
    assert not missing, f"declared but not exported: {missing}"


def test_struct_layouts(native):
    import cudaforge_amd as cf
    assert ctypes.sizeof(cf.MhaDecodeParams) == 64       # mha_decode_int.h:6-15
    assert ctypes.sizeof(cf.MhaFusedParams) == 56        # mha_fused_int.h:7-17
    assert ctypes.sizeof(cf.TensorT) == 160              # platform.h:36-44
    assert ctypes.sizeof(cf.OperatorRegistry) == 32      # src/operator/include/operator.h:34-40


def test_registry_names(native):
    names = {native.operator_at(i).contents.name.decode() for i in range(native.operator_count())}
    hip = {"mha_decode_f32_cuda", "mha_decode_f16_cuda", "mha_decode_attn_f32_cuda", "mha_decode_attn_f16_cuda",
           "mha_fused_f32_cuda", "mha_fused_f16_cuda", "mha_fused_f16io_cuda", "causal_mask_f32_cuda"}
    assert hip <= names
    assert native.operator_init_all() == 0              # idempotent
    assert native.operator_count() == len(names)
    assert not native.operator_find(b"mha_fused_f32_nonexistent")
    # The reference registers mha_fused_f16_cuda as "f32" (FP32 buffers, fp16 math); the
    # fp16-I/O op that F16 graphs dispatch to is mha_fused_f16io_cuda.
    assert native.operator_find(b"mha_fused_f16_cuda").contents.data_type == b"f32"
    assert native.operator_find(b"mha_fused_f16io_cuda").contents.data_type == b"f16"


def _slots(vals):
    return (c_void_p * len(vals))(*vals)


DUMMY = ctypes.create_string_buffer(64)
DP = ctypes.addressof(DUMMY)


@pytest.mark.parametrize("mutate,expect", [
    (lambda p, ins: None, None),
    (lambda p, ins: ins.__setitem__(4, None), -1),            # NULL bias (mha_decode.c:15)
    (lambda p, ins: setattr(p, "num_kv_heads", 3), -1),       # 4 % 3 != 0
    (lambda p, ins: setattr(p, "hidden_size", 100), -1),      # H*d != D
    (lambda p, ins: setattr(p, "cache_len", 8), -1),          # cache_len >= max_seq
    (lambda p, ins: setattr(p, "batch_size", 0), -1),
    (lambda p, ins: setattr(p, "head_dim", 0), -1),
])
def test_decode_argument_validation(native, mutate, expect):
    import cudaforge_amd as cf
    p = cf.MhaDecodeParams(1, 32, 4, 2, 8, 0.35, 0, 8)
    ins = [DP] * 11
    mutate(p, ins)
    if expect is None:
        return      # the valid case is exercised on the GPU
    for name in ("mha_decode_f32_cuda", "mha_decode_f16_cuda"):
        rc = native[name](_slots(ins), _slots([DP] * 3), ctypes.byref(p), None) if False else \
            getattr(native, name)(ctypes.cast(_slots(ins), POINTER(c_void_p)),
                                  ctypes.cast(_slots([DP] * 3), POINTER(c_void_p)), ctypes.addressof(p), None)
        assert rc == expect


def test_decode_null_params_and_ragged_without_lengths(native):
    import cudaforge_amd as cf
    f = native.mha_decode_f32_cuda
    ins = ctypes.cast(_slots([DP] * 11 + [None]), POINTER(c_void_p))
    outs = ctypes.cast(_slots([DP] * 3), POINTER(c_void_p))
    assert f(ins, outs, None, None) == -1
    p = cf.MhaDecodeParams(1, 32, 4, 2, 8, 0.35, -1, 8)    # ragged, slot 11 NULL
    assert f(ins, outs, ctypes.addressof(p), None) == -1
    g = native.mha_decode_attn_f16_cuda
    assert g(ctypes.cast(_slots([DP, DP, DP, None]), POINTER(c_void_p)),
             ctypes.cast(_slots([DP]), POINTER(c_void_p)), ctypes.addressof(p), None) == -1


def test_fused_argument_validation(native):
    import cudaforge_amd as cf
    f = native.mha_fused_f16_cuda
    good = [DP] * 10
    outs = ctypes.cast(_slots([DP]), POINTER(c_void_p))
    p = cf.MhaFusedParams(1, 4, 16, 2, 2, 8, 0.35, False, False)
    bad = list(good)
    bad[0] = None
    assert f(ctypes.cast(_slots(bad), POINTER(c_void_p)), outs, ctypes.addressof(p), None) == -1
    assert f(ctypes.cast(_slots(good), POINTER(c_void_p)), ctypes.cast(_slots([None]), POINTER(c_void_p)),
             ctypes.addressof(p), None) == -1
    assert f(ctypes.cast(_slots(good), POINTER(c_void_p)), outs, None, None) == -1
    p.hidden_size = 15
    assert f(ctypes.cast(_slots(good), POINTER(c_void_p)), outs, ctypes.addressof(p), None) == -1
    p.hidden_size, p.num_kv_heads = 16, 3
    assert native.mha_fused_f32_cuda(ctypes.cast(_slots(good), POINTER(c_void_p)), outs, ctypes.addressof(p),
                                     None) == -1
    assert native.mha_fused_f16io_cuda(ctypes.cast(_slots(good), POINTER(c_void_p)), outs, ctypes.addressof(p),
                                       None) == -1
    p.num_kv_heads = 2
    bad[0], bad[8] = DP, None     # WO missing
    assert f(ctypes.cast(_slots(bad), POINTER(c_void_p)), outs, ctypes.addressof(p), None) == -1


# ----------------------------------------------------------------------- graph ---

_cpu_regs = []


@pytest.fixture(scope="module")
def cpu_ops(native):
    """Register the oracle as the CPU ops mha_fused_f32 / mha_decode_f32 / causal_mask_f32
    (the reference's CPU registrations, operator_registry.def:35-37)."""
    import cudaforge_amd as cf
    from cudaforge_amd._native import OP_FUNC
    for name, fn in (("mha_fused_f32", "oracle_op_mha_fused_f32"), ("mha_decode_f32", "oracle_op_mha_decode_f32"),
                     ("causal_mask_f32", "oracle_op_causal_mask_f32")):
        if native.operator_find(name.encode()):
            continue
        entry = cf.OperatorRegistry(name.encode(), b"f32", OP_FUNC(O.cpu_op_pointer(fn)), 1, 0)
        _cpu_regs.append(entry)
        assert native.operator_register(ctypes.addressof(entry)) == 0
    return native


def test_graph_topological_order_and_cycle(native):
    g = Graph(native)
    _, a = g.tensor(np.zeros(4, np.float32))
    _, b = g.tensor(np.zeros(4, np.float32))
    _, c = g.tensor(np.zeros(4, np.float32))
    n2 = g.node(OP_RELU, [b], [c])
    n1 = g.node(OP_RELU, [a], [b])
    assert native.graph_build(g.g) == 0
    gs = ctypes.cast(g.g, POINTER(c_int * 8)).contents   # first field num_nodes
    assert gs[0] == 2
    order_ptr = ctypes.cast(g.g + 32, POINTER(POINTER(c_int))).contents   # topo_order (after tensors)
    assert [order_ptr[0], order_ptr[1]] == [n1, n2]
    g.destroy()
    g = Graph(native)
    _, a = g.tensor(np.zeros(4, np.float32))
    _, b = g.tensor(np.zeros(4, np.float32))
    g.node(OP_RELU, [a], [b])
    g.node(OP_RELU, [b], [a])
    assert native.graph_build(g.g) == -1
    g.destroy()


def test_graph_name_resolution(cpu_ops):
    lib = cpu_ops
    c = FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True)
    buf = ctypes.create_string_buffer(64)
    g, nid, _, _ = build_fused_graph(lib, c)
    assert lib.graph_resolve_op(g.g, nid, True, buf, 64) and buf.value == b"mha_fused_f32_cuda"
    assert lib.graph_resolve_op(g.g, nid, False, buf, 64) and buf.value == b"mha_fused_f32"
    g.destroy()
    g, nid, _, _ = build_fused_graph(lib, c, f16_out=True)
    assert lib.graph_resolve_op(g.g, nid, True, buf, 64) and buf.value == b"mha_fused_f16io_cuda"
    g.destroy()


def test_graph_execute_cpu_matches_oracle(cpu_ops):
    """tests/test_bert_mha.c:167-306: one MHA_Fused node, INPUT/OUTPUT wrappers, CPU run."""
    lib = cpu_ops
    c = FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True)
    g, nid, tX, tY = build_fused_graph(lib, c)
    ins = (c_void_p * 1)(tX)
    outs = (c_void_p * 1)(tY)
    assert lib.graph_execute(g.g, ins, outs, False) == 0
    got = g.read(tY, c.X.shape)
    assert np.array_equal(got, c.oracle())
    # session wrapper (inference_engine.c:31-37)
    s = lib.inference_session_from_graph(g.g, 1, 1)
    assert s and lib.inference_session_num_inputs(s) == 1
    assert lib.inference_session_run(s, ins, outs, 0) == 0
    assert np.array_equal(g.read(tY, c.X.shape), c.oracle())
    lib.inference_session_destroy(s)       # owns and destroys the graph


def test_graph_replay_state_machine_cpu(cpu_ops):
    """HIP-graph replay only concerns GPU executions: CPU executions leave the state at 0,
    graph_set_replay resets it, and the state API accepts NULL."""
    lib = cpu_ops
    c = FusedCase(1, 4, 2, 2, 8, fill="lcg", residual=True)
    g, nid, tX, tY = build_fused_graph(lib, c)
    ins, outs = (c_void_p * 1)(tX), (c_void_p * 1)(tY)
    for _ in range(3):
        assert lib.graph_execute(g.g, ins, outs, False) == 0
        assert lib.graph_replay_state(g.g) == 0
    assert np.array_equal(g.read(tY, c.X.shape), c.oracle())
    lib.graph_set_replay(g.g, 0)
    assert lib.graph_replay_state(g.g) == 0
    assert lib.graph_replay_state(None) == 0
    g.destroy()


def test_graph_decode_kv_cache_steps_cpu(cpu_ops):
    """OP_MHA_DECODE with in-place caches and graph_update_cache_len over two steps."""
    lib = cpu_ops
    c = DecodeCase(1, 4, 2, 8, 8, cache_len=0, seed=4, wstd=0.3)
    g = Graph(lib)
    tX, iX = g.tensor(c.X)
    tK, iK = g.tensor(c.Kc)
    tV, iV = g.tensor(c.Vc)
    tY, iY = g.tensor(np.zeros_like(c.X))
    ws = [g.tensor(w)[0] for w in (c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO)]
    p = O.decode_params(1, c.D, c.H, c.H_kv, c.d, 0, c.max_seq)
    g.node(OP_MHA_DECODE, [iX, iK, iV], [iY, iK, iV], ws, p)
    lib.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
    lib.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
    lib.graph_set_kv_cache(g.g, iK, iV)
    assert lib.graph_build(g.g) == 0
    want = c.oracle()
    ins, outs = (c_void_p * 1)(tX), (c_void_p * 1)(tY)
    assert lib.graph_execute(g.g, ins, outs, False) == 0
    assert np.array_equal(g.read(tY, c.X.shape), want[0])
    assert np.array_equal(g.read(tK, c.Kc.shape), want[1])
    # step 2
    c2 = DecodeCase(1, 4, 2, 8, 8, cache_len=1, seed=4, wstd=0.3)
    c2.Kc, c2.Vc = want[1], want[2]
    c2.X = O.normal(c.X.shape, 77)
    ctypes.memmove(ctypes.cast(tX, POINTER(__import__("cudaforge_amd").TensorT)).contents.data,
                   c2.X.ctypes.data, c2.X.nbytes)
    lib.graph_update_cache_len(g.g, 1)
    assert lib.graph_execute(g.g, ins, outs, False) == 0
    want2 = c2.oracle()
    assert np.array_equal(g.read(tY, c.X.shape), want2[0])
    assert np.array_equal(g.read(tV, c.Vc.shape), want2[2])
    g.destroy()


def test_graph_unresolved_op_returns_minus_two(native):
    g = Graph(native)
    _, a = g.tensor(np.zeros(4, np.float32))
    _, b = g.tensor(np.zeros(4, np.float32))
    g.node(OP_RELU, [a], [b])
    assert native.graph_build(g.g) == 0
    assert native.graph_execute(g.g, None, None, False) == -2
    g.destroy()


def test_session_load_reports_missing_onnx(native):
    assert not native.inference_session_load(b"model.onnx")


def test_tensor_api(native):
    import cudaforge_amd as cf
    shape = (c_int64 * 3)(2, 3, 4)
    t = native.tensor_create(DT_F16, 3, shape)
    tt = ctypes.cast(t, POINTER(cf.TensorT)).contents
    assert tt.numel == 24 and list(tt.strides[:3]) == [12, 4, 1] and tt.data and not tt.data_device
    u = native.tensor_create(DT_F16, 3, shape)
    assert native.tensor_allclose(t, u, 0.0, 0.0)
    ctypes.cast(ctypes.cast(tt.data, c_void_p), POINTER(ctypes.c_uint16))[5] = 0x3C00   # 1.0
    assert not native.tensor_allclose(t, u, 1e-3, 1e-3)
    assert native.tensor_copy_to_host(t) == 0            # no device mirror: no-op
    native.tensor_destroy(t)
    native.tensor_destroy(u)
    assert not native.tensor_create(DT_F32, 9, shape)


@pytest.mark.parametrize("B,H,H_kv,d,cl,max_seq,f16", [
    (16, 32, 8, 128, 4095, 4096, 1), (4, 32, 8, 128, -1, 32768, 1), (1, 12, 12, 64, 1023, 1024, 0),
    (1, 8, 2, 128, 39999, 40000, 1), (64, 32, 8, 128, 127, 128, 1), (3, 6, 2, 32, 249, 255, 1),
    (2, 4, 4, 80, 0, 16, 0), (1, 8, 8, 128, 8_000_000 - 1, 8_000_000, 1)])
def test_decode_split_plan_invariants(native, B, H, H_kv, d, cl, max_seq, f16):
    """The split planner (host only): chunks are whole 32-position blocks on the fp16
    kernel path, cover every attended position, stay within the kernel's limits (at most
    1024 splits; chunk <= 4096 where scores live in LDS) and leave no split empty; an
    8M-position cache plans too."""
    import cudaforge_amd as cf
    p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, 0.1, cl, max_seq)
    chunk, n = ctypes.c_int64(0), ctypes.c_int64(0)
    assert native.mha_decode_plan(ctypes.addressof(p), f16, ctypes.byref(chunk), ctypes.byref(n)) == 0
    chunk, n = chunk.value, n.value
    t_max = max_seq if cl < 0 else cl + 1
    fast_f16 = f16 and d in (64, 128) and (H // H_kv) in (1, 2, 4, 8)
    assert 1 <= chunk <= (1 << 20 if fast_f16 else 4096) and 1 <= n <= 1024
    assert n * chunk >= t_max and (n - 1) * chunk < t_max
    if fast_f16:
        assert chunk % 32 == 0


@pytest.mark.parametrize("B,H,H_kv,d,max_seq", [(16, 32, 8, 128, 4096), (4, 32, 8, 128, 32768), (3, 6, 2, 32, 255)])
def test_device_uniform_length_plans_as_uniform_over_capacity(native, B, H, H_kv, d, max_seq):
    """cache_len -2 (lengths in slot 11, all equal: the graph's device-held length) plans
    like a uniform length over the whole capacity, so a recorded step fits every length;
    cache_len -1 (ragged) plans four times as many splits."""
    import cudaforge_amd as cf

    def plan(cl):
        p = cf.MhaDecodeParams(B, H * d, H, H_kv, d, 0.1, cl, max_seq)
        chunk, n = ctypes.c_int64(0), ctypes.c_int64(0)
        assert native.mha_decode_plan(ctypes.addressof(p), 1, ctypes.byref(chunk), ctypes.byref(n)) == 0
        return chunk.value, n.value

    assert plan(-2) == plan(max_seq - 1)
    assert plan(-1)[1] >= plan(-2)[1]


def test_buffer_generation_counter(native):
    """gpu_buffer_generation_bump moves the counter that invalidates recordings."""
    g0 = native.gpu_buffer_generation()
    native.gpu_buffer_generation_bump()
    assert native.gpu_buffer_generation() == g0 + 1


def test_graph_decode_length_past_capacity_cpu(cpu_ops):
    """The executor rejects cache_len >= max_seq with -1 before running the node, as the
    reference op does (mha_decode.c:14-16)."""
    lib = cpu_ops
    c = DecodeCase(1, 4, 2, 8, 8, cache_len=7, seed=4, wstd=0.3)
    g = Graph(lib)
    tX, iX = g.tensor(c.X)
    tK, iK = g.tensor(c.Kc)
    tV, iV = g.tensor(c.Vc)
    tY, iY = g.tensor(np.zeros_like(c.X))
    ws = [g.tensor(w)[0] for w in (c.WQ, c.bQ, c.WK, c.bK, c.WV, c.bV, c.WO, c.bO)]
    g.node(OP_MHA_DECODE, [iX, iK, iV], [iY, iK, iV], ws, O.decode_params(1, c.D, c.H, c.H_kv, c.d, 7, 8))
    lib.graph_set_input(g.g, g.node(OP_INPUT, [], [iX]))
    lib.graph_set_output(g.g, g.node(OP_OUTPUT, [iY], []))
    lib.graph_set_kv_cache(g.g, iK, iV)
    assert lib.graph_build(g.g) == 0
    ins, outs = (c_void_p * 1)(tX), (c_void_p * 1)(tY)
    assert lib.graph_execute(g.g, ins, outs, False) == 0
    lib.graph_update_cache_len(g.g, 8)
    assert lib.graph_execute(g.g, ins, outs, False) == -1
    g.destroy()


def test_launch_time_divisor_is_exact(native):
    """The kernels divide grid and row indices by launch-time values through a multiplier
    and shift (cdna4.h FastDiv), exact for 0 <= n < 2^31.  The same source runs on the
    host here: every n below 70 000 for divisors 1..300, the largest n, powers of two and
    their neighbours, and random pairs across the range, against integer division."""
    q = native.cf_fastdiv_quotient
    rng = np.random.default_rng(2026)
    top = 2**31 - 1
    for d in range(1, 301):
        ns = np.arange(0, 70000, 7 if d > 40 else 1)
        assert all(q(int(n), d) == n // d for n in ns), d
        for n in (top, top - 1, top - d, 2**30, 2**30 - 1, d * (top // d), d * (top // d) - 1):
            assert q(n, d) == n // d, (n, d)
    for k in range(31):
        for d in (2**k - 1, 2**k, 2**k + 1):
            if d >= 1:
                for n in (0, 1, d - 1, d, d + 1, top, top - 1):
                    assert q(n, d) == n // d, (n, d)
    for n, d in zip(rng.integers(0, top, 20000), rng.integers(1, top, 20000)):
        assert q(int(n), int(d)) == int(n) // int(d), (n, d)
    for n, d in zip(rng.integers(0, top, 20000), rng.integers(1, 5000, 20000)):
        assert q(int(n), int(d)) == int(n) // int(d), (n, d)
