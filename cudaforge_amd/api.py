"""ctypes helpers over the C-ABI: params structs, device buffers, streams, op calls."""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_bool, c_float, c_int, c_int64, c_void_p

import numpy as np

from ._native import GpuCaps, OperatorRegistryEntry, load_library


class MhaDecodeParams(ctypes.Structure):
    """mha_decode_params_t (include/mha_decode_int.h; reference mha_decode_int.h:6-15)."""

    _fields_ = [
        ("batch_size", c_int64),
        ("hidden_size", c_int64),
        ("num_heads", c_int64),
        ("num_kv_heads", c_int64),
        ("head_dim", c_int64),
        ("scale", c_float),
        ("cache_len", c_int64),
        ("max_seq", c_int64),
    ]


class RopeParams(ctypes.Structure):
    """rope_params_t (include/rope_int.h; reference rope_int.h:6-11)."""

    _fields_ = [("seq_len", c_int64), ("head_dim", c_int64), ("num_heads", c_int64), ("base", c_float)]


class MhaDecodeRopeParams(ctypes.Structure):
    """mha_decode_rope_params_t (include/rope_ops.h): decode params + the RoPE base."""

    _fields_ = [("decode", MhaDecodeParams), ("rope_base", c_float), ("reserved", ctypes.c_int32)]


class LayerNormParams(ctypes.Structure):
    """layernorm_params_t (include/layernorm_int.h; reference layernorm_int.h:6-10)."""

    _fields_ = [("N", c_int64), ("normalized_size", c_int64), ("epsilon", c_float)]


class MatmulParams(ctypes.Structure):
    """matmul_params_t (include/matmul_int.h; reference matmul_int.h:7-17)."""

    _fields_ = [("M", c_int64), ("N", c_int64), ("K", c_int64), ("transpose_a", c_bool), ("transpose_b", c_bool),
                ("batch_size", c_int64), ("stride_a", c_int64), ("stride_b", c_int64), ("stride_c", c_int64),
                ("tuning_config", c_int)]


class CastParams(ctypes.Structure):
    """cast_params_t (include/cast_int.h; reference cast_int.h:12-16), ONNX dtype codes."""

    _fields_ = [("src_dtype", c_int), ("dst_dtype", c_int), ("numel", c_int64)]


ONNX_FLOAT, ONNX_FLOAT16, ONNX_INT64 = 1, 10, 7


class MhaFusedParams(ctypes.Structure):
    """mha_fused_params_t (include/mha_fused_int.h; reference mha_fused_int.h:7-17)."""

    _fields_ = [
        ("batch_size", c_int64),
        ("seq_len", c_int64),
        ("hidden_size", c_int64),
        ("num_heads", c_int64),
        ("num_kv_heads", c_int64),
        ("head_dim", c_int64),
        ("scale", c_float),
        ("has_residual", c_bool),
        ("causal", c_bool),
    ]


GRAPH_MHA_MAX_NODES = 24


class GraphMhaMatch(ctypes.Structure):
    """graph_mha_match_t (include/graph.h): one self-attention subgraph that graph_execute
    runs as a single OP_MHA_FUSED node."""

    _fields_ = [
        ("out_node", ctypes.c_int),
        ("num_nodes", ctypes.c_int),
        ("nodes", ctypes.c_int * GRAPH_MHA_MAX_NODES),
        ("input_tid", ctypes.c_int),
        ("residual_tid", ctypes.c_int),
        ("output_tid", ctypes.c_int),
        ("weights", ctypes.c_void_p * 8),
        ("params", MhaFusedParams),
    ]


def graph_detect_mha(graph, max_matches=8):
    """The attention subgraphs graph_execute would fuse (list of GraphMhaMatch)."""
    arr = (GraphMhaMatch * max_matches)()
    n = load_library().graph_detect_mha(graph, ctypes.cast(arr, ctypes.c_void_p), max_matches)
    return [arr[i] for i in range(n)]


class CausalMaskParams(ctypes.Structure):
    _fields_ = [("seq_len", c_int64)]


class TensorT(ctypes.Structure):
    """tensor_t (include/platform.h; reference platform.h:36-44)."""

    _fields_ = [
        ("dtype", c_int),
        ("ndim", c_int),
        ("shape", c_int64 * 8),
        ("strides", c_int64 * 8),
        ("numel", c_int64),
        ("data", c_void_p),
        ("data_device", c_void_p),
    ]


OperatorRegistry = OperatorRegistryEntry

DT_F32, DT_F16, DT_BF16, DT_I32 = 0, 1, 2, 3


def gpu_available() -> bool:
    return bool(load_library().gpu_available())


def init_gpu(device: int = 0) -> None:
    lib = load_library()
    rc = lib.gpu_platform_init(device)
    if rc != 0:
        raise RuntimeError(f"gpu_platform_init({device}) failed: {rc} {lib.gpu_error_string(rc)!r}")


def device_caps(device: int = 0) -> GpuCaps:
    lib = load_library()
    caps = GpuCaps()
    rc = lib.gpu_get_gpu_caps(ctypes.byref(caps), device)
    if rc != 0:
        raise RuntimeError(f"gpu_get_gpu_caps failed: {rc}")
    return caps


def _check(rc: int, what: str) -> None:
    if rc != 0:
        lib = load_library()
        msg = lib.gpu_error_string(rc) if rc > 0 else b"invalid argument"
        raise RuntimeError(f"{what} failed: rc={rc} ({msg.decode() if msg else ''})")


class Stream:
    """A HIP stream (default priority, non-blocking) owned by the Python object."""

    def __init__(self, null: bool = False):
        self.lib = load_library()
        self.handle = c_void_p(None)
        self.owned = not null
        if not null:
            _check(self.lib.gpu_stream_create(ctypes.byref(self.handle)), "gpu_stream_create")

    def synchronize(self) -> None:
        _check(self.lib.gpu_stream_synchronize(self.handle), "gpu_stream_synchronize")

    def stream_t(self):
        """A pointer to a stream_t holding this stream (stream_t is one void*)."""
        self._st = (c_void_p * 1)(self.handle)
        return ctypes.cast(self._st, c_void_p)

    def close(self) -> None:
        if self.owned and self.handle:
            self.lib.gpu_stream_destroy(self.handle)
            self.handle = c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.lib = load_library()
        self.handle = c_void_p(None)
        _check(self.lib.gpu_event_create(ctypes.byref(self.handle)), "gpu_event_create")

    def record(self, stream: Stream | None = None) -> None:
        _check(self.lib.gpu_event_record(self.handle, stream.handle if stream else None), "gpu_event_record")

    def synchronize(self) -> None:
        _check(self.lib.gpu_event_synchronize(self.handle), "gpu_event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float(0.0)
        _check(self.lib.gpu_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle), "gpu_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                self.lib.gpu_event_destroy(self.handle)
        except Exception:
            pass


class DeviceBuffer:
    """Device memory from the platform allocator, with numpy upload/download."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape=None):
        self.lib = load_library()
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        self.ptr = self.lib.gpu_device_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError(f"gpu_device_alloc({self.nbytes}) failed")

    @classmethod
    def from_numpy(cls, arr: np.ndarray, stream: Stream | None = None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes, arr.dtype, arr.shape)
        buf.upload(arr, stream)
        return buf

    @classmethod
    def empty(cls, shape, dtype) -> "DeviceBuffer":
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        return cls(n, dt, shape)

    def upload(self, arr: np.ndarray, stream: Stream | None = None) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes == self.nbytes, (arr.nbytes, self.nbytes)
        _check(self.lib.gpu_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes, stream.handle if stream else None),
               "gpu_memcpy_h2d")
        # hipMemcpyAsync from pageable memory may return before the copy; make it safe to
        # drop `arr` afterwards.
        _check(self.lib.gpu_stream_synchronize(stream.handle if stream else None), "gpu_stream_synchronize")

    def download(self, stream: Stream | None = None) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _check(self.lib.gpu_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, stream.handle if stream else None),
               "gpu_memcpy_d2h")
        return out

    @classmethod
    def normal(cls, shape, dtype, seed: int, std: float = 1.0, mean: float = 0.0) -> "DeviceBuffer":
        """Synthetic N(mean, std) data made on the device (synthetic_fill_normal:
        splitmix64 + Box-Muller, the CPU oracle's generator), fp16 or fp32."""
        buf = cls.empty(shape, dtype)
        if buf.dtype not in (np.dtype(np.float16), np.dtype(np.float32)):
            raise ValueError("normal() fills float16 or float32 buffers")
        n = buf.nbytes // buf.dtype.itemsize
        _check(buf.lib.synthetic_fill_normal(buf.ptr, n, 1 if buf.dtype == np.float16 else 0, seed & (2**64 - 1),
                                             mean, std, None), "synthetic_fill_normal")
        _check(buf.lib.gpu_stream_synchronize(None), "gpu_stream_synchronize")
        return buf

    def fill_zero(self, stream: Stream | None = None) -> None:
        _check(self.lib.gpu_memset(self.ptr, 0, self.nbytes, stream.handle if stream else None), "gpu_memset")

    def free(self) -> None:
        if self.ptr:
            self.lib.gpu_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return x


def find_op(name: str):
    lib = load_library()
    entry = lib.operator_find(name.encode())
    if not entry:
        raise KeyError(f"operator {name!r} is not registered")
    return entry.contents


def time_op(name: str, inputs, outputs, params, stream: Stream | None, warmup: int, iters: int,
            extra_inputs=()) -> float:
    """Average milliseconds per call of a registered operator, timed by operator_time
    (a C loop between HIP events on `stream`, so Python overhead is excluded)."""
    lib = load_library()
    ins = list(inputs) + list(extra_inputs)
    in_arr = (c_void_p * max(len(ins), 1))(*[_ptr(x) for x in ins])
    out_arr = (c_void_p * max(len(outputs), 1))(*[_ptr(x) for x in outputs])
    ms = c_float(0.0)
    st = stream.stream_t() if stream is not None else None
    rc = lib.operator_time(name.encode(), ctypes.cast(in_arr, POINTER(c_void_p)),
                           ctypes.cast(out_arr, POINTER(c_void_p)),
                           ctypes.cast(ctypes.pointer(params), c_void_p), st, warmup, iters, ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError(f"operator_time({name}) returned {rc}")
    return ms.value / iters


def time_op_sets(name: str, input_sets, output_sets, params, stream: Stream | None, warmup: int,
                 iters: int) -> float:
    """Average milliseconds per call, rotating over several (inputs, outputs) sets: lists
    of equal-length input lists and output lists; call j uses set j % len(input_sets).
    Timed by operator_time_sets.  With a working set larger than the last-level cache,
    every call reads HBM."""
    lib = load_library()
    if len(input_sets) != len(output_sets) or not input_sets:
        raise ValueError("one output list per input set")
    n_in, n_out = len(input_sets[0]), len(output_sets[0])
    if any(len(x) != n_in for x in input_sets) or any(len(x) != n_out for x in output_sets):
        raise ValueError("sets must have equal lengths")
    ins = [_ptr(x) for s in input_sets for x in s]
    outs = [_ptr(x) for s in output_sets for x in s]
    in_arr = (c_void_p * len(ins))(*ins)
    out_arr = (c_void_p * len(outs))(*outs)
    ms = c_float(0.0)
    st = stream.stream_t() if stream is not None else None
    rc = lib.operator_time_sets(name.encode(), ctypes.cast(in_arr, POINTER(c_void_p)), n_in,
                                ctypes.cast(out_arr, POINTER(c_void_p)), n_out, len(input_sets),
                                ctypes.cast(ctypes.pointer(params), c_void_p), st, warmup, iters, ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError(f"operator_time_sets({name}) returned {rc}")
    return ms.value / iters


def call_op(name: str, inputs, outputs, params, stream: Stream | None = None, extra_inputs=()) -> int:
    """Call a registered operator through its registry function pointer, exactly as the
    reference tests do (operator_find(...)->func(inputs, outputs, params, stream))."""
    entry = find_op(name)
    ins = list(inputs) + list(extra_inputs)
    in_arr = (c_void_p * max(len(ins), 1))(*[_ptr(x) for x in ins])
    out_arr = (c_void_p * max(len(outputs), 1))(*[_ptr(x) for x in outputs])
    st = stream.stream_t() if stream is not None else None
    return entry.func(ctypes.cast(in_arr, POINTER(c_void_p)), ctypes.cast(out_arr, POINTER(c_void_p)),
                      ctypes.cast(ctypes.pointer(params), c_void_p) if params is not None else None, st)


def call_entry(name: str, inputs, outputs, params, stream: Stream | None = None) -> int:
    """Call an exported operator-signature C function by its symbol name (for entry
    points that are not in the registry, such as mha_decode_attn_f16_noalloc)."""
    lib = load_library()
    fn = getattr(lib, name)
    in_arr = (c_void_p * max(len(inputs), 1))(*[_ptr(x) for x in inputs])
    out_arr = (c_void_p * max(len(outputs), 1))(*[_ptr(x) for x in outputs])
    st = stream.stream_t() if stream is not None else None
    return fn(ctypes.cast(in_arr, POINTER(c_void_p)), ctypes.cast(out_arr, POINTER(c_void_p)),
              ctypes.cast(ctypes.pointer(params), c_void_p) if params is not None else None, st)
