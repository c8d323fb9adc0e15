"""Loading of libcudaforge_amd.so and ctypes prototypes for its C-ABI."""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

# CUDAFORGE_AMD_LIB selects another build of the library (the host-sanitizer build).
LIB_PATH = os.environ.get("CUDAFORGE_AMD_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                "libcudaforge_amd.so")


class NativeLibraryMissing(RuntimeError):
    """The HIP library is not built; there is deliberately no fallback."""


_lib = None


class GpuCaps(ctypes.Structure):
    _fields_ = [
        ("device_id", c_int),
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("cu_count", c_int),
        ("wavefront_size", c_int),
        ("max_threads_per_block", c_int),
        ("max_threads_per_cu", c_int),
        ("regs_per_block", c_int),
        ("lds_per_block", c_int),
        ("l2_bytes", c_int),
        ("clock_khz", c_int),
        ("mem_clock_khz", c_int),
        ("mem_bus_width", c_int),
        ("total_memory", c_size_t),
        ("hbm_peak_gbs", c_double),
        ("fp16_mfma_peak_tflops", c_double),
        ("fp32_peak_tflops", c_double),
    ]


OP_FUNC = ctypes.CFUNCTYPE(c_int, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p)


class OperatorRegistryEntry(ctypes.Structure):
    _fields_ = [
        ("name", c_char_p),
        ("data_type", c_char_p),
        ("func", OP_FUNC),
        ("version", c_int),
        ("flags", ctypes.c_uint32),
    ]


def _proto(lib):
    sigs = {
        # platform
        "gpu_available": (c_int, []),
        "gpu_init": (c_int, [c_int]),
        "gpu_platform_init": (c_int, [c_int]),
        "gpu_platform_finalize": (None, []),
        "gpu_print_caps": (c_int, [c_int]),
        "gpu_device_alloc": (c_void_p, [c_size_t]),
        "gpu_device_free": (None, [c_void_p]),
        "gpu_host_alloc_pinned": (c_void_p, [c_size_t]),
        "gpu_host_free_pinned": (None, [c_void_p]),
        "gpu_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
        "gpu_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
        "gpu_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
        "gpu_memset": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
        "gpu_stream_create": (c_int, [POINTER(c_void_p)]),
        "gpu_stream_synchronize": (c_int, [c_void_p]),
        "gpu_stream_destroy": (c_int, [c_void_p]),
        "gpu_device_synchronize": (c_int, []),
        "gpu_get_device_count": (c_int, [POINTER(c_int)]),
        "gpu_current_device": (c_int, []),
        "gpu_get_gpu_caps": (c_int, [POINTER(GpuCaps), c_int]),
        "gpu_get_last_error": (c_int, []),
        "gpu_error_string": (c_char_p, [c_int]),
        "gpu_event_create": (c_int, [POINTER(c_void_p)]),
        "gpu_event_destroy": (c_int, [c_void_p]),
        "gpu_event_record": (c_int, [c_void_p, c_void_p]),
        "gpu_event_synchronize": (c_int, [c_void_p]),
        "gpu_event_elapsed_ms": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
        "gpu_workspace_get": (c_void_p, [c_size_t]),
        "gpu_workspace_get_stream": (c_void_p, [c_void_p, c_size_t]),
        "gpu_workspace_size": (c_size_t, []),
        "gpu_workspace_release": (None, []),
        "gpu_inject_alloc_failures": (None, [c_int]),
        "gpu_buffer_generation": (ctypes.c_uint64, []),
        "gpu_buffer_generation_bump": (None, []),
        # registry
        "operator_init_all": (c_int, []),
        "operator_find": (POINTER(OperatorRegistryEntry), [c_char_p]),
        "operator_count": (c_int, []),
        "operator_at": (POINTER(OperatorRegistryEntry), [c_int]),
        "operator_register": (c_int, [c_void_p]),
        "operator_time": (c_int, [c_char_p, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p, c_int, c_int,
                                  POINTER(c_float)]),
        "operator_time_sets": (c_int, [c_char_p, POINTER(c_void_p), c_int, POINTER(c_void_p), c_int, c_int,
                                       c_void_p, c_void_p, c_int, c_int, POINTER(c_float)]),
        "mha_decode_attn_kernel_times": (c_int, [POINTER(c_void_p), c_int, c_int, POINTER(c_void_p), c_void_p,
                                                 c_void_p, c_int, c_int, c_int, POINTER(c_float), POINTER(c_float)]),
        "mha_fused_kernel_times": (c_int, [POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p, c_int, c_int,
                                           c_int, POINTER(c_float)]),
        "synthetic_fill_normal": (c_int, [c_void_p, c_int64, c_int, ctypes.c_uint64, c_float, c_float, c_void_p]),
        # decode planning knobs
        "mha_decode_set_split_chunk": (None, [c_int64]),
        "mha_fused_set_rowcat": (None, [c_int]),
        "cf_gemv_set_dma_tile": (None, [c_int32]),
        "cf_gemv_set_dma_ksplit": (None, [c_int32]),
        "cf_gemv_set_small": (None, [c_int32]),
        "cf_decode_attn_set_merge_wave_wg": (None, [c_int32]),
        "cf_decode_attn_set_stages": (None, [c_int32]),
        "cf_decode_attn_set_merge_rows": (None, [c_int32]),
        "cf_decode_attn_set_merge_rows_split": (None, [c_int32]),
        "cf_decode_attn_set_wide": (None, [c_int32]),
        "cf_decode_attn_set_kreg": (None, [c_int32]),
        "cf_decode_attn_kreg_ok": (c_int32, [c_int32]),
        "cf_fastdiv_quotient": (c_int32, [c_int32, c_int32]),
        "cf_gemm_set_stages": (None, [c_int32]),
        "cf_gemm_set_group_m": (None, [c_int32]),
        "cf_gemm_set_bn": (None, [c_int32]),
        "cf_gemm_set_bk": (None, [c_int32]),
        "cf_gemm_set_ksplit": (None, [c_int32]),
        "cf_gemm_set_ws": (None, [c_int32]),
        "cf_gemm_set_ws_shape": (None, [c_int32, c_int32]),
        "cf_flash_set_mode": (None, [c_int32]),
        "cf_flash_set_causal_pairs": (None, [c_int32]),
        "mha_decode_plan": (c_int, [c_void_p, c_int, POINTER(c_int64), POINTER(c_int64)]),
        "cf_decode_attn_scratch_bytes": (c_size_t, []),
        # host platform / tensors
        "platform_init": (c_int, []),
        "platform_finalize": (None, []),
        "platform_get_core_count": (c_int, []),
        "data_type_get_info": (c_void_p, [c_int]),
        "tensor_create": (c_void_p, [c_int, c_int, POINTER(c_int64)]),
        "tensor_destroy": (None, [c_void_p]),
        "tensor_copy_to_device": (c_int, [c_void_p]),
        "tensor_upload": (c_int, [c_void_p]),
        "tensor_copy_to_host": (c_int, [c_void_p]),
        "tensor_allclose": (ctypes.c_bool, [c_void_p, c_void_p, c_float, c_float]),
        # graph / session
        "graph_create": (c_void_p, []),
        "graph_add_tensor": (c_int, [c_void_p, c_void_p]),
        "graph_add_node": (c_int, [c_void_p, c_int, c_int, POINTER(c_int), c_int, POINTER(c_int), c_int,
                                   POINTER(c_void_p), c_void_p, c_size_t]),
        "graph_set_input": (c_int, [c_void_p, c_int]),
        "graph_set_output": (c_int, [c_void_p, c_int]),
        "graph_build": (c_int, [c_void_p]),
        "graph_set_replay": (None, [c_void_p, c_int]),
        "graph_replay_state": (c_int, [c_void_p]),
        "graph_destroy": (None, [c_void_p]),
        "graph_set_kv_cache": (None, [c_void_p, c_int, c_int]),
        "graph_update_cache_len": (None, [c_void_p, c_int64]),
        "graph_set_permanent_fusion": (None, [c_void_p, c_int]),
        "graph_execute": (c_int, [c_void_p, POINTER(c_void_p), POINTER(c_void_p), ctypes.c_bool]),
        "graph_resolve_op": (POINTER(OperatorRegistryEntry), [c_void_p, c_int, ctypes.c_bool, c_char_p, c_size_t]),
        "graph_detect_mha": (c_int, [c_void_p, c_void_p, c_int]),
        "rope_table_device": (c_void_p, [c_float, c_int64, c_int64]),
        "inference_engine_init": (c_int, []),
        "inference_engine_finalize": (None, []),
        "inference_session_load": (c_void_p, [c_char_p]),
        "inference_session_from_graph": (c_void_p, [c_void_p, c_int, c_int]),
        "inference_session_run": (c_int, [c_void_p, POINTER(c_void_p), POINTER(c_void_p), c_int]),
        "inference_session_num_inputs": (c_int, [c_void_p]),
        "inference_session_num_outputs": (c_int, [c_void_p]),
        "inference_session_destroy": (None, [c_void_p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    for name in ("mha_decode_f32_cuda", "mha_decode_f16_cuda", "mha_decode_attn_f32_cuda",
                 "mha_decode_attn_f16_cuda", "mha_fused_f32_cuda", "mha_fused_f16_cuda", "mha_fused_f16io_cuda",
                 "causal_mask_f32_cuda", "rope_f32_cuda", "rope_f16_cuda", "mha_decode_rope_f32_cuda",
                 "mha_decode_rope_f16_cuda", "mha_decode_attn_f16_noalloc"):
        fn = getattr(lib, name)
        fn.restype = c_int
        fn.argtypes = [POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p]
    return lib


def load_library(path: str | None = None):
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise NativeLibraryMissing(
            f"{p} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no CPU fallback)")
    _lib = _proto(ctypes.CDLL(p, mode=ctypes.RTLD_GLOBAL))
    _lib.platform_init()
    _lib.operator_init_all()
    return _lib


class _LazyLib:
    def __getattr__(self, name):
        return getattr(load_library(), name)


lib = _LazyLib()
