"""ctypes binding of libuttt_hip.so, the C ABI declared in include/uttt_hip.h.

Every product op of this package goes through `call()`; there is no CPU or
PyTorch fallback.  If the library is missing or a call fails the op raises
RuntimeError with the library's message (the reference's callers treat an
ImportError of the kernel module as "use the slow loop", so this module never
raises ImportError: a missing build must fail loudly at the first call).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libuttt_hip.so")

c_int, c_i64, c_sz, c_p = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# dtype codes of the C ABI
F32, BF16, F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

# name -> (restype, argtypes); must list every function of include/uttt_hip.h
SIGNATURES = {
    "uttt_abi_version": (c_int, []),
    "uttt_last_error": (ctypes.c_char_p, []),
    "uttt_row_id_map_workspace_bytes": (c_sz, [c_int, c_int, c_int]),
    "uttt_make_row_id_map": (
        c_int,
        [c_p, c_int, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_p, c_p, c_p, c_sz, c_p],
    ),
    "uttt_permute_fwd": (
        c_int,
        [c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_p, c_i64, c_i64, c_i64, c_p, c_int, c_p, c_p],
    ),
    "uttt_permute_bwd": (
        c_int,
        [c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_int, c_p, c_p, c_p, c_p],
    ),
    "uttt_unpermute_fwd": (
        c_int,
        [c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_int, c_p, c_i64, c_i64, c_i64, c_p, c_p],
    ),
    "uttt_unpermute_bwd": (
        c_int,
        [c_p, c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_int, c_p, c_i64, c_i64, c_i64,
         c_p, c_p, c_i64, c_i64, c_i64, c_p],
    ),
    "uttt_permute_kv_lrs_fwd": (
        c_int,
        [c_p, c_int, c_p, c_int, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_p,
         c_i64, c_i64, c_i64, c_p, c_p, c_p, c_p, c_p, c_int, c_p],
    ),
    "uttt_permute_kv_lrs_bwd": (
        c_int,
        [c_p, c_p, c_int, c_p, c_p, c_p, c_int, c_p, c_int, c_p, c_i64, c_i64, c_i64, c_int,
         c_int, c_int, c_p, c_int, c_int, c_p, c_p, c_p, c_p, c_p, c_p, c_p],
    ),
    "uttt_grouped_gate_up": (
        c_int, [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p, c_int, c_p],
    ),
    "uttt_grouped_gate_up_gathers": (c_int, [ctypes.c_longlong, c_int]),
    "uttt_grouped_gate_up_gather": (
        c_int, [c_p, c_p, c_int, c_p, ctypes.c_longlong, c_p, c_int, c_int, c_int, c_int, c_int,
                c_p, c_p],
    ),
    "uttt_grouped_gemm_nt": (
        c_int, [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p, c_p],
    ),
    "uttt_grouped_gemm_tn": (
        c_int, [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p, c_p],
    ),
    "uttt_update_stage1_workspace_bytes": (c_sz, [c_int, c_int, c_int]),
    "uttt_grouped_update_stage1": (
        c_int,
        [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_p, c_int, c_int, c_int, c_int, c_int,
         c_p, c_p, c_int, c_p, c_p, c_p, c_sz, c_p],
    ),
    "uttt_grouped_wgrad_pair_workspace_bytes": (c_sz, [c_int] * 5),
    "uttt_dense_gather_heads": (
        c_int,
        [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_p, c_p, c_p, c_p,
         c_p, c_p],
    ),
    "uttt_dense_scatter_heads": (c_int, [c_p, c_int, c_int, c_int, c_int, c_p, c_p]),
    "uttt_dense_read_supported": (c_int, [c_int, c_int]),
    "uttt_dense_read": (
        c_int, [c_p, c_int, c_int, c_int, c_int, c_p, c_p, c_int, c_p, c_p],
    ),
    "uttt_dense_pack_weights": (c_int, [c_p, c_p, c_int, c_int, c_int, c_p, c_p]),
    "uttt_dense_read_packed": (
        c_int, [c_p, c_int, c_int, c_int, c_int, c_p, c_int, c_p, c_p],
    ),
    "uttt_dense_update_supported": (c_int, [c_int, c_int]),
    "uttt_dense_pack_update_weights": (c_int, [c_p, c_p, c_int, c_int, c_int, c_p, c_p]),
    "uttt_dense_update_stage1": (
        c_int, [c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_p, c_p, c_p, c_p],
    ),
    "uttt_dense_update_stage1_layers": (
        c_int, [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_p, c_p,
                c_p, c_p],
    ),
    "uttt_dense_wgrad_pair_layers_workspace_bytes": (c_sz, [c_int, c_int, c_int, c_int, c_int]),
    "uttt_dense_wgrad_pair_layers": (
        c_int, [c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int, c_p, c_p, c_p, c_sz,
                c_p],
    ),
    "uttt_grouped_wgrad_pair": (
        c_int,
        [c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p, c_p, c_p, c_sz, c_p],
    ),
    "uttt_grouped_wgrad": (
        c_int, [c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p, c_int, c_p],
    ),
    "uttt_update_bwd_workspace_bytes": (c_sz, [c_int, c_int, c_int]),
    "uttt_grouped_update_bwd": (
        c_int,
        [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int,
         c_int, c_int, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_sz, c_p],
    ),
    "uttt_transpose_2byte": (c_int, [c_p, c_int, c_int, c_int, c_p, c_p]),
    "uttt_row_norms": (c_int, [c_p, c_int, c_i64, c_int, c_p, c_p]),
    "uttt_write_prenorm": (c_int, [c_p, c_p, c_int, c_p, c_i64, c_int, c_p, c_p, c_p]),
    "uttt_rows_preprocess": (c_int, [c_p, c_int, c_i64, c_int, c_i64, c_int, c_int, c_p, c_p,
                                     c_int, c_int, c_int, c_int, c_int, c_p, c_i64, c_p]),
    "uttt_rows_preprocess_bwd": (c_int, [c_p, c_int, c_p, c_i64, c_int, c_i64, c_i64, c_int,
                                         c_int, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_p,
                                         c_p]),
    "uttt_debug_set_supertile_min_tiles": (ctypes.c_longlong, [ctypes.c_longlong]),
    "uttt_debug_set_apply_path": (c_int, [c_int]),
    "uttt_debug_set_gemm_layout": (c_int, [c_int]),
    "uttt_debug_set_ns_path": (c_int, [c_int]),
    "uttt_debug_set_s1_staged": (c_int, [c_int]),
    "uttt_grouped_gemm_nt2": (c_int, [c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int,
                                      c_p, c_p]),
    "uttt_grouped_gemm_tn2": (c_int, [c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int,
                                      c_p, c_p]),
    "uttt_swiglu_bwd_bwd_workspace_bytes": (c_sz, [c_int, c_int, c_int]),
    "uttt_swiglu_bwd_bwd": (
        c_int,
        [c_p, c_p, c_int, c_p, c_p, c_p, c_int, c_p, c_p, c_int, c_int, c_int, c_p, c_p, c_p, c_p,
         c_p, c_p, c_p, c_p, c_sz, c_p],
    ),
    "uttt_router_workspace_bytes": (c_sz, [c_int, c_int, c_int, c_int]),
    "uttt_router_select": (
        c_int,
        [c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_int, c_int, c_int, c_int, c_int, c_int,
         ctypes.c_float, ctypes.c_float, ctypes.c_float, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_sz,
         c_p],
    ),
    "uttt_route_tokens": (
        c_int,
        [c_p, c_int, c_p, c_i64, c_int, c_int, c_int, c_int, c_p, c_i64, c_int, c_int, c_int,
         ctypes.c_float, ctypes.c_float, ctypes.c_float, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p,
         c_sz, c_p],
    ),
    "uttt_route_tokens_map_workspace_bytes": (c_sz, [c_int, c_int, c_int, c_int]),
    "uttt_route_tokens_map_src_rows": (c_int, [c_int, c_int]),
    "uttt_route_tokens_map": (
        c_int,
        [c_p, c_int, c_p, c_i64, c_int, c_int, c_int, c_int, c_p, c_i64, c_int, c_int, c_int,
         ctypes.c_float, ctypes.c_float, ctypes.c_float, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p,
         c_sz, c_p],
    ),
    "uttt_write_step": (
        c_int,
        [c_p, c_p, c_p, c_int, c_p, c_p, ctypes.c_float, c_int, c_i64, c_int, c_int, c_int, c_int,
         c_p, c_p, c_p, c_p],
    ),
    "uttt_loss_free_store_counts": (c_int, [c_p, c_p, c_int, c_int, c_int, c_int, c_p, c_p, c_p]),
    "uttt_loss_free_bias_step": (
        c_int,
        [c_p, c_p, c_int, c_int, c_int, ctypes.c_float, ctypes.c_float, c_p, c_p],
    ),
    "uttt_write_unit_rows": (
        c_int,
        [c_p, c_i64, c_p, c_int, c_i64, c_i64, c_int, c_int, c_p, c_i64, c_p, c_i64, c_p],
    ),
    "uttt_momentum_add": (c_int, [c_p, c_int, c_p, c_p, c_int, c_i64, c_p, c_p]),
    "uttt_newton_schulz5_workspace_bytes": (ctypes.c_size_t, [c_int, c_int, c_int]),
    "uttt_newton_schulz5": (
        c_int,
        [c_p, c_int, c_int, c_int, c_int, ctypes.c_float, c_p, c_p, ctypes.c_size_t, c_p],
    ),
    "uttt_moe_decode_read_workspace_bytes": (c_sz, [c_int, c_int, c_int, c_int]),
    "uttt_moe_decode_read": (
        c_int,
        [c_p, c_int, c_int, c_int, c_p, c_p, c_int, c_int, c_p, c_int, c_i64, c_i64, c_i64,
         c_p, c_i64, c_i64, c_i64, c_int, c_p, c_p, c_sz, c_p],
    ),
    "uttt_moe_decode_read_noalloc": (
        c_int,
        [c_p, c_int, c_int, c_int, c_p, c_p, c_int, c_int, c_p, c_int, c_i64, c_i64, c_i64,
         c_p, c_i64, c_i64, c_i64, c_int, c_p, c_p],
    ),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libuttt_hip.so once; RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"uttt_amd: {LIB_PATH} is not built; run `python -m uttt_amd.build` "
                    "(there is no fallback path)"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def is_available() -> bool:
    try:
        lib()
        return True
    except (RuntimeError, OSError):
        return False


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().uttt_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise AssertionError(f"unsupported dtype {dt}") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# torch's own raw-handle lookup of the current stream (what its compiled code
# uses): one C call by device index, against ~3 us of Python device resolution
# in torch.cuda.current_stream(device) on every kernel call of the glue
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device (the capture
    stream while a HIP graph is being captured)."""
    idx = t.get_device()
    if _raw_stream is not None and idx >= 0:
        return _raw_stream(idx)
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors) -> None:
    """The HIP path only: CPU tensors are a caller error, never a fallback.
    Meta tensors pass: they only carry shapes through tracing (the registered
    ops' fake implementations), and no kernel ever receives them."""
    for t in tensors:
        if t is not None and t.device.type not in ("cuda", "meta"):
            raise RuntimeError(
                f"uttt_amd ops run on the GPU only; got a tensor on {t.device}"
            )
