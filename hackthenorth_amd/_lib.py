"""ctypes binding of libhtn_decode.so, the C-ABI decode library (include/htn_decode.h).

The library is built in-tree by hackthenorth_amd/csrc/Makefile (driven by
__graft_entry__.build()). There is no fallback: if the library is missing or
fails to load, every op raises, so a GPU run can never silently take another
path.
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhtn_decode.so")

HTN_OK = 0
HTN_EINVAL = -1
HTN_EUNSUPPORTED = -2
HTN_ELAUNCH = -3
HEAD_SCRATCH_BYTES = 65536
ATTENTION_XCD_MISMATCH_BYTE = 8  # HTN_ATTENTION_XCD_MISMATCH_BYTE
ATTENTION_OUTPUT_ERROR_BYTE = 12  # HTN_ATTENTION_OUTPUT_ERROR_BYTE
ATTENTION_OUTPUT_ACC_BYTE = 32768  # HTN_ATTENTION_OUTPUT_ACC_BYTE
HEAD_DIM = 128

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int

# name -> argtypes (restype int unless noted); mirrors include/htn_decode.h.
SIGNATURES = {
    "htn_version": [],
    "htn_fill_normal_bf16": [_P, _I64, _U64, _U64, _I64, _F, _P],
    "htn_fill_randint_i64": [_P, _I64, _U64, _U64, _I64, _P],
    "htn_fill_uniform_f32": [_P, _I64, _U64, _U64, _F, _F, _P],
    "htn_fill_weights_w8": [_P, _I64, _U64, _U64, _I, _P],
    "htn_embed_gather": [_P, _I64, _P, _I64, _I64, _P, _P],
    "htn_embed_gather_pair": [_P, _I64, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _P],
    "htn_rms_norm": [_P, _I64, _P, _P, _I64, _I64, _F, _P],
    "htn_add_rms_norm": [_P, _P, _P, _P, _P, _I64, _I64, _F, _P],
    "htn_swiglu": [_P, _I64, _P, _I64, _P, _I64, _I64, _P],
    "htn_gemv": [_P, _P, _P, _I64, _I64, _P],
    "htn_gemv_norm": [_P, _P, _F, _P, _P, _I64, _I64, _I, _P],
    "htn_gemv_residual": [_P, _P, _P, _P, _I64, _I64, _P],
    "htn_lm_head_argmax": [_P, _P, _F, _P, _I64, _I64, _P, _P, _P, _P],
    "htn_lm_head_argmax_noalloc": [_P, _P, _F, _P, _I64, _I64, _P, _P, _P],
    "htn_head_scratch_capacity": [],
    "htn_gemv_w8": [_P, _P, _P, _I, _P, _I64, _I64, _P],
    "htn_gemv_norm_w8": [_P, _P, _F, _P, _P, _I, _P, _I64, _I64, _I, _P],
    "htn_gemv_residual_w8": [_P, _P, _P, _I, _P, _P, _I64, _I64, _P],
    "htn_lm_head_argmax_w8": [_P, _P, _F, _P, _P, _I, _I64, _I64, _P, _P, _P, _P],
    "htn_gemm_rows_scratch_bytes": [_I64, _I64, _I64, _I, _I],
    "htn_gemm_rows": [_P, _I64, _P, _F, _P, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _P, _P,
                      _P],
    "htn_gemm_tiles_scratch_bytes": [_I64, _I64, _I64, _I],
    "htn_gemm_tiles": [_P, _I64, _P, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _P, _P],
    "htn_gemm_library_workspace_bytes": [],
    "htn_gemm_library": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P],
    "htn_gemm_rows_residual_norm": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _F,
                                    _P, _P, _P],
    "htn_argmax_bf16": [_P, _I64, _I64, _P, _P],
    "htn_gate_up_swiglu_scratch_bytes": [_I64, _I64, _I64],
    "htn_stream_read_blocks": [],
    "htn_stream_read": [_P, _I64, _P, _P],
    "htn_gate_up_swiglu": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P],
    "htn_norm_rope_cache": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _P, _F, _F,
                            _P, _P, _I64, _I64, _I, _P, _P, _I64, _P, _P, _P, _I64, _I64,
                            _I64, _I64, _P],
    "htn_attention_scratch_bytes": [_I64, _I64, _I64, _I64],
    "htn_grouped_attention": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64,
                              _I64, _I64, _I64, _I64, _P, _P],
    "htn_prologue_attention": [_P, _I64, _I64, _I64, _P, _P, _F, _F, _P, _P, _I64, _I64, _I,
                               _P, _P, _I64, _P, _P, _I64, _I64, _I64, _P, _P],
    "htn_prologue_attention_prefetch": [_P, _I64, _I64, _I64, _P, _P, _F, _F, _P, _P, _I64, _I64,
                                        _I, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _P, _P,
                                        _I64, _I64, _I, _P],
    "htn_attention_output_scratch_bytes": [_I64, _I64, _I64, _I64, _I64],
    "htn_attention_output_fused_calls": [],
    "htn_prologue_attention_output": [_P, _I64, _I64, _I64, _P, _P, _F, _F, _P, _P, _I64, _I64,
                                      _I, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _I, _I64,
                                      _P, _P, _P, _P],
    "htn_xcc_ids": [_P, _I64, _P],
    "htn_attention_merge_in_kernel": [],
    "htn_attention_disable_in_kernel_merge": [],
}
RESTYPES = {"htn_attention_scratch_bytes": _I64, "htn_gemm_rows_scratch_bytes": _I64,
            "htn_gemm_tiles_scratch_bytes": _I64,
            "htn_gemm_library_workspace_bytes": _I64,
            "htn_gate_up_swiglu_scratch_bytes": _I64, "htn_stream_read_blocks": _I64,
            "htn_attention_output_scratch_bytes": _I64, "htn_attention_output_fused_calls": _I64,
            "htn_head_scratch_capacity": _I64}
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU, EPI_ARGMAX, EPI_RESIDUAL_NORM = 0, 1, 2, 3, 4

_lib = None
_lock = threading.Lock()


def load():
    """Load the library once; raise ImportError with the path when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `make -C hackthenorth_amd/csrc` "
                    "(or __graft_entry__.build()); there is no non-HIP fallback")
            lib = ctypes.CDLL(LIB_PATH)
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = RESTYPES.get(name, ctypes.c_int)
            if lib.htn_version() != 1:
                raise ImportError(f"{LIB_PATH}: unexpected library version")
            _lib = lib
    return _lib


def check(rc, op):
    if rc == HTN_OK:
        return
    if rc in (HTN_EINVAL, HTN_EUNSUPPORTED):
        raise ValueError(f"{op}: {'invalid argument' if rc == HTN_EINVAL else 'unsupported shape'}"
                         f" (code {rc})")
    raise RuntimeError(f"{op}: HIP launch failed (code {rc})")


def call(name, *args):
    check(getattr(load(), name)(*args), name)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("hackthenorth_amd ops run on the GPU only; got a CPU tensor")
