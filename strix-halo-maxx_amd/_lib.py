"""ctypes binding of the C-ABI library libshmaxx.so (declared in include/shmaxx.h).

Mirrors the reference's loader (moondream/gpu/hgemm.py:21-33, hattn.py:5-15): one CDLL, explicit argtypes, int
status returns, raw device pointers and the caller's HIP stream. There is no fallback: if the library is missing the
first call raises, so a GPU run can never silently use another implementation.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libshmaxx.so")

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_long
F = ctypes.c_float

# name -> argtypes (every entry point returns int status)
SIGNATURES = {
    "mx_gemm_bf16": [P, I, I, P, L, P, L, P, P, L, I, P, L, I, I, I, I, I, I, P, L, P, L],
    "mx_gemm_check": [I, I, P, L, P, L, P, P, L, P, L, I, I, I, I, I, P, L, P, L],
    "mx_gemm_pick": [I, I, I],
    "mx_gemm_ws_elems": [I, I, I, I],
    "mx_track_head_blob_elems": [I, I, I],
    "mx_resize_patchify_u8": [P, P, I, I, P, L, I, I, I],
    "mx_gemm_reduce": [P, P, I, L, L, P, P, L, I, P, L, I, I, I, I],
    "mx_gemm_i8_partial": [P, I, I, P, L, P, L, P, L, L, I, I, I, I],
    "mx_gemm_i8_reduce": [P, P, I, L, L, P, P, P, P, L, I, P, L, I, I, I],
    "mx_ssm_step_rows": [P, P, P, P, P, L, P, L, P, P, P, P, P, P, P, P, P, P, L, I, I, P, P, I, P, L],
    "mx_track_heads": [P, P, L, I, I, I, P, I, F, F, P, F, F, I, P, P, L, P],
    "mx_gemm_ws_counters": [I, I, I, I],
    "mx_gemm_ncfg": [],
    "mx_gemm_cfg_tile": [I, ctypes.POINTER(I), ctypes.POINTER(I)],
    "mx_gemm_cfg_kind": [I],
    "mx_gemm_bf16_partial": [P, I, I, P, L, P, L, P, L, L, I, I, I, I],
    "mx_gemm_i8": [P, I, P, L, P, L, P, P, P, P, L, I, P, L, I, I, I, I, I, P, L],
    "mx_quant_rows_i8": [P, P, L, P, L, P, I, I],
    "mx_quant_weight_i8": [P, P, L, P, L, P, I, I],
    "mx_sdpa": [P, P, L, L, L, P, L, L, L, P, L, L, L, P, L, L, L, I, I, I, I, I, F, I, I],
    "mx_sdpa_check": [P, L, P, L, P, L, P, L, I, I, I, I, I],
    "mx_sdpa_tiling": [I, I, I, I, P],
    "mx_layernorm": [P, P, L, P, P, P, L, I, I, F],
    "mx_residual_layernorm": [P, P, I, L, L, P, P, L, P, L, P, P, P, L, I, I, F],
    "mx_residual_rmsnorm": [P, P, I, L, L, P, P, L, P, L, P, P, L, I, I, F],
    "mx_rmsnorm": [P, P, L, P, P, L, I, I, F],
    "mx_patchify_u8": [P, P, P, L, I, I, I, I],
    "mx_rope_kv": [P, P, L, P, P, P, P, I, I, I, I, I, I, I],
    "mx_ln_gemv2": [P, P, P, P, F, P, L, P, I, I, I, P, P, I],
    "mx_gemv_dual_res": [P, P, P, P, I, P, P, P, I, P, P, I],
    "mx_ln_gemv2_i8": [P, P, P, P, F, P, L, P, P, I, I, I, P, P, I],
    "mx_gemv_dual_res_i8": [P, P, P, P, P, I, P, P, P, P, I, P, P, I],
    "mx_lm_argmax_nparts": [I],
    "mx_ln_gemv_argmax": [P, P, P, P, F, P, L, P, I, I, P, P, I],
    "mx_embed_step": [P, P, I, P, I, P, I, P, I, P],
    "mx_decode_attn": [P, P, P, P, P, I, I, P, I, F, P, P, P],
    "mx_decode_attn_fc2": [P, P, P, P, P, I, I, P, F, I, P, P, P, P, P, I, P, I],
    "mx_gemv_res2": [P, P, P, I, P, P, P, I, P, P, I],
    "mx_decode_attn_fc2_i8": [P, P, P, P, P, I, I, P, F, I, P, P, P, P, P, P, I, P, I],
    "mx_gemv_res2_i8": [P, P, P, I, P, P, P, P, I, P, P, I],
    "mx_decode_step_mk": [P, P, I, I, P, P, P, P, I, P, P, F, F, P, P, I, P, I, P, P, P],
    "mx_decode_step_mk_i8": [P, P, I, I, P, P, P, P, I, P, P, F, F, P, P, I, P, I, P, P, P],
    "mx_decode_mk_words": [],
    "mx_decode_mk_grid": [],
    "mx_decode_mk_layer_bytes": [],
    "mx_ssm_step": [P, P, P, P, P, L, P, L, P, P, P, P, P, P, P, P, P, P, L, I, I],
    "mx_ssm_prep": [P, P, L, L, P, P, P, P, P, P, P, P, P, P, I, I, I],
    "mx_rglru_scan": [P, P, P, P, I, I, I, P, L, L, P, L, L],
    "mx_rglru_step": [P, P, L, P, P, P, P, P, P, P, P, L, I, I],
    "mx_counter_add": [P, P, I],
    "mx_gemm_bf16_noalloc": [P, I, I, P, L, P, L, P, P, L, I, P, L, I, I, I, I, I, I],
    "mx_gemm_noalloc_max_ws": [],
    "mx_gemm_bf16_res_ln": [P, P, L, P, L, P, P, L, P, L, P, P, P, L, I, I, I, I, F, P, L, P, L],
    "mx_gemm_bf16_res_rms": [P, P, L, P, L, P, P, L, P, L, P, P, L, I, I, I, I, F, P, L, P, L],
    "mx_gemm_res_ln_stats_words": [I, I],
    "mx_gemm_res_ln_sync_words": [I],
}

STATUS = {0: "ok", -1: "bad config", -2: "unsupported shape/stride", -3: "split-K workspace too small",
          -4: "operand layout/alignment", -5: "HIP launch failed", -6: "null pointer"}

RESTYPE = {"mx_gemm_ws_elems": L, "mx_gemm_ws_counters": L, "mx_track_head_blob_elems": L,
           "mx_gemm_noalloc_max_ws": L, "mx_sdpa_tiling": None, "mx_gemm_res_ln_stats_words": L,
           "mx_gemm_res_ln_sync_words": L}

_lib = None


class MxError(RuntimeError):
    pass


def load():
    """Load libshmaxx.so (built by build.py) and declare every entry point."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MxError(f"{LIB_PATH} is missing: build it first (python __graft_entry__.py build)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = RESTYPE.get(name, I)
        _lib = lib
    return _lib


def check(rc, what):
    if rc != 0:
        raise MxError(f"{what} returned {rc} ({STATUS.get(rc, 'unknown')})")


def call(name, *args):
    """Call entry point `name`; raise MxError on a non-zero status."""
    rc = getattr(load(), name)(*args)
    check(rc, name)
    return rc


def stream():
    """The HIP stream handle of torch's current stream (launches are asynchronous on it)."""
    import torch
    return torch.cuda.current_stream().cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()
