"""ctypes binding of libiian_pa.so (the C ABI declared in include/iian_pa.h).

Loading fails loudly: there is no fallback path.  Build the library first with
``python -m iian_amd.build``.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libiian_pa.so"

OK = 0
ERR_NULL = -1
ERR_ARG = -2
ERR_UNSUPPORTED = -3
ERR_WORKSPACE = -4
ERR_HIP = -5
ERR_SCRATCH = -6
NOALLOC_SCRATCH_BYTES = 64 << 20

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q8_0 = 8

# name -> (restype, argtypes); exactly the entry points of include/iian_pa.h
_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
SIGNATURES = {
    "iian_pa_status_string": (C.c_char_p, [C.c_int]),
    "iian_pa_supported": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    "iian_pa_kv_write": (C.c_int, [_P, _P, _I64, _I64, _P, _P, _I64, C.c_int, _P]),
    "iian_pa_kv_write_kv": (C.c_int, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, C.c_int, C.c_int, _P]),
    "iian_pa_workspace_size": (C.c_size_t, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "iian_pa_attention": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, _I32, _P, _I32, _P, _P, _P,
                                    _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                    C.c_float, C.c_float, _I32, _I32, _P, _P, C.c_size_t, _P]),
    "iian_pa_attention_noalloc": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, _I32, _P, _I32, _P, _P, _P,
                                            _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                            C.c_float, C.c_float, _I32, _I32, _P, _P]),
    "iian_pa_write_attention": (C.c_int, [_P, _P, _P, _P, _P, _P, C.c_int, C.c_int, _I32, _P, _I32, _P, _P, _P,
                                          _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                          C.c_float, C.c_float, _I32, _I32, _P, _P, C.c_size_t, _P]),
    "iian_pa_build_batch": (C.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P]),
    "iian_pa_swa_free_blocks": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _P, _I32]),
    "iian_pa_rope_kv_write": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _I64,
                                        C.c_int, C.c_int, _P]),
    "iian_pa_runtime_create": (C.c_int, [_P, _P]),
    "iian_pa_runtime_destroy": (None, [_P]),
    "iian_pa_runtime_begin_step": (C.c_int, [_P, _P, _P, _P, _P, _P, _I32]),
    "iian_pa_runtime_layer": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, C.c_float, _I32, _I32, _P]),
    "iian_pa_runtime_errors": (C.c_int, [_P, _P, _P]),
    "iian_pa_dequant_q8_0": (C.c_int, [_P, _P, _I64, _P, _I64, _I64, _P]),
}


class RuntimeConfig(C.Structure):
    """iian_pa_runtime_config of include/iian_pa.h."""
    _fields_ = [(n, C.c_int32) for n in ("max_seqs", "max_tokens", "max_blocks_per_seq", "max_total_blocks",
                                         "n_head", "n_head_kv", "head_dim", "head_dim_v", "block_size", "num_blocks",
                                         "type_k", "type_v")]


class RopeParams(C.Structure):
    """iian_pa_rope_params of include/iian_pa.h."""
    _fields_ = [("n_dims", C.c_int32), ("mode", C.c_int32), ("n_ctx_orig", C.c_int32),
                ("freq_base", C.c_float), ("freq_scale", C.c_float), ("ext_factor", C.c_float),
                ("attn_factor", C.c_float), ("beta_fast", C.c_float), ("beta_slow", C.c_float),
                ("freq_factors", C.c_void_p)]

_lib = None


class PagedAttnError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed: {status} ({status_string(status)})")


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m iian_amd.build` "
                           "(there is no CPU fallback for the paged-attention kernels)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().iian_pa_status_string(status).decode()


def check(fn: str, status: int) -> None:
    if status != OK:
        raise PagedAttnError(fn, status)
