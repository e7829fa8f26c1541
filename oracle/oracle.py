"""ctypes binding of the CPU oracle (oracle/pa_oracle.c) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the product package (iian_amd/).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libpa_oracle.so"
REF_LIB = HERE / "_ref" / "libggml_q8_ref.so"

F32, F16, Q8_0 = 0, 1, 8
QK8_0, Q8_0_BYTES = 32, 34

_lib = None
_ref = None


def build(ref: bool = False) -> None:
    """make -C oracle [ref]; the ref target needs the reference tree."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P, I64, I32 = C.c_void_p, C.c_int64, C.c_int32
        L.pao_f32_to_f16.restype = C.c_uint16
        L.pao_f32_to_f16.argtypes = [C.c_float]
        L.pao_f16_to_f32.restype = C.c_float
        L.pao_f16_to_f32.argtypes = [C.c_uint16]
        for n in ("pao_f32_to_f16_row", "pao_f16_to_f32_row", "pao_quantize_row_q8_0",
                  "pao_quantize_row_q8_0_ref", "pao_dequantize_row_q8_0"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [P, P, I64]
        L.pao_set_rows.restype = C.c_int
        L.pao_set_rows.argtypes = [P, I64, I64, P, P, I64, C.c_int]
        L.pao_rope_cache.restype = None
        L.pao_rope_cache.argtypes = [I32, C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float,
                                     C.c_float, P, P]
        L.pao_rope_rows.restype = C.c_int
        L.pao_rope_rows.argtypes = [P, P, I64, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
                                    C.c_float, C.c_float, C.c_float, C.c_float, P]
        L.pao_rope_corr_dims.restype = None
        L.pao_rope_corr_dims.argtypes = [C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, P]
        L.pao_build_batch.restype = C.c_int64
        L.pao_build_batch.argtypes = [P, P, P, P, I32, I32, I32, P, P, P, P, P, P, P]
        L.pao_paged_attention.restype = C.c_int
        L.pao_paged_attention.argtypes = [P, P, P, C.c_int, C.c_int, P, I32, P, P, P, I32, I32, I32, I32, I32,
                                          I32, I32, C.c_float, C.c_float, I32, I32, P, I32, P, I64]
        _lib = L
    return _lib


def ref_lib() -> Optional[C.CDLL]:
    """ggml's Q8_0 routines compiled from the reference tree, or None."""
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            try:
                build(ref=True)
            except Exception:
                return None
        if not REF_LIB.exists():
            return None
        L = C.CDLL(str(REF_LIB))
        for n in ("ref_quantize_row_q8_0_x86", "ref_quantize_row_q8_0_scalar", "ref_dequantize_row_q8_0"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        _ref = L
    return _ref


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().pao_f32_to_f16_row(_p(x), _p(y), x.size)
    return y


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().pao_f16_to_f32_row(_p(h), _p(y), h.size)
    return y


def row_bytes(type_: int, n: int) -> int:
    return {F32: 4 * n, F16: 2 * n}.get(type_, n // QK8_0 * Q8_0_BYTES)


def quantize_q8_0(x: np.ndarray, variant: str = "x86") -> np.ndarray:
    """Rows of x (last dim % 32 == 0) -> uint8 [..., row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape[:-1] + (x.shape[-1] // QK8_0 * Q8_0_BYTES,), dtype=np.uint8)
    fn = lib().pao_quantize_row_q8_0 if variant == "x86" else lib().pao_quantize_row_q8_0_ref
    fn(_p(x), _p(out), x.size)
    return out


def dequantize_q8_0(b: np.ndarray, n: int) -> np.ndarray:
    """uint8 [..., n/32*34] -> f32 [..., n]."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape[:-1] + (n,), dtype=np.float32)
    lib().pao_dequantize_row_q8_0(_p(b), _p(out), out.size)
    return out


def set_rows(pool: np.ndarray, rows: np.ndarray, slots: np.ndarray, type_: int) -> int:
    """In-place KV write into pool (uint8 [n_cells, row_bytes]); returns the status."""
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    assert pool.dtype == np.uint8 and pool.flags.c_contiguous
    return lib().pao_set_rows(_p(rows), rows.shape[0], rows.shape[1], _p(slots), _p(pool), pool.shape[0], type_)


def paged_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, k_type: int, v_type: int,
                    block_tables: np.ndarray, seq_lens: np.ndarray, seq_idx: np.ndarray, pos: np.ndarray,
                    n_head_kv: int, head_dim_v: int, block_size: int, scale: float, softcap: float = 0.0,
                    causal: bool = True, n_swa: int = 0, n_threads: int = 8,
                    items: Optional[np.ndarray] = None, out: Optional[np.ndarray] = None) -> np.ndarray:
    """paged_attn_impl restated (pa_oracle.c).  q f32 [T, H, D]; pools uint8
    [n_cells, row_bytes]; returns f32 [T, H, Dv] (rows outside `items` are 0
    unless `out` is given)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    T, H, D = q.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    si = np.ascontiguousarray(seq_idx, dtype=np.int32)
    ps = np.ascontiguousarray(pos, dtype=np.int32)
    assert k_pool.flags.c_contiguous and v_pool.flags.c_contiguous
    if out is None:
        out = np.zeros((T, H, head_dim_v), dtype=np.float32)
    it = None if items is None else np.ascontiguousarray(items, dtype=np.int64)
    st = lib().pao_paged_attention(_p(q), _p(k_pool), _p(v_pool), k_type, v_type, _p(bt), bt.shape[1], _p(sl),
                                   _p(si), _p(ps), T, sl.shape[0], H, n_head_kv, D, head_dim_v, block_size,
                                   float(scale), float(softcap), int(causal), int(n_swa), _p(out), int(n_threads),
                                   None if it is None else _p(it), 0 if it is None else it.size)
    if st != 0:
        raise ValueError(f"pao_paged_attention rejected its arguments ({st})")
    return out


def build_batch(block_ids, num_computed, n_new, block_size: int, max_blocks: int) -> dict:
    """Engine::step's UBatch arrays (engine.cpp:491-535) restated (pa_oracle.c
    pao_build_batch): block tables, seq_lens, query_start_loc, pos, slots, plus
    seq_idx and the expanded per-request cell lists."""
    S = len(block_ids)
    off = np.zeros(S + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(b) for b in block_ids])
    flat = np.ascontiguousarray(np.concatenate([np.asarray(b, np.int32) for b in block_ids]) if off[-1]
                                else np.zeros(1, np.int32), dtype=np.int32)
    nc = np.ascontiguousarray(num_computed, dtype=np.int32)
    nn = np.ascontiguousarray(n_new, dtype=np.int32)
    T = int(nn.sum())
    L = nc.astype(np.int64) + nn
    bt = np.empty((S, max_blocks), np.int32)
    sl = np.empty(S, np.int32)
    qsl = np.empty(S + 1, np.int32)
    pos = np.empty(max(T, 1), np.int32)
    slots = np.empty(max(T, 1), np.int64)
    seq_idx = np.empty(max(T, 1), np.int32)
    cells = np.empty(max(int(L.sum()), 1), np.int64)
    got = lib().pao_build_batch(_p(flat), _p(off), _p(nc), _p(nn), S, block_size, max_blocks, _p(bt), _p(sl),
                                _p(qsl), _p(pos), _p(slots), _p(seq_idx), _p(cells))
    if got < 0:
        raise ValueError("pao_build_batch rejected its arguments")
    return dict(block_tables=bt, seq_lens=sl, query_start_loc=qsl, pos=pos[:T], slots=slots[:T],
                seq_idx=seq_idx[:T], cells=np.split(cells[:int(L.sum())], np.cumsum(L)[:-1]))


def rope_cache(pos: int, n_dims: int, n_ctx_orig: int = 0, freq_base: float = 10000.0, freq_scale: float = 1.0,
               ext_factor: float = 0.0, attn_factor: float = 1.0, beta_fast: float = 32.0, beta_slow: float = 1.0,
               freq_factors: Optional[np.ndarray] = None) -> np.ndarray:
    """(cos, sin) per pair of one position (pa_oracle.c pao_rope_cache)."""
    out = np.empty(n_dims, np.float32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
    lib().pao_rope_cache(int(pos), n_dims, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor, beta_fast,
                         beta_slow, None if ff is None else _p(ff), _p(out))
    return out


def rope_rows(x: np.ndarray, pos: np.ndarray, n_heads: int, head_dim: int, n_dims: int, mode: int = 0,
              n_ctx_orig: int = 0, freq_base: float = 10000.0, freq_scale: float = 1.0, ext_factor: float = 0.0,
              attn_factor: float = 1.0, beta_fast: float = 32.0, beta_slow: float = 1.0,
              freq_factors: Optional[np.ndarray] = None) -> np.ndarray:
    """ggml_rope_ext forward on f32 rows [T, n_heads*head_dim] (pao_rope_rows)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    ps = np.ascontiguousarray(pos, dtype=np.int32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
    st = lib().pao_rope_rows(_p(x), _p(y), x.shape[0], n_heads, head_dim, _p(ps), n_dims, mode, n_ctx_orig,
                             freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow,
                             None if ff is None else _p(ff))
    if st != 0:
        raise ValueError("pao_rope_rows rejected its arguments")
    return y


def rope_corr_dims(n_dims: int, n_ctx_orig: int, freq_base: float, beta_fast: float, beta_slow: float):
    out = np.empty(2, np.float32)
    lib().pao_rope_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, _p(out))
    return out
