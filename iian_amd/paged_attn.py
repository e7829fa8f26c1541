"""Host-side mirror of iian's paged-attention operator over the gfx950 C ABI.

Names and argument meaning follow the reference (CocoRoF/iian):

* ``PagedAttnParams``        src/iian/paged_attn.h:16-22 (the UBatch pointer
                             becomes the explicit ``PagedBatch`` argument)
* ``paged_attn_supported``   src/iian/paged_attn.cpp:15-18
* ``set_rows``               ggml_set_rows as build_attn uses it for the KV
                             write, src/iian/graph.cpp:314-322
* ``build_paged_attn``       src/iian/paged_attn.h:29-30 / paged_attn.cpp:159-169:
                             q [T][H][D] f32 -> out [T][H][Dv] f32
* ``PagedBatch.from_ubatch`` the UBatch of include/iian/graph.h:22-38 as the
                             engine fills it (src/iian/engine.cpp:491-535),
                             compressed losslessly to block tables

Where the reference aborts on a violated precondition (GGML_ASSERT in
paged_attn.cpp:161-162 and ggml-cpu/ops.cpp:5263) this layer raises
``PagedAttnError`` / ``ValueError`` instead.  All device work goes through
libiian_pa.so; torch is used only for device memory and streams.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Callable, Optional, Sequence

import numpy as np
import torch

from . import _lib

GGML_TYPE_F32 = _lib.TYPE_F32
GGML_TYPE_F16 = _lib.TYPE_F16
GGML_TYPE_Q8_0 = _lib.TYPE_Q8_0
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def row_bytes(type_: int, n: int) -> int:
    """ggml_row_size for the pool types."""
    if type_ == GGML_TYPE_F32:
        return 4 * n
    if type_ == GGML_TYPE_F16:
        return 2 * n
    if type_ == GGML_TYPE_Q8_0:
        if n % QK8_0:
            raise ValueError("Q8_0 rows need a multiple of 32 elements")
        return n // QK8_0 * Q8_0_BLOCK_BYTES
    raise ValueError(f"unsupported ggml type {type_}")


@dataclass
class PagedAttnParams:
    """src/iian/paged_attn.h:16-22."""
    scale: float = 1.0
    softcap: float = 0.0      # 0 = off
    causal: bool = True
    n_swa: int = 0            # 0 = full attention for this layer


class KVPool:
    """One layer's K or V cell pool: ``n_cells`` rows of ``n_embd`` elements of
    ``type_`` (src/iian/kv_cache.cpp:156-169), zero-initialised like the
    reference's ggml_backend_buffer_clear (kv_cache.cpp:173)."""

    def __init__(self, n_cells: int, n_embd: int, type_: int, device="cuda"):
        self.n_cells = n_cells
        self.n_embd = n_embd
        self.type = type_
        self.row_bytes = row_bytes(type_, n_embd)
        self.data = torch.zeros((n_cells, self.row_bytes), dtype=torch.uint8, device=device)

    @classmethod
    def wrap(cls, data: torch.Tensor, n_embd: int, type_: int) -> "KVPool":
        """Use an existing [n_cells, row_bytes] byte tensor as the pool."""
        self = cls.__new__(cls)
        self.n_cells = data.shape[0]
        self.n_embd = n_embd
        self.type = type_
        self.row_bytes = row_bytes(type_, n_embd)
        if data.dtype != torch.uint8 or data.dim() != 2 or data.shape[1] != self.row_bytes or not data.is_contiguous():
            raise ValueError("pool tensor must be contiguous uint8 [n_cells, row_bytes]")
        self.data = data
        return self

    def view_f16(self) -> torch.Tensor:
        if self.type != GGML_TYPE_F16:
            raise ValueError("not an f16 pool")
        return self.data.view(torch.float16)


@dataclass
class PagedBatch:
    """Device-side description of a micro-batch (the UBatch of
    include/iian/graph.h:22-38 with each sequence's cell list given as its
    block table; cell_pos[i] == i always holds, engine.cpp:505)."""
    block_tables: torch.Tensor      # int32 [S, max_blocks]
    seq_lens: torch.Tensor          # int32 [S]
    query_start_loc: torch.Tensor   # int32 [S+1]
    pos: torch.Tensor               # int32 [T]
    slots: torch.Tensor             # int64 [T]
    max_query_len: int
    block_size: int = 16

    @property
    def n_tokens(self) -> int:
        return int(self.pos.shape[0])

    @property
    def n_seqs(self) -> int:
        return int(self.seq_lens.shape[0])

    @classmethod
    def from_ubatch(cls, pos: Sequence[int], seq_idx: Sequence[int], slots: Sequence[int],
                    seq_cells: Sequence[Sequence[int]], block_size: int = 16,
                    seq_cell_pos: Optional[Sequence[Sequence[int]]] = None, device="cuda") -> "PagedBatch":
        """Compress a reference UBatch (per-token pos/seq_idx/slots, per-sequence
        absolute cells) into block tables.  Raises ValueError when the cells are
        not block-structured (cell i must be table[i // bs] * bs + i % bs,
        kv_cache.h:135-137), when cell_pos[i] != i, or when a sequence's tokens
        are not contiguous in the batch (engine.cpp:508-513 builds them so)."""
        seq_idx = np.asarray(seq_idx, dtype=np.int64)
        S = len(seq_cells)
        T = len(pos)
        if len(seq_idx) != T or len(slots) != T:
            raise ValueError("pos, seq_idx and slots must have one entry per token")
        if T and (seq_idx.min() < 0 or seq_idx.max() >= S):
            raise ValueError("seq_idx out of range")
        if T and np.any(np.diff(seq_idx) < 0):
            raise ValueError("tokens of a sequence must be contiguous and sequences in order")
        counts = np.bincount(seq_idx, minlength=S) if T else np.zeros(S, dtype=np.int64)
        qsl = np.zeros(S + 1, dtype=np.int32)
        qsl[1:] = np.cumsum(counts)
        lens = np.array([len(c) for c in seq_cells], dtype=np.int32)
        max_blocks = max(1, int(((lens.max() if S else 0) + block_size - 1) // block_size))
        bt = np.zeros((S, max_blocks), dtype=np.int32)
        for s, cells in enumerate(seq_cells):
            cells = np.asarray(cells, dtype=np.int64)
            if seq_cell_pos is not None and not np.array_equal(np.asarray(seq_cell_pos[s]), np.arange(len(cells))):
                raise ValueError("cell_pos[i] must equal i")
            nb = (len(cells) + block_size - 1) // block_size
            for b in range(nb):
                seg = cells[b * block_size:(b + 1) * block_size]
                blk = seg[0] // block_size
                if seg[0] % block_size or not np.array_equal(seg, blk * block_size + np.arange(len(seg))):
                    raise ValueError(f"sequence {s}: cells are not block-structured at block {b}")
                bt[s, b] = blk
        t = lambda a, dt: torch.as_tensor(np.asarray(a), dtype=dt, device=device)
        return cls(block_tables=t(bt, torch.int32), seq_lens=t(lens, torch.int32),
                   query_start_loc=t(qsl, torch.int32), pos=t(pos, torch.int32), slots=t(slots, torch.int64),
                   max_query_len=int(counts.max()) if S else 0, block_size=block_size)


@dataclass
class RequestBlocks:
    """Device copies of the per-request state iian_pa_build_batch reads: the
    packed block ids of every scheduled request (KVRequestState::block_ids,
    include/iian/kv_cache.h:93-97), the offsets of each request's ids, and its
    computed-token and new-token counts (Request::num_computed_tokens,
    ScheduledRequest::n_new_tokens)."""
    block_ids: torch.Tensor      # int32 [sum of blocks]
    block_off: torch.Tensor      # int32 [S+1]
    num_computed: torch.Tensor   # int32 [S]
    n_new: torch.Tensor          # int32 [S]

    @classmethod
    def pack(cls, block_ids: Sequence[Sequence[int]], num_computed: Sequence[int], n_new: Sequence[int],
             device="cuda") -> "RequestBlocks":
        S = len(block_ids)
        if len(num_computed) != S or len(n_new) != S:
            raise ValueError("one block list, computed count and new count per request")
        off = np.zeros(S + 1, dtype=np.int64)
        off[1:] = np.cumsum([len(b) for b in block_ids])
        if off[-1] > np.iinfo(np.int32).max:
            raise ValueError("too many blocks")
        flat = np.concatenate([np.asarray(b, dtype=np.int32) for b in block_ids]) if off[-1] else np.zeros(1, np.int32)
        t = lambda a: torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32), device=device)
        return cls(block_ids=t(flat), block_off=t(off), num_computed=t(num_computed), n_new=t(n_new))


def build_batch(req: RequestBlocks, n_tokens: int, block_size: int, max_blocks: int, num_blocks: int,
                max_query_len: Optional[int] = None, out: Optional[PagedBatch] = None,
                err_flag: Optional[torch.Tensor] = None, bind: bool = False) -> PagedBatch:
    """The step's PagedBatch built on the device by iian_pa_build_batch from
    the requests' block ids and counts (the work of Engine::step's UBatch
    loop, src/iian/engine.cpp:491-535, without expanding cells on the host).
    `out` (optional) supplies the output tensors, which makes the call
    allocation-free."""
    S = int(req.n_new.shape[0])
    dev = req.n_new.device
    for name in ("block_ids", "block_off", "num_computed", "n_new"):
        t = getattr(req, name)
        if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"req.{name} must be a contiguous int32 1-d tensor on {dev}")
    if req.block_off.shape[0] != S + 1 or req.num_computed.shape[0] != S:
        raise ValueError("block_off must have S+1 entries and num_computed S")
    if out is None:
        out = PagedBatch(block_tables=torch.empty((S, max_blocks), dtype=torch.int32, device=dev),
                         seq_lens=torch.empty(S, dtype=torch.int32, device=dev),
                         query_start_loc=torch.empty(S + 1, dtype=torch.int32, device=dev),
                         pos=torch.empty(n_tokens, dtype=torch.int32, device=dev),
                         slots=torch.empty(n_tokens, dtype=torch.int64, device=dev),
                         max_query_len=0, block_size=block_size)
    else:
        if tuple(out.block_tables.shape) != (S, max_blocks) or out.pos.shape[0] != n_tokens:
            raise ValueError("out does not match the batch shape")
        _check_batch(out, dev)
    out.max_query_len = int(max_query_len) if max_query_len is not None else out.max_query_len
    out.block_size = block_size
    args = (_stream(), req.block_ids.data_ptr(), req.block_off.data_ptr(), req.num_computed.data_ptr(),
            req.n_new.data_ptr(), S, n_tokens, block_size, max_blocks, num_blocks, out.block_tables.data_ptr(),
            out.seq_lens.data_ptr(), out.query_start_loc.data_ptr(), out.pos.data_ptr(), out.slots.data_ptr(),
            _ptr(err_flag))
    if bind:
        return out, args
    _lib.check("iian_pa_build_batch", _lib.load().iian_pa_build_batch(*args))
    return out


def bind_build_batch(req: RequestBlocks, n_tokens: int, block_size: int, max_blocks: int, num_blocks: int,
                     out: PagedBatch, err_flag: Optional[torch.Tensor] = None) -> Callable[[], None]:
    """build_batch checked once and bound to these buffers and the current
    stream: the returned function issues iian_pa_build_batch again with one
    ctypes call, as an engine holding its arguments would."""
    _, args = build_batch(req, n_tokens, block_size, max_blocks, num_blocks, out=out, err_flag=err_flag, bind=True)
    fn = _lib.load().iian_pa_build_batch

    def call() -> None:
        st = fn(*args)
        if st:
            _lib.check("iian_pa_build_batch", st)
    return call


def swa_free_blocks(batch: PagedBatch, n_swa: int, clear_table: bool = False) -> torch.Tensor:
    """Per sequence, the leading blocks a sliding-window layer (window n_swa)
    will never read again at this step or later (the reference's planned
    out-of-window block freeing, docs/ROADMAP.md:33): int32 [S].  With
    clear_table, those block-table entries are set to -1."""
    S = batch.n_seqs
    dev = batch.pos.device
    _check_batch(batch, dev)
    n_free = torch.empty(S, dtype=torch.int32, device=dev)
    st = _lib.load().iian_pa_swa_free_blocks(_stream(), batch.query_start_loc.data_ptr(), batch.pos.data_ptr(), S,
                                             batch.n_tokens, int(n_swa), batch.block_size, n_free.data_ptr(),
                                             batch.block_tables.data_ptr() if clear_table else None,
                                             int(batch.block_tables.shape[1]))
    _lib.check("iian_pa_swa_free_blocks", st)
    return n_free


class PagedAttnRuntime:
    """The engine-side runtime (iian_pa_runtime_*): device buffers of one
    step allocated once; begin_step per engine step from the scheduler's
    per-request block ids and counts, layer per attention layer.  Replaces the
    host UBatch expansion of Engine::step (src/iian/engine.cpp:491-535) and
    the paged branch of build_attn (src/iian/graph.cpp:314-337)."""

    def __init__(self, max_seqs: int, max_tokens: int, max_blocks_per_seq: int, max_total_blocks: int, n_head: int,
                 n_head_kv: int, head_dim: int, head_dim_v: int, block_size: int, num_blocks: int, type_k: int,
                 type_v: int):
        self._lib = _lib.load()
        self.cfg = _lib.RuntimeConfig(max_seqs, max_tokens, max_blocks_per_seq, max_total_blocks, n_head, n_head_kv,
                                      head_dim, head_dim_v, block_size, num_blocks, type_k, type_v)
        h = C.c_void_p()
        _lib.check("iian_pa_runtime_create", self._lib.iian_pa_runtime_create(C.byref(self.cfg), C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            self._lib.iian_pa_runtime_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def begin_step(self, block_ids: Sequence[Sequence[int]], num_computed: Sequence[int],
                   n_new: Sequence[int]) -> None:
        S = len(block_ids)
        arrs = [np.ascontiguousarray(b, dtype=np.int32) for b in block_ids]
        ptrs = (C.c_void_p * max(S, 1))(*[a.ctypes.data if a.size else None for a in arrs])
        nb = np.array([a.size for a in arrs], np.int32)
        nc = np.ascontiguousarray(num_computed, dtype=np.int32)
        nn = np.ascontiguousarray(n_new, dtype=np.int32)
        self._T = None
        st = self._lib.iian_pa_runtime_begin_step(self._h, _stream(), ptrs, nb.ctypes.data, nc.ctypes.data,
                                                  nn.ctypes.data, S)
        _lib.check("iian_pa_runtime_begin_step", st)
        self._T = int(nn.sum())

    def layer(self, q: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor, k_pool: KVPool, v_pool: KVPool,
              params: PagedAttnParams, out: torch.Tensor, rope: Optional[RopeParams] = None,
              q_rot: Optional[torch.Tensor] = None) -> None:
        c = self.cfg
        T = getattr(self, "_T", None)
        if T is None:
            raise ValueError("layer() needs a successful begin_step() first")
        dev = q.device
        shapes = ((q, (T, c.n_head, c.head_dim)), (k_rows, (T, c.n_head_kv * c.head_dim)),
                  (v_rows, (T, c.n_head_kv * c.head_dim_v)), (out, (T, c.n_head, c.head_dim_v)))
        for t, shp in shapes:
            if tuple(t.shape) != shp:
                raise ValueError(f"expected a tensor of shape {shp} for this step, got {tuple(t.shape)}")
        for t, _ in shapes:
            if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda or t.device != dev:
                raise ValueError("q, k_rows, v_rows and out must be contiguous f32 tensors on one GPU")
        n_cells = c.num_blocks * c.block_size
        for pool, ty, e in ((k_pool, c.type_k, c.n_head_kv * c.head_dim), (v_pool, c.type_v, c.n_head_kv * c.head_dim_v)):
            if pool.type != ty or pool.n_cells != n_cells or pool.n_embd != e or pool.data.device != dev:
                raise ValueError(f"pools must hold {n_cells} cells of {e} elements of the configured types on q's device")
        prm = None
        if rope is not None:
            if q_rot is None:
                raise ValueError("rope needs q_rot (q itself for an in-place rotation)")
            if (q_rot.dtype != torch.float32 or not q_rot.is_contiguous() or q_rot.device != dev
                    or q_rot.shape != q.shape):
                raise ValueError("q_rot must be a contiguous f32 tensor shaped like q on q's device")
            ff = rope.freq_factors
            if ff is not None and (ff.dtype != torch.float32 or ff.numel() < rope.n_dims // 2 or ff.device != dev):
                raise ValueError("freq_factors must be f32 with n_dims/2 values on q's device")
            prm = _lib.RopeParams(rope.n_dims, rope.mode, rope.n_ctx_orig, rope.freq_base, rope.freq_scale,
                                  rope.ext_factor, rope.attn_factor, rope.beta_fast, rope.beta_slow,
                                  _ptr(rope.freq_factors))
        st = self._lib.iian_pa_runtime_layer(self._h, _stream(), q.data_ptr(), _ptr(q_rot), k_rows.data_ptr(),
                                             v_rows.data_ptr(), C.byref(prm) if prm is not None else None,
                                             k_pool.data.data_ptr(), v_pool.data.data_ptr(), float(params.scale),
                                             float(params.softcap), int(bool(params.causal)), int(params.n_swa),
                                             out.data_ptr())
        _lib.check("iian_pa_runtime_layer", st)

    def errors(self) -> int:
        e = C.c_int32(0)
        _lib.check("iian_pa_runtime_errors", self._lib.iian_pa_runtime_errors(self._h, _stream(), C.byref(e)))
        return int(e.value)


def paged_attn_supported(type_k: int, type_v: int, max_alibi_bias: float, head_dim: int = 128,
                         head_dim_v: Optional[int] = None) -> bool:
    """src/iian/paged_attn.cpp:15-18, as supported by the gfx950 kernels."""
    lib = _lib.load()
    return bool(lib.iian_pa_supported(type_k, type_v, head_dim, head_dim if head_dim_v is None else head_dim_v,
                                      float(max_alibi_bias)))


def set_rows(pool: KVPool, rows: torch.Tensor, slots: torch.Tensor, err_flag: Optional[torch.Tensor] = None) -> KVPool:
    """ggml_set_rows(pool, rows, slots) (src/iian/graph.cpp:319-320): row
    slots[t] of the pool <- convert(rows[t]).  rows: f32 [T, n_embd]."""
    if rows.dtype != torch.float32 or rows.dim() != 2 or rows.shape[1] != pool.n_embd:
        raise ValueError("rows must be f32 [n_tokens, n_embd]")
    if slots.dtype != torch.int64 or slots.shape != (rows.shape[0],):
        raise ValueError("slots must be int64 [n_tokens]")
    rows = rows.contiguous()
    lib = _lib.load()
    st = lib.iian_pa_kv_write(_stream(), rows.data_ptr(), rows.shape[0], rows.shape[1], slots.data_ptr(),
                              pool.data.data_ptr(), pool.n_cells, pool.type, _ptr(err_flag))
    _lib.check("iian_pa_kv_write", st)
    return pool


def _set_rows_kv_args(k_pool: KVPool, v_pool: KVPool, k_rows: torch.Tensor, v_rows: torch.Tensor,
                      slots: torch.Tensor, err_flag: Optional[torch.Tensor]):
    """Checks a call of iian_pa_kv_write_kv and returns its argument tuple
    (the row tensors must already be contiguous)."""
    for pool, rows in ((k_pool, k_rows), (v_pool, v_rows)):
        if rows.dtype != torch.float32 or rows.dim() != 2 or rows.shape[1] != pool.n_embd:
            raise ValueError("rows must be f32 [n_tokens, n_embd]")
    if k_rows.shape[0] != v_rows.shape[0] or k_pool.n_cells != v_pool.n_cells:
        raise ValueError("K and V must have the same token count and cell count")
    if slots.dtype != torch.int64 or slots.shape != (k_rows.shape[0],):
        raise ValueError("slots must be int64 [n_tokens]")
    if not (k_rows.is_contiguous() and v_rows.is_contiguous()):
        raise ValueError("rows must be contiguous")
    return (_stream(), k_rows.data_ptr(), v_rows.data_ptr(), k_rows.shape[0], k_rows.shape[1], v_rows.shape[1],
            slots.data_ptr(), k_pool.data.data_ptr(), v_pool.data.data_ptr(), k_pool.n_cells, k_pool.type,
            v_pool.type, _ptr(err_flag))


def set_rows_kv(k_pool: KVPool, v_pool: KVPool, k_rows: torch.Tensor, v_rows: torch.Tensor, slots: torch.Tensor,
                err_flag: Optional[torch.Tensor] = None) -> None:
    """The layer's two set_rows calls (K pool, then V pool, same slots;
    src/iian/graph.cpp:319-320) as one launch when the pool types match."""
    args = _set_rows_kv_args(k_pool, v_pool, k_rows.contiguous(), v_rows.contiguous(), slots, err_flag)
    _lib.check("iian_pa_kv_write_kv", _lib.load().iian_pa_kv_write_kv(*args))


def bind_set_rows_kv(k_pool: KVPool, v_pool: KVPool, k_rows: torch.Tensor, v_rows: torch.Tensor,
                     slots: torch.Tensor, err_flag: Optional[torch.Tensor] = None) -> Callable[[], None]:
    """set_rows_kv checked once and bound to these buffers and the current
    stream (contiguous rows), as bind_paged_attn."""
    args = _set_rows_kv_args(k_pool, v_pool, k_rows, v_rows, slots, err_flag)
    fn = _lib.load().iian_pa_kv_write_kv

    def call() -> None:
        st = fn(*args)
        if st:
            _lib.check("iian_pa_kv_write_kv", st)
    return call


@dataclass
class RopeParams:
    """The rope arguments of ggml_rope_ext as build_rope passes them
    (src/iian/graph.cpp:250-253).  mode: 0 = NORMAL, 2 = NEOX."""
    n_dims: int
    mode: int = 0
    n_ctx_orig: int = 0
    freq_base: float = 10000.0
    freq_scale: float = 1.0
    ext_factor: float = 0.0
    attn_factor: float = 1.0
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    freq_factors: Optional[torch.Tensor] = None   # f32 [n_dims/2] on the device


def rope_set_rows_kv(k_pool: KVPool, v_pool: KVPool, k_rows: torch.Tensor, v_rows: torch.Tensor,
                     slots: torch.Tensor, pos: torch.Tensor, rope: RopeParams, n_head_kv: int,
                     q: Optional[torch.Tensor] = None, q_out: Optional[torch.Tensor] = None,
                     err_flag: Optional[torch.Tensor] = None, bind: bool = False) -> Optional[torch.Tensor]:
    """build_rope on K (and q) fused with the layer's two set_rows calls
    (src/iian/graph.cpp:250-253, 319-320), one launch: k_pool[slots[t]] <-
    rope(k_rows[t], pos[t]), v_pool[slots[t]] <- v_rows[t], and, when q
    ([T, H, D]) is given, q rotated into q_out (a new tensor, or q itself when
    q_out is q).  Returns the rotated q, or None."""
    T = k_rows.shape[0]
    for pool, rows in ((k_pool, k_rows), (v_pool, v_rows)):
        if rows.dtype != torch.float32 or rows.dim() != 2 or rows.shape[1] != pool.n_embd or not rows.is_cuda:
            raise ValueError("rows must be f32 [n_tokens, n_embd] GPU tensors")
    if v_rows.shape[0] != T or k_pool.n_cells != v_pool.n_cells:
        raise ValueError("K and V must have the same token count and cell count")
    if k_pool.n_embd % n_head_kv or v_pool.n_embd % n_head_kv:
        raise ValueError("pool rows must hold n_head_kv heads")
    if slots.dtype != torch.int64 or slots.shape != (T,) or pos.dtype != torch.int32 or pos.shape != (T,):
        raise ValueError("slots must be int64 [T] and pos int32 [T]")
    dev = k_rows.device
    if not (slots.is_contiguous() and pos.is_contiguous()) or slots.device != dev or pos.device != dev:
        raise ValueError("slots and pos must be contiguous and on the rows' device")
    if v_rows.device != dev or k_pool.data.device != dev or v_pool.data.device != dev:
        raise ValueError("rows and pools must be on one device")
    D = k_pool.n_embd // n_head_kv
    H = 0
    if q is not None:
        if (q.dtype != torch.float32 or q.dim() != 3 or q.shape[0] != T or q.shape[2] != D or not q.is_contiguous()
                or q.device != dev):
            raise ValueError("q must be contiguous f32 [T, H, D] on the rows' device")
        H = q.shape[1]
        if q_out is None:
            q_out = torch.empty_like(q)
        elif (q_out.shape != q.shape or q_out.dtype != q.dtype or not q_out.is_contiguous()
              or q_out.device != dev):
            raise ValueError("q_out must match q (shape, dtype, device) and be contiguous")
    elif q_out is not None:
        raise ValueError("q_out without q")
    ff = rope.freq_factors
    if ff is not None and (ff.dtype != torch.float32 or ff.numel() < rope.n_dims // 2 or ff.device != dev):
        raise ValueError("freq_factors must be f32 with n_dims/2 values on the rows' device")
    prm = _lib.RopeParams(rope.n_dims, rope.mode, rope.n_ctx_orig, rope.freq_base, rope.freq_scale, rope.ext_factor,
                          rope.attn_factor, rope.beta_fast, rope.beta_slow, _ptr(ff))
    if bind and not (k_rows.is_contiguous() and v_rows.is_contiguous()):
        raise ValueError("bound rows must be contiguous")
    k_rows, v_rows = k_rows.contiguous(), v_rows.contiguous()
    args = (_stream(), k_rows.data_ptr(), v_rows.data_ptr(), _ptr(q), _ptr(q_out), pos.data_ptr(), slots.data_ptr(),
            T, H, n_head_kv, D, v_pool.n_embd // n_head_kv, C.byref(prm), k_pool.data.data_ptr(),
            v_pool.data.data_ptr(), k_pool.n_cells, k_pool.type, v_pool.type, _ptr(err_flag))
    if bind:
        return q_out, (args, prm)
    _lib.check("iian_pa_rope_kv_write", _lib.load().iian_pa_rope_kv_write(*args))
    return q_out


def bind_rope_set_rows_kv(k_pool: KVPool, v_pool: KVPool, k_rows: torch.Tensor, v_rows: torch.Tensor,
                          slots: torch.Tensor, pos: torch.Tensor, rope: RopeParams, n_head_kv: int,
                          q: Optional[torch.Tensor] = None, q_out: Optional[torch.Tensor] = None,
                          err_flag: Optional[torch.Tensor] = None) -> Callable[[], None]:
    """rope_set_rows_kv checked once and bound to these buffers (contiguous
    rows; q_out given when q is) and the current stream, as bind_paged_attn."""
    if q is not None and q_out is None:
        raise ValueError("a bound call needs q_out when q is given")
    _, (args, prm) = rope_set_rows_kv(k_pool, v_pool, k_rows, v_rows, slots, pos, rope, n_head_kv, q=q, q_out=q_out,
                                      err_flag=err_flag, bind=True)
    fn = _lib.load().iian_pa_rope_kv_write

    def call() -> None:
        st = fn(*args)
        if st:
            _lib.check("iian_pa_rope_kv_write", st)
    call.params = prm   # the rope parameter block the bound arguments point at
    return call


def workspace_size(n_tokens: int, n_seqs: int, n_head: int, n_head_kv: int, head_dim_v: int, max_blocks: int,
                   block_size: int) -> int:
    return int(_lib.load().iian_pa_workspace_size(n_tokens, n_seqs, n_head, n_head_kv, head_dim_v, max_blocks,
                                                  block_size))


def new_workspace(n_tokens: int, n_seqs: int, n_head: int, n_head_kv: int, head_dim_v: int, max_blocks: int,
                  block_size: int, device="cuda") -> torch.Tensor:
    """A workspace for build_paged_attn, reusable across calls on one stream
    (it needs no initialisation)."""
    n = workspace_size(n_tokens, n_seqs, n_head, n_head_kv, head_dim_v, max_blocks, block_size)
    return torch.empty(n, dtype=torch.uint8, device=device)


def _check_batch(batch: PagedBatch, device: torch.device) -> None:
    """The batch arrays are read by the kernels as contiguous int32 (int64
    for slots) device arrays of the documented shapes: anything else would be
    misread, so it is rejected here."""
    S = batch.n_seqs
    want = (("block_tables", torch.int32, 2), ("seq_lens", torch.int32, 1), ("query_start_loc", torch.int32, 1),
            ("pos", torch.int32, 1))
    for name, dt, nd in want:
        t = getattr(batch, name)
        if t.dtype != dt or t.dim() != nd or not t.is_contiguous() or t.device != device:
            raise ValueError(f"batch.{name} must be a contiguous {dt} {nd}-d tensor on {device}")
    if batch.query_start_loc.shape[0] != S + 1:
        raise ValueError("batch.query_start_loc must have n_seqs + 1 entries")
    if batch.block_tables.shape[0] != S:
        raise ValueError("batch.block_tables must have one row per sequence")


def _attn_call(q: torch.Tensor, k_cache: KVPool, v_cache: KVPool, n_head_kv: int, params: PagedAttnParams,
               batch: PagedBatch, out: Optional[torch.Tensor], workspace: Optional[torch.Tensor],
               err_flag: Optional[torch.Tensor]):
    """Checks a call of iian_pa_attention and returns (out, its argument tuple)."""
    if q.dtype != torch.float32 or q.dim() != 3:
        raise ValueError("q must be f32 [n_tokens, n_head, head_dim]")   # paged_attn.cpp:161
    if not q.is_contiguous():
        raise ValueError("q head vectors must be contiguous")            # paged_attn.cpp:162
    T, H, D = q.shape
    if k_cache.n_embd % n_head_kv or v_cache.n_embd % n_head_kv:
        raise ValueError("pool rows must hold n_head_kv heads")
    if k_cache.n_embd // n_head_kv != D:
        raise ValueError("k head size differs from q head size")
    Dv = v_cache.n_embd // n_head_kv
    if not q.is_cuda:
        raise ValueError("q must be a GPU tensor")
    if T != batch.n_tokens:
        raise ValueError("q and batch disagree on n_tokens")
    _check_batch(batch, q.device)
    for pool in (k_cache, v_cache):
        if pool.data.device != q.device:
            raise ValueError("pools must be on q's device")
    if k_cache.n_cells != v_cache.n_cells or k_cache.n_cells % batch.block_size:
        raise ValueError("pools must hold the same whole number of blocks")
    num_blocks = k_cache.n_cells // batch.block_size
    if out is None:
        out = torch.empty((T, H, Dv), dtype=torch.float32, device=q.device)
    elif (out.dtype != torch.float32 or tuple(out.shape) != (T, H, Dv) or out.device != q.device
          or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous f32 [{T}, {H}, {Dv}] tensor on q's device")
    if err_flag is not None and (err_flag.dtype != torch.int32 or err_flag.device != q.device or err_flag.numel() < 1):
        raise ValueError("err_flag must be an int32 tensor on q's device")
    max_blocks = int(batch.block_tables.shape[1])
    need = workspace_size(T, batch.n_seqs, H, n_head_kv, Dv, max_blocks, batch.block_size)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    elif workspace.numel() < need:
        raise ValueError(f"workspace holds {workspace.numel()} bytes, {need} needed")
    args = (_stream(), q.data_ptr(), k_cache.data.data_ptr(), v_cache.data.data_ptr(), k_cache.type, v_cache.type,
            num_blocks, batch.block_tables.data_ptr(), max_blocks, batch.seq_lens.data_ptr(),
            batch.query_start_loc.data_ptr(), batch.pos.data_ptr(), T, batch.n_seqs, batch.max_query_len, H,
            n_head_kv, D, Dv, batch.block_size, float(params.scale), float(params.softcap),
            int(bool(params.causal)), int(params.n_swa), out.data_ptr(), workspace.data_ptr(), workspace.numel(),
            _ptr(err_flag))
    return out, args


def build_paged_attn(q: torch.Tensor, k_cache: KVPool, v_cache: KVPool, n_head_kv: int,
                     params: PagedAttnParams, batch: PagedBatch, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None,
                     err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged attention of q [T, H, D] over the pools (paged_attn.cpp:90-169);
    returns f32 [T, H, Dv].  A workspace from new_workspace() may be passed in
    and reused across calls."""
    out, args = _attn_call(q, k_cache, v_cache, n_head_kv, params, batch, out, workspace, err_flag)
    _lib.check("iian_pa_attention", _lib.load().iian_pa_attention(*args))
    return out


def bind_paged_attn(q: torch.Tensor, k_cache: KVPool, v_cache: KVPool, n_head_kv: int, params: PagedAttnParams,
                    batch: PagedBatch, out: torch.Tensor, workspace: torch.Tensor,
                    err_flag: Optional[torch.Tensor] = None) -> Callable[[], None]:
    """The call build_paged_attn would make, checked once and bound to these
    buffers and the current stream: the returned function issues it again
    with one ctypes call, as a C caller holding its arguments would.  The
    buffers must outlive it."""
    _, args = _attn_call(q, k_cache, v_cache, n_head_kv, params, batch, out, workspace, err_flag)
    fn = _lib.load().iian_pa_attention

    def call() -> None:
        st = fn(*args)
        if st:
            _lib.check("iian_pa_attention", st)
    return call


def _write_attn_args(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: KVPool, v_cache: KVPool,
                     n_head_kv: int, params: PagedAttnParams, batch: PagedBatch, out: Optional[torch.Tensor],
                     workspace: Optional[torch.Tensor], err_flag: Optional[torch.Tensor]):
    """Checks a call of iian_pa_write_attention and returns (out, its argument tuple)."""
    out, args = _attn_call(q, k_cache, v_cache, n_head_kv, params, batch, out, workspace, err_flag)
    T, _, D = q.shape
    for name, t, pool in (("k_new", k_new, k_cache), ("v_new", v_new, v_cache)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != q.device:
            raise ValueError(f"{name} must be a contiguous f32 tensor on q's device")
        if t.numel() != T * pool.n_embd or (t.dim() >= 1 and t.shape[0] != T):
            raise ValueError(f"{name} must hold one pool row of f32 per token: [{T}, {pool.n_embd}]")
    return out, args[:2] + (k_new.data_ptr(), v_new.data_ptr()) + args[2:]


def write_paged_attn(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: KVPool, v_cache: KVPool,
                     n_head_kv: int, params: PagedAttnParams, batch: PagedBatch, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None,
                     err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The layer's set_rows of the new K/V rows at their positions' cells
    (src/iian/graph.cpp:319-320) and its paged attention
    (graph.cpp:331-336) in one launch, for f16 decode and spec-verify steps
    (iian_pa_write_attention); raises PagedAttnError (IIAN_PA_ERR_UNSUPPORTED)
    for other calls, which take set_rows_kv and build_paged_attn."""
    out, args = _write_attn_args(q, k_new, v_new, k_cache, v_cache, n_head_kv, params, batch, out, workspace,
                                 err_flag)
    _lib.check("iian_pa_write_attention", _lib.load().iian_pa_write_attention(*args))
    return out


def bind_write_paged_attn(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: KVPool,
                          v_cache: KVPool, n_head_kv: int, params: PagedAttnParams, batch: PagedBatch,
                          out: torch.Tensor, workspace: torch.Tensor,
                          err_flag: Optional[torch.Tensor] = None) -> Callable[[], None]:
    """write_paged_attn checked once and bound to these buffers and the
    current stream, as bind_paged_attn."""
    _, args = _write_attn_args(q, k_new, v_new, k_cache, v_cache, n_head_kv, params, batch, out, workspace,
                               err_flag)
    fn = _lib.load().iian_pa_write_attention

    def call() -> None:
        st = fn(*args)
        if st:
            _lib.check("iian_pa_write_attention", st)
    return call


def dequant_q8_0(pool: KVPool, rows_idx: torch.Tensor) -> torch.Tensor:
    """f32 values of the given Q8_0 pool rows (ggml-quants.c:553-567)."""
    if pool.type != GGML_TYPE_Q8_0:
        raise ValueError("not a Q8_0 pool")
    rows_idx = rows_idx.to(torch.int64).contiguous()
    out = torch.empty((rows_idx.shape[0], pool.n_embd), dtype=torch.float32, device=pool.data.device)
    st = _lib.load().iian_pa_dequant_q8_0(_stream(), pool.data.data_ptr(), pool.n_cells, rows_idx.data_ptr(),
                                          rows_idx.shape[0], pool.n_embd, out.data_ptr())
    _lib.check("iian_pa_dequant_q8_0", st)
    return out
