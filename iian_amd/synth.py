"""Seeded synthetic workloads at the benchmark configurations (random data of
the real shapes; there are no checkpoints or datasets here).

Each workload is one layer-call of the paged-attention path: the KV write of
this step's new tokens followed by paged attention over the block pool.
Block tables are seeded random permutations of the physical block ids, so a
sequence's blocks are scattered over the pool as in a long-running engine
(src/iian/kv_cache.cpp:214-229 hands out blocks from a free list).

Configurations (BASELINE.json ``configs``):
  cfg1            Qwen2.5-0.5B decode: H14/Hkv2/D64, 8 seqs, L~U[64,1024], 1024-block pool
  cfg2            Llama-3-8B decode: H32/Hkv8/D128, 64 seqs, L log-uniform [512,8192],
                  65536-block pool, plus the KV write of the 64 new tokens
                  (cfg2_f32: the same with F32 K/V pools, the general fp32 kernel)
  cfg3            Qwen3-8B mixed batch: 4 prefill chunks of 512 tokens over a prior
                  context P~U[1024,4096] whose first 1024 tokens (64 blocks) are shared
                  by all 4 sequences, plus 32 decode tokens with L~U[1024,4096]
                  (cfg3_prefill: the prefill chunks alone; cfg3_p0: one chunk with no prior)
  cfg4            Llama-3-8B Q8_0 KV: 128 seqs, 4096 prior + 5 spec-verify queries
  cfg5_<l>_<k>    Gemma3-12B: H16/Hkv8/D256, 32 seqs, L~U[8192,32768]; l in
                  {local (n_swa=1024), global}; k in {decode, prefill (256-token chunk)}
  phi3_decode     Phi-3.5-mini decode (head size 96): H32/Hkv32/D96, 64 seqs,
                  L log-uniform [512,8192], f16 KV
  phi3_prefill    Phi-3.5-mini chunked prefill: H32/Hkv32/D96, 4 chunks of 512 tokens
                  over a prior context P~U[1024,4096], f16 KV
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np
import torch

from .paged_attn import (GGML_TYPE_F16, GGML_TYPE_F32, GGML_TYPE_Q8_0, KVPool, PagedAttnParams, PagedBatch,
                         set_rows)


@dataclass
class Spec:
    name: str
    H: int
    Hkv: int
    D: int
    seq_lens: np.ndarray          # cells per sequence, this step's tokens included
    n_q: np.ndarray               # query tokens per sequence (the last n_q cells)
    num_blocks: int
    kv_type: int = GGML_TYPE_F16
    n_swa: int = 0
    softcap: float = 0.0
    shared_prefix_blocks: int = 0  # leading blocks shared by the first `shared_seqs` sequences
    shared_seqs: int = 0
    block_size: int = 16
    seed: int = 0

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)


def spec(name: str, seed: Optional[int] = None, small: bool = False) -> Spec:
    """The named configuration.  ``small`` shrinks sequence count and context
    (same heads, head size, formats and masks) for fast CPU-checked runs."""
    base = {"cfg1": 1, "cfg2": 2, "cfg2_f32": 2, "cfg3": 3, "cfg3_prefill": 3, "cfg4": 4, "phi3_decode": 6,
            "phi3_prefill": 7}.get(name, 5)
    rng = np.random.default_rng(seed if seed is not None else base)
    sd = seed if seed is not None else base
    if name == "cfg1":
        S = 8
        L = rng.integers(64, 1025, S)
        return Spec(name, 14, 2, 64, L, np.ones(S, np.int64), 1024, seed=sd)
    if name in ("cfg2", "cfg2_f32"):
        S = 8 if small else 64
        hi = 1024 if small else 8192
        L = np.exp(rng.uniform(math.log(512), math.log(hi), S)).astype(np.int64)
        return Spec(name, 32, 8, 128, L, np.ones(S, np.int64), 65536 if not small else 4096,
                    kv_type=GGML_TYPE_F32 if name == "cfg2_f32" else GGML_TYPE_F16, seed=sd)
    if name.startswith("cfg3"):
        n_pre, chunk, n_dec = (2, 64, 4) if small else (4, 512, 32)
        if name == "cfg3_prefill":  # the prefill chunks alone (the prefill kernel without the decode rows)
            n_dec = 0
        p_lo, p_hi = (128, 256) if small else (1024, 4096)
        P = rng.integers(p_lo, p_hi + 1, n_pre)
        if name == "cfg3_p0":       # a prefill chunk with no prior context
            P[-1] = 0
        Ld = rng.integers(p_lo, p_hi + 1, n_dec)
        L = np.concatenate([P + chunk, Ld])
        nq = np.concatenate([np.full(n_pre, chunk), np.ones(n_dec, np.int64)])
        shared = (256 if small else 1024) // 16
        nb = int(sum((l + 15) // 16 for l in L)) + 64
        return Spec(name, 32, 8, 128, L, nq, max(nb, 1024) * (1 if small else 4), shared_prefix_blocks=shared,
                    shared_seqs=n_pre if name != "cfg3_p0" else n_pre - 1, seed=sd)
    if name == "cfg4":
        S = 8 if small else 128
        prior = 256 if small else 4096
        L = np.full(S, prior + 5, np.int64)
        nb = int(S * ((prior + 5 + 15) // 16)) * 2
        return Spec(name, 32, 8, 128, L, np.full(S, 5, np.int64), nb, kv_type=GGML_TYPE_Q8_0, seed=sd)
    if name == "phi3_decode":
        S = 8 if small else 64
        hi = 1024 if small else 8192
        L = np.exp(rng.uniform(math.log(512), math.log(hi), S)).astype(np.int64)
        nb = int(sum((l + 15) // 16 for l in L)) * 2
        return Spec(name, 32, 32, 96, L, np.ones(S, np.int64), nb, seed=sd)
    if name == "phi3_prefill":
        n_pre, chunk = (2, 64) if small else (4, 512)
        p_lo, p_hi = (128, 256) if small else (1024, 4096)
        L = rng.integers(p_lo, p_hi + 1, n_pre) + chunk
        nb = int(sum((l + 15) // 16 for l in L)) * 2
        return Spec(name, 32, 32, 96, L, np.full(n_pre, chunk, np.int64), nb, seed=sd)
    if name.startswith("cfg5"):
        _, layer, kind = name.split("_")
        S = 4 if small else 32
        lo, hi = (1024, 3072) if small else (8192, 32768)
        L = rng.integers(lo, hi + 1, S)
        nq = np.full(S, 1 if kind == "decode" else (64 if small else 256), np.int64)
        nb = int(sum((l + 15) // 16 for l in L)) + 64
        return Spec(name, 16, 8, 256, L, nq, nb, n_swa=(1024 if not small else 512) if layer == "local" else 0,
                    seed=sd)
    raise ValueError(f"unknown configuration {name}")


@dataclass
class Workload:
    spec: Spec
    block_tables: np.ndarray       # int32 [S, max_blocks], unused entries -1
    seq_idx: np.ndarray            # int32 [T]
    pos: np.ndarray                # int32 [T]
    slots: np.ndarray              # int64 [T]
    qsl: np.ndarray                # int32 [S+1]
    params: PagedAttnParams
    q: torch.Tensor                # f32 [T, H, D]
    k_new: torch.Tensor            # f32 [T, Hkv*D] rows of this step's KV write
    v_new: torch.Tensor
    k_pool: KVPool
    v_pool: KVPool
    batch: PagedBatch
    extra: Dict[str, float] = field(default_factory=dict)

    @property
    def T(self) -> int:
        return int(self.pos.shape[0])


def _tables(sp: Spec, rng: np.random.Generator) -> np.ndarray:
    bs = sp.block_size
    nblk = (sp.seq_lens + bs - 1) // bs
    max_blocks = int(nblk.max())
    perm = rng.permutation(sp.num_blocks).astype(np.int32)
    bt = np.full((len(sp.seq_lens), max_blocks), -1, dtype=np.int32)
    cur = 0
    shared = perm[:sp.shared_prefix_blocks]
    cur += sp.shared_prefix_blocks
    for s, nb in enumerate(nblk):
        own = 0
        if s < sp.shared_seqs:
            k = min(sp.shared_prefix_blocks, nb)
            bt[s, :k] = shared[:k]
            own = k
        need = int(nb) - own
        if cur + need > sp.num_blocks:
            raise ValueError("pool too small for the drawn contexts")
        bt[s, own:nb] = perm[cur:cur + need]
        cur += need
    return bt


def request_blocks(sp: Spec):
    """The per-request state behind the workload's batch, as the scheduler
    holds it: each request's block ids (its block-table row, the blocks its
    context uses), its computed-token count (context before this step) and
    its new-token count.  Same seeded tables as build()."""
    rng = np.random.default_rng(sp.seed + 1000)
    bt = _tables(sp, rng)
    bs = sp.block_size
    nblk = (sp.seq_lens + bs - 1) // bs
    ids = [bt[s, :nblk[s]].copy() for s in range(len(sp.seq_lens))]
    n_new = sp.n_q.astype(np.int32)
    return ids, (sp.seq_lens - sp.n_q).astype(np.int32), n_new


def _fill_randn(dst: torch.Tensor, gen: torch.Generator, chunk: int = 1 << 26) -> None:
    """dst (f16 view, any shape) <- N(0,1) values cast to f16, in chunks."""
    flat = dst.view(-1)
    for i in range(0, flat.numel(), chunk):
        n = min(chunk, flat.numel() - i)
        flat[i:i + n] = torch.randn(n, generator=gen, device=dst.device, dtype=torch.float32).to(torch.float16)


def build(sp: Spec, device: str = "cuda", replicas: int = 1) -> Workload:
    """Materialise the workload on `device`: metadata from numpy's seeded
    generator, tensor values from torch's seeded generator on that device.
    With replicas > 1 the pool holds that many disjoint copies of the
    workload's blocks (pool blocks r*num_blocks + id), each with its own
    values, and Workload.extra['replica_batches'] holds one batch per copy:
    cycling through them keeps a small workload's KV out of the caches
    between steps."""
    rng = np.random.default_rng(sp.seed + 1000)
    bs = sp.block_size
    bt = _tables(sp, rng)
    if replicas > 1:
        sp = Spec(**{**sp.__dict__, "num_blocks": sp.num_blocks * replicas})
        used0 = bt >= 0
        base_num = sp.num_blocks // replicas
        bt_all = [np.where(used0, bt + r * base_num, -1).astype(np.int32) for r in range(replicas)]
    else:
        bt_all = [bt]
    S = len(sp.seq_lens)
    seq_idx, pos, slots = [], [], []
    for s in range(S):
        L, nq = int(sp.seq_lens[s]), int(sp.n_q[s])
        for p in range(L - nq, L):
            seq_idx.append(s)
            pos.append(p)
            slots.append(int(bt[s, p // bs]) * bs + p % bs)
    seq_idx = np.array(seq_idx, np.int32)
    pos = np.array(pos, np.int32)
    slots = np.array(slots, np.int64)
    qsl = np.zeros(S + 1, np.int32)
    qsl[1:] = np.cumsum(sp.n_q)
    T = len(pos)
    gen = torch.Generator(device=device)
    gen.manual_seed(sp.seed)
    n_embd = sp.Hkv * sp.D
    q = torch.randn((T, sp.H, sp.D), generator=gen, device=device, dtype=torch.float32)
    k_new = torch.randn((T, n_embd), generator=gen, device=device, dtype=torch.float32)
    v_new = torch.randn((T, n_embd), generator=gen, device=device, dtype=torch.float32)
    n_cells = sp.num_blocks * bs
    k_pool = KVPool(n_cells, n_embd, sp.kv_type, device=device)
    v_pool = KVPool(n_cells, n_embd, sp.kv_type, device=device)
    used = np.unique(np.concatenate([b[b >= 0] for b in bt_all])).astype(np.int64)
    used_t = torch.as_tensor(used, device=device)
    if sp.kv_type == GGML_TYPE_F16:
        for pool in (k_pool, v_pool):
            blocks = pool.data.view(sp.num_blocks, bs * pool.row_bytes)
            vals = torch.empty((len(used), bs * n_embd), dtype=torch.float16, device=device)
            _fill_randn(vals, gen)
            blocks[used_t] = vals.view(torch.uint8)
    else:
        # quantise N(0,1) rows into the used blocks with the library's own KV write
        rows_per = max(1, (1 << 24) // n_embd)
        cells = (used_t[:, None] * bs + torch.arange(bs, device=device)[None, :]).reshape(-1)
        for pool in (k_pool, v_pool):
            for i in range(0, cells.numel(), rows_per):
                c = cells[i:i + rows_per]
                rows = torch.randn((c.numel(), n_embd), generator=gen, device=device, dtype=torch.float32)
                set_rows(pool, rows, c.contiguous())
    batch = PagedBatch(
        block_tables=torch.as_tensor(bt, device=device), seq_lens=torch.as_tensor(sp.seq_lens.astype(np.int32), device=device),
        query_start_loc=torch.as_tensor(qsl, device=device), pos=torch.as_tensor(pos, device=device),
        slots=torch.as_tensor(slots, device=device), max_query_len=int(sp.n_q.max()), block_size=bs)
    params = PagedAttnParams(scale=sp.scale, softcap=sp.softcap, causal=True, n_swa=sp.n_swa)
    w = Workload(sp, bt, seq_idx, pos, slots, qsl, params, q, k_new, v_new, k_pool, v_pool, batch)
    if replicas > 1:
        w.extra["replica_batches"] = [batch] + [
            PagedBatch(block_tables=torch.as_tensor(b, device=device), seq_lens=batch.seq_lens,
                       query_start_loc=batch.query_start_loc, pos=batch.pos,
                       slots=torch.as_tensor(slots + (r + 1) * (sp.num_blocks // replicas) * bs, device=device),
                       max_query_len=batch.max_query_len, block_size=bs)
            for r, b in enumerate(bt_all[1:])]
    return w


def attended_cells(sp: Spec, pos: np.ndarray, seq_idx: np.ndarray) -> np.ndarray:
    """Unmasked (query, cell) pairs per token under causal + sliding-window masks."""
    L = sp.seq_lens[seq_idx]
    hi = np.minimum(L, pos.astype(np.int64) + 1)
    lo = np.maximum(0, pos.astype(np.int64) - sp.n_swa + 1) if sp.n_swa > 0 else np.zeros_like(hi)
    return np.maximum(0, hi - lo)


def algorithmic_bytes(w: Workload, include_kv_write: bool = True) -> int:
    """Minimum HBM traffic of one layer-call: every attended KV-head row once
    (K and V), Q and O once, the block tables and per-token metadata, plus the
    KV write (f32 rows in, converted rows out, slots)."""
    sp = w.spec
    e = {GGML_TYPE_F16: 2.0, GGML_TYPE_F32: 4.0}.get(sp.kv_type, 34.0 / 32.0)
    S = len(sp.seq_lens)
    kv = 0
    for s in range(S):
        q0, q1 = w.qsl[s], w.qsl[s + 1]
        p = w.pos[q0:q1].astype(np.int64)
        L = int(sp.seq_lens[s])
        hi = min(L, int(p.max()) + 1)
        lo = max(0, int(p.min()) - sp.n_swa + 1) if sp.n_swa > 0 else 0
        kv += max(0, hi - lo)
    T = w.T
    total = kv * sp.Hkv * 2 * sp.D * e                  # K and V rows of every attended cell
    total += T * sp.H * sp.D * 4 * 2                    # Q in, O out
    total += int(((sp.seq_lens + 15) // 16).sum()) * 4  # block tables
    total += T * 4 + (S + 1) * 4 + S * 4                # pos, query_start_loc, seq_lens
    if include_kv_write:
        total += T * sp.Hkv * sp.D * 2 * (4 + e) + T * 8
    return int(total)


def attention_flops(w: Workload) -> int:
    """4*H*D flops per unmasked (query, cell) pair (QK^T and PV)."""
    sp = w.spec
    pairs = attended_cells(sp, w.pos, w.seq_idx).sum()
    return int(4 * sp.H * sp.D * pairs)
