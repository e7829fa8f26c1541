"""Shared test helpers: seeded small paged-attention cases and an independent
float64 brute-force attention (softmax(scale*qK^T + mask) V written from the
definition, not from the oracle's code)."""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

F32, F16, Q8_0 = 0, 1, 8


def row_bytes(type_: int, n: int) -> int:
    return {F32: 4 * n, F16: 2 * n}.get(type_, n // 32 * 34)


def decode_rows_f64(pool: np.ndarray, type_: int, n: int) -> np.ndarray:
    """Pool rows (uint8 [R, row_bytes]) -> float64 [R, n], by the format definitions."""
    if type_ == F32:
        return pool.view(np.float32).astype(np.float64)
    if type_ == F16:
        return pool.view(np.float16).astype(np.float64)
    blocks = pool.reshape(pool.shape[0], n // 32, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float64)          # [R, nb, 1]
    qs = blocks[:, :, 2:].view(np.int8).astype(np.float64)                   # [R, nb, 32]
    return (qs * d).reshape(pool.shape[0], n)


@dataclass
class Case:
    q: np.ndarray            # f32 [T, H, D]
    k_pool: np.ndarray       # uint8 [n_cells, row_bytes]
    v_pool: np.ndarray
    k_type: int
    v_type: int
    bt: np.ndarray           # int32 [S, max_blocks]
    seq_lens: np.ndarray     # int32 [S]
    seq_idx: np.ndarray      # int32 [T]
    pos: np.ndarray          # int32 [T]
    qsl: np.ndarray          # int32 [S+1]
    H: int
    Hkv: int
    D: int
    bs: int
    scale: float
    softcap: float = 0.0
    causal: bool = True
    n_swa: int = 0
    Dv: int = 0              # 0: same as D

    def __post_init__(self):
        if not self.Dv:
            self.Dv = self.D

    @property
    def T(self):
        return self.q.shape[0]


def make_case(rng: np.random.Generator, H: int, Hkv: int, D: int, lens, nq, bs: int = 16, k_type: int = F16,
              v_type: Optional[int] = None, num_blocks: Optional[int] = None, shared_blocks: int = 0,
              shared_seqs: int = 0, softcap: float = 0.0, causal: bool = True, n_swa: int = 0,
              pos_mode: str = "tail", quantize=None, Dv: Optional[int] = None) -> Case:
    """Random case: sequence s has lens[s] cells and its nq[s] query tokens sit
    at the last nq[s] positions (pos_mode 'tail') or at random positions
    ('random').  Blocks are a seeded random permutation of the pool; the first
    `shared_blocks` blocks of the first `shared_seqs` sequences are the same
    physical blocks.  `quantize(rows f32) -> uint8 rows` is required for Q8_0.
    V rows hold Hkv*Dv elements (Dv defaults to D)."""
    v_type = k_type if v_type is None else v_type
    Dv = D if Dv is None else Dv
    lens = np.asarray(lens, dtype=np.int64)
    nq = np.asarray(nq, dtype=np.int64)
    S = len(lens)
    nblk = (lens + bs - 1) // bs
    need = int(nblk.sum()) + 8
    num_blocks = num_blocks or max(need * 2, 16)
    perm = rng.permutation(num_blocks).astype(np.int32)
    max_blocks = int(max(1, nblk.max()))
    bt = np.full((S, max_blocks), -1, dtype=np.int32)
    cur = shared_blocks
    for s in range(S):
        own = 0
        if s < shared_seqs:
            k = min(shared_blocks, int(nblk[s]))
            bt[s, :k] = perm[:k]
            own = k
        bt[s, own:nblk[s]] = perm[cur:cur + nblk[s] - own]
        cur += int(nblk[s]) - own
    n_cells = num_blocks * bs

    def pool(type_, n_embd):
        x = rng.standard_normal((n_cells, n_embd)).astype(np.float32)
        if type_ == F32:
            return x.view(np.uint8).reshape(n_cells, -1).copy()
        if type_ == F16:
            return x.astype(np.float16).view(np.uint8).reshape(n_cells, -1).copy()
        return quantize(x)

    k_pool, v_pool = pool(k_type, Hkv * D), pool(v_type, Hkv * Dv)
    seq_idx, pos = [], []
    for s in range(S):
        if pos_mode == "tail":
            ps = np.arange(lens[s] - nq[s], lens[s])
        else:
            ps = np.sort(rng.integers(0, max(1, lens[s]), nq[s]))
        seq_idx += [s] * int(nq[s])
        pos += list(ps)
    qsl = np.zeros(S + 1, np.int32)
    qsl[1:] = np.cumsum(nq)
    T = len(pos)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    return Case(q, k_pool, v_pool, k_type, v_type, bt, lens.astype(np.int32), np.array(seq_idx, np.int32),
                np.array(pos, np.int32), qsl, H, Hkv, D, bs, 1.0 / math.sqrt(D), softcap, causal, n_swa, Dv)


def brute_force(c: Case, items=None) -> np.ndarray:
    """float64 softmax attention from the definition (paged_attn.cpp:121-144 semantics)."""
    T, H, D = c.q.shape
    Dv = c.Dv
    gqa = H // c.Hkv
    out = np.zeros((T, H, Dv), dtype=np.float64)
    cache = {}
    todo = range(T * H) if items is None else items
    for it in todo:
        t, h = divmod(int(it), H)
        s = int(c.seq_idx[t])
        L = int(c.seq_lens[s])
        if s not in cache:
            i = np.arange(L)
            cells = c.bt[s, i // c.bs].astype(np.int64) * c.bs + i % c.bs
            cache[s] = (decode_rows_f64(c.k_pool[cells], c.k_type, c.Hkv * D).reshape(L, c.Hkv, D),
                        decode_rows_f64(c.v_pool[cells], c.v_type, c.Hkv * Dv).reshape(L, c.Hkv, Dv))
        K, V = cache[s]
        hk = h // gqa
        p1 = int(c.pos[t])
        i = np.arange(L)
        mask = np.zeros(L, bool)
        if c.causal:
            mask |= i > p1
        if c.n_swa > 0:
            mask |= (p1 - i) >= c.n_swa
        if mask.all():
            continue
        sc = K[:, hk, :] @ c.q[t, h].astype(np.float64) * c.scale
        if c.softcap > 0:
            sc = c.softcap * np.tanh(sc / c.softcap)
        sc = np.where(mask, -np.inf, sc)
        p = np.exp(sc - sc.max())
        out[t, h] = (p @ V[:, hk, :]) / p.sum()
    return out


def row_rel_err(y: np.ndarray, r: np.ndarray) -> np.ndarray:
    """Per (t, h) row: max|y - r| / max(max|r|, 1e-6)."""
    num = np.abs(y.astype(np.float64) - r.astype(np.float64)).max(axis=-1)
    den = np.maximum(np.abs(r).max(axis=-1), 1e-6)
    return num / den
