"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle.

Bars: KV-write placement and Q8_0 values bit-exact; attention max relative
error per (token, head) row, max|y - r| / max|r|, at most 2e-3 (BASELINE
north star; fp32 accumulation in both).
"""
import zlib

import numpy as np
import pytest
import torch

from helpers import F16, F32, Q8_0, decode_rows_f64, make_case, row_rel_err

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


def banner(msg):
    print(f"\n[gpu] {msg}", flush=True)


# ---------------------------------------------------------------- KV write

@pytest.mark.parametrize("type_,n_embd", [(F16, 1024), (F16, 100), (F32, 256), (Q8_0, 1024), (Q8_0, 256)])
def test_kv_write_bit_exact(pa, oracle, type_, n_embd):
    banner(f"kv_write type={type_} n_embd={n_embd}")
    rng = np.random.default_rng(100 + type_ + n_embd)
    n_cells, T = 4096, 64
    rb = pa.row_bytes(type_, n_embd)
    init = rng.integers(0, 256, (n_cells, rb), dtype=np.uint8)
    rows = rng.standard_normal((T, n_embd)).astype(np.float32)
    rows[0, :32] = 0.0
    if n_embd >= 64:
        rows[1, :32] = 0.0
        rows[1, 0] = 127.0
        rows[1, 1:6] = [2.5, -2.5, 0.5, 1.5, 126.5]
        rows[2] *= 1e-30
        rows[3] *= 3e4
    slots = rng.choice(n_cells, T, replace=False).astype(np.int64)
    pool = pa.KVPool.wrap(torch.as_tensor(init).cuda(), n_embd, type_)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows(pool, torch.as_tensor(rows).cuda(), torch.as_tensor(slots).cuda(), err)
    got = pool.data.cpu().numpy()
    want = init.copy()
    assert oracle.set_rows(want, rows, slots, type_) == 0
    assert int(err.item()) == 0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("tk,tv,ek,ev", [(F16, F16, 1024, 1024), (Q8_0, Q8_0, 1024, 512), (F16, F16, 256, 100),
                                         (F32, F32, 256, 256), (F16, Q8_0, 512, 512)])
def test_kv_write_kv_bit_exact(pa, oracle, tk, tv, ek, ev):
    """One call writes both pools; each must equal its own set_rows oracle
    (rows of different lengths exercise the shared grid's tail)."""
    banner(f"kv_write_kv types={tk},{tv} n_embd={ek},{ev}")
    rng = np.random.default_rng(300 + tk + tv + ek + ev)
    n_cells, T = 2048, 96
    pools, wants, rows = [], [], []
    for t, e in ((tk, ek), (tv, ev)):
        init = rng.integers(0, 256, (n_cells, pa.row_bytes(t, e)), dtype=np.uint8)
        r = rng.standard_normal((T, e)).astype(np.float32)
        pools.append(pa.KVPool.wrap(torch.as_tensor(init).cuda(), e, t))
        wants.append(init.copy())
        rows.append(r)
    slots = rng.choice(n_cells, T, replace=False).astype(np.int64)
    slots[5] = n_cells          # out of range: skipped in both pools, flagged
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows_kv(pools[0], pools[1], torch.as_tensor(rows[0]).cuda(), torch.as_tensor(rows[1]).cuda(),
                   torch.as_tensor(slots).cuda(), err)
    keep = np.arange(T) != 5
    for pool, want, r, t in zip(pools, wants, rows, (tk, tv)):
        assert oracle.set_rows(want, r[keep], slots[keep], t) == 0
        assert np.array_equal(pool.data.cpu().numpy(), want)
    assert int(err.item()) & 1


def test_kv_write_out_of_range_slot_is_flagged_not_written(pa):
    banner("kv_write out-of-range slot")
    n_cells = 64
    pool = pa.KVPool(n_cells, 128, F16)
    rows = torch.ones((3, 128), dtype=torch.float32, device="cuda")
    slots = torch.tensor([5, 64, -1], dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows(pool, rows, slots, err)
    got = pool.data.cpu().numpy()
    assert int(err.item()) & 1
    assert got[5].view(np.float16).tolist() == [1.0] * 128
    assert not np.delete(got, 5, axis=0).any()


def test_dequant_q8_0_bit_exact(pa, oracle):
    banner("dequant q8_0")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((256, 1024)).astype(np.float32)
    x[7] *= 1e-30
    qb = oracle.quantize_q8_0(x)
    pool = pa.KVPool.wrap(torch.as_tensor(qb).cuda(), 1024, Q8_0)
    idx = torch.as_tensor(rng.choice(256, 100, replace=False).astype(np.int64)).cuda()
    got = pa.dequant_q8_0(pool, idx).cpu().numpy()
    want = oracle.dequantize_q8_0(qb[idx.cpu().numpy()], 1024)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- attention

def to_device(pa, c):
    k = pa.KVPool.wrap(torch.as_tensor(c.k_pool).cuda(), c.Hkv * c.D, c.k_type)
    v = pa.KVPool.wrap(torch.as_tensor(c.v_pool).cuda(), c.Hkv * c.Dv, c.v_type)
    nq = np.diff(c.qsl)
    batch = pa.PagedBatch(block_tables=torch.as_tensor(c.bt).cuda(), seq_lens=torch.as_tensor(c.seq_lens).cuda(),
                          query_start_loc=torch.as_tensor(c.qsl).cuda(), pos=torch.as_tensor(c.pos).cuda(),
                          slots=torch.zeros(c.T, dtype=torch.int64, device="cuda"), max_query_len=int(nq.max()),
                          block_size=c.bs)
    return k, v, batch


def gpu_attention(pa, c, err=None, max_query_len=None):
    k, v, batch = to_device(pa, c)
    if max_query_len is not None:
        batch.max_query_len = max_query_len
    prm = pa.PagedAttnParams(scale=c.scale, softcap=c.softcap, causal=c.causal, n_swa=c.n_swa)
    out = pa.build_paged_attn(torch.as_tensor(c.q).cuda(), k, v, c.Hkv, prm, batch, err_flag=err)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_attention(oracle, c, items=None):
    return oracle.paged_attention(c.q, c.k_pool, c.v_pool, c.k_type, c.v_type, c.bt, c.seq_lens, c.seq_idx, c.pos,
                                  c.Hkv, c.Dv, c.bs, c.scale, softcap=c.softcap, causal=c.causal, n_swa=c.n_swa,
                                  n_threads=16, items=items)


SMALL = {
    # name: (H, Hkv, D, lens, nq, kwargs)            which kernel
    "decode_gqa7_d64": (14, 2, 64, [64, 200, 1000, 17, 1], [1, 1, 1, 1, 1], {}),        # decode, 1 tile
    "decode_gqa4_d128": (32, 8, 128, [513, 77, 2048, 33], [1, 1, 1, 1], {}),            # decode + stream-K merge
    "decode_gqa2_d256": (16, 8, 256, [1500, 40], [1, 1], {}),
    "decode_long_splits": (8, 2, 128, [9000, 5000], [1, 1], {}),                        # 18 splits
    "decode_one_long_seq": (32, 8, 128, [32000], [1], {}),          # 125 pieces per (sequence, kv head)
    "spec_verify_5": (32, 8, 128, [700, 101, 4101], [5, 5, 5], {}),                     # decode, 2 row tiles
    "spec_verify_d64": (14, 2, 64, [300, 90], [3, 4], {}),
    "prefill_d128": (32, 8, 128, [600, 200], [512, 70], {}),                            # prefill kernel
    "prefill_d64": (14, 2, 64, [400], [130], {}),
    "prefill_d256": (16, 8, 256, [700, 300], [256, 33], {}),
    "mixed_prefill_decode": (32, 8, 128, [900, 1500, 700, 64], [256, 1, 1, 64], {}),
    "swa_decode": (16, 8, 256, [3000, 900, 1030], [1, 1, 1], {"n_swa": 1024}),
    "swa_prefill": (16, 8, 256, [2000, 1200], [256, 100], {"n_swa": 512}),
    "softcap": (8, 2, 128, [333, 77], [1, 40], {"softcap": 30.0}),
    "not_causal": (8, 2, 64, [300, 50], [20, 1], {"causal": False}),
    "prefix_shared": (32, 8, 128, [1200, 1100, 900, 300], [128, 64, 1, 1],
                      {"shared_blocks": 32, "shared_seqs": 3}),
    "block_size_32": (8, 2, 128, [500, 61], [1, 40], {"bs": 32}),
    # f16 prefill tiles loaded with a scalar block base: 64-cell blocks with a
    # window that starts tiles at odd multiples of 32 (a tile's cells span two
    # blocks), and the smallest block size
    "swa_prefill_d128_bs64": (8, 2, 128, [2000, 1200], [256, 100], {"n_swa": 480, "bs": 64}),
    "prefill_d128_bs8": (8, 2, 128, [700, 300], [200, 64], {"bs": 8}),
    # 12 row blocks per (sequence, kv head) and 4 pairs per XCD: the fourth
    # pair's slots start in the second round of CU slots, so it takes its row
    # blocks in reverse (a round that 12 does not divide)
    "prefill_nrb12_reversed": (32, 8, 128, [600, 500, 450, 700], [384, 384, 384, 384], {}),
    "random_positions": (8, 2, 64, [300, 200], [6, 40], {"pos_mode": "random"}),
    # prefill row blocks split in two KV halves: chunks with no prior context,
    # whose first row blocks see one tile (the first half attends nothing), and
    # a batch with more row blocks than one round of slots (not split)
    "prefill_split_p0_d128": (32, 8, 128, [40, 300, 1000], [40, 300, 1], {}),
    "prefill_unsplit_many_rb_d64": (14, 2, 64, [700] * 8 + [900, 50], [600] * 8 + [1, 1], {}),
    # ragged prefill batches (one chunk over a prefix several times longer than
    # the others'): f16 (the mixed launch) and Q8_0, head size 64, a sliding
    # window, positions that are not the engine's layout, a softcap with
    # decode rows in the same launch
    "prefill_split_ragged_d128": (32, 8, 128, [4000, 700, 900, 1200], [256, 256, 256, 256], {}),
    "q8_prefill_split_ragged": (32, 8, 128, [4000, 700, 900, 1200], [256, 256, 256, 256], {"k_type": Q8_0}),
    "prefill_split_ragged_d64": (14, 2, 64, [3000, 300], [200, 200], {}),
    "prefill_split_swa": (32, 8, 128, [5000, 600], [256, 256], {"n_swa": 2000}),
    "prefill_split_random_pos": (8, 2, 128, [3000, 200], [100, 100], {"pos_mode": "random"}),
    "prefill_split_softcap_decode": (32, 8, 128, [3500, 800, 64], [128, 1, 1], {"softcap": 30.0}),
    # Q8_0 pools (decode / spec-verify kernel)
    "q8_decode_gqa4_d128": (32, 8, 128, [513, 77, 2048, 33], [1, 1, 1, 1], {"k_type": Q8_0}),
    "q8_spec_verify_5": (32, 8, 128, [700, 101, 4101], [5, 5, 5], {"k_type": Q8_0}),
    "q8_decode_gqa7_d64": (14, 2, 64, [64, 200, 1000, 17, 1], [1, 1, 1, 1, 1], {"k_type": Q8_0}),
    "q8_spec_d64": (14, 2, 64, [300, 90], [3, 4], {"k_type": Q8_0}),
    "q8_decode_gqa2_d256": (16, 8, 256, [1500, 40], [1, 1], {"k_type": Q8_0}),
    "q8_swa_d256": (16, 8, 256, [3000, 900], [1, 2], {"k_type": Q8_0, "n_swa": 1024}),
    "q8_long_splits": (8, 2, 128, [9000, 5000], [1, 1], {"k_type": Q8_0}),
    "q8_spec_one_long_seq": (32, 8, 128, [32000], [5], {"k_type": Q8_0}),   # 250 pieces x 2 row tiles
    # spec-verify at head size 128 (two row tiles per kv head) with a window
    # and softcap, and over an odd number of kv heads
    "q8_spec_swa_softcap": (16, 4, 128, [3000, 130, 33], [5, 5, 4], {"k_type": Q8_0, "n_swa": 700,
                                                                          "softcap": 30.0}),
    "q8_spec_odd_kv_heads": (12, 3, 128, [900, 45], [5, 3], {"k_type": Q8_0}),
    "q8_block_size_32": (8, 2, 128, [500, 61], [1, 4], {"k_type": Q8_0, "bs": 32}),
    "q8_softcap": (8, 2, 128, [333, 77], [1, 3], {"k_type": Q8_0, "softcap": 30.0}),
    # Q8_0 pools through the prefill kernel
    "q8_prefill_d128": (32, 8, 128, [600, 200], [512, 70], {"k_type": Q8_0}),
    "q8_prefill_d64": (14, 2, 64, [400], [130], {"k_type": Q8_0}),
    "q8_prefill_d256": (16, 8, 256, [700, 300], [256, 33], {"k_type": Q8_0}),
    "q8_mixed_prefill_decode": (32, 8, 128, [900, 1500, 700, 64], [256, 1, 1, 64], {"k_type": Q8_0}),
    "q8_swa_prefill": (16, 8, 256, [2000, 1200], [256, 100], {"k_type": Q8_0, "n_swa": 512}),
    "q8_prefill_softcap": (8, 2, 128, [333, 77], [1, 40], {"k_type": Q8_0, "softcap": 30.0}),
    # head size 96 (Phi-3) f16 decode and spec-verify on the MFMA decode kernel: 12-byte V
    # slices, 6 output dims per lane, the merge's 48 live lanes
    "d96_decode_gqa1": (32, 32, 96, [800, 1200, 70, 4000], [1, 1, 1, 1], {}),
    "d96_decode_gqa4_splits": (32, 8, 96, [9000, 513, 77], [1, 1, 1], {}),
    "d96_spec_verify_5": (32, 8, 96, [700, 101, 4101], [5, 5, 5], {}),
    "d96_swa_softcap": (16, 4, 96, [3000, 900], [1, 2], {"n_swa": 700, "softcap": 30.0}),
    "d96_random_positions_bs32": (8, 2, 96, [600, 300], [6, 3], {"pos_mode": "random", "bs": 32}),
    # head pairs (two kv heads per wave): 8 rows per head fill the 16-row tile,
    # long contexts split into 16-row records; an odd kv-head count keeps one head per wave
    "d96_pairs_full_tile_splits": (32, 8, 96, [9000, 3000, 40], [2, 2, 2], {}),
    "d96_odd_kv_heads": (12, 3, 96, [1500, 700], [1, 1], {}),
    # head size 96 f16 prefill on the MFMA prefill kernel (register-staged 64-cell
    # tiles, 3 output tiles of 32 dims), alone and with decode rows in the same launch
    "d96_prefill_gqa1": (32, 32, 96, [600, 200], [512, 70], {}),
    "d96_mixed_prefill_decode": (32, 32, 96, [900, 1500, 700, 64], [256, 1, 1, 64], {}),
    "d96_prefill_swa_softcap": (16, 4, 96, [2000, 1200], [256, 100], {"n_swa": 512, "softcap": 30.0}),
    "d96_prefill_bs8_random_pos": (8, 2, 96, [700, 300], [200, 64], {"bs": 8, "pos_mode": "random"}),
    "d96_prefill_ragged": (32, 8, 96, [3000, 300], [200, 200], {}),
    "d96_prefill_not_causal": (8, 2, 96, [300, 50], [40, 1], {"causal": False}),
    # spec-verify launch (rows per kv head up to 32) holding sequences of 4 and 8 rows too
    "mixed_rows": (32, 8, 128, [600, 90, 1500], [1, 5, 2], {}),
    "q8_mixed_rows": (32, 8, 128, [600, 90, 1500], [1, 5, 2], {"k_type": Q8_0}),
}


@pytest.mark.parametrize("name", sorted(SMALL))
def test_attention_small_cases(pa, oracle, name):
    H, Hkv, D, lens, nq, kw = SMALL[name]
    banner(f"attention {name} H={H} Hkv={Hkv} D={D} lens={lens} nq={nq} {kw}")
    c = make_case(np.random.default_rng(zlib.crc32(name.encode())), H, Hkv, D, lens, nq,
                  quantize=oracle.quantize_q8_0, **kw)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = gpu_attention(pa, c, err)
    want = oracle_attention(oracle, c)
    e = row_rel_err(got, want)
    print(f"[gpu] {name}: max row rel err {e.max():.3e}", flush=True)
    assert int(err.item()) == 0
    assert np.isfinite(got).all()
    assert e.max() <= TOL, (name, e.max())


def staged_q8_v(v_row_bytes: np.ndarray, n_elems: int) -> np.ndarray:
    """f16(q*d) of every element of Q8_0 rows, as f32: q (int8) times the
    block's f16 scale d is exact in f32 and rounded once to f16."""
    blocks = v_row_bytes.reshape(v_row_bytes.shape[0], n_elems // 32, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float32)          # [rows, blocks, 1]
    q = blocks[:, :, 2:].copy().view(np.int8).astype(np.float32)             # [rows, blocks, 32]
    with np.errstate(over="ignore"):
        return (q * d).astype(np.float16).astype(np.float32).reshape(v_row_bytes.shape[0], n_elems)


@pytest.mark.parametrize("kind", ["decode", "spec", "prefill"])
def test_q8_attention_stages_v_as_f16_of_q_times_d(pa, oracle, kind):
    """Pins the V values the Q8_0 attention kernels compute with: a query row
    that sees exactly one cell has softmax weight 1 on it, so its output is
    that cell's V as staged, exactly: f16(q*d) (K enters exactly).  The V
    rows span block scales from 1e-6 to ~400.  Element 0 of every row sits in
    a block of scale 600, where 127*d is past the f16 range: those outputs are
    not finite (the staged value is +-inf, and the tile's masked cells, weight
    0, turn it into NaN), the documented limit of this staging."""
    banner(f"q8 staged V values, {kind}")
    rng = np.random.default_rng({"decode": 77, "spec": 79, "prefill": 78}[kind])
    H, Hkv, D = 32, 8, 128
    # spec: 5-token verify batches (two row tiles per kv head); the first
    # token of each sequence sees only cell 0
    lens, nq = {"decode": ([1] * 48, [1] * 48), "spec": ([5] * 24, [5] * 24), "prefill": ([160], [160])}[kind]
    c = make_case(rng, H, Hkv, D, lens, nq, k_type=Q8_0, quantize=oracle.quantize_q8_0)
    n_cells = c.v_pool.shape[0]
    x = rng.standard_normal((n_cells, Hkv * D)).astype(np.float32)
    scale = 10.0 ** rng.uniform(-6, 2.6, (n_cells, Hkv * D // 32, 1)).astype(np.float32)
    x = (x.reshape(n_cells, -1, 32) * scale).reshape(n_cells, -1)
    x[:, 0] = 127.0 * 600.0
    c.v_pool = oracle.quantize_q8_0(x)
    got = gpu_attention(pa, c)
    staged = staged_q8_v(c.v_pool, Hkv * D)
    gqa = H // Hkv
    finite = np.ones((H, D), dtype=bool)
    finite[:gqa, 0] = False   # element 0 of kv head 0
    # each checked query row sees one cell: cell 0 of its sequence
    for t in {"decode": range(c.T), "spec": range(0, c.T, 5), "prefill": [0]}[kind]:
        cell = int(c.bt[int(c.seq_idx[t]), 0]) * c.bs
        want = staged[cell].reshape(Hkv, D)[np.arange(H) // gqa]
        # exact equality as floats: the weighted sum over the tile's cells
        # cannot keep the sign of a zero (-0 + 0 = +0), every other bit must match
        bad = np.flatnonzero(got[t][finite] != want[finite])
        if len(bad):
            print(f"[gpu] row {t}: {len(bad)} differ; got {got[t][finite][bad[:8]]} want {want[finite][bad[:8]]}",
                  flush=True)
        assert len(bad) == 0, t
        assert not np.isfinite(got[t][~finite]).any(), t


SEGMENT_CASES = {
    # f16 decode calls small enough for the segment-workgroup kernel (every
    # segment within 2 tiles per wave: 32 tiles at D = 64, 16 at D = 128)
    "seg_d64": (14, 2, 64, [64, 200, 1000, 17, 1], [1, 1, 1, 1, 1], {}),
    "seg_d128": (32, 8, 128, [500, 77, 300, 33, 1, 480], [1, 1, 1, 1, 1, 1], {}),
    # query positions well before the end: the kernel attends [0, L) and the
    # causal masks remove the tiles past each row's position
    "seg_d64_random_pos": (8, 2, 64, [900, 640, 100], [2, 1, 2], {"pos_mode": "random"}),
    "seg_d128_spec2": (16, 4, 128, [480, 33, 200], [2, 2, 1], {}),                   # 8 rows per kv head
    "seg_d64_softcap": (8, 2, 64, [640, 33], [1, 1], {"softcap": 20.0}),
    "seg_d128_bs32": (16, 4, 128, [511, 64, 129], [1, 1, 1], {"bs": 32}),
    "seg_d64_bs8": (8, 2, 64, [1000, 300], [1, 1], {"bs": 8}),   # pieces past the first table window
    "seg_d256": (16, 8, 256, [200, 77, 256, 1], [1, 1, 1, 1], {}),   # 8 tiles over 4 waves
    "seg_d256_spec": (16, 8, 256, [250, 40], [4, 8], {}),            # 8 and 16 rows per kv head
}


@pytest.mark.parametrize("name", sorted(SEGMENT_CASES))
def test_segment_decode_matches_stream_k(pa, oracle, name):
    """Small decode calls run the segment-workgroup kernel (one launch, an LDS
    merge) when the block table bounds every segment's tiles; padding the
    table with unused columns makes the same call take the stream-K kernel and
    its merge launch.  Both against the oracle, and against each other."""
    H, Hkv, D, lens, nq, kw = SEGMENT_CASES[name]
    banner(f"segment decode {name} H={H} Hkv={Hkv} D={D} lens={lens} {kw}")
    c = make_case(np.random.default_rng(zlib.crc32(name.encode())), H, Hkv, D, lens, nq, **kw)
    want = oracle_attention(oracle, c)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    seg = gpu_attention(pa, c, err)
    assert int(err.item()) == 0
    pad_cols = (4096 + c.bs - 1) // c.bs - c.bt.shape[1]
    c.bt = np.concatenate([c.bt, np.full((c.bt.shape[0], pad_cols), -1, np.int32)], axis=1)
    sk = gpu_attention(pa, c, err)
    assert int(err.item()) == 0
    e_seg, e_sk = row_rel_err(seg, want), row_rel_err(sk, want)
    print(f"[gpu] {name}: segment kernel {e_seg.max():.3e}, stream-K {e_sk.max():.3e}", flush=True)
    assert np.isfinite(seg).all() and np.isfinite(sk).all()
    assert e_seg.max() <= TOL and e_sk.max() <= TOL, (name, e_seg.max(), e_sk.max())
    assert row_rel_err(seg, sk).max() <= TOL


def window_case(name, rng):
    """Sliding-window decode calls with a segment for every CU of an MI355X
    (S * Hkv = 256), which run the segment-workgroup kernel."""
    H, Hkv, D, n_swa, kw = WINDOW_SEGMENT_CASES[name]
    kw = dict(kw)
    S = 256 // Hkv
    lens = rng.integers(40, 3 * n_swa, S)
    nq = rng.integers(1, 16 // (H // Hkv) + 1, S) if kw.pop("spec", False) else np.ones(S, np.int64)
    return make_case(rng, H, Hkv, D, lens, nq, n_swa=n_swa, **kw)


WINDOW_SEGMENT_CASES = {
    "swa_d256": (16, 8, 256, 256, {}),
    # positions far from the end of each sequence: the window the kernel
    # guesses from the length is wrong, and the waves reload their entries
    "swa_d256_random_pos": (16, 8, 256, 256, {"pos_mode": "random"}),
    "swa_d128_spec": (32, 8, 128, 300, {"spec": True}),               # 4 .. 16 rows per kv head
    "swa_d64_bs8": (16, 8, 64, 500, {"bs": 8}),                       # windows past 64 table entries
    "swa_d128_softcap": (32, 8, 128, 200, {"softcap": 25.0}),
}


@pytest.mark.parametrize("name", sorted(WINDOW_SEGMENT_CASES))
def test_segment_window_decode_matches_stream_k(pa, oracle, name):
    """Sliding-window decode calls whose segments fill the device run the
    segment-workgroup kernel; a max_query_len that asks for 32-row decode tiles
    makes the same call take the stream-K kernel and its merge launch.  Both
    against the oracle, and against each other."""
    if torch.cuda.get_device_properties(0).multi_processor_count > 256:
        pytest.skip("the cases give 256 segments: fewer than this device's CUs")
    banner(f"segment window decode {name} {WINDOW_SEGMENT_CASES[name]}")
    c = window_case(name, np.random.default_rng(zlib.crc32(name.encode())))
    want = oracle_attention(oracle, c)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    seg = gpu_attention(pa, c, err)
    assert int(err.item()) == 0
    sk = gpu_attention(pa, c, err, max_query_len=16 // (c.H // c.Hkv) + 1)
    assert int(err.item()) == 0
    e_seg, e_sk = row_rel_err(seg, want), row_rel_err(sk, want)
    print(f"[gpu] {name}: segment kernel {e_seg.max():.3e}, stream-K {e_sk.max():.3e}", flush=True)
    assert np.isfinite(seg).all() and np.isfinite(sk).all()
    assert e_seg.max() <= TOL and e_sk.max() <= TOL, (name, e_seg.max(), e_sk.max())
    assert row_rel_err(seg, sk).max() <= TOL


@pytest.mark.parametrize("k_type,nq,D", [(F16, 1, 128), (F16, 5, 128), (F16, 64, 128), (Q8_0, 1, 128), (Q8_0, 5, 128),
                                        (Q8_0, 64, 128), (F16, 1, 96), (F16, 5, 96), (F16, 64, 96), (F16, 64, 64),
                                        (F16, 64, 256)])
def test_attention_growing_scores(pa, oracle, k_type, nq, D):
    """K rows scaled by a ramp 1 .. 16 along each sequence, so every row's
    running max keeps rising by many log2 units: exercises the online-softmax
    rescale of O and l on most tiles (random N(0,1) data barely moves the max
    after the first tile), and peaked softmax rows whose scores a single f16 q
    would get wrong by more than the tolerance.  nq = 1, 5: decode and
    spec-verify kernels; nq = 64: prefill kernels, whose lo product of q runs
    in bf8 over f16 pools (a CPU emulation of these cases at D = 128 puts it at
    4.6e-4 and 7.4e-4, against 4.3e-3 and 8.6e-3 with no lo product)."""
    banner(f"growing scores k_type={k_type} nq={nq} D={D}")
    rng = np.random.default_rng(46 + nq + k_type)
    c = make_case(rng, 32, 8, D, [1300, 2100, 90], [nq] * 3, k_type=k_type, quantize=oracle.quantize_q8_0)
    n_embd = c.Hkv * c.D
    rows = decode_rows_f64(c.k_pool, c.k_type, n_embd).astype(np.float32)
    for s in range(len(c.seq_lens)):
        L = int(c.seq_lens[s])
        i = np.arange(L)
        cells = c.bt[s, i // c.bs].astype(np.int64) * c.bs + i % c.bs
        rows[cells] *= (1.0 + 15.0 * i / max(L - 1, 1))[:, None].astype(np.float32)
    c.k_pool = (oracle.f32_to_f16_bits(rows).view(np.uint8).reshape(rows.shape[0], -1) if k_type == F16
                else oracle.quantize_q8_0(rows))
    got = gpu_attention(pa, c)
    e = row_rel_err(got, oracle_attention(oracle, c))
    print(f"[gpu] growing scores k_type={k_type} nq={nq}: max row rel err {e.max():.3e}", flush=True)
    assert np.isfinite(got).all()
    assert e.max() <= TOL, e.max()


@pytest.mark.parametrize("k_type,H,Hkv,D", [(Q8_0, 32, 8, 128), (F16, 16, 8, 256), (Q8_0, 16, 8, 256),
                                           (F16, 32, 8, 128)])
def test_mixed_batch_on_a_side_stream_of_the_caller(pa, oracle, k_type, H, Hkv, D):
    """A prefill + decode batch over a Q8_0 pool or at head size 256 forks its
    decode rows onto the library's side stream and joins them back (f16 at
    head size 128 runs both in one launch): issued on a non-default torch
    stream, three back-to-back calls into three outputs are all complete once
    that stream is synchronised."""
    banner(f"mixed batch on a caller stream k_type={k_type} D={D}")
    rng = np.random.default_rng(47 + D + k_type)
    c = make_case(rng, H, Hkv, D, [900, 1500, 700, 3000], [200, 1, 1, 1], k_type=k_type,
                  quantize=oracle.quantize_q8_0)
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    qs = [rng.standard_normal(c.q.shape).astype(np.float32) for _ in range(3)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        qd = [torch.as_tensor(x).cuda() for x in qs]
        outs = [pa.build_paged_attn(x, k, v, c.Hkv, prm, batch) for x in qd]
    s.synchronize()
    for x, o in zip(qs, outs):
        c.q = x
        assert row_rel_err(o.cpu().numpy(), oracle_attention(oracle, c)).max() <= TOL


def test_bound_call_matches_the_plain_call(pa, oracle):
    """bind_paged_attn issues the same call: bit-identical output, twice."""
    banner("bound attention call")
    rng = np.random.default_rng(77)
    c = make_case(rng, 32, 8, 128, [900, 40, 3000], [1, 1, 1])
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    q = torch.as_tensor(c.q).cuda()
    ws = pa.new_workspace(c.T, 3, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    want = pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, workspace=ws).cpu().numpy()
    out = torch.full((c.T, c.H, c.D), float("nan"), device="cuda")
    call = pa.bind_paged_attn(q, k, v, c.Hkv, prm, batch, out, ws)
    call()
    call()
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


def test_attention_all_masked_rows_are_zero(pa, oracle):
    banner("all-masked rows")
    rng = np.random.default_rng(42)
    c = make_case(rng, 8, 2, 128, [100, 40, 0 + 16], [2, 1, 1])
    c.pos[:] = [-5, -1, -2, 10]          # every cell after the first three queries
    got = gpu_attention(pa, c)
    assert np.all(got[:3] == 0.0)
    assert row_rel_err(got[3:], oracle_attention(oracle, c)[3:]).max() <= TOL


def test_workspace_reuse_across_calls(pa, oracle):
    """One workspace serves consecutive calls: three calls (different queries,
    then a different batch) all match the oracle."""
    banner("workspace reuse")
    rng = np.random.default_rng(45)
    c = make_case(rng, 32, 8, 128, [5000, 700, 3000, 64], [1, 1, 1, 1])
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    ws = pa.new_workspace(64, 8, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    for it in range(3):
        if it == 2:
            c.seq_lens[:] = [4000, 500, 3000, 20]      # shorter: stays inside every block table
            c.pos[:] = c.seq_lens - 1
            k, v, batch = to_device(pa, c)
        c.q = rng.standard_normal(c.q.shape).astype(np.float32)
        got = pa.build_paged_attn(torch.as_tensor(c.q).cuda(), k, v, c.Hkv, prm, batch, workspace=ws)
        torch.cuda.synchronize()
        e = row_rel_err(got.cpu().numpy(), oracle_attention(oracle, c))
        assert e.max() <= TOL, (it, e.max())


# decode kernel (f16; Q8_0 spec-verify), the mixed prefill launch, whose
# decode workers merge split segments through tagged counters in the
# workspace, and a Q8_0 mixed batch, whose decode rows run on the side stream
# (a fork and join inside the captured graph)
SPLIT_CASES = [(F16, (1, 1, 1, 1)), (Q8_0, (5, 5, 5, 5)), (F16, (128, 1, 1, 1)), (Q8_0, (128, 1, 1, 1))]


@pytest.mark.parametrize("k_type,nqs", SPLIT_CASES)
def test_split_merge_with_garbage_workspace(pa, oracle, k_type, nqs):
    """The workspace needs no initialisation: every record and segment entry
    the merge reads is written earlier in the same call, and a merge counter
    holding another call's tag counts as zero.  Filled with 0xff, with random
    bytes, or zeroed, the workspace gives the same bits (the merging piece
    reads every record in order) and the oracle's result."""
    banner(f"split merge over garbage workspaces k_type={k_type} nq={nqs}")
    rng = np.random.default_rng(48 + sum(nqs))
    c = make_case(rng, 32, 8, 128, [6000, 700, 3000, 2500], list(nqs), k_type=k_type, quantize=oracle.quantize_q8_0)
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    q = torch.as_tensor(c.q).cuda()
    ws = pa.new_workspace(c.T, 4, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    outs = []
    for fill in ("ff", "random", "zero"):
        if fill == "ff":
            ws.fill_(255)
        elif fill == "random":
            ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, generator=torch.Generator().manual_seed(7)))
        else:
            ws.zero_()
        outs.append(pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, workspace=ws).cpu().numpy())
    assert row_rel_err(outs[0], oracle_attention(oracle, c)).max() <= TOL
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


GRAPH_LENS = [5000, 700, 3000, 2500]


@pytest.mark.parametrize("k_type,nqs,lens", [(k, n, GRAPH_LENS) for k, n in SPLIT_CASES] +
                         [(F16, (1, 1, 1, 1), [500, 300, 77, 200])])   # the segment-workgroup kernel
def test_graph_replays_match_eager(pa, oracle, k_type, nqs, lens):
    """A call captured in a graph and replayed four times, with eager calls
    of another batch on the same workspace in between, gives the eager call's
    bits on every replay (a replay reuses its call's merge-counter tag; the
    merging piece resets each counter it completes)."""
    banner(f"graph replays k_type={k_type} nq={nqs} lens={lens}")
    rng = np.random.default_rng(49 + sum(nqs))
    c = make_case(rng, 32, 8, 128, lens, list(nqs), k_type=k_type, quantize=oracle.quantize_q8_0)
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    q = torch.as_tensor(c.q).cuda()
    ws = pa.new_workspace(c.T, 4, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    eager = pa.build_paged_attn(q, k, v, c.Hkv, prm, batch).cpu().numpy()
    assert row_rel_err(eager, oracle_attention(oracle, c)).max() <= TOL
    q2 = torch.as_tensor(rng.standard_normal(c.q.shape).astype(np.float32)).cuda()
    other = pa.build_paged_attn(q2, k, v, c.Hkv, prm, batch).cpu().numpy()
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, out=out, workspace=ws)   # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, out=out, workspace=ws)
    for it in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), it
        o2 = pa.build_paged_attn(q2, k, v, c.Hkv, prm, batch, workspace=ws)
        torch.cuda.synchronize()
        assert np.array_equal(o2.cpu().numpy(), other), it


def test_q8_many_sequences_split_over_workers(pa, oracle):
    """Q8_0 spec-verify over at least as many sequences as stream-K workers
    (130 sequences of 5 query tokens: 128 workers of 2-wave workgroups on an
    MI355X), ragged, so segments split at worker boundaries.  Against the
    oracle, over workspaces filled with garbage (same bits every time), and
    through graph replays."""
    banner("q8 many sequences split over workers")
    rng = np.random.default_rng(50)
    c = make_case(rng, 32, 8, 128, rng.integers(60, 700, 130), [5] * 130, k_type=Q8_0,
                  quantize=oracle.quantize_q8_0)
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    q = torch.as_tensor(c.q).cuda()
    ws = pa.new_workspace(c.T, 130, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    outs = []
    for fill in ("ff", "random", "zero"):
        if fill == "ff":
            ws.fill_(255)
        elif fill == "random":
            ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, generator=torch.Generator().manual_seed(8)))
        else:
            ws.zero_()
        outs.append(pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, workspace=ws).cpu().numpy())
    e = row_rel_err(outs[0], oracle_attention(oracle, c))
    print(f"[gpu] q8 many sequences: max row rel err {e.max():.3e}", flush=True)
    assert e.max() <= TOL
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    out = torch.empty_like(q)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, out=out, workspace=ws)
    for it in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), outs[0]), it


def test_attention_bad_block_id_is_clamped_and_flagged(pa):
    banner("bad block id")
    rng = np.random.default_rng(43)
    c = make_case(rng, 8, 2, 128, [100, 40], [1, 1])
    c.bt[1, 1] = 1 << 30
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = gpu_attention(pa, c, err)
    assert int(err.item()) & 2
    assert np.isfinite(got).all()


def test_attention_block_permutation_invariance_bitwise(pa):
    banner("block permutation invariance")
    rng = np.random.default_rng(44)
    c = make_case(rng, 32, 8, 128, [3000, 700, 64], [1, 5, 1])
    base = gpu_attention(pa, c)
    nb = c.k_pool.shape[0] // c.bs
    perm = rng.permutation(nb)
    kp, vp = np.empty_like(c.k_pool), np.empty_like(c.v_pool)
    kp.reshape(nb, -1)[perm] = c.k_pool.reshape(nb, -1)
    vp.reshape(nb, -1)[perm] = c.v_pool.reshape(nb, -1)
    c.k_pool, c.v_pool = kp, vp
    c.bt = np.where(c.bt >= 0, perm[np.maximum(c.bt, 0)], -1).astype(np.int32)
    assert np.array_equal(base, gpu_attention(pa, c))


# ---------------------------------------------------------------- full-size configurations

def config_parity(pa, oracle, name, n_items=None, seed=None):
    from iian_amd import synth
    sp = synth.spec(name, seed=seed)
    banner(f"config {name}: S={len(sp.seq_lens)} T={int(sp.n_q.sum())} H={sp.H} Hkv={sp.Hkv} D={sp.D} "
           f"n_swa={sp.n_swa} kv_type={sp.kv_type}")
    w = synth.build(sp, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows(w.k_pool, w.k_new, w.batch.slots, err)
    pa.set_rows(w.v_pool, w.v_new, w.batch.slots, err)
    out = pa.build_paged_attn(w.q, w.k_pool, w.v_pool, sp.Hkv, w.params, w.batch, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got = out.cpu().numpy()
    kp, vp = w.k_pool.data.cpu().numpy(), w.v_pool.data.cpu().numpy()
    items = None
    if n_items is not None and n_items < w.T * sp.H:
        items = np.sort(np.random.default_rng(1).choice(w.T * sp.H, n_items, replace=False)).astype(np.int64)
    want = oracle.paged_attention(w.q.cpu().numpy(), kp, vp, sp.kv_type, sp.kv_type, w.block_tables, sp.seq_lens,
                                  w.seq_idx, w.pos, sp.Hkv, sp.D, sp.block_size, sp.scale, softcap=sp.softcap,
                                  causal=True, n_swa=sp.n_swa, n_threads=16, items=items)
    g, r = got.reshape(-1, sp.D), want.reshape(-1, sp.D)
    if items is not None:
        g, r = g[items], r[items]
    e = row_rel_err(g, r)
    print(f"[gpu] {name}: rows checked {len(e)}, max row rel err {e.max():.3e}, mean {e.mean():.3e}", flush=True)
    assert np.isfinite(got).all()
    assert e.max() <= TOL, (name, e.max())
    # the KV write of this step landed bit-exactly in both pools
    rows_k = oracle.f32_to_f16_bits(w.k_new.cpu().numpy()) if sp.kv_type == F16 else oracle.quantize_q8_0(
        w.k_new.cpu().numpy())
    assert np.array_equal(kp[w.slots].reshape(rows_k.shape[0], -1).view(np.uint8),
                          rows_k.view(np.uint8).reshape(rows_k.shape[0], -1))


@pytest.mark.parametrize("name,n_items", [
    ("cfg1", None), ("cfg2", None), ("cfg3", 4096), ("cfg3_prefill", 4096), ("cfg3_p0", 4096), ("cfg4", 2048),
    ("cfg5_global_decode", None), ("cfg5_local_decode", None),
    ("cfg5_global_prefill", 1024), ("cfg5_local_prefill", 1024), ("phi3_decode", None),
])
def test_config_parity(pa, oracle, name, n_items):
    config_parity(pa, oracle, name, n_items)
