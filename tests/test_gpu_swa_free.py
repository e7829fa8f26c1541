"""Sliding-window block freeing (iian_pa_swa_free_blocks; the reference's
planned out-of-window block eviction, docs/ROADMAP.md:33).

For a sliding-window layer, the blocks the call reports as freeable are never
read again: with their block-table entries set to -1 and their pool bytes
overwritten with NaN, attention gives the same bits as before and sets no
error bit (a read of a -1 entry would set bit 1; a read of a NaN cell would
poison the row).  The count itself is checked against its closed form."""
import numpy as np
import pytest
import torch

from helpers import F16, F32, Q8_0, make_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


def expected_free(qsl, pos, n_swa, bs):
    out = []
    for s in range(len(qsl) - 1):
        ps = pos[qsl[s]:qsl[s + 1]]
        out.append(0 if len(ps) == 0 else (max(0, int(ps.min()) - n_swa + 1) & ~31) // bs)
    return np.array(out)


def check_free_and_attend(pa, k_pool, v_pool, batch, params, Hkv, q, n_swa):
    """Returns the freed fraction of the table's used blocks."""
    bs = batch.block_size
    want = pa.build_paged_attn(q, k_pool, v_pool, Hkv, params, batch).cpu().numpy()
    nf = pa.swa_free_blocks(batch, n_swa).cpu().numpy()
    qsl, pos = batch.query_start_loc.cpu().numpy(), batch.pos.cpu().numpy()
    assert np.array_equal(nf, expected_free(qsl, pos, n_swa, bs))
    bt = batch.block_tables.cpu().numpy()
    freed = np.concatenate([bt[s, :nf[s]] for s in range(len(nf))]).astype(np.int64)
    nf2 = pa.swa_free_blocks(batch, n_swa, clear_table=True)
    assert np.array_equal(nf2.cpu().numpy(), nf)
    bt2 = batch.block_tables.cpu().numpy()
    for s in range(len(nf)):
        assert (bt2[s, :nf[s]] == -1).all() and np.array_equal(bt2[s, nf[s]:], bt[s, nf[s]:])
    if freed.size:
        rows = (torch.as_tensor(freed, device="cuda")[:, None] * bs + torch.arange(bs, device="cuda")[None, :]).reshape(-1)
        k_pool.data[rows] = 0xFF
        v_pool.data[rows] = 0xFF
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = pa.build_paged_attn(q, k_pool, v_pool, Hkv, params, batch, err_flag=err).cpu().numpy()
    assert int(err.item()) == 0
    assert np.array_equal(got, want)
    used = sum(int((bt[s] >= 0).sum()) for s in range(len(nf)))
    return freed.size / max(used, 1)


@pytest.mark.parametrize("name", ["cfg5_local_decode", "cfg5_local_prefill"])
def test_swa_free_at_gemma3_shapes(pa, name):
    from iian_amd import synth
    sp = synth.spec(name)
    print(f"\n[gpu] swa free {name}", flush=True)
    w = synth.build(sp)
    frac = check_free_and_attend(pa, w.k_pool, w.v_pool, w.batch, w.params, sp.Hkv, w.q, sp.n_swa)
    print(f"[gpu] {name}: {frac:.1%} of the used blocks freeable", flush=True)
    assert frac > 0.9


@pytest.mark.parametrize("k_type,D,nq,bs", [(Q8_0, 128, [1, 5, 1], 16), (F32, 96, [1, 40, 1], 16),
                                            (F16, 128, [200, 1, 3], 8), (F16, 64, [1, 1, 1], 12)])
def test_swa_free_small_cases(pa, oracle, k_type, D, nq, bs):
    """Q8_0 decode / spec-verify, the general kernel (F32, head size 96,
    block size 12), the f16 prefill kernel at block size 8."""
    print(f"\n[gpu] swa free k_type={k_type} D={D} nq={nq} bs={bs}", flush=True)
    rng = np.random.default_rng(81 + D + bs)
    c = make_case(rng, 16, 4, D, [3000, 1500, 2200], nq, k_type=k_type, n_swa=700, bs=bs,
                  quantize=oracle.quantize_q8_0)
    k = pa.KVPool.wrap(torch.as_tensor(c.k_pool).cuda(), c.Hkv * c.D, c.k_type)
    v = pa.KVPool.wrap(torch.as_tensor(c.v_pool).cuda(), c.Hkv * c.Dv, c.v_type)
    batch = pa.PagedBatch(block_tables=torch.as_tensor(c.bt).cuda(), seq_lens=torch.as_tensor(c.seq_lens).cuda(),
                          query_start_loc=torch.as_tensor(c.qsl).cuda(), pos=torch.as_tensor(c.pos).cuda(),
                          slots=torch.zeros(c.T, dtype=torch.int64, device="cuda"), max_query_len=int(max(nq)),
                          block_size=bs)
    prm = pa.PagedAttnParams(scale=c.scale, n_swa=c.n_swa)
    frac = check_free_and_attend(pa, k, v, batch, prm, c.Hkv, torch.as_tensor(c.q).cuda(), c.n_swa)
    assert frac > 0.5
