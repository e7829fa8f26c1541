"""GPU: iian_pa_write_attention, the step's KV write fused into the f16 decode
kernels, against the two calls it replaces (iian_pa_kv_write_kv at the slots
of the tokens' positions, then iian_pa_attention) on copies of the same
pools.  Bars: both pools, the output and *err_flag equal bit for bit (the same
kernels read the same bytes); the output within the attention tolerance of the
CPU oracle on the written pools; calls outside the f16 decode kernels refused
before any launch, pools untouched.
"""
import zlib

import numpy as np
import pytest
import torch

from helpers import F16, Q8_0, make_case, row_rel_err
from test_gpu_parity import TOL, oracle_attention, to_device

pytestmark = pytest.mark.gpu

UNSUPPORTED = -3   # IIAN_PA_ERR_UNSUPPORTED


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


def banner(msg):
    print(f"\n[gpu] {msg}", flush=True)


def slots_of(bt: np.ndarray, seq_idx: np.ndarray, pos: np.ndarray, bs: int) -> np.ndarray:
    """slot = block_tables[s][pos / bs] * bs + pos % bs (-1 where the position has no block)."""
    out = np.full(len(pos), -1, np.int64)
    for t, (s, p) in enumerate(zip(seq_idx, pos)):
        if 0 <= p < bt.shape[1] * bs and bt[s, p // bs] >= 0:
            out[t] = int(bt[s, p // bs]) * bs + p % bs
    return out


def fused_vs_two_calls(pa, k, v, batch, q, k_new, v_new, n_head_kv, prm, slots):
    """Runs both paths from the same pool contents; asserts the bit-for-bit
    bar and returns (output, pools after the write, err_flag)."""
    k2 = pa.KVPool.wrap(k.data.clone(), k.n_embd, k.type)
    v2 = pa.KVPool.wrap(v.data.clone(), v.n_embd, v.type)
    err_a = torch.zeros(1, dtype=torch.int32, device="cuda")
    err_b = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows_kv(k, v, k_new, v_new, slots, err_a)
    out_a = pa.build_paged_attn(q, k, v, n_head_kv, prm, batch, err_flag=err_a)
    out_b = pa.write_paged_attn(q, k_new, v_new, k2, v2, n_head_kv, prm, batch, err_flag=err_b)
    torch.cuda.synchronize()
    assert int(err_a.item()) == int(err_b.item())
    assert torch.equal(k.data, k2.data) and torch.equal(v.data, v2.data)
    assert torch.equal(out_a.view(torch.int32), out_b.view(torch.int32))
    return out_b, k2, v2, int(err_b.item())


@pytest.mark.parametrize("name", ["cfg1", "cfg2", "phi3_decode", "cfg5_global_decode", "cfg5_local_decode"])
def test_write_attention_configs_match_two_calls(pa, name):
    """The decode configurations at full size: Qwen2 head size 64, Llama-3
    128 (stream-K workers and the merge launch), Phi-3 96 (kv head pairs),
    Gemma3 256 global and sliding-window layers."""
    from iian_amd import synth
    sp = synth.spec(name)
    banner(f"write+attention {name}: S={len(sp.seq_lens)} H={sp.H} Hkv={sp.Hkv} D={sp.D} n_swa={sp.n_swa}")
    w = synth.build(sp, device="cuda")
    _, _, _, err = fused_vs_two_calls(pa, w.k_pool, w.v_pool, w.batch, w.q, w.k_new.contiguous(),
                                      w.v_new.contiguous(), sp.Hkv, w.params, w.batch.slots)
    assert err == 0


CASES = {
    # (H, Hkv, D, lens, nq, make_case kwargs, pad the table to 4096 cells)
    "seg_d64": (14, 2, 64, [64, 200, 1000, 17, 1], [1, 1, 1, 1, 1], {}, False),
    "sk_d64_random_pos": (8, 2, 64, [900, 640, 100], [2, 1, 2], {"pos_mode": "random"}, True),
    "seg_d64_bs8": (8, 2, 64, [1000, 300], [1, 1], {"bs": 8}, False),
    "seg_d128_spec2": (16, 4, 128, [480, 33, 200], [2, 2, 1], {}, False),
    "sk_d128_spec2": (16, 4, 128, [480, 33, 200], [2, 2, 1], {}, True),
    "sk_d128_32rows": (32, 8, 128, [700, 90, 1300], [8, 3, 1], {}, True),   # two 16-row tiles
    "sk_d128_softcap_bs32": (32, 8, 128, [511, 64, 129], [1, 2, 1], {"softcap": 20.0, "bs": 32}, True),
    "sk_d96_pairs": (16, 4, 96, [800, 77, 1500], [2, 1, 2], {}, True),       # head pairs, 8 rows per pair
    "sk_d96_single": (24, 2, 96, [800, 77, 1500], [1, 1, 1], {}, True),      # 12 rows per kv head
    "seg_d256_spec": (16, 8, 256, [250, 40], [4, 8], {}, False),
    "sk_d256": (16, 8, 256, [900, 40, 2000], [1, 2, 1], {}, True),
    "sk_d128_swa": (32, 8, 128, [2000, 700, 90], [1, 3, 1], {"n_swa": 300}, True),
}


def case_inputs(pa, name):
    H, Hkv, D, lens, nq, kw, pad = CASES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    c = make_case(rng, H, Hkv, D, lens, nq, **kw)
    if pad:   # unused table columns: the call takes the stream-K kernel, not the segment workgroups
        cols = (4096 + c.bs - 1) // c.bs - c.bt.shape[1]
        c.bt = np.concatenate([c.bt, np.full((c.bt.shape[0], cols), -1, np.int32)], axis=1)
    k, v, batch = to_device(pa, c)
    g = torch.Generator(device="cuda").manual_seed(7)
    k_new = torch.randn((c.T, Hkv * D), generator=g, device="cuda")
    v_new = torch.randn((c.T, Hkv * D), generator=g, device="cuda")
    prm = pa.PagedAttnParams(scale=c.scale, softcap=c.softcap, causal=c.causal, n_swa=c.n_swa)
    return c, k, v, batch, k_new, v_new, prm


@pytest.mark.parametrize("name", sorted(CASES))
def test_write_attention_cases(pa, oracle, name):
    c, k, v, batch, k_new, v_new, prm = case_inputs(pa, name)
    banner(f"write+attention case {name}: H={c.H} Hkv={c.Hkv} D={c.D} lens={list(c.seq_lens)} "
           f"nq={list(np.diff(c.qsl))}")
    slots = torch.as_tensor(slots_of(c.bt, c.seq_idx, c.pos, c.bs), device="cuda")
    q = torch.as_tensor(c.q).cuda()
    out, k2, v2, err = fused_vs_two_calls(pa, k, v, batch, q, k_new, v_new, c.Hkv, prm, slots)
    assert err == 0
    # the new rows are in the pools, and the output is the oracle's over them
    c.k_pool, c.v_pool = k2.data.cpu().numpy(), v2.data.cpu().numpy()
    s = slots.cpu().numpy()
    want_k = k_new.cpu().numpy().astype(np.float16).view(np.uint8)
    assert np.array_equal(c.k_pool[s], want_k.reshape(len(s), -1))
    e = row_rel_err(out.cpu().numpy(), oracle_attention(oracle, c))
    print(f"[gpu] {name}: max row rel err {e.max():.3e}", flush=True)
    assert e.max() <= TOL, (name, e.max())


def test_write_attention_unwritable_rows_are_flagged_not_written(pa):
    """A new token at a position beyond its sequence's length, or in a block
    outside the pool, is not written and sets bit 0, as the KV write does for
    a slot outside the pool; the attention flags the bad block id (bit 1)."""
    c, k, v, batch, k_new, v_new, prm = case_inputs(pa, "sk_d128_spec2")
    T = c.T
    pos = c.pos.copy()
    pos[0] = c.seq_lens[c.seq_idx[0]]           # one past its sequence's end
    s_last = int(c.seq_idx[T - 1])
    bt = c.bt.copy()
    bt[s_last, pos[T - 1] // c.bs] = k.n_cells // c.bs   # a block id outside the pool
    batch.pos = torch.as_tensor(pos).cuda()
    batch.block_tables = torch.as_tensor(bt).cuda()
    slots = slots_of(bt, c.seq_idx, pos, c.bs)
    slots[0] = -1                                # the two-call path: no cell for either token
    slots[T - 1] = -1
    q = torch.as_tensor(c.q).cuda()
    _, _, _, err = fused_vs_two_calls(pa, k, v, batch, q, k_new, v_new, c.Hkv, prm,
                                      torch.as_tensor(slots, device="cuda"))
    assert err == 1 | 2, err


def test_write_attention_refuses_other_calls_before_any_launch(pa):
    """Q8_0 pools and prefill-sized calls take the two calls: the fused entry
    returns IIAN_PA_ERR_UNSUPPORTED and writes nothing."""
    from iian_amd import synth
    c, k, v, batch, k_new, v_new, prm = case_inputs(pa, "sk_d128_spec2")
    q = torch.as_tensor(c.q).cuda()
    # prefill-sized: 16 tokens of one sequence at 4 query heads per kv head (64 rows)
    rng = np.random.default_rng(3)
    cp = make_case(rng, 16, 4, 128, [400, 90], [16, 1])
    kp, vp, bp = to_device(pa, cp)
    before = (kp.data.clone(), vp.data.clone())
    kn = torch.randn((cp.T, 4 * 128), device="cuda")
    with pytest.raises(pa.PagedAttnError) as e:
        pa.write_paged_attn(torch.as_tensor(cp.q).cuda(), kn, kn.clone(), kp, vp, 4, prm, bp)
    assert e.value.status == UNSUPPORTED
    sp = synth.spec("cfg4", small=True)
    w = synth.build(sp, device="cuda")
    before_q8 = w.k_pool.data.clone()
    with pytest.raises(pa.PagedAttnError) as e:
        pa.write_paged_attn(w.q, w.k_new.contiguous(), w.v_new.contiguous(), w.k_pool, w.v_pool, sp.Hkv, w.params,
                            w.batch)
    assert e.value.status == UNSUPPORTED
    torch.cuda.synchronize()
    assert torch.equal(kp.data, before[0]) and torch.equal(vp.data, before[1])
    assert torch.equal(w.k_pool.data, before_q8)


@pytest.mark.parametrize("name", ["sk_d128_spec2", "seg_d128_spec2"])
def test_write_attention_graph_replays(pa, name):
    """The fused call captured in a graph (it allocates nothing) and replayed
    four times, with the pools reset to their contents before the write and
    an eager call of other new rows in between: every replay gives the eager
    fused call's pools and output, bit for bit."""
    c, k, v, batch, k_new, v_new, prm = case_inputs(pa, name)
    banner(f"write+attention graph replays {name}")
    q = torch.as_tensor(c.q).cuda()
    k0, v0 = k.data.clone(), v.data.clone()
    ws = pa.new_workspace(c.T, batch.n_seqs, c.H, c.Hkv, c.D, c.bt.shape[1], c.bs)
    out = torch.empty((c.T, c.H, c.D), dtype=torch.float32, device="cuda")
    want = pa.write_paged_attn(q, k_new, v_new, k, v, c.Hkv, prm, batch, workspace=ws).clone()
    want_k, want_v = k.data.clone(), v.data.clone()
    k_other, v_other = torch.randn_like(k_new), torch.randn_like(v_new)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up outside the capture
        pa.write_paged_attn(q, k_new, v_new, k, v, c.Hkv, prm, batch, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pa.write_paged_attn(q, k_new, v_new, k, v, c.Hkv, prm, batch, out=out, workspace=ws)
    for it in range(4):
        k.data.copy_(k0)
        v.data.copy_(v0)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), it
        assert torch.equal(k.data, want_k) and torch.equal(v.data, want_v), it
        pa.write_paged_attn(q, k_other, v_other, k, v, c.Hkv, prm, batch, workspace=ws)   # eager, other rows
        torch.cuda.synchronize()
