"""The engine runtime (iian_pa_runtime_*): an engine step driven through it,
from the scheduler's per-request block ids and counts on the host, gives the
same bits as the direct path (device batch build, fused RoPE + KV write,
attention) on the same inputs, over consecutive steps that reuse its pinned
staging; its error word stays clear, and a request whose blocks do not cover
its context is refused before any device work."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4"])
def test_runtime_step_matches_direct_path(pa, name):
    from iian_amd import synth
    sp = synth.spec(name, small=True)
    print(f"\n[gpu] runtime {name}", flush=True)
    w = synth.build(sp)
    ids, nc, nn = synth.request_blocks(sp)
    T = int(nn.sum())
    max_blocks = w.block_tables.shape[1]
    rt = pa.PagedAttnRuntime(max_seqs=len(ids) + 4, max_tokens=T + 16, max_blocks_per_seq=max_blocks + 4,
                             max_total_blocks=sum(len(b) for b in ids) + 64, n_head=sp.H, n_head_kv=sp.Hkv,
                             head_dim=sp.D, head_dim_v=sp.D, block_size=sp.block_size, num_blocks=sp.num_blocks,
                             type_k=sp.kv_type, type_v=sp.kv_type)
    rope = pa.RopeParams(n_dims=sp.D, mode=2, freq_base=1e6)
    kd, vd = w.k_pool.data.clone(), w.v_pool.data.clone()
    for step in range(2):
        sub = slice(0, len(ids) if step == 0 else max(1, len(ids) // 2))
        sids, snc, snn = ids[sub], nc[sub], nn[sub]
        Ts = int(snn.sum())
        q = torch.randn((Ts, sp.H, sp.D), device="cuda")
        kr = torch.randn((Ts, sp.Hkv * sp.D), device="cuda")
        vr = torch.randn((Ts, sp.Hkv * sp.D), device="cuda")
        # direct path on copies of the pools
        kp2 = pa.KVPool.wrap(kd, sp.Hkv * sp.D, sp.kv_type)
        vp2 = pa.KVPool.wrap(vd, sp.Hkv * sp.D, sp.kv_type)
        req = pa.RequestBlocks.pack(sids, snc, snn)
        b = pa.build_batch(req, Ts, sp.block_size, max_blocks + 4, sp.num_blocks, max_query_len=int(snn.max()))
        q_rot = pa.rope_set_rows_kv(kp2, vp2, kr, vr, b.slots, b.pos, rope, sp.Hkv, q=q)
        want = pa.build_paged_attn(q_rot, kp2, vp2, sp.Hkv, w.params, b)
        # the runtime
        out = torch.empty_like(want)
        qr = torch.empty_like(q)
        rt.begin_step(sids, snc, snn)
        rt.layer(q, kr, vr, w.k_pool, w.v_pool, w.params, out, rope=rope, q_rot=qr)
        torch.cuda.synchronize()
        assert rt.errors() == 0
        assert torch.equal(out, want), (name, step)
        assert torch.equal(qr, q_rot)
        assert torch.equal(w.k_pool.data, kd) and torch.equal(w.v_pool.data, vd)
    with pytest.raises(pa.PagedAttnError):
        rt.begin_step([ids[0][:1]], [int(nc[0])], [int(nn[0])])   # one block cannot cover the context
    rt.close()
