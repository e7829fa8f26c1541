"""The engine runtime (iian_pa_runtime_*).

* At the full cfg2, cfg3 and cfg4 shapes, two consecutive engine steps driven
  through it (the configuration's batch, then a decode step of every request
  that attends the cells the first step wrote) match the CPU oracle's chain
  on the same host inputs: the UBatch build of Engine::step
  (src/iian/engine.cpp:491-535; pao_build_batch), RoPE on q and K
  (graph.cpp:250-253; pao_rope_rows), the K and V set_rows
  (graph.cpp:319-320; pao_set_rows) and the paged attention op
  (paged_attn.cpp:90-146; pao_paged_attention).  Rotated q and both pools are
  bit-exact; attention rows are within 2e-3 (rows sampled at cfg3 and cfg4 as
  the full-size parity test does).
* At small shapes it gives the same bits as the direct path (device batch
  build, fused RoPE + KV write, attention) over consecutive steps that reuse
  its pinned staging; its error word stays clear, and a request whose blocks
  do not cover its context is refused before any device work."""
import numpy as np
import pytest
import torch

from helpers import row_rel_err

TOL = 2e-3

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


# (config, rope mode, freq base, sampled attention rows of step 0 / step 1; None = every row)
FULL = [("cfg2", 0, 500000.0, None, None), ("cfg3", 2, 1000000.0, 4096, None), ("cfg4", 0, 500000.0, 2048, 2048)]


@pytest.mark.parametrize("name,mode,base,n0,n1", FULL, ids=[f[0] for f in FULL])
def test_runtime_steps_match_oracle_chain(pa, oracle, name, mode, base, n0, n1):
    from iian_amd import synth
    sp = synth.spec(name)
    w = synth.build(sp)
    ids, nc, nn = synth.request_blocks(sp)
    ids = [list(map(int, b)) for b in ids]
    S, bs, H, Hkv, D = len(ids), sp.block_size, sp.H, sp.Hkv, sp.D
    max_blocks = max(len(b) for b in ids) + 4
    print(f"\n[gpu] runtime vs oracle chain {name}: S={S} T={int(nn.sum())} pool={sp.num_blocks} blocks", flush=True)
    rt = pa.PagedAttnRuntime(max_seqs=S, max_tokens=int(nn.sum()), max_blocks_per_seq=max_blocks,
                             max_total_blocks=sum(len(b) for b in ids) + S, n_head=H, n_head_kv=Hkv, head_dim=D,
                             head_dim_v=D, block_size=bs, num_blocks=sp.num_blocks, type_k=sp.kv_type,
                             type_v=sp.kv_type)
    rope = pa.RopeParams(n_dims=D, mode=mode, freq_base=base)
    kp_h, vp_h = w.k_pool.data.cpu().numpy(), w.v_pool.data.cpu().numpy()
    free = np.setdiff1d(np.arange(sp.num_blocks), np.concatenate([np.asarray(b) for b in ids]))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(sp.seed + 77)
    items_rng = np.random.default_rng(sp.seed + 78)
    for step, n_items in enumerate((n0, n1)):
        if step == 1:   # the next engine step: every request decodes one token after the ones just written
            nc = (nc + nn).astype(np.int32)
            nn = np.ones(S, np.int32)
            for s_ in range(S):
                if int(nc[s_]) + 1 > len(ids[s_]) * bs:
                    ids[s_].append(int(free[0]))
                    free = free[1:]
        T = int(nn.sum())
        b = oracle.build_batch(ids, nc, nn, bs, max_blocks)
        q = torch.randn((T, H, D), generator=gen, device="cuda")
        kr = torch.randn((T, Hkv * D), generator=gen, device="cuda")
        vr = torch.randn((T, Hkv * D), generator=gen, device="cuda")
        out = torch.empty((T, H, D), dtype=torch.float32, device="cuda")
        q_rot = torch.empty_like(q)
        rt.begin_step(ids, nc, nn)
        rt.layer(q, kr, vr, w.k_pool, w.v_pool, w.params, out, rope=rope, q_rot=q_rot)
        torch.cuda.synchronize()
        assert rt.errors() == 0
        # the oracle chain on the same host inputs
        rr = dict(mode=mode, freq_base=base)
        q_h = oracle.rope_rows(q.cpu().numpy().reshape(T, H * D), b["pos"], H, D, D, **rr).reshape(T, H, D)
        k_h = oracle.rope_rows(kr.cpu().numpy(), b["pos"], Hkv, D, D, **rr)
        assert oracle.set_rows(kp_h, k_h, b["slots"], sp.kv_type) == 0
        assert oracle.set_rows(vp_h, vr.cpu().numpy(), b["slots"], sp.kv_type) == 0
        assert np.array_equal(q_rot.cpu().numpy(), q_h), (name, step)
        sl = torch.as_tensor(b["slots"], device="cuda")
        assert np.array_equal(w.k_pool.data[sl].cpu().numpy(), kp_h[b["slots"]]), (name, step)
        assert np.array_equal(w.v_pool.data[sl].cpu().numpy(), vp_h[b["slots"]]), (name, step)
        items = None
        if n_items is not None and n_items < T * H:
            items = np.sort(items_rng.choice(T * H, n_items, replace=False)).astype(np.int64)
        want = oracle.paged_attention(q_h, kp_h, vp_h, sp.kv_type, sp.kv_type, b["block_tables"], b["seq_lens"],
                                      b["seq_idx"], b["pos"], Hkv, D, bs, sp.scale, softcap=sp.softcap, causal=True,
                                      n_swa=sp.n_swa, n_threads=16, items=items)
        g, r = out.cpu().numpy().reshape(-1, D), want.reshape(-1, D)
        if items is not None:
            g, r = g[items], r[items]
        e = row_rel_err(g, r)
        print(f"[gpu] runtime {name} step {step}: T={T} rows checked {len(e)}, max row rel err {e.max():.3e}",
              flush=True)
        assert np.isfinite(g).all()
        assert e.max() <= TOL, (name, step, e.max())
    # every other cell of both pools is untouched: the device pools equal the oracle's after both steps
    assert np.array_equal(w.k_pool.data.cpu().numpy(), kp_h)
    assert np.array_equal(w.v_pool.data.cpu().numpy(), vp_h)
    rt.close()
