"""GPU parity of iian_pa_build_batch (pa_batch.hip): the step's block tables,
seq_lens, query_start_loc, pos and slots built on the device from the
requests' block ids and counts must equal, bit for bit, both the oracle's
restatement of Engine::step (src/iian/engine.cpp:491-535) and
PagedBatch.from_ubatch run on the host UBatch, at the cfg2, cfg3 and cfg4
shapes; attention over the device-built batch equals attention over the
host-built one."""
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


def kernel_us(fn, reps=50):
    """Average device time of fn() on the current stream (HIP events)."""
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) * 1000.0 / reps


@pytest.mark.parametrize("name,pad", [("cfg2", 0), ("cfg3", 0), ("cfg4", 0), ("cfg3_p0", 0), ("cfg2", 37)])
def test_build_batch_bit_exact(pa, oracle, name, pad):
    from iian_amd import synth
    sp = synth.spec(name)
    ids, nc, nn = synth.request_blocks(sp)
    bs = sp.block_size
    max_blocks = max(len(b) for b in ids) + pad
    print(f"\n[gpu] build_batch {name}: S={len(ids)} T={int(nn.sum())} max_blocks={max_blocks}", flush=True)
    want = oracle.build_batch(ids, nc, nn, bs, max_blocks)
    req = pa.RequestBlocks.pack(ids, nc, nn)
    T = int(nn.sum())
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = pa.build_batch(req, T, bs, max_blocks, sp.num_blocks, max_query_len=int(nn.max()), err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert np.array_equal(got.block_tables.cpu().numpy(), want["block_tables"])
    assert np.array_equal(got.seq_lens.cpu().numpy(), want["seq_lens"])
    assert np.array_equal(got.query_start_loc.cpu().numpy(), want["query_start_loc"])
    assert np.array_equal(got.pos.cpu().numpy(), want["pos"])
    assert np.array_equal(got.slots.cpu().numpy(), want["slots"])
    if pad == 0:   # the host construction the GPU path replaces gives the same arrays
        host = pa.PagedBatch.from_ubatch(want["pos"], want["seq_idx"], want["slots"], want["cells"], block_size=bs,
                                         device="cpu")
        for f in ("block_tables", "seq_lens", "query_start_loc", "pos", "slots"):
            assert np.array_equal(getattr(got, f).cpu().numpy(), getattr(host, f).numpy()), f
    us = kernel_us(lambda: pa.build_batch(req, T, bs, max_blocks, sp.num_blocks, out=got))
    print(f"[gpu] build_batch {name}: {us:.1f} us per call", flush=True)


def test_attention_over_device_built_batch(pa, oracle):
    """cfg2 small: attention reading the device-built batch gives the same
    bits as attention reading the host-built one."""
    from iian_amd import synth
    sp = synth.spec("cfg2", small=True)
    w = synth.build(sp)
    ids, nc, nn = synth.request_blocks(sp)
    req = pa.RequestBlocks.pack(ids, nc, nn)
    dev = pa.build_batch(req, w.T, sp.block_size, w.batch.block_tables.shape[1], sp.num_blocks,
                         max_query_len=int(nn.max()))
    a = pa.build_paged_attn(w.q, w.k_pool, w.v_pool, sp.Hkv, w.params, w.batch).cpu().numpy()
    b = pa.build_paged_attn(w.q, w.k_pool, w.v_pool, sp.Hkv, w.params, dev).cpu().numpy()
    assert np.array_equal(a, b)


def test_build_batch_flags_inconsistent_requests(pa):
    """A request whose blocks do not cover its context, and a block id outside
    the pool, are flagged (bits 3, 0 and 1); the missing token's slot is -1,
    which the KV write skips."""
    req = pa.RequestBlocks.pack([[3, 4], [5], [99]], [20, 0, 0], [20, 1, 1])   # 40 tokens in 2 blocks
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    b = pa.build_batch(req, 22, 16, 4, 64, err_flag=err)
    torch.cuda.synchronize()
    e = int(err.item())
    assert e & 8 and e & 1 and e & 2
    slots = b.slots.cpu().numpy()
    # request 0's new tokens are positions 20..39: 20..31 in its second block (id 4), 32..39 in a missing third
    assert slots[:12].tolist() == [4 * 16 + 4 + i for i in range(12)] and (slots[12:20] == -1).all()
    assert slots[20] == 5 * 16 and slots[21] == 99 * 16
    assert b.query_start_loc.cpu().tolist() == [0, 20, 21, 22]


def test_build_batch_fills_tokens_past_the_counts(pa):
    """n_tokens above the sum of the new-token counts: bit 3 is set, and the
    tokens past the last request get pos 0 and slot -1, so a KV write of
    n_tokens rows skips them (bit 0) and leaves the pool untouched."""
    req = pa.RequestBlocks.pack([[3, 4], [5]], [10, 0], [6, 1])   # 7 new tokens
    T = 12
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    b = pa.build_batch(req, T, 16, 4, 64, err_flag=err)
    b.pos.fill_(12345)            # stale contents must be overwritten
    b.slots.fill_(7)
    pa.build_batch(req, T, 16, 4, 64, err_flag=err, out=b)
    torch.cuda.synchronize()
    assert int(err.item()) & 8
    assert b.pos.cpu().tolist()[7:] == [0] * 5
    assert b.slots.cpu().tolist()[7:] == [-1] * 5
    assert b.slots.cpu().tolist()[:7] == [3 * 16 + 10 + i for i in range(6)] + [5 * 16]
    pool = pa.KVPool(64 * 16, 64, pa.GGML_TYPE_F16, device="cuda")
    pool.data.zero_()
    err2 = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa.set_rows(pool, torch.ones((T, 64), device="cuda"), b.slots, err2)
    torch.cuda.synchronize()
    assert int(err2.item()) & 1
    rows = pool.data.view(64 * 16, -1).cpu()
    written = (rows != 0).any(dim=1).nonzero().flatten().tolist()
    assert written == sorted([3 * 16 + 10 + i for i in range(6)] + [5 * 16])
