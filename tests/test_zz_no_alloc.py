"""iian_pa_attention_noalloc (the entry point that allocates nothing) against
iian_pa_attention, through the C ABI.

Each case makes two calls in a row on the library's per-GPU scratch, the
second with a smaller input, and requires the same bits as the
workspace-taking entry point on the same arguments: both run the same
kernels with the same plan, and the scratch keeps the first call's contents
when the second starts.  Cases: f16 decode whose segments split over stream-K
workers (records + merge launch), a mixed f16 batch (in-launch merge through
tagged counters), a Q8_0 mixed batch (prefill and decode kernels in order on
the caller's stream instead of a side stream), the general fp32 path with
split ranges, and a head size of 512 on the general path whose split ranges
are capped by the scratch size (there the two entry points plan different
range counts, so the outputs agree within fp32 rounding, not bit for bit).
"""
import ctypes as C

import numpy as np
import pytest
import torch

from helpers import F16, F32, Q8_0, make_case, row_rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


def device_case(c):
    import iian_amd as pa
    k = pa.KVPool.wrap(torch.as_tensor(c.k_pool).cuda(), c.Hkv * c.D, c.k_type)
    v = pa.KVPool.wrap(torch.as_tensor(c.v_pool).cuda(), c.Hkv * c.Dv, c.v_type)
    nq = np.diff(c.qsl)
    batch = pa.PagedBatch(block_tables=torch.as_tensor(c.bt).cuda(), seq_lens=torch.as_tensor(c.seq_lens).cuda(),
                          query_start_loc=torch.as_tensor(c.qsl).cuda(), pos=torch.as_tensor(c.pos).cuda(),
                          slots=torch.zeros(c.T, dtype=torch.int64, device="cuda"), max_query_len=int(nq.max()),
                          block_size=c.bs)
    return torch.as_tensor(c.q).cuda(), k, v, batch


def call_noalloc(lib, c, q, k, v, batch, out, err):
    st = lib.iian_pa_attention_noalloc(
        torch.cuda.current_stream().cuda_stream, q.data_ptr(), k.data.data_ptr(), v.data.data_ptr(), c.k_type,
        c.v_type, k.n_cells // c.bs, batch.block_tables.data_ptr(), batch.block_tables.shape[1],
        batch.seq_lens.data_ptr(), batch.query_start_loc.data_ptr(), batch.pos.data_ptr(), c.T, len(c.seq_lens),
        batch.max_query_len, c.H, c.Hkv, c.D, c.Dv, c.bs, float(c.scale), float(c.softcap), int(c.causal),
        int(c.n_swa), out.data_ptr(), err.data_ptr())
    return st


CASES = [
    # (name, H, Hkv, D, lens big, nq big, lens small, nq small, kwargs)
    ("f16_decode_splits", 32, 8, 128, [9000, 700, 3000, 64], [1, 1, 1, 1], [2000, 90], [1, 1], {}),
    ("f16_mixed_one_launch", 32, 8, 128, [900, 5000, 700], [200, 1, 1], [600, 3000], [64, 1], {}),
    ("q8_mixed_in_order", 32, 8, 128, [900, 5000, 700], [200, 1, 1], [600, 3000], [64, 1], {"k_type": Q8_0}),
    ("f32_general_splits", 8, 2, 96, [6000, 700], [1, 3], [1500], [1], {"k_type": F32}),
    # head size 512 on the general path: 64 ranges of records would need 67.4 MB, more than the
    # scratch holds, so the no-allocation call plans fewer ranges than the workspace call (same
    # values within fp32 rounding, not the same bits)
    ("f16_general_d512_scratch_cap", 16, 1, 512, [1500], [32], [1200], [32], {"exact": False}),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_workspace_entry_on_two_calls(pa, oracle, case):
    name, H, Hkv, D, lens1, nq1, lens2, nq2, kw = case
    print(f"\n[gpu] noalloc {name}", flush=True)
    lib = pa._lib.load()
    rng = np.random.default_rng(61)
    kw = dict(kw)
    exact = kw.pop("exact", True)
    for lens, nq in ((lens1, nq1), (lens2, nq2)):
        c = make_case(rng, H, Hkv, D, lens, nq, quantize=oracle.quantize_q8_0, **kw)
        q, k, v, batch = device_case(c)
        prm = pa.PagedAttnParams(scale=c.scale, softcap=c.softcap, causal=c.causal, n_swa=c.n_swa)
        want = pa.build_paged_attn(q, k, v, c.Hkv, prm, batch).cpu().numpy()
        out = torch.full((c.T, H, c.Dv), float("nan"), dtype=torch.float32, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        assert call_noalloc(lib, c, q, k, v, batch, out, err) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert int(err.item()) == 0
        if exact:
            assert np.array_equal(got, want), (name, len(lens), np.abs(got - want).max())
        else:
            assert row_rel_err(got, want).max() <= 1e-5, (name, len(lens), np.abs(got - want).max())
        e = row_rel_err(got, oracle.paged_attention(c.q, c.k_pool, c.v_pool, c.k_type, c.v_type, c.bt, c.seq_lens,
                                                    c.seq_idx, c.pos, c.Hkv, c.Dv, c.bs, c.scale, n_threads=16))
        assert e.max() <= 2e-3, (name, e.max())
