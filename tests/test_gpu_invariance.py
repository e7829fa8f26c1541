"""Batching and chunking invariance of the attention op, at the operator level.

The reference's paged-engine test (tests/e2e/test-batching.cpp:79-218, the
`paged` variant) asserts that greedy outputs do not depend on how requests are
batched or how a prompt is chunked.  Here the same property is checked on the
op's outputs directly:

* chunked prefill: a prompt's query tokens attended in one call, or in two
  consecutive calls (the second over the cells the first chunk would have
  written), give the same rows bit for bit.  A prefill row's cells are walked
  in the same tile order either way and masked cells add exact zeros, so the
  row block a token lands in does not change its arithmetic.  With a sliding
  window a row block's tiles start at its own window's first cell, so the
  cells are grouped into tiles differently; a row's reference max (the one
  its exponentials are taken against, moved lazily) then moves at other
  tiles, which changes the f16 rounding of P, and rows agree to the 2e-3 bar
  (5.6e-4 measured) instead of bit for bit;
* batch composition: a prefill chunk attended alone or beside other
  sequences gives the same rows bit for bit.  Decode rows are split into
  stream-K pieces along the whole call's line of tiles, and each piece takes
  its exponentials against its own running max, so the f16 rounding of P
  follows the split: they agree to the 2e-3 bar (2e-4 measured).

Every call is also checked against the CPU oracle at the usual 2e-3 bar.
"""
import numpy as np
import pytest
import torch

from helpers import Q8_0, Case, make_case, row_rel_err
from test_gpu_parity import TOL, banner, gpu_attention, oracle_attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


def sub_case(c: Case, parts) -> Case:
    """The case made of `parts`: (sequence s of c, its query tokens [a, b),
    seq_len) each, over c's pools and block-table rows."""
    q, bt, lens, seq_idx, pos, nq = [], [], [], [], [], []
    for i, (s, a, b, L) in enumerate(parts):
        t0 = c.qsl[s]
        q.append(c.q[t0 + a:t0 + b])
        pos.append(c.pos[t0 + a:t0 + b])
        seq_idx += [i] * (b - a)
        bt.append(c.bt[s])
        lens.append(L)
        nq.append(b - a)
    qsl = np.zeros(len(parts) + 1, np.int32)
    qsl[1:] = np.cumsum(nq)
    return Case(np.concatenate(q), c.k_pool, c.v_pool, c.k_type, c.v_type, np.stack(bt), np.array(lens, np.int32),
                np.array(seq_idx, np.int32), np.concatenate(pos).astype(np.int32), qsl, c.H, c.Hkv, c.D, c.bs,
                c.scale, c.softcap, c.causal, c.n_swa, c.Dv)


def checked(pa, oracle, c, what):
    got = gpu_attention(pa, c)
    e = row_rel_err(got, oracle_attention(oracle, c)).max()
    print(f"[gpu] {what}: max row rel err vs oracle {e:.3e}", flush=True)
    assert e <= TOL, (what, e)
    return got


CHUNKING = {
    # name: (H, Hkv, D, lens, nq, kwargs)
    "f16_d128": (32, 8, 128, [900, 400], [256, 100], {}),
    "f16_d64": (14, 2, 64, [700, 300], [200, 90], {}),
    "f16_d96": (32, 32, 96, [600, 300], [160, 64], {}),
    "f16_d256": (16, 8, 256, [800, 400], [256, 120], {}),
    "q8_d128": (32, 8, 128, [900, 400], [256, 100], {"k_type": Q8_0}),
    "f16_d128_swa_softcap": (16, 4, 128, [1500, 700], [300, 100], {"n_swa": 400, "softcap": 30.0}),
}


@pytest.mark.parametrize("name", sorted(CHUNKING))
def test_prefill_chunking(pa, oracle, name):
    H, Hkv, D, lens, nq, kw = CHUNKING[name]
    banner(f"chunking {name} H={H} Hkv={Hkv} D={D} lens={lens} nq={nq} {kw}")
    c = make_case(np.random.default_rng(sum(map(ord, name))), H, Hkv, D, lens, nq,
                  quantize=oracle.quantize_q8_0, **kw)
    whole = checked(pa, oracle, c, f"{name} one call")
    # the first chunk sees the cells up to its own last token, as the engine's
    # seq_len would be before the second chunk is written
    first = [(s, 0, n // 2, L - n + n // 2) for s, (L, n) in enumerate(zip(lens, nq))]
    second = [(s, n // 2, n, L) for s, (L, n) in enumerate(zip(lens, nq))]
    a = checked(pa, oracle, sub_case(c, first), f"{name} first chunks")
    b = checked(pa, oracle, sub_case(c, second), f"{name} second chunks")
    parts = []
    for s, n in enumerate(nq):
        t0 = c.qsl[s]
        parts.append((t0, t0 + n // 2, t0 + n))
    want_a = np.concatenate([whole[t0:tm] for t0, tm, _ in parts])
    want_b = np.concatenate([whole[tm:t1] for _, tm, t1 in parts])
    for got, want, which in ((a, want_a, "first"), (b, want_b, "second")):
        if c.n_swa == 0:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                f"{which} chunks differ from the one-call rows"
        else:
            e = row_rel_err(got, want).max()
            print(f"[gpu] {name}: {which} chunks against one call: max row rel diff {e:.3e}", flush=True)
            assert e <= TOL, (name, which, e)


COMPOSITION = {
    # name: (H, Hkv, D, lens, nq, kwargs); sequence 0 is the prefill chunk, the rest decode rows
    "f16_d128": (32, 8, 128, [900, 1500, 700, 3000], [256, 1, 1, 1], {}),
    "f16_d256": (16, 8, 256, [800, 2000, 600], [256, 1, 1], {}),
    "q8_d128": (32, 8, 128, [900, 1500, 700], [256, 1, 1], {"k_type": Q8_0}),
    "f16_d96": (32, 32, 96, [600, 1200, 500], [128, 1, 1], {}),
}


@pytest.mark.parametrize("name", sorted(COMPOSITION))
def test_batch_composition(pa, oracle, name):
    H, Hkv, D, lens, nq, kw = COMPOSITION[name]
    banner(f"composition {name} H={H} Hkv={Hkv} D={D} lens={lens} nq={nq} {kw}")
    c = make_case(np.random.default_rng(sum(map(ord, name)) + 7), H, Hkv, D, lens, nq,
                  quantize=oracle.quantize_q8_0, **kw)
    together = checked(pa, oracle, c, f"{name} prefill and decode rows in one call")
    alone = checked(pa, oracle, sub_case(c, [(0, 0, nq[0], lens[0])]), f"{name} the prefill chunk alone")
    dec = checked(pa, oracle, sub_case(c, [(s, 0, nq[s], lens[s]) for s in range(1, len(lens))]),
                  f"{name} the decode rows alone")
    n0 = nq[0]
    assert np.array_equal(alone.view(np.uint32), together[:n0].view(np.uint32)), \
        "a prefill chunk's rows depend on the other sequences of its batch"
    e = row_rel_err(dec, together[n0:]).max()
    print(f"[gpu] {name}: decode rows alone against in the batch: max row rel diff {e:.3e}", flush=True)
    assert e <= TOL, (name, e)
