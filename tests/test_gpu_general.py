"""GPU parity of the general fp32 path (pa_general.hip) against the CPU oracle.

It covers what the reference accepts beyond the MFMA kernels
(paged_attn.cpp:15-18, 148-155, Dv from the V pool at :163): F32 pools, the
mixed (F16, F32) and (F32, F16) pools, head sizes such as Phi-3's 96 and 80,
Dv != D, and block sizes that are not a power of two >= 8; plus Q8_0 paired
with the other types.  Same bar as the MFMA kernels: max relative error per
(token, head) row at most 2e-3; the fp32 arithmetic lands near 1e-6.
"""
import zlib

import numpy as np
import pytest
import torch

from helpers import F16, F32, Q8_0, make_case, row_rel_err
from test_gpu_parity import banner, gpu_attention, oracle_attention, to_device

pytestmark = pytest.mark.gpu

TOL = 2e-3
# fp32 throughout: the general path should sit far below the shared bar
TOL_F32 = 2e-5


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


GENERAL = {
    # name: (H, Hkv, D, lens, nq, kwargs)
    "f32_decode_gqa4_d128": (32, 8, 128, [513, 77, 2048, 33], [1, 1, 1, 1], {"k_type": F32}),
    "f32_prefill_d128": (8, 2, 128, [600, 200], [300, 70], {"k_type": F32}),
    "f32_mixed_d64": (14, 2, 64, [900, 1500, 64], [128, 1, 1], {"k_type": F32}),
    "f16k_f32v_decode": (32, 8, 128, [700, 101, 4101], [1, 5, 1], {"k_type": F16, "v_type": F32}),
    "f32k_f16v_prefill": (8, 2, 128, [500, 90], [200, 1], {"k_type": F32, "v_type": F16}),
    "phi3_d96_decode_f32": (32, 32, 96, [800, 1200, 70], [1, 1, 1], {"k_type": F32}),   # f16 decode: MFMA kernel
    # f16 prefill at head size 96 runs on the MFMA prefill kernel from 8-cell
    # blocks up; 4-cell blocks keep this Phi-3 prefill on the general kernel
    "phi3_d96_prefill_gqa4": (40, 10, 96, [700, 300], [256, 33], {"bs": 4}),
    "d80_f16_mixed": (16, 4, 80, [600, 64, 900], [100, 1, 1], {}),
    "d80_f32_decode": (8, 8, 80, [300, 1000], [1, 1], {"k_type": F32}),
    "dv64_d128_f16": (32, 8, 128, [600, 90, 1500], [1, 5, 200], {"Dv": 64}),
    "dv128_d64_f32": (8, 2, 64, [300, 700], [40, 1], {"k_type": F32, "Dv": 128}),
    "d256_f32_decode": (16, 8, 256, [1500, 40], [1, 1], {"k_type": F32}),
    "d512_f16": (8, 2, 512, [300, 70], [3, 30], {}),
    "d4_f32": (4, 2, 4, [100, 30], [2, 1], {"k_type": F32}),
    "bs12_f16_d128": (8, 2, 128, [500, 61, 1000], [1, 40, 1], {"bs": 12}),
    "bs4_f16_d64": (8, 2, 64, [300, 100], [20, 1], {"bs": 4}),
    "bs1_f32": (4, 1, 64, [70, 19], [5, 1], {"bs": 1, "k_type": F32}),
    "q8k_f16v_d128": (32, 8, 128, [600, 200], [1, 70], {"k_type": Q8_0, "v_type": F16}),
    "q8_d96": (16, 4, 96, [400, 100], [1, 50], {"k_type": Q8_0}),
    "f16k_q8v_d64": (8, 2, 64, [300, 1000], [1, 1], {"k_type": F16, "v_type": Q8_0}),
    "f32_softcap": (8, 2, 128, [333, 77], [1, 40], {"k_type": F32, "softcap": 30.0}),
    "f32_swa_d96": (8, 2, 96, [3000, 900], [1, 100], {"k_type": F32, "n_swa": 256}),
    "f32_not_causal": (8, 2, 64, [300, 50], [20, 1], {"k_type": F32, "causal": False}),
    "f32_random_positions": (8, 2, 64, [300, 200], [6, 40], {"k_type": F32, "pos_mode": "random"}),
    "f32_long_splits": (8, 2, 128, [9000, 5000], [1, 1], {"k_type": F32}),
    # head sizes that are not multiples of 4 (rows staged element-wise into
    # zero-padded LDS rows) and above 512 (4-cell tiles, four output quads per
    # lane), through both the single-range and the split-and-merge launches
    "d70_f16_prefill": (8, 2, 70, [500, 90], [100, 1], {}),
    "d3_f32_decode": (4, 2, 3, [300, 40], [1, 1], {"k_type": F32}),
    "d130_dv33_f16": (8, 4, 130, [700, 200], [1, 40], {"Dv": 33}),
    "d1_dv5_f32_splits": (4, 1, 1, [6000, 100], [1, 1], {"k_type": F32, "Dv": 5}),
    "d576_dv512_f16_mla_like": (16, 1, 576, [900, 300], [1, 20], {"Dv": 512}),
    "d1024_f32_splits": (4, 2, 1024, [3000, 80], [1, 2], {"k_type": F32}),
    "d1000_f16_prefill": (4, 2, 1000, [400, 90], [70, 1], {}),
    "q8_d1024": (4, 2, 1024, [600, 100], [1, 30], {"k_type": Q8_0}),
    "d99_f16k_q8v_dv96": (8, 2, 99, [500, 300], [1, 12], {"v_type": Q8_0, "Dv": 96}),
    "f32_one_long_seq": (32, 8, 128, [32000], [1], {"k_type": F32}),
    "f32_prefix_shared": (32, 8, 128, [1200, 1100, 900, 300], [128, 64, 1, 1],
                          {"k_type": F32, "shared_blocks": 32, "shared_seqs": 3}),
}


@pytest.mark.parametrize("name", sorted(GENERAL))
def test_general_path_matches_oracle(pa, oracle, name):
    H, Hkv, D, lens, nq, kw = GENERAL[name]
    banner(f"general {name} H={H} Hkv={Hkv} D={D} lens={lens} nq={nq} {kw}")
    c = make_case(np.random.default_rng(zlib.crc32(name.encode())), H, Hkv, D, lens, nq,
                  quantize=oracle.quantize_q8_0, **kw)
    assert pa.paged_attn_supported(c.k_type, c.v_type, 0.0, c.D, c.Dv)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = gpu_attention(pa, c, err)
    want = oracle_attention(oracle, c)
    e = row_rel_err(got, want)
    print(f"[gpu] {name}: max row rel err {e.max():.3e}", flush=True)
    assert int(err.item()) == 0
    assert np.isfinite(got).all()
    assert e.max() <= (TOL_F32 if Q8_0 not in (c.k_type, c.v_type) else TOL), (name, e.max())


def test_general_all_masked_rows_are_zero(pa, oracle):
    banner("general all-masked rows")
    rng = np.random.default_rng(52)
    c = make_case(rng, 8, 2, 96, [100, 40, 16], [2, 1, 1], k_type=F32)
    c.pos[:] = [-5, -1, -2, 10]
    got = gpu_attention(pa, c)
    assert np.all(got[:3] == 0.0)
    assert row_rel_err(got[3:], oracle_attention(oracle, c)[3:]).max() <= TOL_F32


def test_general_split_records_with_garbage_workspace(pa, oracle):
    """Split records are written before the merge reads them in the same
    call: a workspace full of 0xff, random bytes or zeros gives the same bits."""
    banner("general split merge over garbage workspaces")
    rng = np.random.default_rng(53)
    c = make_case(rng, 32, 8, 128, [6000, 700, 3000, 2500], [1, 1, 1, 1], k_type=F32)
    k, v, batch = to_device(pa, c)
    prm = pa.PagedAttnParams(scale=c.scale)
    q = torch.as_tensor(c.q).cuda()
    ws = pa.new_workspace(c.T, 4, c.H, c.Hkv, c.Dv, c.bt.shape[1], c.bs)
    outs = []
    for fill in ("ff", "random", "zero"):
        if fill == "ff":
            ws.fill_(255)
        elif fill == "random":
            ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, generator=torch.Generator().manual_seed(8)))
        else:
            ws.zero_()
        outs.append(pa.build_paged_attn(q, k, v, c.Hkv, prm, batch, workspace=ws).cpu().numpy())
    assert row_rel_err(outs[0], oracle_attention(oracle, c)).max() <= TOL_F32
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("k_type,lens,nq,declared", [
    (F16, [500, 300, 900], [1, 3, 1], 1),        # decode launch: its row budget still covers the 3 tokens
    (F16, [600, 500], [200, 1], 64),             # prefill launch: rows past 64 tokens are not covered
    (Q8_0, [600, 500], [5, 1], 2),               # Q8_0 spec-verify launch
    (F32, [600, 500], [100, 1], 16),             # general path
])
def test_understated_max_query_len_is_flagged(pa, oracle, k_type, lens, nq, declared):
    """A sequence with more query tokens than the caller's max_query_len sets
    bit 2 of the error word; the sequences within the declared length are
    still exact."""
    banner(f"understated max_query_len k_type={k_type} nq={nq} declared={declared}")
    rng = np.random.default_rng(54 + declared)
    c = make_case(rng, 32, 8, 128, lens, nq, k_type=k_type, quantize=oracle.quantize_q8_0)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = gpu_attention(pa, c, err, max_query_len=declared)
    assert int(err.item()) & 4
    want = oracle_attention(oracle, c)
    ok_tokens = np.concatenate([np.arange(c.qsl[s], c.qsl[s + 1]) for s in range(len(lens)) if nq[s] <= declared])
    assert row_rel_err(got[ok_tokens], want[ok_tokens]).max() <= TOL
    # a correctly declared call leaves the bit clear
    err.zero_()
    gpu_attention(pa, c, err)
    assert int(err.item()) == 0
