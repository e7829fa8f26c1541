"""GPU parity of iian_pa_rope_kv_write (pa_rope.hip): RoPE of K fused with
the layer's K and V writes (src/iian/graph.cpp:250-253, 319-320), plus the
same rotation of q.  The pool bytes must equal, bit for bit, the oracle's
RoPE (pa_oracle.c pao_rope_rows, ggml's CPU rope restated) followed by its
set_rows, for f16, Q8_0 and f32 pools; the rotated q must equal the oracle's
bit for bit."""
import zlib

import numpy as np
import pytest
import torch

from helpers import F16, F32, Q8_0

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pa():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    import iian_amd
    iian_amd._lib.load()
    return iian_amd


CASES = {
    # name: (T, H, Hkv, D, Dv, types, rope kwargs, freq factors?)
    # Llama-3: NORMAL, base 500000, rope_freqs factors
    "llama3_f16": (64, 32, 8, 128, 128, (F16, F16), dict(n_dims=128, mode=0, freq_base=500000.0), True),
    # Qwen: NEOX, base 1e6, Q8_0 pools (cfg4's format)
    "qwen_neox_q8": (640, 32, 8, 128, 128, (Q8_0, Q8_0), dict(n_dims=128, mode=2, freq_base=1e6), False),
    # Gemma3: NEOX at head size 256
    "gemma3_neox_d256": (96, 16, 8, 256, 256, (F16, F16), dict(n_dims=256, mode=2, freq_base=1e6), False),
    # Phi-3: NEOX at head size 96 with LongRoPE factors, f32 pools
    "phi3_longrope_f32": (80, 32, 32, 96, 96, (F32, F32), dict(n_dims=96, mode=2, freq_base=10000.0), True),
    # partial rotary (n_rot < head size), mixed pool types
    "partial_rotary_mixed": (50, 8, 2, 128, 64, (F16, Q8_0), dict(n_dims=64, mode=0, freq_base=10000.0), False),
    # YaRN
    "yarn_f16": (70, 8, 4, 128, 128, (F16, F16),
                 dict(n_dims=128, mode=2, freq_base=10000.0, freq_scale=0.25, ext_factor=1.0, n_ctx_orig=4096,
                      attn_factor=1.0, beta_fast=32.0, beta_slow=1.0), False),
}


def pool_bytes(t, n):
    return n // 32 * 34 if t == Q8_0 else n * {F32: 4, F16: 2}[t]


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("q_mode", ["separate", "in_place"])
def test_rope_kv_write_bit_exact(pa, oracle, name, q_mode):
    T, H, Hkv, D, Dv, (tk, tv), rk, has_ff = CASES[name]
    print(f"\n[gpu] rope_kv_write {name} q={q_mode}", flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    n_cells = 4 * T + 64
    k_rows = rng.standard_normal((T, Hkv * D)).astype(np.float32)
    v_rows = rng.standard_normal((T, Hkv * Dv)).astype(np.float32)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = rng.integers(0, 32768, T).astype(np.int32)
    slots = rng.choice(n_cells, T, replace=False).astype(np.int64)
    ff = rng.uniform(1.0, 30.0, rk["n_dims"] // 2).astype(np.float32) if has_ff else None
    kinit = rng.integers(0, 256, (n_cells, pool_bytes(tk, Hkv * D)), dtype=np.uint8)
    vinit = rng.integers(0, 256, (n_cells, pool_bytes(tv, Hkv * Dv)), dtype=np.uint8)

    kp = pa.KVPool.wrap(torch.as_tensor(kinit).cuda(), Hkv * D, tk)
    vp = pa.KVPool.wrap(torch.as_tensor(vinit).cuda(), Hkv * Dv, tv)
    rope = pa.RopeParams(freq_factors=None if ff is None else torch.as_tensor(ff).cuda(), **rk)
    qd = torch.as_tensor(q).cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q_out = pa.rope_set_rows_kv(kp, vp, torch.as_tensor(k_rows).cuda(), torch.as_tensor(v_rows).cuda(),
                                torch.as_tensor(slots).cuda(), torch.as_tensor(pos).cuda(), rope, Hkv, q=qd,
                                q_out=qd if q_mode == "in_place" else None, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0

    okw = {k: v for k, v in rk.items()}
    k_rot = oracle.rope_rows(k_rows, pos, Hkv, D, freq_factors=ff, **okw)
    q_rot = oracle.rope_rows(q.reshape(T, H * D), pos, H, D, freq_factors=ff, **okw).reshape(T, H, D)
    kw, vw = kinit.copy(), vinit.copy()
    assert oracle.set_rows(kw, k_rot, slots, tk) == 0
    assert oracle.set_rows(vw, v_rows, slots, tv) == 0
    kg, vg = kp.data.cpu().numpy(), vp.data.cpu().numpy()
    bad = np.argwhere(kg != kw)
    assert bad.size == 0, f"{len(bad)} K pool bytes differ, first at {bad[:3].tolist()}"
    assert np.array_equal(vg, vw)
    qg = q_out.cpu().numpy()
    assert np.array_equal(qg.view(np.uint32), q_rot.view(np.uint32))
    if q_mode == "in_place":
        assert q_out.data_ptr() == qd.data_ptr()


def test_rope_kv_write_out_of_range_slot(pa, oracle):
    """A slot outside the pool is skipped and flagged (bit 0); q is still rotated."""
    T, H, Hkv, D = 4, 4, 2, 64
    rng = np.random.default_rng(70)
    kp, vp = pa.KVPool(32, Hkv * D, F16), pa.KVPool(32, Hkv * D, F16)
    k = torch.as_tensor(rng.standard_normal((T, Hkv * D)).astype(np.float32)).cuda()
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([5, 6, 7, 8], np.int32)
    slots = torch.tensor([3, 32, -1, 4], dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    qo = pa.rope_set_rows_kv(kp, vp, k, k.clone(), slots, torch.as_tensor(pos).cuda(), pa.RopeParams(n_dims=64), Hkv,
                             q=torch.as_tensor(q).cuda(), err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    got = kp.data.cpu().numpy()
    assert not np.delete(got, [3, 4], axis=0).any()
    want = oracle.rope_rows(q.reshape(T, -1), pos, H, D, 64).reshape(T, H, D)
    assert np.array_equal(qo.cpu().numpy(), want)
