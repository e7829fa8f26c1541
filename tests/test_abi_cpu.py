"""C-ABI checks that need no GPU: the library loads, exports every entry point
of include/iian_pa.h, and rejects invalid arguments on the host before any
device work (the reference aborts on these, paged_attn.cpp:161-162 and
ggml-cpu/ops.cpp:5263; the ABI returns status codes instead)."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def lib():
    from iian_amd import _lib
    return _lib.load()


def header_symbols():
    text = (ROOT / "include" / "iian_pa.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(iian_pa_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol(lib):
    from iian_amd import _lib
    syms = header_symbols()
    assert len(syms) >= 6
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_lib.SIGNATURES)


def test_status_strings(lib):
    from iian_amd import _lib
    for code in (_lib.OK, _lib.ERR_NULL, _lib.ERR_ARG, _lib.ERR_UNSUPPORTED, _lib.ERR_WORKSPACE, _lib.ERR_HIP,
                 _lib.ERR_SCRATCH):
        assert _lib.status_string(code) not in ("", "unknown status")
    assert _lib.status_string(12345) == "unknown status"


def test_supported_matrix(lib):
    """iian_pa_supported accepts what paged_attn_supported accepts
    (paged_attn.cpp:15-18: K and V each F16 or F32, in any pairing, no ALiBi;
    any head size, Dv from the V pool, :163), widened to Q8_0: every head
    size from 1 to 1024 (multiples of 32 for a Q8_0 pool)."""
    from iian_amd import paged_attn_supported as sup
    F32, F16, Q8 = 0, 1, 8
    for tk in (F32, F16, Q8):
        for tv in (F32, F16, Q8):
            for d in (32, 64, 96, 128, 160, 256, 512):
                assert sup(tk, tv, 0.0, d), (tk, tv, d)
                assert sup(tk, tv, 0.0, d, 64) and sup(tk, tv, 0.0, 64, d)      # Dv != D
            assert not sup(tk, tv, 8.0, 128)                                   # ALiBi (paged_attn.cpp:17)
    for d in (1, 2, 3, 4, 6, 8, 50, 80, 100, 112, 130, 200, 508, 516, 1000, 1023):
        assert sup(F16, F16, 0.0, d) and sup(F32, F16, 0.0, d) and sup(F16, F32, 0.0, 64, d)
        assert not sup(Q8, F16, 0.0, d) and not sup(F16, Q8, 0.0, 64, d)      # Q8_0 rows: 32-element blocks
    for d in (576, 1024):
        assert sup(F16, F16, 0.0, d) and sup(Q8, Q8, 0.0, d) and sup(F32, F16, 0.0, 64, d)
    # beyond what the general kernel stages
    for d in (0, -4, 1025, 1056, 2048):
        assert not sup(F16, F16, 0.0, d) and not sup(F32, F32, 0.0, 64, d) and not sup(Q8, Q8, 0.0, d)
    assert not sup(2, F16, 0.0, 128) and not sup(F16, 2, 0.0, 128)           # Q4_0 pools are not KV types here


def test_workspace_size(lib):
    """Stream-K partial records: the size follows the sequence count, kv heads
    and head size, not the context length or the token count."""
    from iian_amd import workspace_size
    a = workspace_size(64, 64, 32, 8, 128, 512, 16)
    b = workspace_size(64, 64, 32, 8, 128, 1024, 16)
    c = workspace_size(64, 128, 32, 8, 128, 512, 16)
    d = workspace_size(64, 64, 32, 8, 256, 512, 16)
    assert 0 < a == b < c and a < d
    assert workspace_size(-1, 64, 32, 8, 128, 512, 16) == 0
    assert workspace_size(64, 64, 32, 0, 128, 512, 16) == 0
    assert workspace_size(0, 0, 32, 8, 128, 512, 16) > 0
    # a prefill-heavy batch needs no more than its sequence count asks for
    big = workspace_size(2080, 36, 32, 8, 128, 290, 16)
    assert big == workspace_size(8000, 36, 32, 8, 128, 290, 16)
    assert big < workspace_size(2080, 2080, 32, 8, 128, 290, 16)


def call_attention(lib, **over):
    """iian_pa_attention with a valid-looking argument set (fake but aligned
    device addresses: every case here must be rejected before any launch)."""
    a = dict(stream=None, q=0x1000, k=0x2000, v=0x3000, tk=1, tv=1, num_blocks=64, bt=0x4000, max_blocks=4,
             seq_lens=0x5000, qsl=0x6000, pos=0x7000, T=4, S=2, maxq=2, H=8, Hkv=2, D=128, Dv=128, bs=16,
             scale=0.1, softcap=0.0, causal=1, n_swa=0, out=0x8000, ws=0x9000, ws_bytes=1 << 30, err=None)
    a.update(over)
    return lib.iian_pa_attention(a["stream"], a["q"], a["k"], a["v"], a["tk"], a["tv"], a["num_blocks"], a["bt"],
                                 a["max_blocks"], a["seq_lens"], a["qsl"], a["pos"], a["T"], a["S"], a["maxq"],
                                 a["H"], a["Hkv"], a["D"], a["Dv"], a["bs"], a["scale"], a["softcap"], a["causal"],
                                 a["n_swa"], a["out"], a["ws"], a["ws_bytes"], a["err"])


@pytest.mark.parametrize("over,code", [
    ({"q": None}, -1), ({"k": None}, -1), ({"bt": None}, -1), ({"out": None}, -1), ({"pos": None}, -1),
    ({"H": 6, "Hkv": 4}, -2), ({"Hkv": 0}, -2), ({"T": -1}, -2), ({"maxq": 5}, -2), ({"num_blocks": 0}, -2),
    ({"n_swa": -1}, -2), ({"softcap": -1.0}, -2), ({"scale": float("nan")}, -2), ({"q": 0x1004}, -2),
    ({"tk": 8, "tv": 8, "D": 80, "Dv": 80}, -3), ({"tk": 2, "tv": 2}, -3), ({"D": 1028, "Dv": 1028}, -3),
    ({"D": 2048, "Dv": 2048}, -3), ({"Dv": 1056}, -3), ({"D": 0, "Dv": 0}, -3), ({"bs": 0}, -2),
    ({"num_blocks": (1 << 28) + 1}, -3),                      # more than 2^32 cells on the MFMA path
    ({"tk": 0, "tv": 0, "max_blocks": 1 << 28}, -3),          # 2^32 cells in one sequence on the general path
    ({"ws": None}, -4), ({"ws_bytes": 16}, -4),
])
def test_attention_rejects_invalid_arguments(lib, over, code):
    assert call_attention(lib, **over) == code


def call_write_attention(lib, **over):
    """iian_pa_write_attention with fake aligned addresses, as call_attention."""
    a = dict(stream=None, q=0x1000, kn=0x10000, vn=0x11000, k=0x2000, v=0x3000, tk=1, tv=1, num_blocks=64,
             bt=0x4000, max_blocks=4, seq_lens=0x5000, qsl=0x6000, pos=0x7000, T=4, S=2, maxq=2, H=8, Hkv=2, D=128,
             Dv=128, bs=16, scale=0.1, softcap=0.0, causal=1, n_swa=0, out=0x8000, ws=0x9000, ws_bytes=1 << 30,
             err=None)
    a.update(over)
    return lib.iian_pa_write_attention(a["stream"], a["q"], a["kn"], a["vn"], a["k"], a["v"], a["tk"], a["tv"],
                                       a["num_blocks"], a["bt"], a["max_blocks"], a["seq_lens"], a["qsl"], a["pos"],
                                       a["T"], a["S"], a["maxq"], a["H"], a["Hkv"], a["D"], a["Dv"], a["bs"],
                                       a["scale"], a["softcap"], a["causal"], a["n_swa"], a["out"], a["ws"],
                                       a["ws_bytes"], a["err"])


@pytest.mark.parametrize("over,code", [
    ({"kn": None}, -1), ({"vn": None}, -1), ({"q": None}, -1), ({"kn": 0x10004}, -2), ({"vn": 0x11008}, -2),
    ({"tk": 8, "tv": 8}, -3),                        # Q8_0 pools: the two calls
    ({"tk": 0, "tv": 0}, -3),                        # f32 pools (the general kernel)
    ({"D": 128, "Dv": 64}, -3),                      # K and V head sizes differ
    ({"D": 80, "Dv": 80}, -3),                       # a head size only the general kernel takes
    ({"bs": 4}, -3),                                 # blocks below 8 cells
    ({"T": 40, "maxq": 20}, -3),                     # 80 rows per kv head: a prefill call
    ({"ws": None}, -4),
])
def test_write_attention_rejects_calls_outside_the_decode_kernels(lib, over, code):
    assert call_write_attention(lib, **over) == code


def test_write_attention_empty_batch_is_ok(lib):
    assert call_write_attention(lib, T=0) == 0
    assert call_write_attention(lib, S=0, kn=None) == 0


def test_attention_empty_batch_is_ok(lib):
    assert call_attention(lib, T=0) == 0
    assert call_attention(lib, S=0) == 0


def test_kv_write_rejects_invalid_arguments(lib):
    # every call here must return before any launch (the pointers are fake)
    f = lib.iian_pa_kv_write
    assert f(None, None, 4, 128, 0x2000, 0x3000, 64, 1, None) == -1
    assert f(None, 0x1000, 4, 128, None, 0x3000, 64, 1, None) == -1
    assert f(None, 0x1000, -1, 128, 0x2000, 0x3000, 64, 1, None) == -2
    assert f(None, 0x1000, 4, 100, 0x2000, 0x3000, 64, 8, None) == -2      # Q8_0 needs 32-multiples
    assert f(None, 0x1000, 4, 128, 0x2000, 0x3000, 64, 2, None) == -3      # Q4_0 not a KV write type here
    assert f(None, 0x1000, 0, 128, 0x2000, 0x3000, 64, 1, None) == 0       # nothing to do


def test_kv_write_kv_rejects_invalid_arguments(lib):
    f = lib.iian_pa_kv_write_kv
    ok = dict(k=0x1000, v=0x1100, n=4, ek=128, ev=128, slots=0x2000, kp=0x3000, vp=0x4000, cells=64, tk=1, tv=1)

    def call(**over):
        a = dict(ok, **over)
        return f(None, a["k"], a["v"], a["n"], a["ek"], a["ev"], a["slots"], a["kp"], a["vp"], a["cells"], a["tk"],
                 a["tv"], None)
    assert call(v=None) == -1 and call(vp=None) == -1 and call(slots=None) == -1
    assert call(n=-1) == -2 and call(ev=0) == -2
    assert call(tv=8, ev=100) == -2                                     # Q8_0 needs 32-multiples
    assert call(tk=2) == -3
    assert call(n=0) == 0


def test_dequant_rejects_invalid_arguments(lib):
    f = lib.iian_pa_dequant_q8_0
    assert f(None, None, 64, 0x2000, 4, 128, 0x3000) == -1
    assert f(None, 0x1000, 64, 0x2000, 4, 100, 0x3000) == -2
    assert f(None, 0x1000, 64, 0x2000, 0, 128, 0x3000) == 0


def test_ubatch_compression_roundtrip():
    """UBatch (per-sequence absolute cells, engine.cpp:501-507) -> block tables."""
    from iian_amd import PagedBatch
    bs = 16
    tables = [[5, 9, 2], [7], [3, 11]]
    lens = [40, 16, 17]
    seq_cells = [[t[i // bs] * bs + i % bs for i in range(n)] for t, n in zip(tables, lens)]
    pos = [39, 15, 15, 16]
    seq_idx = [0, 1, 2, 2]
    slots = [seq_cells[s][p] for s, p in zip(seq_idx, pos)]
    b = PagedBatch.from_ubatch(pos, seq_idx, slots, seq_cells, block_size=bs, device="cpu")
    assert b.block_tables.tolist() == [[5, 9, 2], [7, 0, 0], [3, 11, 0]]
    assert b.seq_lens.tolist() == lens
    assert b.query_start_loc.tolist() == [0, 1, 2, 4]
    assert b.max_query_len == 2
    assert b.slots.tolist() == slots
    with pytest.raises(ValueError):
        PagedBatch.from_ubatch(pos, [0, 2, 1, 2], slots, seq_cells, device="cpu")      # not contiguous
    bad = [list(c) for c in seq_cells]
    bad[0][3] += 1
    with pytest.raises(ValueError):
        PagedBatch.from_ubatch(pos, seq_idx, slots, bad, device="cpu")                 # not block-structured
    with pytest.raises(ValueError):
        PagedBatch.from_ubatch(pos, seq_idx, slots, seq_cells, device="cpu",
                               seq_cell_pos=[list(range(40)), list(range(16)), [1] * 17])


def test_host_wrappers_validate_before_launch():
    from iian_amd import KVPool, PagedAttnParams, PagedBatch, build_paged_attn
    pool = KVPool.wrap(torch.zeros((64, 512), dtype=torch.uint8), 256, 1)
    b = PagedBatch.from_ubatch([3], [0], [3], [[0, 1, 2, 3]], device="cpu")
    with pytest.raises(ValueError):
        build_paged_attn(torch.zeros((1, 4, 128), dtype=torch.float16), pool, pool, 2, PagedAttnParams(), b)
    with pytest.raises(ValueError):
        build_paged_attn(torch.zeros((1, 4, 64), dtype=torch.float32), pool, pool, 2, PagedAttnParams(), b)
    with pytest.raises(ValueError):
        build_paged_attn(torch.zeros((1, 4, 128), dtype=torch.float32).transpose(0, 1), pool, pool, 2,
                         PagedAttnParams(), b)


def test_bound_calls_check_their_arguments_when_bound():
    """bind_paged_attn / bind_set_rows_kv run the same checks as the plain
    wrappers, once, before anything is bound."""
    from iian_amd import KVPool, PagedAttnParams, PagedBatch, bind_paged_attn, bind_set_rows_kv
    pool = KVPool.wrap(torch.zeros((64, 512), dtype=torch.uint8), 256, 1)
    b = PagedBatch.from_ubatch([3], [0], [3], [[0, 1, 2, 3]], device="cpu")
    out = torch.empty((1, 4, 128), dtype=torch.float32)
    ws = torch.empty(16, dtype=torch.uint8)
    with pytest.raises(ValueError):   # f16 q
        bind_paged_attn(torch.zeros((1, 4, 128), dtype=torch.float16), pool, pool, 2, PagedAttnParams(), b, out, ws)
    with pytest.raises(ValueError):   # q not on a GPU
        bind_paged_attn(torch.zeros((1, 4, 128), dtype=torch.float32), pool, pool, 2, PagedAttnParams(), b, out, ws)
    rows = torch.zeros((3, 256), dtype=torch.float32)
    with pytest.raises(ValueError):   # int32 slots
        bind_set_rows_kv(pool, pool, rows, rows, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError):   # non-contiguous rows
        bind_set_rows_kv(pool, pool, torch.zeros((256, 3)).t(), rows, torch.zeros(3, dtype=torch.int64))


def test_noalloc_rejects_a_call_beyond_its_scratch(lib):
    """iian_pa_attention_noalloc checks its need against the 64 MiB scratch on
    the host and returns IIAN_PA_ERR_SCRATCH before any launch (pointers are
    fake: nothing may reach the device)."""
    from iian_amd import _lib
    f = lib.iian_pa_attention_noalloc
    # 40000 decode sequences x 8 kv heads: ~2.7 GB of stream-K records
    st = f(None, 0x1000, 0x2000, 0x3000, 1, 1, 1 << 20, 0x4000, 4, 0x5000, 0x6000, 0x7000, 40000, 40000, 1, 32, 8,
           128, 128, 16, 0.1, 0.0, 1, 0, 0x8000, None)
    assert st == _lib.ERR_SCRATCH
    assert "64 MiB" in _lib.status_string(st)
    # argument checks come first, as in iian_pa_attention
    assert f(None, None, 0x2000, 0x3000, 1, 1, 64, 0x4000, 4, 0x5000, 0x6000, 0x7000, 4, 2, 2, 8, 2, 128, 128, 16,
             0.1, 0.0, 1, 0, 0x8000, None) == _lib.ERR_NULL
    assert f(None, 0x1000, 0x2000, 0x3000, 1, 1, 64, 0x4000, 4, 0x5000, 0x6000, 0x7000, 4, 2, 2, 8, 2, 1028, 1028, 16,
             0.1, 0.0, 1, 0, 0x8000, None) == _lib.ERR_UNSUPPORTED


def test_runtime_rejects_invalid_configs(lib):
    """iian_pa_runtime_create validates its configuration before allocating
    anything (no device work on these paths)."""
    from iian_amd import _lib
    ok = dict(max_seqs=8, max_tokens=64, max_blocks_per_seq=32, max_total_blocks=256, n_head=32, n_head_kv=8,
              head_dim=128, head_dim_v=128, block_size=16, num_blocks=1024, type_k=1, type_v=1)

    def create(**over):
        cfg = _lib.RuntimeConfig(**dict(ok, **over))
        h = C.c_void_p()
        st = lib.iian_pa_runtime_create(C.byref(cfg), C.byref(h))
        assert not h.value
        return st
    assert create(max_seqs=0) == _lib.ERR_ARG
    assert create(n_head=30) == _lib.ERR_ARG            # not a multiple of n_head_kv
    assert create(block_size=0) == _lib.ERR_ARG
    assert create(head_dim=1028) == _lib.ERR_UNSUPPORTED
    assert create(type_k=2) == _lib.ERR_UNSUPPORTED
    assert lib.iian_pa_runtime_create(None, None) == _lib.ERR_NULL
    lib.iian_pa_runtime_destroy(None)
    assert lib.iian_pa_runtime_begin_step(None, None, None, None, None, None, 1) == _lib.ERR_NULL
    assert lib.iian_pa_runtime_layer(None, None, None, None, None, None, None, None, None, 1.0, 0.0, 1, 0,
                                     None) == _lib.ERR_NULL


def test_runtime_layer_checks_the_step_shapes():
    """PagedAttnRuntime.layer checks q, the rows, out and the pools against
    the configuration and the token count of the last begin_step before the
    C runtime reads rt->T rows (a runtime object without device buffers:
    nothing may reach the library)."""
    from iian_amd import _lib
    from iian_amd.paged_attn import KVPool, PagedAttnParams, PagedAttnRuntime
    rt = PagedAttnRuntime.__new__(PagedAttnRuntime)
    rt.cfg = _lib.RuntimeConfig(8, 64, 32, 256, 8, 2, 64, 64, 16, 4, 1, 1)
    rt._h = C.c_void_p()
    T = 5
    q, out = torch.zeros((T, 8, 64)), torch.zeros((T, 8, 64))
    kr, vr = torch.zeros((T, 128)), torch.zeros((T, 128))
    pool = KVPool.wrap(torch.zeros((64, 256), dtype=torch.uint8), 128, 1)
    prm = PagedAttnParams()
    with pytest.raises(ValueError, match="begin_step"):
        rt.layer(q, kr, vr, pool, pool, prm, out)
    rt._T = T
    for bad in (dict(q=torch.zeros((T + 1, 8, 64))), dict(kr=torch.zeros((T, 64))), dict(vr=torch.zeros((T - 1, 128))),
                dict(out=torch.zeros((T, 8, 32)))):
        a = dict(q=q, kr=kr, vr=vr, out=out, **{})
        a.update(bad)
        with pytest.raises(ValueError, match="shape"):
            rt.layer(a["q"], a["kr"], a["vr"], pool, pool, prm, a["out"])
    with pytest.raises(ValueError, match="GPU"):   # right shapes, host tensors
        rt.layer(q, kr, vr, pool, pool, prm, out)


def test_rope_kv_write_rejects_unaligned_rows_and_split_q8_blocks(lib):
    """iian_pa_rope_kv_write loads and stores adjacent f32 pairs as 8-byte
    accesses and quantises each Q8_0 head row in its own blocks: unaligned
    buffers and Q8_0 heads that are not whole 32-value blocks (or above 512
    values) are refused on the host (fake pointers: nothing may reach the
    device)."""
    from iian_amd import _lib
    prm = _lib.RopeParams(64, 0, 0, 10000.0, 1.0, 0.0, 1.0, 32.0, 1.0, None)
    f = lib.iian_pa_rope_kv_write

    def call(k_rows=0x1000, q=0x3000, D=64, Dv=64, tk=1, tv=1):
        return f(None, k_rows, 0x2000, q, q, 0x4000, 0x5000, 4, 4, 2, D, Dv, C.byref(prm), 0x6000, 0x7000, 64, tk,
                 tv, None)
    assert call(k_rows=0x1004) == _lib.ERR_ARG
    assert call(q=0x3004) == _lib.ERR_ARG
    assert call(D=80, Dv=64, tk=8, tv=1) == _lib.ERR_UNSUPPORTED     # 80-value heads: blocks would span heads
    assert call(D=64, Dv=48, tk=1, tv=8) == _lib.ERR_UNSUPPORTED
    assert call(D=576, Dv=64, tk=8, tv=1) == _lib.ERR_UNSUPPORTED
    wide = _lib.RopeParams(576, 0, 0, 10000.0, 1.0, 0.0, 1.0, 32.0, 1.0, None)   # more pairs than the table holds
    assert f(None, 0x1000, 0x2000, 0x3000, 0x3000, 0x4000, 0x5000, 4, 4, 2, 640, 64, C.byref(wide), 0x6000, 0x7000,
             64, 1, 1, None) == _lib.ERR_UNSUPPORTED
