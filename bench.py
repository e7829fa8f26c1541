"""Benchmark of the paged-attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config cfg2] [--no-cpu-baseline]

A step is one layer-call of the path at Llama-3-8B decode shapes (BASELINE
config 2): the slot-mapped KV write of the 64 new tokens (K and V pools) and
paged GQA decode attention over the block pool, inputs resident in HBM.
``value`` is the achieved algorithmic HBM bandwidth of the whole step (GB/s);
``attn_tok_per_s`` the query tokens per second of one layer-call.
``roofline`` is measured live for the dominant launch (the attention call) with
HIP events on the stream it runs on: one pair around K back-to-back calls
(``avg_launch_us``), and one pair around each call of K steps
(``avg_launch_us_evented``, which adds the event records' own cost to short
calls); ``cpu_baseline`` times the CPU oracle
(a restatement of the reference's paged_attn_impl) on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "paged decode attn achieved HBM GB/s (% of peak) + attn tok/s, Llama-3-8B shapes"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
WORKLOADS = {
    "cfg1": "Qwen2.5-0.5B paged decode, H14/Hkv2/D64, 8 seqs, ctx U[64,1024], 1024-block f16 pool",
    "cfg2": "Llama-3-8B paged decode, H32/Hkv8/D128, 64 seqs, ctx log-uniform [512,8192], "
            "16-token f16 blocks in a 65536-block pool, + KV write of 64 tokens",
    "cfg2_f32": "Llama-3-8B paged decode as cfg2 with F32 K/V pools (the general fp32 kernel), + KV write "
                "of 64 tokens",
    "cfg3": "Qwen3-8B mixed batch, H32/Hkv8/D128: 4 prefill chunks x 512 over prior U[1024,4096] "
            "(1024-token shared prefix) + 32 decode tokens, f16 KV",
    "cfg3_prefill": "Qwen3-8B, H32/Hkv8/D128: the 4 prefill chunks of cfg3 alone (x 512 tokens over prior "
                    "U[1024,4096], 1024-token shared prefix), f16 KV",
    "cfg4": "Llama-3-8B Q8_0 KV, 128 seqs x 4096 prior + 5 spec-verify queries",
    "cfg5_global_decode": "Gemma3-12B global layer decode, H16/Hkv8/D256, 32 seqs, ctx U[8192,32768]",
    "cfg5_local_decode": "Gemma3-12B local layer decode (n_swa=1024), H16/Hkv8/D256, 32 seqs",
    "cfg5_global_prefill": "Gemma3-12B global layer, 256-token prefill chunk per seq, 32 seqs",
    "cfg5_local_prefill": "Gemma3-12B local layer (n_swa=1024), 256-token prefill chunk per seq, 32 seqs",
    "phi3_decode": "Phi-3.5-mini paged decode, H32/Hkv32/D96, 64 seqs, ctx log-uniform [512,8192], f16 KV",
    "phi3_prefill": "Phi-3.5-mini chunked prefill, H32/Hkv32/D96, 4 chunks x 512 tokens over prior U[1024,4096], "
                    "f16 KV",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def pmc_traffic(config: str):
    """HBM bytes per attention launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (scaled by a calibration copy), recorded in profiles/."""
    f = ROOT / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get(config)
    return None if rec is None else int(rec["traffic_bytes_per_launch"])


def launch_kernels(sp, pa, max_blocks: int, block_size: int, cus: int) -> str:
    """The kernels one iian_pa_attention call of this workload launches (as
    run_attention in pa_abi.hip picks them on a device of `cus` CUs)."""
    gqa = sp.H // sp.Hkv
    rows = [int(n) * gqa for n in sp.n_q]
    if sp.D == 96 and sp.kv_type == pa.GGML_TYPE_F16 and max(rows) <= 32:
        return "pa_decode_f16_kernel<96> + pa_merge_kernel<96>"
    if (sp.D not in (64, 96, 128, 256) or (sp.D == 96 and sp.kv_type != pa.GGML_TYPE_F16)
            or sp.kv_type not in (pa.GGML_TYPE_F16, pa.GGML_TYPE_Q8_0)):
        return "pa_general_kernel + pa_general_merge_kernel"
    has_dec = any(0 < r <= 32 for r in rows)
    has_pf = any(r > 32 for r in rows)
    d = sp.D
    if sp.kv_type == pa.GGML_TYPE_Q8_0:
        dec = f"pa_decode_q8_kernel<{d}> + pa_merge_kernel<{d}>"
        pf = f"pa_prefill_kernel<{d}, Q8_0>" if d <= 128 else f"pa_prefill16_kernel<{d}, Q8_0>"
    else:
        dec = f"pa_decode_f16_kernel<{d}> + pa_merge_kernel<{d}>"
        pf = f"pa_prefill_kernel<{d}, f16>" if d <= 128 else f"pa_prefill16_kernel<{d}, f16>"
        if has_pf and d <= 128:   # the mixed-batch instantiation, also without decode rows
            extra = " (decode pieces in the same grid, merged there)" if has_dec else ""
            return f"pa_prefill_kernel<{d}, f16, mixed>{extra}"
        # decode-only calls with short or window-bounded segments: one
        # workgroup per (sequence, kv head)
        seg_waves = {64: 16, 128: 8, 256: 4}.get(d, 0)
        tiles = (max_blocks * block_size + 31) // 32
        if sp.n_swa > 0:
            wtiles = min(tiles, (sp.n_swa + max(sp.n_q) - 1 + 62) // 32)
            seg = wtiles <= 16 * seg_waves and len(sp.n_q) * sp.Hkv >= cus
        else:
            seg = tiles <= 2 * seg_waves
        if not has_pf and max(rows) <= 16 and seg_waves and seg:
            return f"pa_decode_seg_kernel<{d}, {seg_waves}>"
    if has_dec and has_pf:
        return f"{pf} || {dec} (two streams)"
    return pf if has_pf else dec


# The host-core share of one GPU on the GPU boxes: worker pools are sized to
# it whatever nproc reports there.
CPU_SHARE = 16


def host_cpu():
    """(nproc, cores this process may run on, lscpu model name)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = nproc
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return nproc, avail, model


def cpu_baseline(w, threads: int, runs: int = 5):
    """Median wall time of the CPU oracle over the same step (KV write + all
    (token, head) items) on `threads` host threads, 1 warm-up then `runs`."""
    import numpy as np
    from oracle import oracle
    sp = w.spec
    kp = w.k_pool.data.cpu().numpy()
    vp = w.v_pool.data.cpu().numpy()
    q = w.q.cpu().numpy()
    kn, vn = w.k_new.cpu().numpy(), w.v_new.cpu().numpy()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        oracle.set_rows(kp, kn, w.slots, sp.kv_type)
        oracle.set_rows(vp, vn, w.slots, sp.kv_type)
        oracle.paged_attention(q, kp, vp, sp.kv_type, sp.kv_type, w.block_tables, sp.seq_lens, w.seq_idx, w.pos,
                               sp.Hkv, sp.D, sp.block_size, sp.scale, softcap=sp.softcap, n_swa=sp.n_swa,
                               n_threads=threads)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
    return float(np.median(times))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--rotate-below-mb", type=int, default=512,
                    help="cycle through disjoint copies of the KV blocks when a step reads less than this")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the timed steps, run one plain device copy of this many MiB (HBM counter scale)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU's share: this build runs on a single MI355X "
              "(multi-GPU sharding is designed, not built); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import iian_amd as pa
    from iian_amd import synth

    torch.cuda.init()
    sp = synth.spec(args.config)
    log(f"building workload {args.config}: S={len(sp.seq_lens)} T={int(sp.n_q.sum())} H={sp.H} Hkv={sp.Hkv} "
        f"D={sp.D} sum(L)={int(sp.seq_lens.sum())}")
    # A workload whose KV fits in the 256 MB MALL would be timed from cache:
    # such workloads cycle through disjoint copies of their blocks (each step
    # reads a copy no step touched for at least ~1 GB of traffic).
    w = synth.build(sp, device="cuda")
    kv_bytes = synth.algorithmic_bytes(w, include_kv_write=False)
    replicas = 1
    if kv_bytes < args.rotate_below_mb << 20:
        replicas = min(512, -(-(1 << 30) // max(kv_bytes, 1)))
        del w
        torch.cuda.empty_cache()
        w = synth.build(sp, device="cuda", replicas=replicas)
        log(f"{kv_bytes / 1e6:.1f} MB per step: cycling through {replicas} disjoint copies of the blocks")
    batches = w.extra.get("replica_batches", [w.batch])
    b_step = synth.algorithmic_bytes(w, include_kv_write=True)
    b_attn = synth.algorithmic_bytes(w, include_kv_write=False)
    flops = synth.attention_flops(w)
    mfma_bound = int(sp.n_q.max()) * (sp.H // sp.Hkv) > 32
    ws = pa.new_workspace(w.T, len(sp.seq_lens), sp.H, sp.Hkv, sp.D, w.block_tables.shape[1], sp.block_size)
    out = torch.empty((w.T, sp.H, sp.D), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    cur = [0]   # the replica the next step uses

    # The step's two library calls, each checked once and bound to its
    # buffers (one ctypes call per issue, as a C++ engine holding its
    # arguments calls the C ABI), for every copy of the batch cycled through.
    k_rows, v_rows = w.k_new.contiguous(), w.v_new.contiguous()   # held for the bound calls' lifetime
    kv_calls = [pa.bind_set_rows_kv(w.k_pool, w.v_pool, k_rows, v_rows, b.slots) for b in batches]
    attn_calls = [pa.bind_paged_attn(w.q, w.k_pool, w.v_pool, sp.Hkv, w.params, b, out=out, workspace=ws)
                  for b in batches]

    def kv_write():
        kv_calls[cur[0]]()

    def attention():
        attn_calls[cur[0]]()

    def two_calls():
        kv_write()
        attention()
        cur[0] = (cur[0] + 1) % len(batches)

    # f16 decode steps: the KV write and the attention in one launch
    # (iian_pa_write_attention), where the library takes the call
    fused_calls = [pa.bind_write_paged_attn(w.q, k_rows, v_rows, w.k_pool, w.v_pool, sp.Hkv, w.params, b, out=out,
                                            workspace=ws) for b in batches]
    try:
        fused_calls[0]()
        torch.cuda.synchronize()
    except pa.PagedAttnError:
        fused_calls = None

    def fused():
        fused_calls[cur[0]]()
        cur[0] = (cur[0] + 1) % len(batches)

    step = fused if fused_calls else two_calls
    step_calls = ("iian_pa_write_attention (KV write and attention, one launch)" if fused_calls
                  else "iian_pa_kv_write_kv + iian_pa_attention")

    # untimed warm-up: the W steps asked for, continued until 0.5 s have passed
    # so the GPU clocks have left their idle state before the timed region
    n_warm = 0
    t_warm = time.perf_counter()
    while n_warm < args.warmup or time.perf_counter() - t_warm < 0.5:
        step()
        n_warm += 1
        if n_warm % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"warmup done ({n_warm} steps)")

    # timed region: exactly K steps, synchronised on both sides
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    log(f"timed {args.steps} steps ({step_calls}): {ms_step * 1e3:.1f} us/step")
    two_call_ms = None
    if fused_calls:   # the same K steps as the two calls they replace
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            two_calls()
        torch.cuda.synchronize()
        two_call_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        log(f"the same steps as two calls (kv write, attention): {two_call_ms * 1e3:.1f} us/step")

    # dominant launch: the attention call alone, HIP events on its stream.
    # First a pair around each call of K steps (the KV write between calls),
    # then one pair around K back-to-back calls.  The second is the launch's
    # average duration: an event record between kernels costs about 2.7 us of
    # its own at most configurations, and the back-to-back average agrees with
    # the kernel trace's (rocprofv3) where the per-call pairs exceed it.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in ev:
        kv_write()
        a.record(stream)
        attention()
        b.record(stream)
        cur[0] = (cur[0] + 1) % len(batches)
    torch.cuda.synchronize()
    attn_ev_ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        attention()
        cur[0] = (cur[0] + 1) % len(batches)
    e1.record(stream)
    torch.cuda.synchronize()
    attn_ms = e0.elapsed_time(e1) / args.steps
    attn_gbs = b_attn / (attn_ms * 1e-3) / 1e9
    attn_tfs = flops / (attn_ms * 1e-3) / 1e12
    log(f"attention: {attn_ms * 1e3:.1f} us/launch back to back ({attn_ev_ms * 1e3:.1f} us between per-call "
        f"events), {attn_gbs:.0f} GB/s algorithmic, {attn_tfs:.1f} TFLOP/s")

    # per-step work beside the layer-call, each timed alone with HIP events:
    # the device-side batch build (once per step, iian_pa_build_batch) and the
    # fused RoPE + KV write (once per layer, iian_pa_rope_kv_write)
    ids, nc, nn = synth.request_blocks(synth.spec(args.config))
    req = pa.RequestBlocks.pack(ids, nc, nn)
    nb_dev = pa.build_batch(req, w.T, sp.block_size, w.block_tables.shape[1], sp.num_blocks,
                            max_query_len=int(sp.n_q.max()))
    rope = pa.RopeParams(n_dims=sp.D, mode=0, freq_base=500000.0)
    q_rot = torch.empty_like(w.q)

    def timed(fn, reps=max(20, args.steps // 4)):   # back to back, one pair of events (us per call)
        fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(reps):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps * 1e3

    # bound calls (one ctypes call per issue), as kv_write and attention above
    build_us = timed(pa.bind_build_batch(req, w.T, sp.block_size, w.block_tables.shape[1], sp.num_blocks, nb_dev))
    rope_call = pa.bind_rope_set_rows_kv(w.k_pool, w.v_pool, k_rows, v_rows, w.batch.slots, w.batch.pos, rope,
                                         sp.Hkv, q=w.q, q_out=q_rot)
    rope_us = timed(rope_call)
    kvw_us = timed(kv_write)
    # the unfused sequence the fused launch replaces: RoPE of q and K into f32
    # rows (the same kernel with an f32 "pool" of T rows at slots 0..T-1; it
    # also copies V there, 4*T*Hkv*Dv bytes the reference's rope would not
    # move), then the layer's two set_rows (iian_pa_kv_write_kv)
    k_tmp = pa.KVPool(w.T, sp.Hkv * sp.D, pa.GGML_TYPE_F32)
    v_tmp = pa.KVPool(w.T, sp.Hkv * sp.D, pa.GGML_TYPE_F32)
    ident = torch.arange(w.T, dtype=torch.int64, device="cuda")
    rope_only = pa.bind_rope_set_rows_kv(k_tmp, v_tmp, k_rows, v_rows, ident, w.batch.pos, rope, sp.Hkv, q=w.q,
                                         q_out=q_rot)
    k_rot = k_tmp.data.view(torch.float32).view(w.T, sp.Hkv * sp.D)
    kv_after = pa.bind_set_rows_kv(w.k_pool, w.v_pool, k_rot, v_rows, w.batch.slots)

    def unfused():
        rope_only()
        kv_after()
    unfused_us = timed(unfused)
    log(f"beside the call: build_batch {build_us:.1f} us, rope+kv write {rope_us:.1f} us (unfused rope then kv "
        f"write {unfused_us:.1f} us), kv write {kvw_us:.1f} us")

    if args.copy_calibration:
        # a copy kernel that reads and writes exactly n bytes: its FETCH_SIZE /
        # WRITE_SIZE under rocprofv3 --pmc scale the counters of the kernels above
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {n} bytes read, {n} bytes written")

    value = b_step / (ms_step * 1e-3) / 1e9
    kernels = launch_kernels(sp, pa, int(w.batch.block_tables.shape[1]), w.batch.block_size,
                             torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": n_warm,
        "warmup_requested": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the arithmetic type: f16 MFMA operands (fp32 sums), or fp32 throughout on the general kernel
        "dtype": "f32" if "general" in kernels else "f16",
        "data": "synthetic",
        "step_calls": step_calls,
        "two_call_ms_per_step": round(two_call_ms, 5) if two_call_ms else None,
        "config": {
            "workload": f"{args.config}: " + WORKLOADS.get(args.config, args.config),
            "n_seqs": len(sp.seq_lens), "n_tokens": w.T, "sum_ctx": int(sp.seq_lens.sum()),
            "algorithmic_bytes_per_step": b_step,
            "kv_copies_cycled": replicas,
        },
        "beside_the_call_us": {"build_batch": round(build_us, 2), "rope_kv_write": round(rope_us, 2),
                               "rope_then_kv_write_unfused": round(unfused_us, 2), "kv_write": round(kvw_us, 2)},
        "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        "attn_tok_per_s": round(w.T / (attn_ms * 1e-3), 1),
        "roofline": {
            "bound": "mfma" if mfma_bound else "hbm",
            "kernel": "iian_pa_attention (" + kernels + ")",
            "achieved": round(attn_tfs if mfma_bound else attn_gbs, 1),
            "peak": MFMA_F16_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBS,
            "unit": "TFLOP/s" if mfma_bound else "GB/s",
            "frac": round(attn_tfs / MFMA_F16_PEAK_TFLOPS if mfma_bound else attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic(args.config),
            "algorithmic_bytes_per_launch": b_attn,
            "flops_per_launch": flops,
            "avg_launch_us": round(attn_ms * 1e3, 2),
            "avg_launch_us_evented": round(attn_ev_ms * 1e3, 2),
        },
    }
    if not args.no_cpu_baseline:
        nproc, avail, model = host_cpu()
        # nproc threads and the reference engine's default hardware_concurrency()/2
        # (src/iian/engine.cpp:119), each capped at the host-core share of one GPU
        t_share = max(1, min(avail, CPU_SHARE))
        t_half = max(1, min(nproc // 2, CPU_SHARE))
        log(f"timing the CPU oracle on the same step: {model}, nproc {nproc}, {avail} cores available, "
            f"{t_share} threads, {t_half} threads and 1")
        med = cpu_baseline(w, t_share)
        med_half = cpu_baseline(w, t_half) if t_half != t_share else med
        med1 = cpu_baseline(w, 1, runs=3 if med * t_share < 3.0 else 1)
        res["cpu_baseline"] = {
            "value": round(b_step / med / 1e9, 2), "unit": "GB/s", "cores": t_share, "kind": "port",
            "sample": f"the full {args.config} step (KV write + all {w.T * sp.H} (token, head) items), "
                      f"median of 5 runs after 1 warm-up, {med * 1e3:.1f} ms/step on {t_share} threads",
            "cpu_model": model, "nproc": nproc, "cores_available": avail,
            "threads_policy": f"min(nproc, hardware_concurrency()/2 = {nproc // 2}) capped at the "
                              f"{CPU_SHARE}-core host share of one GPU on this pool: {t_share} and {t_half} threads",
            "half_concurrency": {"threads": t_half, "value": round(b_step / med_half / 1e9, 2),
                                 "ms_per_step": round(med_half * 1e3, 1)},
            "single_thread": {"value": round(b_step / med1 / 1e9, 3), "ms_per_step": round(med1 * 1e3, 1)},
        }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
