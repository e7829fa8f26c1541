"""Benchmark of the paged-attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config cfg2] [--no-cpu-baseline]

A step is one layer-call of the path at Llama-3-8B decode shapes (BASELINE
config 2): the slot-mapped KV write of the 64 new tokens (K and V pools) and
paged GQA decode attention over the block pool, inputs resident in HBM.
``value`` is the achieved algorithmic HBM bandwidth of the whole step (GB/s);
``attn_tok_per_s`` the query tokens per second of one layer-call.
``roofline`` is measured live for the dominant launch (the attention call) with
HIP events on the stream it runs on; ``cpu_baseline`` times the CPU oracle
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
    "cfg3": "Qwen3-8B mixed batch, H32/Hkv8/D128: 4 prefill chunks x 512 over prior U[1024,4096] "
            "(1024-token shared prefix) + 32 decode tokens, f16 KV",
    "cfg3_prefill": "Qwen3-8B, H32/Hkv8/D128: the 4 prefill chunks of cfg3 alone (x 512 tokens over prior "
                    "U[1024,4096], 1024-token shared prefix), f16 KV",
    "cfg4": "Llama-3-8B Q8_0 KV, 128 seqs x 4096 prior + 5 spec-verify queries",
    "cfg5_global_decode": "Gemma3-12B global layer decode, H16/Hkv8/D256, 32 seqs, ctx U[8192,32768]",
    "cfg5_local_decode": "Gemma3-12B local layer decode (n_swa=1024), H16/Hkv8/D256, 32 seqs",
    "cfg5_global_prefill": "Gemma3-12B global layer, 256-token prefill chunk per seq, 32 seqs",
    "cfg5_local_prefill": "Gemma3-12B local layer (n_swa=1024), 256-token prefill chunk per seq, 32 seqs",
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


def launch_kernels(sp, pa) -> str:
    """The kernels one iian_pa_attention call of this workload launches."""
    gqa = sp.H // sp.Hkv
    rows = [int(n) * gqa for n in sp.n_q]
    has_dec = any(0 < r <= 32 for r in rows)
    has_pf = any(r > 32 for r in rows)
    d = sp.D
    if sp.kv_type == pa.GGML_TYPE_Q8_0:
        dec = f"pa_decode_q8_kernel<{d}> + pa_merge_kernel<{d}>"
        pf = f"pa_prefill_kernel<{d}, Q8_0>" if d <= 128 else f"pa_prefill16_kernel<{d}, Q8_0>"
    else:
        dec = f"pa_decode_f16_kernel<{d}> + pa_merge_kernel<{d}>"
        pf = f"pa_prefill_kernel<{d}, f16>" if d <= 128 else f"pa_prefill16_kernel<{d}, f16>"
        if has_dec and has_pf and d <= 128:
            return f"pa_prefill_kernel<{d}, f16, mixed> (decode pieces in the same grid) + pa_merge_kernel<{d}>"
    if has_dec and has_pf:
        return f"{pf} || {dec} (two streams)"
    return pf if has_pf else dec


def cpu_baseline(w, runs: int = 5):
    """Median wall time of the CPU oracle over the same step (KV write + all
    (token, head) items), using every host core."""
    import numpy as np
    from oracle import oracle
    sp = w.spec
    threads = min(os.cpu_count() or 1, 16)   # the host-core share of one GPU
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
    med = float(np.median(times))
    return med, threads


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
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
    w = synth.build(sp, device="cuda")
    b_step = synth.algorithmic_bytes(w, include_kv_write=True)
    b_attn = synth.algorithmic_bytes(w, include_kv_write=False)
    flops = synth.attention_flops(w)
    mfma_bound = int(sp.n_q.max()) * (sp.H // sp.Hkv) > 32
    ws = pa.new_workspace(w.T, len(sp.seq_lens), sp.H, sp.Hkv, sp.D, w.block_tables.shape[1], sp.block_size)
    out = torch.empty((w.T, sp.H, sp.D), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def kv_write():
        pa.set_rows_kv(w.k_pool, w.v_pool, w.k_new, w.v_new, w.batch.slots)

    def attention():
        pa.build_paged_attn(w.q, w.k_pool, w.v_pool, sp.Hkv, w.params, w.batch, out=out, workspace=ws)

    def step():
        kv_write()
        attention()

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
    log(f"timed {args.steps} steps: {ms_step * 1e3:.1f} us/step")

    # dominant launch: the attention call alone, HIP events on its stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in ev:
        kv_write()
        a.record(stream)
        attention()
        b.record(stream)
    torch.cuda.synchronize()
    attn_ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
    attn_gbs = b_attn / (attn_ms * 1e-3) / 1e9
    attn_tfs = flops / (attn_ms * 1e-3) / 1e12
    log(f"attention: {attn_ms * 1e3:.1f} us/launch, {attn_gbs:.0f} GB/s algorithmic, {attn_tfs:.1f} TFLOP/s")

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
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: " + WORKLOADS.get(args.config, args.config),
            "n_seqs": len(sp.seq_lens), "n_tokens": w.T, "sum_ctx": int(sp.seq_lens.sum()),
            "algorithmic_bytes_per_step": b_step,
        },
        "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        "attn_tok_per_s": round(w.T / (attn_ms * 1e-3), 1),
        "roofline": {
            "bound": "mfma" if mfma_bound else "hbm",
            "kernel": "iian_pa_attention (" + launch_kernels(sp, pa) + ")",
            "achieved": round(attn_tfs if mfma_bound else attn_gbs, 1),
            "peak": MFMA_F16_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBS,
            "unit": "TFLOP/s" if mfma_bound else "GB/s",
            "frac": round(attn_tfs / MFMA_F16_PEAK_TFLOPS if mfma_bound else attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic(args.config),
            "algorithmic_bytes_per_launch": b_attn,
            "flops_per_launch": flops,
            "avg_launch_us": round(attn_ms * 1e3, 2),
        },
    }
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on the same step")
        med, threads = cpu_baseline(w)
        res["cpu_baseline"] = {
            "value": round(b_step / med / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the full {args.config} step (KV write + all {w.T * sp.H} (token, head) items), "
                      f"median of 5 runs after 1 warm-up, {med * 1e3:.1f} ms/step",
        }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
