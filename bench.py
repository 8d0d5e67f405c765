"""Benchmark of the paged Q8_0 KV hot path on one MI355X.

Default workload (BASELINE.json metric, SURVEY headline row): B=64 sequences,
every one at L=32768 tokens after appending this step's token; 16 query heads
/ 2 KV heads, head_dim 256, 64-token pages in a shuffled shared pool with 10%
free-page slack; K/V ~ N(0,1) bf16 quantized to Q8_0 by the append kernel;
bf16 query ~ N(0,1); softmax scale 1/16; f32 output; seed 0.

One step = append one K/V row per sequence (position L-1, the same slot every
step, so every step is the same work) + split-K decode + LSE combine, all on
one stream: two launches, the decode launch quantizing and writing the new
rows itself before it reads them (--append-launch: a separate append launch
first).  Inputs are resident in HBM before the timed region.

Printed: ONE JSON line (rank 0) with the whole-step algorithmic HBM rate
(`value`, GB/s), us/step, the decode kernel's roofline figures measured with
HIP events around its launches inside the timed region, and the reference CPU
path (the C restatement in oracle/) timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0

METRIC = "Q8 paged flash-decode HBM GB/s (% of 8 TB/s) + µs/step at B=64, 32k ctx"


def load_rkv():
    name = "remora_lab_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "remora-lab_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--q-heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=2)
    ap.add_argument("--head-dim", type=int, default=256)
    ap.add_argument("--page-size", type=int, default=64)
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--append-launch", action="store_true",
                    help="append the step's rows with a separate rkv_pool_append launch instead "
                         "of inside the decode launch")
    ap.add_argument("--cpu-sample-seqs", type=int, default=4,
                    help="sequences of the oracle CPU baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 2 GiB device copy (rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE "
                         "calibration of known bytes)")
    return ap.parse_args()


def copy_calibration(steps: int) -> int:
    import torch
    n = 1 << 31
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "seconds": dt,
                      "GB/s_read+write": 2 * n / dt / 1e9}), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(sequences shard across GPUs with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(max(args.steps, 1))
    import torch
    rkv = load_rkv()
    torch.manual_seed(args.seed)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    B, L, Hq, Hkv, D, PT = args.batch, args.ctx, args.q_heads, args.kv_heads, args.head_dim, args.page_size
    pages_per_seq = (L + PT - 1) // PT
    num_pages = int(math.ceil(B * pages_per_seq * 1.10))
    pool = rkv.Pool(ctx, 1, Hkv, D, PT, num_pages, B, pages_per_seq, seed=args.seed)
    for s in range(B):
        pool.alloc.reserve(s, L)
    pool.sync_tables()
    g = pool.geometry

    # ---- fill the cache through the append kernel (not timed) ------------------
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    chunk = 1 << 16
    total = B * L
    for start in range(0, total, chunk):
        n = min(chunk, total - start)
        idx = torch.arange(start, start + n, device=dev, dtype=torch.int64)
        sid = (idx // L).to(torch.int32)
        pos = (idx % L).to(torch.int32)
        k = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        pool.append(0, sid, pos, k, v)
    ctx.sync()

    # ---- per-step inputs ---------------------------------------------------------
    seq_ids = torch.arange(B, device=dev, dtype=torch.int32)
    positions = torch.full((B,), L - 1, device=dev, dtype=torch.int32)
    k_new = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((B, 1, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty((B, 1, Hq, D), device=dev, dtype=torch.float32)
    scale = 1.0 / math.sqrt(D)
    a = rkv.decode_args(q, out, seq_ids, scale, L, partition_tokens=args.partition_tokens)
    part = rkv.decode_partition_tokens(g, a)
    n_parts = (L + part - 1) // part
    rows = Hq
    # split-K partials, laid out as rkv_decode_q8's workspace
    ml = torch.empty((B, rows, n_parts, 2), device=dev, dtype=torch.float32)
    o = torch.empty((B, rows, n_parts, D), device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream()
    lib = rkv.lib()
    pages_p = pool.layer_pages(0)
    bt_p = pool.block_tables_ptr()
    lens_p = pool.seq_lens_ptr()

    # this step's new K/V rows, appended by the decode launch itself (the
    # default) or by a separate rkv_pool_append launch (--append-launch)
    app = rkv.append_args(seq_ids, positions, k_new, v_new)
    a = rkv.decode_args(q, out, seq_ids, scale, L, partition_tokens=args.partition_tokens,
                        append=None if args.append_launch else app)
    fused = not args.append_launch

    def step(ev=None):
        # [append launch], then the two kernels rkv_pool_decode chains (split-K
        # decode, log-sum-exp combine), called through their kernel-level entry
        # points so events can bracket each kernel on the launch stream
        if ev is not None:
            ev[0].record(stream)
        if not fused:
            pool.append(0, seq_ids, positions, k_new, v_new, stream=stream)
            if ev is not None:
                ev[1].record(stream)
        if n_parts > 1:
            rkv.check(lib.rkv_decode_q8_partials(ctx.h, C.byref(g), C.c_void_p(pages_p),
                                                 C.c_void_p(bt_p), pages_per_seq,
                                                 C.c_void_p(lens_p), B, C.byref(a),
                                                 C.c_void_p(ml.data_ptr()), C.c_void_p(o.data_ptr()),
                                                 C.c_void_p(stream.cuda_stream)))
            if ev is not None:
                ev[2].record(stream)
            rkv.check(lib.rkv_splitk_combine(ctx.h, C.c_void_p(ml.data_ptr()),
                                             C.c_void_p(o.data_ptr()), B, rows, n_parts, D,
                                             C.c_void_p(seq_ids.data_ptr()), C.c_void_p(lens_p), B,
                                             part, C.c_void_p(out.data_ptr()), rkv.F32,
                                             C.c_void_p(stream.cuda_stream)))
        else:
            pool.decode(0, a, stream=stream)
            if ev is not None:
                ev[2].record(stream)
        if ev is not None:
            ev[3].record(stream)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctx.sync()
    dec_from = 0 if fused else 1  # the decode launch starts after the append launch
    t_step = [evs[i][0].elapsed_time(evs[i][3]) * 1e-3 for i in range(args.steps)]
    t_app = [0.0 if fused else evs[i][0].elapsed_time(evs[i][1]) * 1e-3 for i in range(args.steps)]
    t_dec = [evs[i][dec_from].elapsed_time(evs[i][2]) * 1e-3 for i in range(args.steps)]
    t_cmb = [evs[i][2].elapsed_time(evs[i][3]) * 1e-3 for i in range(args.steps)]
    step_s = wall / args.steps  # whole-job rate over the timed region
    dec_s = sum(t_dec) / len(t_dec)

    # ---- algorithmic bytes -----------------------------------------------------------
    row = D // 32 * 34
    kv_bytes = B * L * Hkv * 2 * row
    q_bytes = B * Hq * D * 2
    out_bytes = B * Hq * D * 4
    bt_bytes = B * pages_per_seq * 4
    app_bytes = B * Hkv * 2 * (D * 2 + row)
    step_bytes = kv_bytes + q_bytes + out_bytes + bt_bytes + app_bytes
    # split-K partials are implementation overhead, reported beside the
    # algorithmic figure and not in it
    partial_bytes = B * rows * n_parts * (D + 2) * 4
    # the decode kernel's share of the step: K/V, q, block tables, out, and
    # the appended rows when it appends them itself
    dec_bytes = kv_bytes + q_bytes + bt_bytes + out_bytes + (app_bytes if fused else 0)
    flops = 4 * D * Hq * B * L

    value = step_bytes / step_s / 1e9
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 QK + f16 PV, f32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0 via the append kernel; bf16 q)",
        "config": {"workload": f"headline paged Q8 decode step: B={B}, L={L}, Hq={Hq}, Hkv={Hkv}, "
                               f"D={D}, page={PT}, 10% pool slack, bf16 q, f32 out, scale 1/{int(math.sqrt(D))}",
                   "batch": B, "ctx": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
                   "page_tokens": PT, "partition_tokens": part, "partitions": n_parts,
                   "pool_pages": num_pages,
                   "append": "separate launch" if args.append_launch else "inside the decode launch"},
        "us_per_step": round(step_s * 1e6, 2),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "algorithmic_bytes_per_step": step_bytes,
        "kernel_us": {"append": round(1e6 * sum(t_app) / len(t_app), 2),
                      "decode": round(1e6 * dec_s, 2),
                      "combine": round(1e6 * sum(t_cmb) / len(t_cmb), 2),
                      "event_step": round(1e6 * sum(t_step) / len(t_step), 2)},
        "split_k_partial_bytes": partial_bytes,
        "achieved_tflops": round(flops / step_s / 1e12, 2),
        "roofline": {"bound": "hbm", "kernel": "decode_kernel<256,1,false,2>",
                     "achieved": round(dec_bytes / dec_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_bytes / dec_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(), "algorithmic_bytes_per_launch": dec_bytes},
    }

    # ---- CPU baseline: the reference path restated in C, timed on a sample -------
    if args.cpu_sample_seqs > 0:
        res["cpu_baseline"] = cpu_baseline(rkv, ctx, pool, g, q, out, k_new, v_new, B, L, Hq, Hkv,
                                           D, scale, step_bytes, args.cpu_sample_seqs)
    print(json.dumps(res), flush=True)
    pool.close()
    ctx.close()
    return 0


def read_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), if any."""
    path = os.path.join(ROOT, "profiles", "decode_headline_pmc.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def cpu_baseline(rkv, ctx, pool, g, q, out, k_new, v_new, B, L, Hq, Hkv, D, scale, step_bytes,
                 n_sample):
    """Time the reference CPU path (oracle/rkv_oracle.c: q8 quantize for the
    append rows, flash_decode_reference over each sampled sequence) and scale
    the sample to a whole step.  Also checks those sequences' GPU outputs."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import rko
    rko.lib()
    n_sample = min(n_sample, B)
    rb = D // 32 * 34
    # host copies of the sampled sequences' rows (reference contiguous layout)
    rows = []
    for s in range(n_sample):
        kk = torch.empty(Hkv * L * rb, dtype=torch.uint8, device="cuda")
        vv = torch.empty_like(kk)
        pool.gather(0, s, rkv.K, kk)
        pool.gather(0, s, rkv.V, vv)
        ctx.sync()
        rows.append((rko.rows_to_words(kk.cpu().numpy()), rko.rows_to_words(vv.cpu().numpy())))
    qf = q.float().cpu().numpy()
    gpu_out = out.cpu().numpy()
    kn = k_new.float().cpu().numpy()
    vn = v_new.float().cpu().numpy()
    t0 = time.perf_counter()
    for b in range(B):  # append: quantize every new row (all B rows)
        for h in range(Hkv):
            rko.q8_encode(kn[b, h])
            rko.q8_encode(vn[b, h])
    t_app = time.perf_counter() - t0
    p = rko.fd_params(Hq, Hkv, L, 1024, D)
    max_err = 0.0
    t0 = time.perf_counter()
    for s in range(n_sample):
        qs = (qf[s, 0] * np.float32(scale)).astype(np.float32).reshape(-1)
        ref = rko.flash_decode_reference(p, rows[s][0], rows[s][1], qs)
        max_err = max(max_err, float(np.max(np.abs(ref - gpu_out[s, 0].reshape(-1)))))
    t_dec = time.perf_counter() - t0
    full = t_app + t_dec * B / n_sample
    return {"value": round(step_bytes / full / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"append quantize of all {B} rows + flash_decode_reference (attention.rs:148-215, "
                      f"chunk 1024) over {n_sample} of {B} sequences at L={L}, scaled x{B / n_sample:g}; "
                      f"{t_app + t_dec:.1f} s of CPU work",
            "us_per_step": round(full * 1e6, 1),
            "gpu_vs_cpu_max_abs_err_on_sample": max_err}


if __name__ == "__main__":
    sys.exit(main())
