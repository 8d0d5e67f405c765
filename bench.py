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
# The arithmetic a line's kernels compute in.  With a bf16 query, waves of up
# to 8 rows per kv head take the int8 QK against three int8 query planes;
# 16-row waves (the verify, the prefill) take the f16 QK.
DT_INT8_QK = "int8 QK (bf16 query as three int8 planes) + f16 PV (two-term weights), f32 accumulate"
DT_F16_QK = ("f16 QK (bf16 query exact in f16, K codes widened exactly) + f16 PV (two-term weights), "
             "f32 accumulate")


def load_rkv():
    name = "remora_lab_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "remora-lab_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


class GpuState:
    """The GPU's power cap and clock limits through amdsmi, so that a line
    from a power-capped or lower-clocked box can be told apart from a slower
    build; start() and stop() also sample the graphics and memory clocks and
    the socket power every `period` seconds on a side thread (amdsmi updates
    them on a scale of many ms, so they describe long regions only).  Any
    amdsmi failure is reported in the result, never raised."""

    def __init__(self, period=0.005):
        import threading
        self.period, self.samples, self.static, self.error = period, [], {}, None
        self._stop = threading.Event()
        self._thread = None
        self.h = None
        try:
            import amdsmi
            self.smi = amdsmi
            amdsmi.amdsmi_init()
            hs = amdsmi.amdsmi_get_processor_handles()
            self.h = hs[0] if len(hs) == 1 else self._match(hs)
            gfx = amdsmi.amdsmi_get_clock_info(self.h, amdsmi.AmdSmiClkType.GFX)
            mem = amdsmi.amdsmi_get_clock_info(self.h, amdsmi.AmdSmiClkType.MEM)
            cap = amdsmi.amdsmi_get_power_cap_info(self.h)
            self.static = {"gfx_clk_max_mhz": gfx.get("max_clk"), "mem_clk_max_mhz": mem.get("max_clk"),
                           "power_cap_w": self._watts(cap.get("power_cap")),
                           "default_power_cap_w": self._watts(cap.get("default_power_cap"))}
        except Exception as e:  # no amdsmi, no permission, no device
            self.error = f"{type(e).__name__}: {e}"

    def _match(self, hs):
        import torch
        bus = torch.cuda.get_device_properties(0).pci_bus_id
        for h in hs:
            if int(self.smi.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == bus:
                return h
        return hs[0]

    @staticmethod
    def _watts(v):
        if not isinstance(v, (int, float)):
            return None
        return round(v / 1e6, 1) if v > 1e5 else v  # amdsmi reports caps in microwatts

    def _one(self):
        smi = self.smi
        try:
            g = smi.amdsmi_get_clock_info(self.h, smi.AmdSmiClkType.GFX).get("clk")
            m = smi.amdsmi_get_clock_info(self.h, smi.AmdSmiClkType.MEM).get("clk")
            w = smi.amdsmi_get_power_info(self.h).get("current_socket_power")
            self.samples.append((g, m, w))
            return True
        except Exception as e:
            self.error = f"{type(e).__name__}: {e}"
            return False

    def _sample(self):
        while not self._stop.wait(self.period) and self._one():
            pass

    def start(self):
        """Sample every period on a side thread until stop().  No sample at
        the start or the stop: with the stream drained around a region the
        clocks read there are idle clocks."""
        import threading
        if self.h is not None and self.error is None:
            self._thread = threading.Thread(target=self._sample, daemon=True)
            self._thread.start()
        return self

    def stop(self) -> dict:
        import numpy as np
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
        res = dict(self.static)
        if self.samples:
            for i, k in enumerate(("gfx_clk_mhz", "mem_clk_mhz", "socket_power_w")):
                xs = [x[i] for x in self.samples if isinstance(x[i], (int, float))]
                if xs:
                    res[k + "_p10_p50_p90"] = [float(v) for v in np.percentile(xs, [10, 50, 90])]
            res["samples"] = len(self.samples)
        if self.error:
            res["error"] = self.error
        return res


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--event-every", type=int, default=5,
                    help="record the per-kernel HIP events on every N-th timed step")
    ap.add_argument("--event-steps", type=int, default=24,
                    help="steps of the event pass after the timed region, each with its per-kernel "
                         "events, that the percentiles are taken from (at least 20)")
    ap.add_argument("--no-secondary", dest="secondary", action="store_false",
                    help="headline only: skip configs 2, 3 and 5 in the default line")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sustained-ms", type=float, default=150.0,
                    help="headline: length of the sustained pass (the step back to back) after "
                         "the timed region")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--q-heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=2)
    ap.add_argument("--head-dim", type=int, default=256)
    ap.add_argument("--page-size", type=int, default=64)
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--config", type=int, default=1,
                    help="1 = the headline line (default); 2-5 = BASELINE.json's secondary configs; "
                         "6 = prefix-shared decode (forks + copy-on-write pages); "
                         "7 = chunked prefill attention; 8 = R4KV page spill/restore; "
                         "9 = serving step through the adapter; 10 = host-KV tier (pages in "
                         "pinned host memory)")
    ap.add_argument("--layers", type=int, default=48, help="layer pools of config 4")
    ap.add_argument("--serve-layers", type=int, default=4, help="layers of config 9")
    ap.add_argument("--prefill-batch", type=int, default=8, help="sequences of config 7")
    ap.add_argument("--prefill-ctx", type=int, default=8192, help="cached tokens of config 7")
    ap.add_argument("--prefill-rows", type=int, default=512, help="chunk rows of config 7")
    ap.add_argument("--prefill-segment", type=int, default=0,
                    help="config 7 segment_tokens: 0 = automatic split (with a workspace), "
                         "> 0 = that segment length, -1 = never split")
    ap.add_argument("--append-launch", action="store_true",
                    help="append the step's rows with a separate rkv_pool_append launch instead "
                         "of inside the decode launch")
    ap.add_argument("--cpu-sample-seqs", type=int, default=4,
                    help="sequences of the oracle CPU baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-stream-ceiling", dest="stream_ceiling", action="store_false",
                    help="skip the streaming-read ceiling measured after the headline")
    ap.add_argument("--graph", action="store_true",
                    help="configs 2 and 3: report graph replays as the step time (default: eager)")
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
    stream = torch.cuda.current_stream()
    # this step's new K/V rows, appended by the decode launch itself (the
    # default) or by a separate rkv_pool_append launch (--append-launch)
    app = rkv.append_args(seq_ids, positions, k_new, v_new)
    a = rkv.decode_args(q, out, seq_ids, scale, L, partition_tokens=args.partition_tokens,
                        append=None if args.append_launch else app)
    ws = torch.empty(max(rkv.decode_workspace_bytes(g, a), 4), device=dev, dtype=torch.uint8)
    a = rkv.decode_args(q, out, seq_ids, scale, L, partition_tokens=args.partition_tokens,
                        workspace=ws, append=None if args.append_launch else app)
    fused = not args.append_launch
    rows = Hq

    def step(ev=None):
        # [append launch], then rkv_pool_decode: the split-K decode kernel and
        # the combine kernel; the library records ev[2] between the two
        if ev is not None:
            ev[0].record(stream)
        if not fused:
            pool.append(0, seq_ids, positions, k_new, v_new, stream=stream)
            if ev is not None:
                ev[1].record(stream)
        a.split_event = C.c_void_p(ev[2].cuda_event) if ev is not None else None
        pool.decode(0, a, stream=stream)
        if ev is not None:
            ev[3].record(stream)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    # kernel durations: HIP events on every `event_every`-th timed step (event
    # markers cost the stream a few us each, so not on every step)
    sampled = list(range(0, args.steps, max(args.event_every, 1)))
    evs = {i: [torch.cuda.Event(enable_timing=True) for _ in range(4)] for i in sampled}
    for e in evs.values():  # create the events (torch creates them at their first record)
        for x in e:
            x.record(stream)
    torch.cuda.synchronize()
    gpu = GpuState()
    gpu_state = gpu.stop()  # clock limits and power cap (no sampler in the timed region)
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs.get(i))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctx.sync()
    # the event pass: every step with its events (markers cost the stream a
    # few us per step, so it runs after the timed region), for percentiles
    # over at least 20 samples
    n_pass = max(args.event_steps, 20)
    pass_evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_pass)]
    for e in pass_evs:
        for x in e:
            x.record(stream)
    torch.cuda.synchronize()
    for e in pass_evs:
        step(e)
    torch.cuda.synchronize()
    ctx.sync()
    # the sustained pass: the same step back to back for about
    # --sustained-ms.  The graphics clock falls within a few ms of sustained
    # load and partly recovers later (power management; amdsmi's clock
    # readings are too coarse in time to follow it), and while it is below
    # about 1.5 GHz the decode's per-tile instruction stream, not HBM, sets
    # its pace.  A short timed region can fall in that dip; this records the
    # steady rate beside it.
    n_sus = max(20, int(args.sustained_ms * 1e-3 / max(wall / args.steps, 1e-6)))
    t0 = time.perf_counter()
    for _ in range(n_sus):
        step()
    torch.cuda.synchronize()
    sus_s = (time.perf_counter() - t0) / n_sus
    ctx.sync()
    part = int(ws[:4].view(torch.int32).item())  # the partition length the device chose
    n_parts = (L + part - 1) // part
    dec_from = 0 if fused else 1  # the decode launch starts after the append launch
    t_step = [evs[i][0].elapsed_time(evs[i][3]) * 1e-3 for i in sampled]
    t_app = [0.0 if fused else evs[i][0].elapsed_time(evs[i][1]) * 1e-3 for i in sampled]
    t_dec = [evs[i][dec_from].elapsed_time(evs[i][2]) * 1e-3 for i in sampled]
    t_cmb = [evs[i][2].elapsed_time(evs[i][3]) * 1e-3 for i in sampled]
    p_step = [e[0].elapsed_time(e[3]) * 1e-3 for e in pass_evs]
    p_dec = [e[dec_from].elapsed_time(e[2]) * 1e-3 for e in pass_evs]
    p_cmb = [e[2].elapsed_time(e[3]) * 1e-3 for e in pass_evs]
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
        "dtype": DT_INT8_QK,
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
                      "event_step": round(1e6 * sum(t_step) / len(t_step), 2),
                      "sampled_steps": len(sampled), "sampled_every": args.event_every,
                      # percentiles: the event pass after the timed region
                      "decode_p10_p50_p90": _pcts(p_dec),
                      "combine_p10_p50_p90": _pcts(p_cmb),
                      "event_step_p10_p50_p90": _pcts(p_step),
                      "percentile_samples": n_pass},
        "gpu_state": gpu_state,
        "sustained": {"steps": n_sus, "us_per_step": round(sus_s * 1e6, 2),
                      "gbs": round(step_bytes / sus_s / 1e9, 2)},
        "split_k_partial_bytes": partial_bytes,
        "achieved_tflops": round(flops / step_s / 1e12, 2),
        "roofline": {"bound": "hbm", "kernel": "rkv::decode_kernel<256, 1, false, 2, 1, false>",
                     "achieved": round(dec_bytes / dec_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_bytes / dec_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(), "algorithmic_bytes_per_launch": dec_bytes,
                     "traffic_source": "profiles/decode_headline_pmc.txt: rocprofv3 --pmc FETCH_SIZE "
                                       "and WRITE_SIZE of this kernel, scaled by a copy kernel's "
                                       "counts (a separate profiled run, not this one)"},
    }

    # ---- practical ceiling: a plain streaming read of HBM in the same run ---------
    if args.stream_ceiling:
        ceil = stream_ceiling(rkv, ctx, stream)
        res["stream_read_ceiling"] = ceil
        best = max(ceil["vector_gbs"], ceil["lds_dma_gbs"])
        res["roofline"]["frac_of_stream_ceiling"] = round(res["roofline"]["achieved"] / best, 4)
        # the decode's own tile order over this pool's (shuffled) pages, with
        # nothing computed: the read rate that access pattern reaches here
        if L % 32:
            res["pattern_read_ceiling"] = {"skipped": f"ctx {L} is not a whole number of "
                                                      "32-token tiles"}
        else:
            pat = pattern_ceiling(rkv, ctx, pool, g, B, L, part, pages_per_seq, kv_bytes, stream)
            res["pattern_read_ceiling"] = pat
            # K/V bytes over the decode kernel's time against the same bytes over the pattern's
            res["roofline"]["frac_of_pattern_ceiling"] = round(pat["us"] * 1e-6 / dec_s, 4)

    # ---- CPU baseline: the reference path restated in C, timed on a sample -------
    if args.cpu_sample_seqs > 0:
        res["cpu_baseline"] = cpu_baseline(rkv, ctx, pool, g, q, out, k_new, v_new, B, L, Hq, Hkv,
                                           D, scale, step_bytes, args.cpu_sample_seqs)
    pool.close()

    # ---- configs 2, 3 and 5 in the same run (driver-timed secondary lines) -------
    if args.secondary:
        res["secondary"] = secondary(args)
    print(json.dumps(res), flush=True)
    ctx.close()
    return 0


def secondary(args) -> dict:
    """Configs 2, 3 (device-chosen partitions, and the reference's 128) and 5
    at the headline's --steps/--warmup, each a compact record of its own
    line (run_config): us per step, whole-step GB/s and fraction of 8 TB/s,
    the decode kernel's events and roofline fraction."""
    import copy
    out = {}
    for name, cfg, part in (("config2", 2, 0), ("config3", 3, 0), ("config3_128_partitions", 3, 2048),
                            ("config5", 5, 0)):
        a = copy.copy(args)
        a.config, a.partition_tokens, a.graph = cfg, part, False
        r = run_config(a, emit=False)
        rf = r.get("roofline", {})
        out[name] = {"us_per_step": r["us_per_step"], "gbs": r["value"],
                     "frac_of_hbm_peak": round(r["value"] / HBM_PEAK_GBS, 4),
                     "decode_us": rf.get("decode_us"), "decode_frac": rf.get("frac"),
                     "decode_p10_p50_p90": r.get("decode_p10_p50_p90"),
                     "partition_tokens": r["config"]["partition_tokens"],
                     "partitions": r["config"]["partitions_total"],
                     "algorithmic_bytes_per_step": r["algorithmic_bytes_per_step"]}
        if "graph_us_per_step" in r:
            out[name]["graph_us_per_step"] = r["graph_us_per_step"]
        print(f"[bench] secondary {name}: {r['us_per_step']} us/step", file=sys.stderr, flush=True)
    return out


def _pcts(xs):
    """p10, median and p90 of a list of seconds, in microseconds."""
    import numpy as np
    return [round(1e6 * float(v), 2) for v in np.percentile(np.asarray(xs), [10, 50, 90])]


def stream_ceiling(rkv, ctx, stream, nbytes=4 << 30, reps=5):
    """Read rate of a plain stream over `nbytes` of HBM (rkv_stream_read):
    16-byte vector loads over several grid sizes, and 1 KiB LDS-DMA copies
    (the decode's stage copy, 16 KiB in flight per one-wave workgroup).  The
    best grid's median over `reps` launches, in GB/s."""
    import torch
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    word = torch.zeros(1, dtype=torch.int32, device="cuda")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]

    def rate(mode, blocks):
        rkv.stream_read(ctx, buf, mode, blocks, word, stream=stream)  # warm
        for r in range(reps):
            ev[2 * r].record(stream)
            rkv.stream_read(ctx, buf, mode, blocks, word, stream=stream)
            ev[2 * r + 1].record(stream)
        torch.cuda.synchronize()
        ts = sorted(ev[2 * r].elapsed_time(ev[2 * r + 1]) * 1e-3 for r in range(reps))
        return nbytes / ts[reps // 2] / 1e9

    vec = {b: rate(0, b) for b in (256, 512, 1024, 2048)}
    dma = {b: rate(1, b) for b in (1024, 2048, 4096)}
    bv = max(vec, key=vec.get)
    bd = max(dma, key=dma.get)
    del buf
    return {"bytes": nbytes, "vector_gbs": round(vec[bv], 1), "vector_blocks": bv,
            "lds_dma_gbs": round(dma[bd], 1), "lds_dma_blocks": bd,
            "kernel": "rkv_stream_read (rkv_stream.hip)"}


def pattern_ceiling(rkv, ctx, pool, g, B, L, part, bt_stride, kv_bytes, stream, reps=5):
    """Read rate of the decode's tile order over the pool's own pages
    (rkv_stream_read_tiles): the same partitions, 32-token tiles and
    nontemporal LDS-DMA copies, one tile in flight, no compute; median of
    `reps` launches after one warm-up."""
    import torch
    run = lambda: rkv.stream_read_tiles(ctx, g, pool.layer_pages(0), pool.block_tables_ptr(), bt_stride,
                                        B, L, part, stream=stream)
    run()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3)
    ctx.sync()
    t = sorted(ts)[len(ts) // 2]
    return {"gbs": round(kv_bytes / t / 1e9, 1), "us": round(t * 1e6, 2), "bytes": kv_bytes,
            "kernel": "rkv_stream_read_tiles (rkv_stream.hip): the decode's partitions and 32-token "
                      "tiles over this pool's pages, nt LDS-DMA copies, one tile in flight, nothing computed"}


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
                 n_sample, n_sample_all=16):
    """Time the reference CPU path (oracle/rkv_oracle.c: q8 quantize for the
    append rows, flash_decode_reference over sampled sequences) and scale the
    sample to a whole step: on one core (the reference is single-threaded) and
    on all host cores (OpenMP over sequence x q head).  Also checks those
    sequences' GPU outputs."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import rko
    rko.lib()
    n_sample = min(n_sample, B)
    n_all = min(max(n_sample_all, n_sample), B)
    rb = D // 32 * 34
    # host copies of the sampled sequences' rows (reference contiguous layout)
    rows = []
    for s in range(n_all):
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
    qs = (qf[:n_all, 0] * np.float32(scale)).astype(np.float32)
    max_err = 0.0
    t0 = time.perf_counter()
    refs = []
    for s in range(n_sample):
        ref = rko.flash_decode_reference(p, rows[s][0], rows[s][1], qs[s].reshape(-1))
        refs.append(ref)
    t_dec = time.perf_counter() - t0
    for s, ref in enumerate(refs):
        max_err = max(max_err, float(np.max(np.abs(ref - gpu_out[s, 0].reshape(-1)))))
    full = t_app + t_dec * B / n_sample
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    t0 = time.perf_counter()
    many = rko.flash_decode_reference_many(p, [r[0] for r in rows], [r[1] for r in rows], qs, threads)
    t_many = time.perf_counter() - t0
    max_err = max(max_err, float(np.max(np.abs(many - gpu_out[:n_all, 0]))))
    rel_err = float(np.linalg.norm(many - gpu_out[:n_all, 0]) / np.linalg.norm(many))
    full_all = t_app + t_many * B / n_all
    return {"value": round(step_bytes / full / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"append quantize of all {B} rows + flash_decode_reference (attention.rs:148-215, "
                      f"chunk 1024) over {n_sample} of {B} sequences at L={L}, scaled x{B / n_sample:g}; "
                      f"{t_app + t_dec:.1f} s of CPU work",
            "us_per_step": round(full * 1e6, 1),
            "all_cores": {"value": round(step_bytes / full_all / 1e9, 4), "unit": "GB/s",
                          "cores": threads, "us_per_step": round(full_all * 1e6, 1),
                          "sample": f"the same loop over {n_all} of {B} sequences on {threads} OpenMP "
                                    f"threads (sequence x q head), scaled x{B / n_all:g}; "
                                    f"{t_many:.1f} s wall"},
            "gpu_vs_cpu_max_abs_err_on_sample": max_err,
            "gpu_vs_cpu_rel_err_on_sample": rel_err}


def _cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name"), with its
    family and model numbers and the logical CPU count: a virtual machine may
    report only the vendor's brand in the name (the GPU boxes say "AMD EPYC";
    family 26 is Zen 5, 25 is Zen 3/4)."""
    name, fam, mod = "unknown", None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and name == "unknown":
                    name = val
                elif key == "cpu family" and fam is None:
                    fam = val
                elif key == "model" and mod is None:
                    mod = val
                if name != "unknown" and fam is not None and mod is not None:
                    break
    except OSError:
        pass
    extra = [f"family {fam} model {mod}"] if fam is not None and mod is not None else []
    extra.append(f"{os.cpu_count()} logical CPUs")
    return f"{name} ({', '.join(extra)})"


# ---------------------------------------------------------------------------
# Secondary workloads: `--config N` prints one
# JSON line of the same shape for that workload.  The default run above is
# the headline line the metric is quoted on.
# ---------------------------------------------------------------------------

def _fill_layer(rkv, pool, layer, seqs, lens, Hkv, D, seed, outlier_frac=0.0, chunk=1 << 16):
    """Append rows [0, lens[i]) of sequence seqs[i] to `layer`: bf16 N(0,1)
    K/V (seeded per layer), with ceil(outlier_frac*D) seed-chosen channels
    per kv head scaled x8 before quantization.  Returns nothing; not timed."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    sid = np.concatenate([np.full(int(L), s, np.int32) for s, L in zip(seqs, lens)])
    pos = np.concatenate([np.arange(int(L), dtype=np.int32) for L in lens])
    gen = torch.Generator(device=dev)
    gen.manual_seed(1000 + 7919 * layer + seed)
    mult = None
    if outlier_frac > 0:
        rng = np.random.default_rng(seed * 131 + layer)
        m = np.ones((Hkv, D), np.float32)
        for h in range(Hkv):
            m[h, rng.choice(D, int(math.ceil(outlier_frac * D)), replace=False)] = 8.0
        mult = torch.from_numpy(m).to(dev)
    for a in range(0, len(sid), chunk):
        n = min(chunk, len(sid) - a)
        k = torch.randn((n, Hkv, D), generator=gen, device=dev)
        v = torch.randn((n, Hkv, D), generator=gen, device=dev)
        if mult is not None:
            k *= mult
            v *= mult
        pool.append(layer, torch.from_numpy(sid[a:a + n]).to(dev), torch.from_numpy(pos[a:a + n]).to(dev),
                    k.to(torch.bfloat16), v.to(torch.bfloat16))


class _Decoder:
    """One layer-step through rkv_pool_decode (split-K decode with the rows
    appended inside it, then the combine); the library records the split
    event of `ev` between the two kernels."""

    def __init__(self, rkv, ctx, pool, q, out, seq_ids, scale, max_len, q_len, app, part, stream):
        import torch
        self.rkv, self.pool, self.stream = rkv, pool, stream
        g = pool.geometry
        a = rkv.decode_args(q, out, seq_ids, scale, max_len, q_len=q_len, partition_tokens=part,
                            append=app)
        self.ws = torch.empty(max(rkv.decode_workspace_bytes(g, a), 4), device="cuda", dtype=torch.uint8)
        self.a = rkv.decode_args(q, out, seq_ids, scale, max_len, q_len=q_len, partition_tokens=part,
                                 workspace=self.ws, append=app)
        self.max_len = max_len

    def __call__(self, layer, ev=None):
        if ev is not None:
            ev[0].record(self.stream)
        self.a.split_event = C.c_void_p(ev[1].cuda_event) if ev is not None else None
        self.pool.decode(layer, self.a, stream=self.stream)

    def partition_tokens(self) -> int:
        """The partition length of the last launch (workspace header)."""
        import torch
        return int(self.ws[:4].view(torch.int32).item())

    def partitions_total(self, batch) -> int:
        """Partitions of the last launch over its `batch` entries (workspace
        header: partition length, then first partition and count per entry)."""
        import torch
        return int(self.ws[:4 * (1 + 2 * batch)].view(torch.int32)[2::2].sum().item())


def _line(args, cfg, workload, step_s, dec_s, step_bytes, dec_bytes, flops, extra, dtype=DT_INT8_QK,
          emit=True):
    value = step_bytes / step_s / 1e9
    res = {
        "metric": f"config {cfg}: paged Q8 decode HBM GB/s (% of 8 TB/s) + us/step",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0 via the append kernel; bf16 q)",
        "config": dict(workload=workload, **extra.pop("config", {})),
        "us_per_step": round(step_s * 1e6, 2),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "algorithmic_bytes_per_step": step_bytes,
        "achieved_tflops": round(flops / step_s / 1e12, 2),
    }
    if dec_s:
        res["roofline"] = {"bound": "hbm", "kernel": "decode_kernel",
                           "achieved": round(dec_bytes / dec_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(dec_bytes / dec_s / 1e9 / HBM_PEAK_GBS, 4),
                           "traffic": None, "algorithmic_bytes_per_launch": dec_bytes,
                           "decode_us": round(dec_s * 1e6, 2)}
    res.update(extra)
    if emit:
        print(json.dumps(res), flush=True)
    return res


def _time_steps(args, stream, step, n_events=2, event_pass=False):
    import torch
    for i in range(args.warmup):
        step(i, None)
    torch.cuda.synchronize()
    sampled = list(range(0, args.steps, max(args.event_every, 1)))
    evs = {i: [torch.cuda.Event(enable_timing=True) for _ in range(n_events)] for i in sampled}
    for e in evs.values():  # create the events (torch creates them at their first record)
        for x in e:
            x.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i, evs.get(i))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    dec = sum(e[0].elapsed_time(e[1]) for e in evs.values()) * 1e-3 / len(evs)
    _time_steps.last_pcts = None
    if not event_pass:
        return wall, dec
    # the event pass: every step with its events, for percentiles over at
    # least 20 samples (after the timed region: markers cost the stream)
    n_pass = max(getattr(args, "event_steps", 20), 20)
    pev = [[torch.cuda.Event(enable_timing=True) for _ in range(n_events)] for _ in range(n_pass)]
    for e in pev:
        for x in e:
            x.record(stream)
    torch.cuda.synchronize()
    for i, e in enumerate(pev):
        step(args.warmup + args.steps + i, e)
    torch.cuda.synchronize()
    _time_steps.last_pcts = _pcts([e[0].elapsed_time(e[1]) * 1e-3 for e in pev])
    return wall, dec


def _time_graphs(args, dec, layers):
    """Capture one decode step per layer pool into a HIP graph and time
    args.steps replays (layers in rotation) by wall clock, per step."""
    import torch
    dec.a.split_event = None
    torch.cuda.synchronize()
    graphs = []
    for layer in range(layers):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            dec.pool.decode(layer, dec.a, stream=torch.cuda.current_stream())
        graphs.append(g)
    for i in range(args.warmup):
        graphs[i % layers].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        graphs[i % layers].replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    del graphs
    return wall


def run_config(args, emit=True):
    """Configs 2, 3 and 5: every sequence keeps its length across steps (the
    appended rows overwrite the same slots), pools rotate over `layers` so the
    K/V stream does not fit the 256 MB Infinity Cache.  Config 5 also grows
    each sequence by its 4 draft rows and rolls back to a seeded accepted
    length every step, through the allocator and an async table upload."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    cfg = args.config
    rng = np.random.default_rng(args.seed)
    Hq, Hkv, D, PT = 16, 2, 256, 64
    q_len, outliers, part = 1, 0.0, args.partition_tokens
    if cfg == 2:
        B, layers = 16, 8
        lens = rng.integers(4096, 16385, B)
        outliers = 0.01
        work = (f"config 2 batched decode: B=16, L~U[4096,16384] (sum {int(lens.sum())}), Hq=16, Hkv=2, "
                f"D=256, page 64, 1% outlier channels x8, {layers} rotating layer pools")
    elif cfg == 3:
        B, layers = 1, 2
        lens = np.array([262144])
        work = (f"config 3 long context: B=1, L=262144, Hq=16, Hkv=2, D=256, page 64, "
                f"{'device-chosen' if not part else 262144 // part} split-K partitions + LSE combine, "
                f"{layers} rotating layer pools")
    elif cfg == 5:
        B, layers, q_len = 32, 1, 4
        lens = np.full(B, 32768)
        work = ("config 5 speculative verify: B=32, q_len=4 causal draft rows, Hq=16, Hkv=2, D=256, "
                "page 64, L=32768 committed + 4 drafts, seeded accept length in [0,4] and rollback")
    else:
        raise SystemExit(f"unknown config {cfg}")
    cap = lens + q_len
    pps = int((cap.max() + PT - 1) // PT)
    num_pages = int(math.ceil(sum((int(c) + PT - 1) // PT for c in cap) * 1.10))
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, num_pages, B, pps, seed=args.seed)
    for s in range(B):
        pool.alloc.reserve(s, int(cap[s]) if cfg != 5 else int(lens[s]))
    pool.sync_tables()
    for layer in range(layers):
        _fill_layer(rkv, pool, layer, range(B), lens if cfg == 5 else cap, Hkv, D, args.seed, outliers)
    ctx.sync()
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 5)
    seq_ids = torch.arange(B, device=dev, dtype=torch.int32)
    rows_sid = torch.repeat_interleave(seq_ids, q_len)
    first = torch.from_numpy(lens.astype(np.int32) if cfg == 5 else (cap - q_len).astype(np.int32)).to(dev)
    positions = (first.repeat_interleave(q_len) +
                 torch.arange(q_len, device=dev, dtype=torch.int32).repeat(B)).to(torch.int32)
    k_new = torch.randn((B * q_len, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((B * q_len, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((B, q_len, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty((B, q_len, Hq, D), device=dev, dtype=torch.float32)
    app = rkv.append_args(rows_sid, positions, k_new, v_new)
    dec = _Decoder(rkv, ctx, pool, q, out, seq_ids, 1.0 / math.sqrt(D), int(cap.max()), q_len, app,
                   part, stream)
    acc_rng = np.random.default_rng(args.seed + 17)
    accepts = []
    # config 5's allocator work goes through the pair-batch calls: one
    # foreign call per step and kind instead of one per sequence (32 reserves
    # and 64 truncates through ctypes took about 200 us of host time per
    # step, which kept the GPU idle for part of each step)
    all_seqs = np.arange(B, dtype=np.int32)
    grown = (lens + q_len).astype(np.int32)
    base = lens.astype(np.int32)

    def step(i, ev):
        if cfg == 5:
            pool.alloc.reserve_n(all_seqs, grown)
            pool.sync_tables(stream)
        dec(i % layers, ev)
        if cfg == 5:
            a = acc_rng.integers(0, q_len + 1, B)
            accepts.append(a)
            pool.alloc.truncate_n(all_seqs, (base + a).astype(np.int32))
            pool.alloc.truncate_n(all_seqs, base)  # steady state: drafts never commit

    wall, dec_s = _time_steps(args, stream, step, event_pass=True)
    ctx.sync()
    launch = "eager"
    graph_wall = None
    if cfg in (2, 3):
        # the same step as one HIP graph per layer pool (append + decode +
        # combine), replayed in rotation; it measures slower than the eager
        # launches here, so it is reported beside them and used with --graph
        graph_wall = _time_graphs(args, dec, layers)
        if args.graph:
            wall, launch = graph_wall, "hip graph per layer pool, replayed"
    pt = dec.partition_tokens()
    n_parts = dec.partitions_total(len(cap))  # partitions of the batch
    row = D // 32 * 34
    kv = int(cap.sum()) * Hkv * 2 * row
    qo = B * q_len * Hq * D * (2 + 4)
    bt = sum((int(c) + PT - 1) // PT for c in cap) * 4
    apb = B * q_len * Hkv * 2 * (D * 2 + row)
    step_bytes = kv + qo + bt + apb
    # causal draft rows: row j attends ctx+j+1 positions
    flops = 4 * D * Hq * sum(int(c) - q_len + j + 1 for c in cap for j in range(q_len))
    res = _line(args, cfg, work, wall, dec_s, step_bytes, step_bytes, flops,
                {"config": {"batch": B, "q_len": q_len, "layers_rotated": layers,
                            "partition_tokens": pt, "partitions_total": n_parts,
                            "pool_pages_per_layer": num_pages, "launch": launch},
                 **({"graph_us_per_step": round(graph_wall * 1e6, 2)} if graph_wall else {}),
                 "split_k_partial_bytes": n_parts * q_len * Hq * (D + 2) * 4,
                 "decode_p10_p50_p90": _time_steps.last_pcts,
                 **({"mean_accept": float(np.mean(accepts))} if accepts else {})},
                dtype=DT_F16_QK if q_len * Hq // Hkv > 8 else DT_INT8_QK, emit=emit)
    pool.close()
    ctx.close()
    return res if not emit else 0


def run_config4(args) -> int:
    """Continuous-batching mix: B=64 slots with lognormal lengths (median
    8192, sigma 1.0, clipped to [512, 65536]) over 48 layer pools.  Per step
    and layer: 56 slots decode one token (appended inside the decode launch)
    and 8 rotating slots append a 512-row prefill chunk; each slot finishes
    with probability 0.02 per step, frees its pages and restarts empty.  The
    allocator edits of a step go up in one async table upload."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    rng = np.random.default_rng(args.seed)
    B, layers, Hq, Hkv, D, PT = 64, args.layers, 16, 2, 256, 64
    NPF, CH = 8, 512
    lens = np.clip(np.round(np.exp(rng.normal(math.log(8192), 1.0, B))), 512, 65536).astype(np.int64)
    total_steps = args.warmup + args.steps
    # worst case growth: every slot prefills every step
    max_len = 65536 + total_steps * CH
    pps = (max_len + PT - 1) // PT
    num_pages = int(math.ceil((int(lens.sum()) + B * total_steps * CH // 4) / PT * 1.10)) + B * 8
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, num_pages, B, pps, seed=args.seed)
    for s in range(B):
        pool.alloc.reserve(s, int(lens[s]))
    pool.sync_tables()
    for layer in range(layers):
        _fill_layer(rkv, pool, layer, range(B), lens, Hkv, D, args.seed)
    ctx.sync()
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 9)
    ND = B - NPF
    kd = torch.randn((ND, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    vd = torch.randn((ND, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    kp = torch.randn((NPF * CH, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    vp = torch.randn((NPF * CH, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((ND, 1, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty((ND, 1, Hq, D), device=dev, dtype=torch.float32)
    d_sid = torch.empty(ND, dtype=torch.int32, device=dev)
    d_pos = torch.empty(ND, dtype=torch.int32, device=dev)
    p_sid = torch.empty(NPF * CH, dtype=torch.int32, device=dev)
    p_pos = torch.empty(NPF * CH, dtype=torch.int32, device=dev)
    # host staging of the per-step index vectors: two pinned buffers, each
    # rewritten only after the upload that last read it has run
    h_idx = [torch.empty(2 * ND + 2 * NPF * CH, dtype=torch.int32).pin_memory() for _ in range(2)]
    h_done = [None, None]
    app = rkv.append_args(d_sid, d_pos, kd, vd)
    scale = 1.0 / math.sqrt(D)
    fin_rng = np.random.default_rng(args.seed + 3)
    cur = lens.copy()
    stats = {"decode_tokens": 0, "prefill_rows": 0, "finished": 0}
    dec_cache = {}
    per_step_bytes = []

    def step(i, ev):
        pf = [(i * NPF + j) % B for j in range(NPF)]
        dset = [s for s in range(B) if s not in pf]
        # finishes: free pages, restart empty (new sequences take pages from the free list)
        for s in range(B):
            if fin_rng.random() < 0.02:
                pool.alloc.free(s)
                cur[s] = 0
                stats["finished"] += 1
        dpos = cur[dset].copy()
        for s in dset:
            pool.alloc.reserve(s, int(cur[s]) + 1)
            cur[s] += 1
        ppos0 = cur[pf].copy()
        for s in pf:
            pool.alloc.reserve(s, int(cur[s]) + CH)
            cur[s] += CH
        hb = i & 1
        if h_done[hb] is not None:
            h_done[hb].synchronize()
        h = h_idx[hb].numpy()
        h[:ND] = dset
        h[ND:2 * ND] = dpos
        h[2 * ND:2 * ND + NPF * CH] = np.repeat(pf, CH)
        h[2 * ND + NPF * CH:] = (ppos0[:, None] + np.arange(CH)[None, :]).reshape(-1)
        dev_idx = h_idx[hb].to(dev, non_blocking=True)
        h_done[hb] = torch.cuda.Event()
        h_done[hb].record(stream)
        d_sid.copy_(dev_idx[:ND])
        d_pos.copy_(dev_idx[ND:2 * ND])
        p_sid.copy_(dev_idx[2 * ND:2 * ND + NPF * CH])
        p_pos.copy_(dev_idx[2 * ND + NPF * CH:])
        pool.sync_tables(stream)
        max_len = int(cur[dset].max())
        key = (max_len + 4095) // 4096
        if key not in dec_cache:
            dec_cache[key] = _Decoder(rkv, ctx, pool, q, out, d_sid, scale, key * 4096, 1, app, 0, stream)
        dec = dec_cache[key]
        if ev is not None:
            ev[0].record(stream)
        for layer in range(layers):
            pool.append(layer, p_sid, p_pos, kp, vp, stream=stream)
            dec(layer)
        if ev is not None:
            ev[1].record(stream)
        stats["decode_tokens"] += int(cur[dset].sum())
        stats["prefill_rows"] += NPF * CH
        row = D // 32 * 34
        per_step_bytes.append(layers * (int(cur[dset].sum()) * Hkv * 2 * row + ND * Hq * D * 6 +
                                        sum((int(cur[s]) + PT - 1) // PT for s in dset) * 4 +
                                        (ND + NPF * CH) * Hkv * 2 * (D * 2 + row)))

    wall, tot = _time_steps(args, stream, step)
    ctx.sync()
    timed = per_step_bytes[args.warmup:]
    step_bytes = int(sum(timed) / len(timed))
    _line(args, 4, f"config 4 continuous batching: B=64 (56 decode + 8 x 512-row prefill append per step), "
                   f"lognormal L (median 8192, sigma 1.0, [512, 65536]), {layers} layer pools, "
                   f"2% finish per step", wall, None, step_bytes, step_bytes, 0,
          {"config": {"layers": layers, "pool_pages_per_layer": num_pages},
           "us_per_layer_step": round(wall * 1e6 / layers, 2),
           "event_us_per_step": round(tot * 1e6, 2),
           "finished_total": stats["finished"]})
    pool.close()
    ctx.close()
    return 0


def run_config6(args) -> int:
    """Prefix sharing: 64 sequences forked from one 30752-token prefix (it
    ends inside a page) each grow a private suffix to L=32768, so every
    child's first suffix row lands in a copy-on-write copy of the prefix's
    last page.  The parent is then freed; its pages live on through the
    children's references.  Set-up times the table sync that runs the
    64 x layers page copies.  Each step is the headline's decode (one row
    appended per sequence inside the launch) over the children, rotating over
    4 layer pools.  `value` counts the logical K/V bytes the decode serves;
    the prefix is stored once, so `unique_kv_bytes` is far smaller and most
    reads hit the caches."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    Hq, Hkv, D, PT = 16, 2, 256, 64
    B, layers, L, prefix = 64, 4, 32768, 30752
    pps = L // PT
    unique_pages = (prefix + PT - 1) // PT + B * ((L - prefix + PT - 1) // PT + 1)
    num_pages = int(math.ceil(unique_pages * 1.10))
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, num_pages, B + 1, pps, seed=args.seed)
    parent = B
    pool.alloc.reserve(parent, prefix)
    pool.sync_tables()
    for layer in range(layers):
        _fill_layer(rkv, pool, layer, [parent], [prefix], Hkv, D, args.seed)
    for s in range(B):
        pool.alloc.fork(parent, s, prefix)
    pool.alloc.free(parent)
    for s in range(B):
        pool.alloc.reserve(s, L)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    pool.sync_tables(stream)
    e1.record(stream)
    torch.cuda.synchronize()
    cow_us = e0.elapsed_time(e1) * 1e3
    page_b = rkv.page_bytes(pool.geometry)
    cow_bytes = 2 * B * layers * page_b
    for layer in range(layers):
        suffix_pos = np.arange(prefix, L, dtype=np.int32)
        sid = np.repeat(np.arange(B, dtype=np.int32), L - prefix)
        gen = torch.Generator(device=dev)
        gen.manual_seed(2000 + layer + args.seed)
        for a in range(0, len(sid), 1 << 16):
            n = min(1 << 16, len(sid) - a)
            k = torch.randn((n, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((n, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
            pos = torch.from_numpy(np.tile(suffix_pos, B)[a:a + n]).to(dev)
            pool.append(layer, torch.from_numpy(sid[a:a + n]).to(dev), pos, k, v)
    ctx.sync()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 5)
    seq_ids = torch.arange(B, device=dev, dtype=torch.int32)
    positions = torch.full((B,), L - 1, device=dev, dtype=torch.int32)
    k_new = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((B, 1, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty((B, 1, Hq, D), device=dev, dtype=torch.float32)
    app = rkv.append_args(seq_ids, positions, k_new, v_new)
    dec = _Decoder(rkv, ctx, pool, q, out, seq_ids, 1.0 / math.sqrt(D), L, 1, app,
                   args.partition_tokens, stream)

    def step(i, ev):
        dec(i % layers, ev)

    wall, dec_s = _time_steps(args, stream, step)
    ctx.sync()
    row = D // 32 * 34
    kv = B * L * Hkv * 2 * row
    unique_kv = (prefix + B * (L - prefix)) * Hkv * 2 * row
    step_bytes = kv + B * Hq * D * (2 + 4) + B * pps * 4 + B * Hkv * 2 * (D * 2 + row)
    flops = 4 * D * Hq * B * L
    _line(args, 6, (f"prefix-shared decode: B={B} sequences forked from one {prefix}-token prefix, "
                    f"private suffixes to L={L}, Hq=16, Hkv=2, D=256, page 64, one row appended "
                    f"per sequence in the decode launch, {layers} rotating layer pools"),
          wall, None, step_bytes, step_bytes, flops,
          {"config": {"batch": B, "layers_rotated": layers, "prefix_tokens": prefix,
                      "partition_tokens": dec.partition_tokens(),
                      "pool_pages_per_layer": num_pages},
           "unique_kv_bytes": unique_kv,
           "unique_kv_gbs": round(unique_kv / wall / 1e9, 2),
           "decode_us": round(dec_s * 1e6, 2),
           "cow_sync": {"pairs": B, "layers": layers, "us": round(cow_us, 2),
                        "page_bytes_moved": cow_bytes,
                        "gbs": round(cow_bytes / (cow_us * 1e-6) / 1e9, 2)}})
    pool.close()
    ctx.close()
    return 0


def run_config7(args) -> int:
    """Chunked prefill: 8 sequences, each with ctx=8192 cached tokens and a
    512-row chunk (config 4's prefill rows, at its median context).  One step
    and layer appends the chunk's K/V rows (rkv_pool_append) and runs the
    prefill attention over them (rkv_pool_prefill), rotating over 4 layer
    pools.  Rows of a chunk attend causally: row i sees ctx + i + 1 tokens.
    `value` is attention TFLOP/s, 4*D flops per (query row, visible token),
    against the dense f16 MFMA peak; the prefill kernel (and the split's
    combine, when the launch splits) is HIP-event timed.  --prefill-batch,
    --prefill-ctx and --prefill-rows change the shape (one long-context chunk
    leaves most workgroup slots idle unless its causal ranges are split)."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    Hq, Hkv, D, PT = 16, 2, 256, 64
    B, layers, C0, N = args.prefill_batch, 4, args.prefill_ctx, args.prefill_rows
    L = C0 + N
    pps = (L + PT - 1) // PT
    num_pages = int(math.ceil(B * pps * 1.10))
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, num_pages, B, pps, seed=args.seed)
    for s in range(B):
        pool.alloc.reserve(s, L)
    pool.sync_tables()
    for layer in range(layers):
        _fill_layer(rkv, pool, layer, range(B), [L] * B, Hkv, D, args.seed)
    ctx.sync()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 5)
    rows = B * N
    sid = torch.arange(B, device=dev, dtype=torch.int32).repeat_interleave(N)
    pos = (torch.arange(N, device=dev, dtype=torch.int32) + C0).repeat(B)
    k_new = torch.randn((rows, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((rows, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((rows, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty((rows, Hq, D), device=dev, dtype=torch.float32)
    ent = (list(range(B)), [C0] * B, [N] * B, q, out, 1.0 / math.sqrt(D))
    ws_bytes = rkv.prefill_workspace_bytes(
        pool.geometry, rkv.prefill_args(*ent, segment_tokens=args.prefill_segment))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    pa = rkv.prefill_args(*ent, segment_tokens=args.prefill_segment, workspace=ws)
    stream = torch.cuda.current_stream()

    def step(i, ev):
        layer = i % layers
        pool.append(layer, sid, pos, k_new, v_new, stream=stream)
        if ev is not None:
            ev[0].record(stream)
        pool.prefill(layer, pa, stream=stream)
        if ev is not None:
            ev[1].record(stream)

    wall, kern = _time_steps(args, stream, step)
    ctx.sync()
    row_tokens = B * sum(C0 + i + 1 for i in range(N))
    flops = 4 * D * Hq * row_tokens
    kv_bytes = B * L * Hkv * 2 * (D // 32 * 34)
    peak = 2500.0
    res = {
        "metric": "config 7: chunked prefill attention TFLOP/s (dense f16 MFMA peak 2.5 PFLOP/s)",
        "value": round(flops / wall / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": DT_F16_QK,
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0 via the append kernel; bf16 q)",
        "config": {"workload": (f"chunked prefill: B={B} sequences, ctx={C0} cached + {N}-row chunk "
                                f"each (causal), Hq=16, Hkv=2, D=256, page 64, append + attention "
                                f"per step, {layers} rotating layer pools"),
                   "batch": B, "ctx": C0, "chunk_rows": N, "layers_rotated": layers,
                   "segment_tokens": args.prefill_segment, "split_workspace_bytes": ws_bytes},
        "us_per_step": round(wall * 1e6, 2),
        "flops_per_step": flops,
        # events bracket the whole rkv_pool_prefill call: with a bf16 query and a
        # workspace that holds the widened tiles, the widening pass plus the
        # prefill kernel (and the split combine when the launch splits)
        "roofline": {"bound": "mfma", "kernel": ("rkv::widen_tiles_kernel<256> + "
                                                 "rkv::prefill_kernel<256, false, 2, true, true>"),
                     "achieved": round(flops / kern / 1e12, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(flops / kern / 1e12 / peak, 4), "traffic": None,
                     "prefill_us": round(kern * 1e6, 2)},
        "kv_bytes_per_layer": kv_bytes,
    }
    print(json.dumps(res), flush=True)
    pool.close()
    ctx.close()
    return 0


def run_config9(args) -> int:
    """Serving step through the adapter (rkv_serve_*): 64 live requests with
    lognormal contexts (median 8192, sigma 1.0, clipped to [512, 32768]) over
    `--serve-layers` layers.  Per step: 8 rotating requests prefill a
    512-token chunk (append + causal prefill attention) and the other 56
    decode one token (append inside the decode launch).  Each request
    finishes with probability 0.02 per step; its place goes to a new id that
    starts empty or, one in four, forks the first half of a live request
    (prefix reuse).  One begin_step per step, then prefill and decode
    attention per layer; the value is tokens (prefill rows + decode rows)
    through every layer's attention per second."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    rng = np.random.default_rng(args.seed)
    B, layers, Hq, Hkv, D, PT = 64, args.serve_layers, 16, 2, 256, 64
    NPF, CH = 8, 512
    ND = B - NPF
    lens = np.clip(np.round(np.exp(rng.normal(math.log(8192), 1.0, B))), 512, 32768).astype(np.int64)
    total_steps = args.warmup + args.steps
    cap = 32768 + total_steps * CH + CH
    pps = (cap + PT - 1) // PT
    num_pages = int(math.ceil((int(lens.sum()) + B * total_steps * CH // 4) / PT * 1.25)) + B * 8
    sv = rkv.Serve(ctx, layers, Hkv, D, PT, num_pages, 2 * B, pps, q_heads=Hq, max_decode=B,
                   max_prefill_rows=NPF * CH, seed=args.seed)
    # initial contexts: admit every id, grow it and write its rows directly
    # (no attention for the cache fill; not timed)
    ids = list(range(B))
    sv.begin_step(decode=[(i, 1) for i in ids])
    for i in ids:
        sv.alloc.reserve(sv.slot(i), int(lens[i]))
    sv.sync_tables()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 11)
    sl = np.concatenate([np.full(int(L), sv.slot(i), np.int32) for i, L in zip(ids, lens)])
    po = np.concatenate([np.arange(int(L), dtype=np.int32) for L in lens])
    for layer in range(layers):
        for a0 in range(0, len(sl), 1 << 16):
            n = min(1 << 16, len(sl) - a0)
            k = torch.randn((n, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((n, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
            sv.pool_append(layer, torch.from_numpy(sl[a0:a0 + n]).to(dev),
                           torch.from_numpy(po[a0:a0 + n]).to(dev), k, v)
    ctx.sync()
    stream = torch.cuda.current_stream()
    qp = torch.randn((NPF * CH, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    kp = torch.randn((NPF * CH, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    vp = torch.randn((NPF * CH, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    qd = torch.randn((ND, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    kd = torch.randn((ND, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    vd = torch.randn((ND, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
    op = torch.empty((NPF * CH, Hq, D), dtype=torch.float32, device=dev)
    od = torch.empty((ND, Hq, D), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    fin = np.random.default_rng(args.seed + 3)
    cur = {i: int(lens[i]) for i in ids}
    next_id = [B]
    stats = {"finished": 0, "forks": 0, "decode_kv_bytes": 0, "prefill_flops": 0}
    row = D // 32 * 34

    def step(i, ev):
        # finishes: the position's request is replaced by a new id
        fresh = {}
        for pos in range(B):
            if fin.random() < 0.02:
                sv.finish(ids[pos])
                del cur[ids[pos]]
                ids[pos] = next_id[0]
                next_id[0] += 1
                stats["finished"] += 1
                fresh[pos] = None
        for pos in fresh:
            if fin.random() < 0.25 and len(cur) > 0:
                parent = ids[(pos + 1 + int(fin.integers(B - 1))) % B]
                if parent in cur and parent not in [ids[p] for p in fresh]:
                    fresh[pos] = (parent, cur[parent] // 2)
        pf_pos = [(i * NPF + j) % B for j in range(NPF)]
        pre, dec = [], []
        for pos in range(B):
            sid = ids[pos]
            n = CH if pos in pf_pos else 1
            fk = fresh.get(pos)
            if pos in fresh:
                cur[sid] = fk[1] if fk else 0
                stats["forks"] += 1 if fk else 0
            e = (sid, n, fk[1], fk[0]) if fk else (sid, n)
            (pre if n > 1 else dec).append(e)
            if n == 1:
                stats["decode_kv_bytes"] += layers * (cur[sid] + 1) * Hkv * 2 * row
            else:
                stats["prefill_flops"] += layers * 4 * D * Hq * sum(cur[sid] + j + 1 for j in range(n))
            cur[sid] += n
        sv.begin_step(prefill=pre, decode=dec, stream=stream)
        for layer in range(layers):
            sv.prefill(layer, qp, kp, vp, op, scale, stream=stream)
            sv.decode(layer, qd, kd, vd, od, scale, stream=stream)

    wall, _ = _time_steps(args, stream, step)
    ctx.sync()
    tokens = NPF * CH + ND
    res = {
        "metric": "config 9: serving step through the adapter, tokens through attention per second",
        "value": round(tokens / wall, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "prefill: " + DT_F16_QK + "; decode (8 rows per kv head): " + DT_INT8_QK,
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0; bf16 q)",
        "config": {"workload": f"config 9 serving step (rkv_serve_*): 64 requests, lognormal "
                               f"contexts (median 8192, sigma 1.0, [512, 32768]); per step 8 x "
                               f"{CH}-token prefill chunks + {ND} decode rows, {layers} layers, "
                               f"2% finish per step, 1 in 4 new requests fork a live prefix",
                   "layers": layers, "pool_pages": num_pages},
        "us_per_step": round(wall * 1e6, 2),
        "us_per_layer_step": round(wall * 1e6 / layers, 2),
        "finished_total": stats["finished"], "forks_total": stats["forks"],
        "mean_decode_kv_gb_per_step": round(stats["decode_kv_bytes"] / total_steps / 1e9, 4),
        "mean_prefill_tflop_per_step": round(stats["prefill_flops"] / total_steps / 1e12, 4),
    }
    print(json.dumps(res), flush=True)
    sv.close()
    ctx.close()
    return 0


def run_config10(args) -> int:
    """Host-KV tier (research/host-kv/README.md:1-24): B=8 sequences of
    L=32768 tokens whose pages live in pinned host memory (RKV_PAGES_HOST),
    Hq=16, Hkv=2, D=256, page 64: 285 MB of Q8 K/V in one layer, read over
    the host link by the same kernels as an HBM pool.  Modes, one launch a
    step: decode (q_len 1: 8 query rows per kv head served by each staged
    tile), causal verify q_len 2 and 4 (16 and 32 rows), and a 512-row
    chunked prefill of one sequence (128 rows per tile; its 32 row blocks
    fetch overlapping causal ranges).  `physical` = unique K/V bytes / time;
    `logical` = bytes served to query rows / time (each fetched byte serves
    the tile's rows).  Beside them: the link's read roof (rkv_stream_read
    over the pinned pages, vector loads), a DMA copy of pinned memory to HBM,
    and the same decode on an HBM pool.  `value` is the decode's logical
    GB/s."""
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    Hq, Hkv, D, PT = 16, 2, 256, 64
    B, L = 8, 32768
    G = Hq // Hkv
    pps = L // PT
    num_pages = int(math.ceil(B * pps * 1.10))
    row = D // 32 * 34
    kv_bytes = B * L * Hkv * 2 * row
    stream = torch.cuda.current_stream()
    pools = {}
    for name, mem in (("host", rkv.PAGES_HOST), ("hbm", rkv.PAGES_DEVICE)):
        pool = rkv.Pool(ctx, 1, Hkv, D, PT, num_pages, B, pps, seed=args.seed, page_memory=mem)
        for s_ in range(B):
            pool.alloc.reserve(s_, L)
        pool.sync_tables()
        _fill_layer(rkv, pool, 0, range(B), [L] * B, Hkv, D, args.seed)
        pools[name] = pool
    ctx.sync()
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 10)
    sid = torch.arange(B, device=dev, dtype=torch.int32)
    scale = 1.0 / math.sqrt(D)

    def timed(launch, reps):
        for _ in range(2):
            launch()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
        for r in range(reps):
            ev[2 * r].record(stream)
            launch()
            ev[2 * r + 1].record(stream)
        torch.cuda.synchronize()
        ts = sorted(ev[2 * r].elapsed_time(ev[2 * r + 1]) * 1e-3 for r in range(reps))
        return ts[reps // 2]

    modes = {}
    reps = max(args.steps // 4, 3)
    for pname in ("host", "hbm"):
        pool = pools[pname]
        for q_len in ((1, 2, 4) if pname == "host" else (1,)):
            q = torch.randn((B, q_len, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
            out = torch.empty((B, q_len, Hq, D), device=dev, dtype=torch.float32)
            a = rkv.decode_args(q, out, sid, scale, L, q_len=q_len)
            ws = torch.empty(max(rkv.decode_workspace_bytes(pool.geometry, a), 4), dtype=torch.uint8,
                             device=dev)
            a = rkv.decode_args(q, out, sid, scale, L, q_len=q_len, workspace=ws)
            t = timed(lambda: pool.decode(0, a, stream=stream), reps)
            rows = G * q_len
            modes[f"{pname}_q_len{q_len}"] = {
                "us": round(t * 1e6, 1), "rows_per_tile": rows,
                "physical_gbs": round(kv_bytes / t / 1e9, 2),
                "logical_gbs": round(kv_bytes * rows / t / 1e9, 2)}
    # chunked prefill of sequence 0's last 512 tokens over the host pages
    N = 512
    qp = torch.randn((N, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    op = torch.empty((N, Hq, D), device=dev, dtype=torch.float32)
    ent = ([0], [L - N], [N], qp, op, scale)
    pws_bytes = rkv.prefill_workspace_bytes(pools["host"].geometry, rkv.prefill_args(*ent))
    pws = torch.empty(max(pws_bytes, 1), dtype=torch.uint8, device=dev)
    pa = rkv.prefill_args(*ent, workspace=pws)
    t = timed(lambda: pools["host"].prefill(0, pa, stream=stream), reps)
    tq = 128 // G
    seq_bytes = L * Hkv * 2 * row
    fetched = sum((L - N + min(tq * (b + 1), N)) * Hkv * 2 * row for b in range(N // tq))
    modes["host_prefill512"] = {
        "us": round(t * 1e6, 1), "rows_per_tile": 128, "split_workspace_bytes": pws_bytes,
        "physical_gbs": round(seq_bytes / t / 1e9, 2),
        "block_fetch_gbs": round(fetched / t / 1e9, 2),
        "logical_gbs": round(fetched * 128 / t / 1e9, 2)}
    # the link's read roof and a DMA copy, beside the kernels
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    base = pools["host"].layer_pages(0)
    nread = kv_bytes // 16 * 16
    roof = {}
    for blocks in (256, 1024):
        tr = timed(lambda: rkv.stream_read(ctx, int(base), 0, blocks, word, nbytes=nread,
                                           stream=stream), 3)
        roof[blocks] = nread / tr / 1e9
    src = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    tc = timed(lambda: dst.copy_(src, non_blocking=True), 5)
    dec = modes["host_q_len1"]
    res = {
        "metric": "config 10: host-KV tier decode, logical GB/s (K/V bytes x rows served per "
                  "fetched byte) over pages in pinned host memory",
        "value": dec["logical_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": reps,
        "warmup": 2, "ms_per_step": round(dec["us"] / 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("8-row decode: " + DT_INT8_QK + "; 16- and 32-row verify and the prefill: " + DT_F16_QK),
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0 via the append kernel; bf16 q)",
        "config": {"workload": (f"host-KV tier: B={B}, L={L}, Hq={Hq}, Hkv={Hkv}, D={D}, page {PT}, "
                                f"pages in pinned host memory ({kv_bytes} K/V bytes); decode, verify "
                                f"q_len 2/4, 512-row prefill"),
                   "batch": B, "seq_len": L},
        "modes": modes,
        "link_read_roof_gbs": round(max(roof.values()), 2),
        "link_read_roof_blocks": max(roof, key=roof.get),
        "dma_h2d_copy_gbs": round((256 << 20) / tc / 1e9, 2),
        "hbm_pool_decode_us": modes["hbm_q_len1"]["us"],
    }
    print(json.dumps(res), flush=True)
    for pool in pools.values():
        pool.close()
    ctx.close()
    return 0


def run_config8(args) -> int:
    """Off-HBM tier (R4KV pages): a 4096-token range of one sequence over 48
    layers (Hkv=2, D=256, page 64) is one page of 214 MB.  Timed, with HIP
    events: the device CRC32C over 1 GiB (its HBM roofline); spill into a
    device staging buffer (pack + CRC, no PCIe); spill to pinned host memory
    (+ the D2H copy); restore from pinned host memory (H2D copy, device CRC
    check, one host wait, unpack).  `value` is the spill-to-host rate."""
    import numpy as np
    import torch
    rkv = load_rkv()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = rkv.Ctx(0)
    Hkv, D, PT, layers, T = 2, 256, 64, 48, 4096
    pps = T // PT
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, 2 * pps + 8, 2, pps, seed=args.seed)
    pool.alloc.reserve(0, T)
    pool.alloc.reserve(1, T)
    pool.sync_tables()
    for layer in range(layers):
        _fill_layer(rkv, pool, layer, [0], [T], Hkv, D, args.seed)
    ctx.sync()
    n = pool.r4kv_page_bytes(T, 0, layers - 1)
    staging = torch.empty(n + 256, dtype=torch.uint8, device=dev)
    host = torch.empty(n, dtype=torch.uint8).pin_memory()
    ident = rkv.R4kvHeader(prefix_digest=0xC0FFEE, token_start=0, token_count=T, pos_start=0,
                           layer_lo=0, layer_hi=layers - 1, k_fmt=1, v_fmt=1, epoch=1,
                           generation=1, payload_len=0, sketch_offset=0, flags=0)
    exp = rkv.R4kvExpect(prefix_digest=0xC0FFEE, token_start=0, pos_start=0, layer_lo=0,
                         layer_hi=layers - 1, k_fmt=1, v_fmt=1, check_generation=0,
                         generation_min=0, generation_max=0)
    stream = torch.cuda.current_stream()
    big = torch.randint(0, 256, (1 << 30,), dtype=torch.uint8, device=dev)
    word = torch.zeros(4, dtype=torch.int32, device=dev)
    reps = max(args.steps // 5, 3)

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps, (time.perf_counter() - t0) / reps

    crc_s, _ = timed(lambda: rkv.crc32c(ctx, big, big.numel(), word, stream))
    spill_dev_s, _ = timed(lambda: pool.spill(0, 0, T, 0, layers - 1, ident, staging, staging, stream))
    spill_host_s, _ = timed(lambda: pool.spill(0, 0, T, 0, layers - 1, ident, staging, host, stream))
    page = host.numpy()
    _, restore_s = timed(lambda: pool.restore(1, page, exp, staging, stream))
    ctx.sync()
    res = {
        "metric": "config 8: R4KV page spill to host GB/s (4096 tokens x 48 layers per page)",
        "value": round(n / spill_host_s / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": reps,
        "warmup": 2, "ms_per_step": round(spill_host_s * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8 (Q8_0 page bytes), CRC32C",
        "data": "synthetic (seeded N(0,1) K/V bf16 -> Q8_0 via the append kernel)",
        "config": {"workload": "R4KV spill/restore: one sequence, tokens [0, 4096), layers 0-47, "
                               "Hkv=2, D=256, page 64; page = header + body + CRC32C",
                   "page_bytes": n, "layers": layers, "tokens": T},
        "spill_to_device_us": round(spill_dev_s * 1e6, 1),
        "spill_to_device_gbs": round(n / spill_dev_s / 1e9, 1),
        "spill_to_host_us": round(spill_host_s * 1e6, 1),
        "restore_from_host_us": round(restore_s * 1e6, 1),
        "restore_from_host_gbs": round(n / restore_s / 1e9, 2),
        "roofline": {"bound": "hbm", "kernel": "rkv::crc32c_kernel", "achieved": round((1 << 30) / crc_s / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round((1 << 30) / crc_s / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "crc_bytes": 1 << 30, "crc_us": round(crc_s * 1e6, 1)},
    }
    print(json.dumps(res), flush=True)
    pool.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    _a = parse()
    if _a.config == 10:
        sys.exit(run_config10(_a))
    if _a.config == 8:
        sys.exit(run_config8(_a))
    if _a.config == 7:
        sys.exit(run_config7(_a))
    if _a.config == 4:
        sys.exit(run_config4(_a))
    if _a.config == 6:
        sys.exit(run_config6(_a))
    if _a.config == 9:
        sys.exit(run_config9(_a))
    if _a.config in (2, 3, 5):
        sys.exit(run_config(_a))
    sys.exit(main())
