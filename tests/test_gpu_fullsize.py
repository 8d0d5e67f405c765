"""Parity at BASELINE.json's full sizes: the headline and configs 2-5.

The pools are filled through the product's append kernel from seeded device
rows (bf16 N(0,1), one generator per sequence and layer, so any sequence's
rows can be regenerated).  Sampled sequences are exported with the pool
gather (the reference row layout, attention.rs:144-147) and decoded by the
oracle's flash_decode_reference (attention.rs:148-215) on the host cores.
Checked:
  - page bytes: the gathered rows of sampled tokens equal the oracle's Q8_0
    encoder (r4kv/src/quant.rs:45-90) of the same source rows, bit for bit,
    including the rows the decode launch itself appended;
  - attention: max |gpu - oracle| <= 2e-3 and ||gpu - oracle|| / ||oracle||
    <= 1e-3 over every checked sequence's output (both printed).
"""
import math
import os

import numpy as np
import pytest

from tests.test_gpu_parity import assert_close, outlier_q

pytestmark = pytest.mark.gpu

HQ, HKV, D, PT = 16, 2, 256, 64
RB = D // 32 * 34
SCALE = 1.0 / math.sqrt(D)
THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS") or 16)))


def _torch():
    import torch
    return torch


class Big:
    """A pool of `layers` layers whose sequence s (of `lens[s]` rows) is
    filled from a per-(layer, sequence) seeded generator."""

    def __init__(self, rkv, ctx, layers, lens, cap=None, slack=1.10, seed=0, outliers=0.0,
                 max_seqs=None):
        torch = _torch()
        self.rkv, self.ctx, self.seed = rkv, ctx, seed
        self.lens = [int(x) for x in lens]
        cap = self.lens if cap is None else [int(x) for x in cap]
        B = len(self.lens)
        self.pps = max((c + PT - 1) // PT for c in cap)
        num_pages = int(math.ceil(sum((c + PT - 1) // PT for c in cap) * slack)) + 8
        self.pool = rkv.Pool(ctx, layers, HKV, D, PT, num_pages, max_seqs or B, self.pps, seed=seed)
        self.g = self.pool.geometry
        self.mult = None
        if outliers:
            rng = np.random.default_rng(seed + 77)
            m = np.ones((HKV, D), np.float32)
            for h in range(HKV):
                m[h, rng.choice(D, int(math.ceil(outliers * D)), replace=False)] = 8.0
            self.mult = torch.from_numpy(m).cuda()
        for s, L in enumerate(self.lens):
            if L:
                self.pool.alloc.reserve(s, L)
        self.pool.sync_tables()
        for layer in range(layers):
            for s, L in enumerate(self.lens):
                self.fill(layer, s, 0, L)
        ctx.sync()

    def rows(self, layer, s, start, n, gen_id=0):
        """Source rows [start, start+n) of sequence s (bf16 on the device)."""
        torch = _torch()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(((self.seed * 1000003 + layer) * 7919 + s) * 31 + gen_id)
        k = torch.randn((start + n, HKV, D), generator=gen, device="cuda")[start:]
        v = torch.randn((start + n, HKV, D), generator=gen, device="cuda")[start:]
        if self.mult is not None:
            k = k * self.mult
            v = v * self.mult
        return k.to(torch.bfloat16).contiguous(), v.to(torch.bfloat16).contiguous()

    def fill(self, layer, s, start, n, gen_id=0):
        torch = _torch()
        if n <= 0:
            return
        k, v = self.rows(layer, s, start, n, gen_id)
        sid = torch.full((n,), s, dtype=torch.int32, device="cuda")
        pos = torch.arange(start, start + n, dtype=torch.int32, device="cuda")
        self.pool.append(layer, sid, pos, k, v)

    def gather(self, layer, s):
        """(K rows, V rows) of sequence s: uint8 [HKV][len][RB] on the host."""
        torch = _torch()
        L = self.pool.alloc.seq_len(s)
        out = []
        for kind in (0, 1):
            t = torch.empty(HKV * L * RB, dtype=torch.uint8, device="cuda")
            self.pool.gather(layer, s, kind, t)
            self.ctx.sync()
            out.append(t.cpu().numpy().reshape(HKV, L, RB))
        return out

    def close(self):
        self.pool.close()


def check_rows(rko, got_rows, src, idx, what):
    """got_rows [HKV][len][RB] (one kind) at token indices idx equal the
    oracle's canonical Q8_0 encoding of src ([len(idx)][HKV][D], the source
    rows of those tokens)."""
    want = rko.q8_encode(np.asarray(src, np.float32).reshape(-1)).reshape(len(idx), HKV, RB)
    got = np.ascontiguousarray(got_rows[:, idx].transpose(1, 0, 2))
    bad = int(np.sum(np.any(got != want, axis=-1)))
    print(f"[{what}] {len(idx)} rows x {HKV} heads bit-exact: {bad == 0}", flush=True)
    assert bad == 0, f"{what}: {bad} of {len(idx) * HKV} rows differ"


def oracle_decode(rko, kr, vr, L, q_rows):
    """flash_decode_reference over the first L rows: q_rows [HQ][D] (scaled)."""
    kw = rko.rows_to_words(np.ascontiguousarray(kr[:, :L]))
    vw = rko.rows_to_words(np.ascontiguousarray(vr[:, :L]))
    p = rko.fd_params(HQ, HKV, L, 1024, D)
    return rko.flash_decode_reference_many(p, [kw], [vw], q_rows[None], THREADS)[0]


def run_decode(rkv, pool, layer, q, out, seq_ids, max_len, q_len=1, app=None,
               partition_tokens=0):
    """rkv_pool_decode of one layer with its workspace; returns the workspace
    (its first word is the partition length the launch used)."""
    torch = _torch()
    g = pool.geometry
    a = rkv.decode_args(q, out, seq_ids, SCALE, max_len, q_len=q_len,
                        partition_tokens=partition_tokens, append=app)
    ws = torch.empty(max(rkv.decode_workspace_bytes(g, a), 4), dtype=torch.uint8, device="cuda")
    a = rkv.decode_args(q, out, seq_ids, SCALE, max_len, q_len=q_len,
                        partition_tokens=partition_tokens, workspace=ws, append=app)
    pool.decode(layer, a)
    return ws


def _decode_step_check(rkv, rko, ctx, big, layer, lens, sample, q_np, q_d, out, app_rows,
                       partition_tokens=0, label="", expect_pt=None):
    """One decode launch (this step's row appended inside it) on `layer`;
    checks the appended rows and the sampled sequences' outputs (and, with
    expect_pt, the partition length the device chose)."""
    torch = _torch()
    B = len(lens)
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device="cuda")
    kn, vn = app_rows
    app = rkv.append_args(sid, pos, kn, vn)
    ws = run_decode(rkv, big.pool, layer, q_d, out, sid, max(lens), app=app,
                    partition_tokens=partition_tokens)
    ctx.sync()
    parts = int(ws[:4].view(torch.int32).item()) if partition_tokens == 0 else partition_tokens
    if expect_pt is not None:
        assert parts == expect_pt, f"{label}: the device chose {parts}-token partitions"
    got = out.float().cpu().numpy()
    kn_h, vn_h = kn.float().cpu().numpy(), vn.float().cpu().numpy()
    errs = []
    for s in sample:
        kr, vr = big.gather(layer, s)
        L = lens[s]
        # the appended row (position L-1) and a sample of the filled ones
        src_k, src_v = big.rows(layer, s, 0, L - 1)
        rng = np.random.default_rng(s)
        idx = np.unique(rng.integers(0, L - 1, 512))
        sel = torch.from_numpy(idx).cuda()
        check_rows(rko, kr, src_k[sel].float().cpu().numpy(), idx, f"{label} s{s} K")
        check_rows(rko, vr, src_v[sel].float().cpu().numpy(), idx, f"{label} s{s} V")
        check_rows(rko, kr[:, L - 1:L], kn_h[s:s + 1], np.array([0]), f"{label} s{s} appended K")
        check_rows(rko, vr[:, L - 1:L], vn_h[s:s + 1], np.array([0]), f"{label} s{s} appended V")
        want = oracle_decode(rko, kr, vr, L, (q_np[s, 0] * np.float32(SCALE)).astype(np.float32))
        errs.append((got[s, 0], want))
    g = np.stack([e[0] for e in errs])
    w = np.stack([e[1] for e in errs])
    assert_close(g, w, what=f"{label} partition_tokens={parts} seqs={list(sample)}")


def test_fullsize_headline(rkv, rko, ctx):
    """Headline: B=64, L=32768 (the step's token appended inside the decode
    launch), Hq 16 / Hkv 2, D 256, 64-token pages in a shuffled pool with 10%
    slack, bf16 q, scale 1/16, device-chosen partitions; 12 of 64 sequences
    checked."""
    torch = _torch()
    B, L = 64, 32768
    print(f"headline B={B} L={L}", flush=True)
    big = Big(rkv, ctx, 1, [L - 1] * B, cap=[L] * B, seed=1)
    for s in range(B):
        big.pool.alloc.reserve(s, L)
    big.pool.sync_tables()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    q = torch.randn((B, 1, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    kn = torch.randn((B, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    vn = torch.randn((B, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    out = torch.empty((B, 1, HQ, D), dtype=torch.float32, device="cuda")
    sample = [0, 5, 11, 17, 23, 29, 35, 41, 47, 53, 59, 63]
    _decode_step_check(rkv, rko, ctx, big, 0, [L] * B, sample, q.float().cpu().numpy(), q, out,
                       (kn, vn), label="headline")
    big.close()


def test_fullsize_config2(rkv, rko, ctx):
    """Config 2: B=16, L ~ U[4096, 16384], 1% of channels x8 in K and V, bf16
    q, device-chosen partitions over the ragged lengths; every sequence
    checked."""
    torch = _torch()
    rng = np.random.default_rng(2)
    lens = [int(x) for x in rng.integers(4096, 16385, 16)]
    print(f"config2 lens={lens}", flush=True)
    big = Big(rkv, ctx, 1, [L - 1 for L in lens], cap=lens, seed=2, outliers=0.01)
    for s, L in enumerate(lens):
        big.pool.alloc.reserve(s, L)
    big.pool.sync_tables()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(22)
    B = len(lens)
    q = torch.randn((B, 1, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    kn = torch.randn((B, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    vn = torch.randn((B, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    out = torch.empty((B, 1, HQ, D), dtype=torch.float32, device="cuda")
    _decode_step_check(rkv, rko, ctx, big, 0, lens, list(range(B)), q.float().cpu().numpy(), q,
                       out, (kn, vn), label="config2")
    big.close()


@pytest.mark.parametrize("partition_tokens", [0, 2048])
def test_fullsize_config3(rkv, rko, ctx, partition_tokens):
    """Config 3: one sequence of 262,145 tokens (the last appended by the
    decode launch, as in bench.py's config 3), Hq 16 / Hkv 2, D 256:
    device-chosen partitions (482 of 544 tokens, the last one 481, merged by
    the one-launch combine) and the reference's partitions of 2048 tokens
    (129, the last one 1 token); all 16 heads checked, for an N(0,1) query
    and one with outlier channels."""
    torch = _torch()
    L = 262145
    print(f"config3 L={L} partition_tokens={partition_tokens}", flush=True)
    big = Big(rkv, ctx, 1, [L - 1], cap=[L], seed=3)
    big.pool.alloc.reserve(0, L)
    big.pool.sync_tables()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(33)
    kn = torch.randn((1, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    vn = torch.randn((1, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
    q0 = torch.randn((1, 1, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    q1 = torch.from_numpy(outlier_q(np.random.default_rng(3), (1, 1, HQ, D))).cuda().to(torch.bfloat16)
    for label, q in (("config3", q0), ("config3 outlier q", q1)):
        out = torch.empty((1, 1, HQ, D), dtype=torch.float32, device="cuda")
        _decode_step_check(rkv, rko, ctx, big, 0, [L], [0], q.float().cpu().numpy(), q, out,
                           (kn, vn), partition_tokens=partition_tokens, label=label,
                           expect_pt=544 if partition_tokens == 0 else None)
    big.close()


def test_fullsize_config5(rkv, rko, ctx):
    """Config 5: B=32, 32,768 committed tokens + 4 draft rows (q_len 4, causal:
    draft row j attends ctx + j + 1 positions), drafts appended inside the
    verify launch; then a seeded accept length a in [0, 4] per sequence rolls
    the rejected rows back (rkv_seq_truncate) and a second verify appends new
    drafts at ctx + a.  Rows j of 16 of the 32 sequences (every other one)
    checked each round."""
    torch = _torch()
    B, C, QL = 32, 32768, 4
    print(f"config5 B={B} ctx={C} q_len={QL}", flush=True)
    big = Big(rkv, ctx, 1, [C] * B, cap=[C + 2 * QL] * B, seed=5)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(55)
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    rows_sid = sid.repeat_interleave(QL)
    acc = np.random.default_rng(5).integers(0, QL + 1, B)
    base = np.full(B, C)
    sample = list(range(0, B, 2))
    for rnd in range(2):
        for s in range(B):
            big.pool.alloc.reserve(s, int(base[s]) + QL)
        big.pool.sync_tables()
        pos = torch.from_numpy((base[:, None] + np.arange(QL)[None, :]).reshape(-1).astype(np.int32)).cuda()
        kn = torch.randn((B * QL, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        vn = torch.randn((B * QL, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        q = torch.randn((B, QL, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
        out = torch.empty((B, QL, HQ, D), dtype=torch.float32, device="cuda")
        app = rkv.append_args(rows_sid, pos, kn, vn)
        run_decode(rkv, big.pool, 0, q, out, sid, int(base.max()) + QL, q_len=QL, app=app)
        ctx.sync()
        got = out.float().cpu().numpy()
        qn = q.float().cpu().numpy()
        kn_h = kn.float().cpu().numpy().reshape(B, QL, HKV, D)
        vn_h = vn.float().cpu().numpy().reshape(B, QL, HKV, D)
        gs, ws = [], []
        for s in sample:
            kr, vr = big.gather(0, s)
            Ls = int(base[s]) + QL
            assert kr.shape[1] == Ls
            check_rows(rko, kr[:, Ls - QL:], kn_h[s], np.arange(QL), f"round {rnd} s{s} drafts K")
            check_rows(rko, vr[:, Ls - QL:], vn_h[s], np.arange(QL), f"round {rnd} s{s} drafts V")
            for j in range(QL):
                qs = (qn[s, j] * np.float32(SCALE)).astype(np.float32)
                ws.append(oracle_decode(rko, kr, vr, Ls - QL + j + 1, qs))
                gs.append(got[s, j])
        assert_close(np.stack(gs), np.stack(ws), what=f"config5 round {rnd} rows of {sample}")
        if rnd == 0:
            # accept a[s] drafts, roll the rest back; the next drafts follow them
            for s in range(B):
                big.pool.alloc.truncate(s, int(base[s] + acc[s]))
            big.pool.sync_tables()
            base = base + acc
            for s in sample:
                kr, _ = big.gather(0, s)
                assert kr.shape[1] == base[s]
    big.close()


def test_fullsize_config4(rkv, rko, ctx):
    """Config 4: B=64 sequences with lognormal lengths (median 8192, sigma 1,
    clipped to [512, 65536]); per step 56 sequences decode one token (appended
    inside the decode launch) and 8 append a 512-row bf16 prefill chunk; 2% of
    the sequences finish per step, free their pages and restart from the free
    list.  Three of the 48 layer pools (the per-layer shape is the config's),
    three steps; each step and layer checks 4 decode sequences' outputs and
    one prefill chunk's rows."""
    torch = _torch()
    rng = np.random.default_rng(4)
    B, NPF, CH, LAYERS, STEPS = 64, 8, 512, 3, 3
    lens = np.clip(np.round(np.exp(rng.normal(math.log(8192), 1.0, B))), 512, 65536).astype(np.int64)
    print(f"config4 sum(L)={int(lens.sum())} max={int(lens.max())}", flush=True)
    cap = [int(L) + STEPS * CH for L in lens]
    big = Big(rkv, ctx, LAYERS, lens, cap=cap, slack=1.25, seed=4)
    fin = np.random.default_rng(44)
    gen_id = np.zeros(B, np.int64)  # restarts draw new rows
    cur = lens.copy()
    for step in range(STEPS):
        pf = [(step * NPF + j) % B for j in range(NPF)]
        dset = [s for s in range(B) if s not in pf]
        for s in range(B):
            if fin.random() < 0.02:
                big.pool.alloc.free(s)
                cur[s] = 0
                gen_id[s] += 1
        for s in dset:
            big.pool.alloc.reserve(s, int(cur[s]) + 1)
        for s in pf:
            big.pool.alloc.reserve(s, int(cur[s]) + CH)
        big.pool.sync_tables()
        ND = len(dset)
        for layer in range(LAYERS):
            # prefill chunks: rows [cur, cur + CH) of the 8 sequences
            for s in pf:
                big.fill(layer, s, int(cur[s]), CH, gen_id=100 + 10 * step + int(gen_id[s]))
            gen = torch.Generator(device="cuda")
            gen.manual_seed(400 + 10 * step + layer)
            q = torch.randn((ND, 1, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
            kn = torch.randn((ND, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
            vn = torch.randn((ND, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
            out = torch.empty((ND, 1, HQ, D), dtype=torch.float32, device="cuda")
            sid = torch.tensor(dset, dtype=torch.int32, device="cuda")
            pos = torch.tensor([int(cur[s]) for s in dset], dtype=torch.int32, device="cuda")
            app = rkv.append_args(sid, pos, kn, vn)
            run_decode(rkv, big.pool, layer, q, out, sid, int(cur[dset].max()) + 1, app=app)
            ctx.sync()
            got = out.float().cpu().numpy()
            qn = q.float().cpu().numpy()
            kn_h, vn_h = kn.float().cpu().numpy(), vn.float().cpu().numpy()
            pick = [int(i) for i in np.random.default_rng(step * 10 + layer).choice(ND, 4, replace=False)]
            gs, ws = [], []
            for i in pick:
                s = dset[i]
                kr, vr = big.gather(layer, s)
                L = int(cur[s]) + 1
                check_rows(rko, kr[:, L - 1:L], kn_h[i:i + 1], np.array([0]), f"step {step} layer {layer} s{s} K")
                check_rows(rko, vr[:, L - 1:L], vn_h[i:i + 1], np.array([0]), f"step {step} layer {layer} s{s} V")
                ws.append(oracle_decode(rko, kr, vr, L, (qn[i, 0] * np.float32(SCALE)).astype(np.float32)))
                gs.append(got[i, 0])
            assert_close(np.stack(gs), np.stack(ws), what=f"config4 step {step} layer {layer}")
            s = pf[step % NPF]
            kr, vr = big.gather(layer, s)
            src_k, src_v = big.rows(layer, s, int(cur[s]), CH, gen_id=100 + 10 * step + int(gen_id[s]))
            idx = np.arange(CH)
            check_rows(rko, kr[:, int(cur[s]):int(cur[s]) + CH], src_k.float().cpu().numpy(), idx,
                       f"step {step} layer {layer} chunk s{s} K")
            check_rows(rko, vr[:, int(cur[s]):int(cur[s]) + CH], src_v.float().cpu().numpy(), idx,
                       f"step {step} layer {layer} chunk s{s} V")
        for s in dset:
            cur[s] += 1
        for s in pf:
            cur[s] += CH
    big.close()
