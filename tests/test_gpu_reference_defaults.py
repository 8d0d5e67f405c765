"""The reference's own default geometries through the drop-in, on the GPU.

  - FlashDecodeParams::default(): 24 q heads / 4 kv heads, seq_len 1024,
    chunk 1024, HEAD_DIM 256 (har-serve/src/attention.rs:17-21, 134-137),
    through the flash_decode_q8.comp entry point with the smoke's inputs;
  - KVGeometry::qwen36_27b: 24 q / 4 kv heads, D 256, 32-token pages,
    context_length 262,144 (har-kv/src/geometry.rs:39-59): one sequence of
    that length, decode (6 rows per kv head), q_len 2 (12 rows) and the
    4-draft verify (24 rows), the step's rows appended inside the launch;
  - ServeConfig::default(): page_size 8, kv_layers 8, kv_heads 4, max_batch 4,
    prefill_chunk 1 (har-serve/src/scheduler.rs:103-120) through rkv_serve_*,
    with 24 q heads and D 256; page records of 8 tokens
    (attach_page_if_boundary, scheduler.rs:1045-1077) share 32-token pool
    pages.

Bars as in test_gpu_parity.py: page bytes bit-exact against the oracle's
Q8_0 encoder; attention max-abs 2e-3 and relative 1e-3 against the oracle's
flash_decode_reference (attention.rs:148-215).
"""
import math
import os

import numpy as np
import pytest

from tests.test_gpu_parity import assert_close, outlier_q

pytestmark = pytest.mark.gpu

HQ, HKV, D = 24, 4, 256
RB = D // 32 * 34
THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS") or 16)))


def _torch():
    import torch
    return torch


def test_flash_decode_default_params(rkv, rko, ctx):
    """FlashDecodeParams::default() (24/4, seq_len 1024, chunk 1024) through
    the shader-ABI entry point: K/V words from the har-serve quantizer over
    lcg values, an f32 query, no softmax scale; the smoke's 1e-3 bar
    (har-serve-vulkan-attn-smoke.rs:169-183) and the parity bars."""
    torch = _torch()
    S = 1024
    k = np.empty((HKV, S, RB), np.uint8)
    v = np.empty_like(k)
    for h in range(HKV):
        for p in range(S):
            k[h, p] = rko.q8_quantize_harserve(rko.lcg_values(D, 1000 + (h * S + p) * 31))
            v[h, p] = rko.q8_quantize_harserve(rko.lcg_values(D, 2000 + (h * S + p) * 17))
    kw, vw = rko.rows_to_words(k), rko.rows_to_words(v)
    query = rko.lcg_values(HQ * D, 3000)
    want = rko.flash_decode_reference(rko.fd_params(HQ, HKV, S, 1024, D), kw, vw, query)
    rp = rkv.FlashDecodeParams(HQ, HKV, S, 1024, D)
    scratch = torch.empty(rkv.flash_decode_scratch_bytes(rp), dtype=torch.uint8, device="cuda")
    out = torch.empty(HQ * D, dtype=torch.float32, device="cuda")
    rkv.flash_decode_q8(ctx, rp, torch.from_numpy(kw.view(np.int32)).cuda(),
                        torch.from_numpy(vw.view(np.int32)).cuda(), torch.from_numpy(query).cuda(),
                        out, scratch)
    ctx.sync()
    got = out.cpu().numpy()
    assert float(np.max(np.abs(got - want))) <= 1e-3
    assert_close(got, want, what="FlashDecodeParams::default()")


# ---- KVGeometry::qwen36_27b at its context length -----------------------------

class _LongSeq:
    """One sequence in a 32-token-page pool, filled through the append kernel
    from seeded bf16 rows (regenerable from (seed, start, n))."""

    PT = 32

    def __init__(self, rkv, ctx, length, cap, seed):
        self.rkv, self.ctx, self.seed = rkv, ctx, seed
        pps = (cap + self.PT - 1) // self.PT
        self.pool = rkv.Pool(ctx, 1, HKV, D, self.PT, int(pps * 1.1) + 8, 1, pps, seed=seed)
        self.g = self.pool.geometry
        self.pool.alloc.reserve(0, length)
        self.pool.sync_tables()
        step = 65536
        for s0 in range(0, length, step):
            self.fill(s0, min(step, length - s0))
        ctx.sync()

    def rows(self, start, n, gen_id=0):
        torch = _torch()
        gen = torch.Generator(device="cuda")
        gen.manual_seed((self.seed * 7919 + start) * 31 + gen_id)
        k = torch.randn((n, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((n, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        return k.contiguous(), v.contiguous()

    def fill(self, start, n):
        torch = _torch()
        k, v = self.rows(start, n)
        sid = torch.zeros(n, dtype=torch.int32, device="cuda")
        pos = torch.arange(start, start + n, dtype=torch.int32, device="cuda")
        self.pool.append(0, sid, pos, k, v)

    def gather(self):
        torch = _torch()
        L = self.pool.alloc.seq_len(0)
        out = []
        for kind in (0, 1):
            t = torch.empty(HKV * L * RB, dtype=torch.uint8, device="cuda")
            self.pool.gather(0, 0, kind, t)
            self.ctx.sync()
            out.append(t.cpu().numpy().reshape(HKV, L, RB))
        return out


def _oracle_rows(rko, kr, vr, L, q_rows):
    """flash_decode_reference over the first L rows; q_rows [n][HQ][D] scaled."""
    kw = rko.rows_to_words(np.ascontiguousarray(kr[:, :L]))
    vw = rko.rows_to_words(np.ascontiguousarray(vr[:, :L]))
    p = rko.fd_params(HQ, HKV, L, 1024, D)
    n = len(q_rows)
    return rko.flash_decode_reference_many(p, [kw] * n, [vw] * n, q_rows, THREADS)


def _check_rows(rko, got_rows, src, what):
    """got_rows [HKV][n][RB] equal the oracle's Q8_0 of src [n][HKV][D]."""
    n = src.shape[0]
    want = rko.q8_encode(np.asarray(src, np.float32).reshape(-1)).reshape(n, HKV, RB)
    got = np.ascontiguousarray(got_rows.transpose(1, 0, 2))
    bad = int(np.sum(np.any(got != want, axis=-1)))
    print(f"[{what}] {n} rows x {HKV} heads bit-exact: {bad == 0}", flush=True)
    assert bad == 0, f"{what}: {bad} of {n * HKV} rows differ"


def test_qwen36_27b_context_length(rkv, rko, ctx):
    """One sequence at KVGeometry::qwen36_27b's context_length (262,144
    tokens), 24 q / 4 kv heads, D 256, 32-token pages in a shuffled pool:
      1. decode of token 262,144 (6 rows per kv head, bf16 N(0,1) query and
         one with outlier channels) with its K/V row appended inside the
         launch, device-chosen partitions;
      2. the same with an f32 query at the reference's 128 partitions
         (2048 tokens, the 64-page cap of 32-token pages);
      3. q_len 2 (12 rows per kv head) over two more appended rows;
      4. the 4-draft verify (24 rows per kv head) over four draft rows, then
         a rollback of two of them (rkv_seq_truncate) and a second verify.
    Every head of every row against the oracle; the appended rows and a
    sample of the filled ones bit-exact."""
    torch = _torch()
    L0 = 262143
    print(f"qwen36_27b geometry: HQ={HQ} HKV={HKV} D={D} page 32, L={L0 + 1}", flush=True)
    big = _LongSeq(rkv, ctx, L0, L0 + 16, seed=36)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2736)
    scale = 1.0 / math.sqrt(D)
    sid = torch.zeros(1, dtype=torch.int32, device="cuda")
    hist_k = {}  # appended rows by position, for the bit-exact checks
    hist_v = {}

    def step(q_len, q, partition_tokens=0, label=""):
        L = big.pool.alloc.seq_len(0)
        big.pool.alloc.reserve(0, L + q_len)
        big.pool.sync_tables()
        kn = torch.randn((q_len, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        vn = torch.randn((q_len, HKV, D), generator=gen, device="cuda").to(torch.bfloat16)
        pos = torch.arange(L, L + q_len, dtype=torch.int32, device="cuda")
        app = rkv.append_args(sid.repeat_interleave(q_len), pos, kn, vn)
        out = torch.empty((1, q_len, HQ, D), dtype=torch.float32, device="cuda")
        a = rkv.decode_args(q, out, sid, scale, L + q_len, q_len=q_len,
                            partition_tokens=partition_tokens, append=app)
        ws = torch.empty(max(rkv.decode_workspace_bytes(big.g, a), 4), dtype=torch.uint8,
                         device="cuda")
        a = rkv.decode_args(q, out, sid, scale, L + q_len, q_len=q_len,
                            partition_tokens=partition_tokens, workspace=ws, append=app)
        big.pool.decode(0, a)
        ctx.sync()
        parts = int(ws[:4].view(torch.int32).item()) if partition_tokens == 0 else partition_tokens
        for j in range(q_len):
            hist_k[L + j] = kn[j].float().cpu().numpy()
            hist_v[L + j] = vn[j].float().cpu().numpy()
        kr, vr = big.gather()
        new = np.arange(L, L + q_len)
        _check_rows(rko, kr[:, new], np.stack([hist_k[p] for p in new]), f"{label} appended K")
        _check_rows(rko, vr[:, new], np.stack([hist_v[p] for p in new]), f"{label} appended V")
        qn = q.float().cpu().numpy()[0]
        want = np.stack([_oracle_rows(rko, kr, vr, L + j + 1,
                                      (qn[j] * np.float32(scale))[None])[0]
                         for j in range(q_len)])
        assert_close(out.cpu().numpy()[0], want,
                     what=f"{label} q_len={q_len} partition_tokens={parts}")
        return kr, vr

    # 1. decode, bf16 query, N(0,1) and outlier channels
    q = torch.randn((1, 1, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    kr, vr = step(1, q, label="decode bf16 q")
    # a sample of the filled rows, bit-exact
    idx = np.unique(np.random.default_rng(36).integers(0, L0, 256))
    src_k = []
    src_v = []
    for s0 in range(0, L0, 65536):  # regenerate each filled chunk once
        pick = idx[(idx >= s0) & (idx < s0 + 65536)] - s0
        k, v = big.rows(s0, min(65536, L0 - s0))
        sel = torch.from_numpy(pick).cuda()
        src_k.append(k[sel].float().cpu().numpy())
        src_v.append(v[sel].float().cpu().numpy())
    _check_rows(rko, kr[:, idx], np.concatenate(src_k), "filled K")
    _check_rows(rko, vr[:, idx], np.concatenate(src_v), "filled V")
    del kr, vr
    big.pool.alloc.truncate(0, L0)  # the same position again, other inputs
    qo = torch.from_numpy(outlier_q(np.random.default_rng(27), (1, 1, HQ, D))).cuda()
    step(1, qo.to(torch.bfloat16), label="decode outlier bf16 q")
    # 2. f32 query at the reference's 128 partitions
    big.pool.alloc.truncate(0, L0)
    step(1, qo, partition_tokens=2048, label="decode f32 q, 128 partitions")
    # 3. q_len 2 after the decode's token
    q2 = torch.randn((1, 2, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    step(2, q2, label="q_len 2")
    # 4. verify with 4 drafts, roll two back, verify again
    q4 = torch.randn((1, 4, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
    step(4, q4, label="verify")
    L = big.pool.alloc.seq_len(0)
    big.pool.alloc.truncate(0, L - 2)
    big.pool.sync_tables()
    q4b = torch.from_numpy(outlier_q(np.random.default_rng(28), (1, 4, HQ, D))).cuda()
    step(4, q4b.to(torch.bfloat16), label="verify after rollback")
    big.pool.close()


# ---- ServeConfig::default() through the serving adapter ------------------------

def test_serve_default_config(rkv, rko, ctx):
    """ServeConfig::default(): 8 layers, 4 kv heads, page_size 8, max_batch 4,
    prefill_chunk 1, with FlashDecodeParams::default()'s 24 q heads and
    HEAD_DIM 256.  Four requests arrive over the steps; prefill consumes one
    token per step per prefilling request (prefill_chunk 1), one request
    prefills a longer chunk, one forks a live prefix that ends inside a
    record (35 tokens), one rolls back and one finishes.  Every row of every layer
    against the oracle's flash_decode_reference over that sequence's own
    rows; page records of 8 tokens name the pool page and slots of their
    tokens, and records of one 32-token pool page name the same page."""
    torch = _torch()
    layers, PS, maxb = 8, 8, 4
    scale = 1.0 / math.sqrt(D)
    sv = rkv.Serve(ctx, layers, HKV, D, PS, num_pages=512, max_seqs=maxb + 2,
                   max_pages_per_seq=96, q_heads=HQ, max_decode=maxb, max_prefill_rows=64,
                   seed=8)
    assert sv.geometry.page_tokens == 32 and sv.geometry.num_pages == 128
    rng = np.random.default_rng(81)
    hist = {}  # id -> [layer] -> (K rows, V rows)

    def attend(sid, layer, length, q):
        K, V = hist[sid][layer]

        def words(x):
            enc = np.stack([rko.q8_encode(x[:length, h, :].reshape(-1)).reshape(length, -1)
                            for h in range(HKV)])
            return rko.rows_to_words(enc)
        p = rko.fd_params(HQ, HKV, length, 1024, D)
        return rko.flash_decode_reference(p, words(K), words(V), (q * np.float32(scale)).reshape(-1))

    # (prefill entries (id, tokens[, fork_len, parent]), decode ids, after)
    script = [
        ([(1, 1), (2, 1)], [], []),
        ([(1, 1), (2, 1), (3, 37)], [], []),          # 3 prefills a 37-token chunk
        ([(1, 1), (2, 1)], [3], []),
        ([(4, 1, 35, 3)], [1, 2, 3], []),             # 4 forks 3's first 35 tokens
        ([], [1, 2, 3, 4], [("truncate", 3, 36)]),
        ([], [1, 2, 3, 4], [("finish", 2)]),
        ([(5, 9)], [1, 3, 4], []),
        ([], [1, 3, 4, 5], []),
    ]
    for step, (pre, dec, after) in enumerate(script):
        for e in pre:
            if e[0] not in hist:
                if len(e) > 2:
                    hist[e[0]] = [(k[:e[2]].copy(), v[:e[2]].copy()) for k, v in hist[e[3]]]
                else:
                    z = np.zeros((0, HKV, D), np.float32)
                    hist[e[0]] = [(z, z) for _ in range(layers)]
        ctx_len = {e[0]: len(hist[e[0]][0][0]) for e in pre}
        ctx_len.update({sid: len(hist[sid][0][0]) for sid in dec})
        sv.begin_step(prefill=pre, decode=[(sid, 1) for sid in dec])
        n_pf = sum(e[1] for e in pre)
        for layer in range(layers):
            qp = rng.standard_normal((n_pf, HQ, D)).astype(np.float32)
            kp = rng.standard_normal((n_pf, HKV, D)).astype(np.float32)
            vp = rng.standard_normal((n_pf, HKV, D)).astype(np.float32)
            qd = rng.standard_normal((len(dec), HQ, D)).astype(np.float32)
            kd = rng.standard_normal((len(dec), HKV, D)).astype(np.float32)
            vd = rng.standard_normal((len(dec), HKV, D)).astype(np.float32)
            bf = torch.bfloat16
            qp, kp, vp, qd, kd, vd = (torch.from_numpy(x).to(bf).float().numpy()
                                      for x in (qp, kp, vp, qd, kd, vd))
            op = torch.empty((max(n_pf, 1), HQ, D), dtype=torch.float32, device="cuda")
            od = torch.empty((max(len(dec), 1), HQ, D), dtype=torch.float32, device="cuda")
            if n_pf:
                sv.prefill(layer, torch.from_numpy(qp).cuda().to(bf),
                           torch.from_numpy(kp).cuda().to(bf), torch.from_numpy(vp).cuda().to(bf),
                           op, scale)
            if dec:
                sv.decode(layer, torch.from_numpy(qd).cuda().to(bf),
                          torch.from_numpy(kd).cuda().to(bf), torch.from_numpy(vd).cuda().to(bf),
                          od, scale)
            ctx.sync()
            off = 0
            for e in pre:
                sid, n = e[0], e[1]
                K, V = hist[sid][layer]
                hist[sid][layer] = (np.concatenate([K, kp[off:off + n]]),
                                    np.concatenate([V, vp[off:off + n]]))
                got = op[off:off + n].cpu().numpy()
                want = np.stack([attend(sid, layer, ctx_len[sid] + j + 1, qp[off + j])
                                 for j in range(n)])
                assert_close(got.reshape(n, -1), want,
                             what=f"step {step} layer {layer} prefill id {sid} ({n} rows)")
                off += n
            got = od.cpu().numpy()
            for b, sid in enumerate(dec):
                K, V = hist[sid][layer]
                hist[sid][layer] = (np.concatenate([K, kd[b:b + 1]]),
                                    np.concatenate([V, vd[b:b + 1]]))
                want = attend(sid, layer, ctx_len[sid] + 1, qd[b])
                assert_close(got[b].reshape(-1), want,
                             what=f"step {step} layer {layer} decode id {sid}")
        # page records: one per started 8 tokens, slot (o % 4) * 8 of pool page o // 4
        pb = rkv.page_bytes(sv.geometry)
        for sid in hist:
            L = sv.seq_len(sid)
            assert L == len(hist[sid][0][0])
            locs = [sv.page_location(sid, o) for o in range((L + PS - 1) // PS)]
            for o, loc in enumerate(locs):
                assert loc.first_slot == (o % 4) * PS and loc.slots == PS
                assert loc.offset == loc.page * pb and loc.length == pb
                assert loc.layer_stride == sv.geometry.num_pages * pb and loc.generation >= 1
                assert loc.page == locs[o - o % 4].page
            with pytest.raises(rkv.RkvError):
                sv.page_location(sid, (L + PS - 1) // PS)
        if step == 3:
            # the fork shares 3's first pool page (records 0-3); the page of
            # record 4 (tokens 32..39, the prefix ends at 35) was copied on
            # write when 4 grew into it
            for o in range(4):
                assert sv.page_location(4, o).page == sv.page_location(3, o).page
            assert sv.page_location(4, 4).page != sv.page_location(3, 4).page
        for act in after:
            if act[0] == "finish":
                sv.finish(act[1])
                del hist[act[1]]
            else:
                sv.truncate(act[1], act[2])
                hist[act[1]] = [(k[:act[2]], v[:act[2]]) for k, v in hist[act[1]]]
    # the pool's bytes of every live sequence: the oracle's encoding of its rows
    for sid in hist:
        L = sv.seq_len(sid)
        for layer in (0, layers - 1):
            for kind in (0, 1):
                t = torch.empty(HKV * L * RB, dtype=torch.uint8, device="cuda")
                sv.gather(layer, sv.slot(sid), kind, t)
                ctx.sync()
                rows = t.cpu().numpy().reshape(HKV, L, RB)
                _check_rows(rko, rows, hist[sid][layer][kind], f"id {sid} layer {layer} kind {kind}")
    sv.close()
