"""The serving adapter (rkv_serve_*) driven the way ServeScheduler::step
drives a BatchStepModel (har-serve/src/scheduler.rs:603-960): per step,
chunked prefill entries and one-token decode rows, per layer, with requests
arriving, forking a cached prefix, finishing and rolling back.  Every
attention row is checked against the oracle's flash_decode_reference
(attention.rs:148-165) over that sequence's own rows, at the parity bars of
test_gpu_parity.py; page locations follow the block tables, prefix sharing
and page reuse (har-kv/src/page.rs:100-115)."""
import math

import numpy as np
import pytest

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


class _Model:
    """Host history of every live sequence's K/V rows per layer, and the
    oracle's attention over it."""

    def __init__(self, rko, layers, Hkv, Hq, D):
        self.rko, self.layers, self.Hkv, self.Hq, self.D = rko, layers, Hkv, Hq, D
        self.rows = {}  # id -> [layer] -> (K rows [L][Hkv][D], V rows)

    def admit(self, sid, parent=None, fork_len=0):
        if parent is None:
            z = np.zeros((0, self.Hkv, self.D), np.float32)
            self.rows[sid] = [(z, z) for _ in range(self.layers)]
        else:
            self.rows[sid] = [(k[:fork_len].copy(), v[:fork_len].copy())
                              for k, v in self.rows[parent]]

    def append(self, sid, layer, k, v):
        K, V = self.rows[sid][layer]
        self.rows[sid][layer] = (np.concatenate([K, k]), np.concatenate([V, v]))

    def truncate(self, sid, n):
        self.rows[sid] = [(k[:n], v[:n]) for k, v in self.rows[sid]]

    def attend(self, sid, layer, length, q, scale):
        """flash_decode_reference over the first `length` rows of sid."""
        rko = self.rko
        K, V = self.rows[sid][layer]

        def words(x):
            enc = np.stack([rko.q8_encode(x[:length, h, :].reshape(-1)).reshape(length, -1)
                            for h in range(self.Hkv)])
            return rko.rows_to_words(enc)
        p = rko.fd_params(self.Hq, self.Hkv, length, 1024, self.D)
        return rko.flash_decode_reference(p, words(K), words(V),
                                          (q * np.float32(scale)).reshape(-1))


@pytest.mark.parametrize("D,Hkv,Hq,PT", [(256, 2, 16, 64), (128, 2, 8, 16)])
def test_serve_steps_match_oracle(rkv, rko, ctx, D, Hkv, Hq, PT):
    torch = __import__("torch")
    layers = 2
    scale = 1.0 / math.sqrt(D)
    sv = rkv.Serve(ctx, layers, Hkv, D, PT, num_pages=96, max_seqs=6,
                   max_pages_per_seq=512 // PT + 2, q_heads=Hq, max_decode=6,
                   max_prefill_rows=256, seed=7)
    m = _Model(rko, layers, Hkv, Hq, D)
    rng = np.random.default_rng(D + PT)
    # (prefill entries, decode ids, actions after the step)
    script = [
        ([(11, 128), (12, 77)], [], []),
        ([(11, 128)], [12], []),
        ([(11, 44)], [12], []),
        ([(13, 40, 256, 11)], [11, 12], []),            # 13 forks 11's first 256 tokens
        ([], [11, 12, 13], [("finish", 12)]),
        ([(14, 90)], [11, 13], [("truncate", 13, 290)]),  # 14 reuses 12's pages; 13 rolls back
        ([(15, 3, 200, 11)], [11, 13, 14], []),           # 15 forks inside a page of 11
        ([], [11, 13, 14, 15], [("finish", 11)]),
        ([], [13, 14, 15], []),
    ]
    gens_of_12 = None
    for step, (pre, dec, after) in enumerate(script):
        for e in pre:
            if e[0] not in m.rows:
                m.admit(e[0], *(e[3], e[2]) if len(e) > 2 else ())
        ctx_len = {e[0]: len(m.rows[e[0]][0][0]) for e in pre}
        ctx_len.update({sid: len(m.rows[sid][0][0]) for sid in dec})
        if step == 5:  # 14 is admitted on 12's freed pages
            gens_of_12 = {p: sv.alloc.page_generation(p) for p in freed_12}
        sv.begin_step(prefill=pre, decode=[(sid, 1) for sid in dec])
        n_pf = sum(e[1] for e in pre)
        for layer in range(layers):
            qp = rng.standard_normal((n_pf, Hq, D)).astype(np.float32)
            kp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
            vp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
            qd = rng.standard_normal((len(dec), Hq, D)).astype(np.float32)
            kd = rng.standard_normal((len(dec), Hkv, D)).astype(np.float32)
            vd = rng.standard_normal((len(dec), Hkv, D)).astype(np.float32)
            op = torch.empty((max(n_pf, 1), Hq, D), dtype=torch.float32, device="cuda")
            od = torch.empty((max(len(dec), 1), Hq, D), dtype=torch.float32, device="cuda")
            if n_pf:
                sv.prefill(layer, torch.from_numpy(qp).cuda(), torch.from_numpy(kp).cuda(),
                           torch.from_numpy(vp).cuda(), op, scale)
            if dec:
                sv.decode(layer, torch.from_numpy(qd).cuda(), torch.from_numpy(kd).cuda(),
                          torch.from_numpy(vd).cuda(), od, scale)
            ctx.sync()
            off = 0
            for e in pre:
                sid, n = e[0], e[1]
                m.append(sid, layer, kp[off:off + n], vp[off:off + n])
                got = op[off:off + n].cpu().numpy()
                for j in range(n):
                    want = m.attend(sid, layer, ctx_len[sid] + j + 1, qp[off + j], scale)
                    assert_close(got[j].reshape(-1), want,
                                 what=f"step {step} layer {layer} prefill id {sid} row {j}")
                off += n
            got = od.cpu().numpy()
            for b, sid in enumerate(dec):
                m.append(sid, layer, kd[b:b + 1], vd[b:b + 1])
                want = m.attend(sid, layer, ctx_len[sid] + 1, qd[b], scale)
                assert_close(got[b].reshape(-1), want,
                             what=f"step {step} layer {layer} decode id {sid}")
        for sid in m.rows:
            assert sv.seq_len(sid) == len(m.rows[sid][0][0])
        # page locations: consistent with the geometry; forks share their prefix
        pb = rkv.page_bytes(sv.geometry)
        for sid in m.rows:
            L = sv.seq_len(sid)
            for o in range((L + PT - 1) // PT):
                loc = sv.page_location(sid, o)
                assert loc.offset == loc.page * pb and loc.length == pb
                assert loc.layer_stride == sv.geometry.num_pages * pb and loc.generation >= 1
        if 13 in m.rows and 11 in m.rows:
            for o in range(256 // PT):
                assert sv.page_location(13, o).page == sv.page_location(11, o).page
        for act in after:
            if act[0] == "finish":
                if act[1] == 12:
                    freed_12 = [sv.page_location(12, o).page
                                for o in range((sv.seq_len(12) + PT - 1) // PT)]
                sv.finish(act[1])
                del m.rows[act[1]]
                with pytest.raises(rkv.RkvError):
                    sv.seq_len(act[1])
            else:
                sv.truncate(act[1], act[2])
                m.truncate(act[1], act[2])
        if step == 5:
            # 14 took pages 12 freed: each came back one generation later
            reused = [sv.page_location(14, o) for o in range((90 + PT - 1) // PT)]
            hit = [loc for loc in reused if loc.page in gens_of_12]
            assert hit and all(loc.generation == gens_of_12[loc.page] + 1 for loc in hit)
    sv.close()


def test_serve_refusals_change_nothing(rkv, ctx):
    """Steps the adapter refuses -- out of pages, a repeated id, a decode row
    of two tokens, an unknown fork parent, too many prefill rows -- leave
    every sequence and the set of live ids as they were."""
    D, Hkv, Hq, PT = 128, 2, 8, 16
    sv = rkv.Serve(ctx, 1, Hkv, D, PT, num_pages=10, max_seqs=4, max_pages_per_seq=16,
                   q_heads=Hq, max_decode=4, max_prefill_rows=200, seed=1)
    sv.begin_step(prefill=[(1, 100), (2, 40)])           # 7 + 3 pages: the pool is full
    assert sv.alloc.free_pages() == 0
    bad = [
        dict(prefill=[(3, 10)], decode=[(1, 1)]),          # out of pages (3 is new)
        dict(decode=[(1, 1), (1, 1)]),                      # repeated id
        dict(decode=[(2, 2)]),                              # decode row of two tokens
        dict(prefill=[(5, 4, 8, 99)]),                      # unknown fork parent
        dict(prefill=[(1, 150), (2, 60)]),                  # more rows than max_prefill_rows
    ]
    for kw in bad:
        with pytest.raises(rkv.RkvError):
            sv.begin_step(**kw)
        assert sv.seq_len(1) == 100 and sv.seq_len(2) == 40
        with pytest.raises(rkv.RkvError):
            sv.seq_len(3)
        assert sv.alloc.free_pages() == 0
    # after a finish the same out-of-pages step fits
    sv.finish(2)
    sv.begin_step(prefill=[(3, 10)], decode=[(1, 1)])
    assert sv.seq_len(3) == 10 and sv.seq_len(1) == 101
    sv.close()


def test_serve_long_context_chunk_splits(rkv, rko, ctx):
    """A short chunk after a long cached prompt has too few row blocks to
    fill the chip, so the adapter's prefill splits its causal ranges (the
    plan asks for a workspace); its rows still match the oracle."""
    torch = __import__("torch")
    D, Hkv, Hq, PT = 128, 2, 16, 64
    sv = rkv.Serve(ctx, 1, Hkv, D, PT, num_pages=80, max_seqs=2, max_pages_per_seq=70,
                   q_heads=Hq, max_decode=2, max_prefill_rows=1024, seed=2)
    m = _Model(rko, 1, Hkv, Hq, D)
    m.admit(1)
    rng = np.random.default_rng(31)
    scale = 1.0 / math.sqrt(D)
    for chunk in (1000, 1000, 1000, 64):
        done = len(m.rows[1][0][0])
        sv.begin_step(prefill=[(1, chunk)])
        q = rng.standard_normal((chunk, Hq, D)).astype(np.float32)
        k = rng.standard_normal((chunk, Hkv, D)).astype(np.float32)
        v = rng.standard_normal((chunk, Hkv, D)).astype(np.float32)
        out = torch.empty((chunk, Hq, D), dtype=torch.float32, device="cuda")
        sv.prefill(0, torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                   torch.from_numpy(v).cuda(), out, scale)
        ctx.sync()
        m.append(1, 0, k, v)
        got = out.cpu().numpy()
        for j in (0, chunk // 2, chunk - 1):
            want = m.attend(1, 0, done + j + 1, q[j], scale)
            assert_close(got[j].reshape(-1), want, what=f"ctx {done} chunk {chunk} row {j}")
    # the last call's plan: 4 row blocks x 2 kv heads over 256 CUs is split
    qt = torch.empty((64, Hq, D))
    a = rkv.prefill_args([0], [3000], [64], qt, qt, scale)
    assert rkv.prefill_workspace_bytes(sv.geometry, a) > 0
    sv.close()


def test_serve_steps_alternate_streams(rkv, rko, ctx):
    """Consecutive steps on two streams with no host synchronization between
    them: each step's row layout is uploaded only after the previous step's
    launches on the other stream are done with it, so every decode row still
    matches the oracle."""
    torch = __import__("torch")
    D, Hkv, Hq, PT, ctx_len, n_seq, steps = 256, 2, 16, 64, 2048, 4, 6
    scale = 1.0 / math.sqrt(D)
    sv = rkv.Serve(ctx, 1, Hkv, D, PT, num_pages=n_seq * (ctx_len // PT + 2) + 8, max_seqs=n_seq,
                   max_pages_per_seq=ctx_len // PT + 2, q_heads=Hq, max_decode=n_seq,
                   max_prefill_rows=n_seq * ctx_len, seed=3)
    m = _Model(rko, 1, Hkv, Hq, D)
    rng = np.random.default_rng(11)
    ids = list(range(21, 21 + n_seq))
    for sid in ids:
        m.admit(sid)
    n_pf = n_seq * ctx_len
    kp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
    vp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
    qp = rng.standard_normal((n_pf, Hq, D)).astype(np.float32)
    op = torch.empty((n_pf, Hq, D), dtype=torch.float32, device="cuda")
    sv.begin_step(prefill=[(sid, ctx_len) for sid in ids], decode=[])
    sv.prefill(0, torch.from_numpy(qp).cuda(), torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(),
               op, scale)
    ctx.sync()
    for i, sid in enumerate(ids):
        m.append(sid, 0, kp[i * ctx_len:(i + 1) * ctx_len], vp[i * ctx_len:(i + 1) * ctx_len])
    # every step's inputs and outputs staged before the timed-free loop
    qd = [rng.standard_normal((n_seq, Hq, D)).astype(np.float32) for _ in range(steps)]
    kd = [rng.standard_normal((n_seq, Hkv, D)).astype(np.float32) for _ in range(steps)]
    vd = [rng.standard_normal((n_seq, Hkv, D)).astype(np.float32) for _ in range(steps)]
    dq = [torch.from_numpy(x).cuda() for x in qd]
    dk = [torch.from_numpy(x).cuda() for x in kd]
    dv = [torch.from_numpy(x).cuda() for x in vd]
    od = [torch.zeros((n_seq, Hq, D), dtype=torch.float32, device="cuda") for _ in range(steps)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    print(f"serve: {steps} decode steps alternating two streams, {n_seq} x {ctx_len} tokens", flush=True)
    for step in range(steps):
        st = streams[step % 2]
        sv.begin_step(prefill=[], decode=[(sid, 1) for sid in ids], stream=st)
        sv.decode(0, dq[step], dk[step], dv[step], od[step], scale, stream=st)
    torch.cuda.synchronize()
    for step in range(steps):
        got = od[step].cpu().numpy()
        for b, sid in enumerate(ids):
            m.append(sid, 0, kd[step][b:b + 1], vd[step][b:b + 1])
            want = m.attend(sid, 0, ctx_len + step + 1, qd[step][b], scale)
            assert_close(got[b].reshape(-1), want, what=f"step {step} id {sid}")
    sv.close()


def test_serve_steps_on_released_streams(rkv, rko, ctx):
    """Every step on a stream of its own that the caller releases from the
    pool (rkv_pool_release_stream) and destroys right after queueing the
    step, with no host synchronization: the next step's calls wait for the
    released stream's work through the mark the release recorded, never
    touching the destroyed handle, and every decode row matches the oracle."""
    import ctypes
    import os
    torch = __import__("torch")
    # the HIP runtime torch loaded (the one librkv.so is bound to)
    hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
    D, Hkv, Hq, PT, ctx_len, n_seq, steps = 128, 2, 16, 32, 700, 3, 5
    scale = 1.0 / math.sqrt(D)
    sv = rkv.Serve(ctx, 1, Hkv, D, PT, num_pages=n_seq * (ctx_len // PT + 3) + 8, max_seqs=n_seq,
                   max_pages_per_seq=ctx_len // PT + 3, q_heads=Hq, max_decode=n_seq,
                   max_prefill_rows=n_seq * ctx_len, seed=4)
    m = _Model(rko, 1, Hkv, Hq, D)
    rng = np.random.default_rng(12)
    ids = list(range(31, 31 + n_seq))
    for sid in ids:
        m.admit(sid)
    n_pf = n_seq * ctx_len
    kp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
    vp = rng.standard_normal((n_pf, Hkv, D)).astype(np.float32)
    qp = rng.standard_normal((n_pf, Hq, D)).astype(np.float32)
    op = torch.empty((n_pf, Hq, D), dtype=torch.float32, device="cuda")
    sv.begin_step(prefill=[(sid, ctx_len) for sid in ids], decode=[])
    sv.prefill(0, torch.from_numpy(qp).cuda(), torch.from_numpy(kp).cuda(),
               torch.from_numpy(vp).cuda(), op, scale)
    ctx.sync()
    for i, sid in enumerate(ids):
        m.append(sid, 0, kp[i * ctx_len:(i + 1) * ctx_len], vp[i * ctx_len:(i + 1) * ctx_len])
    qd = [rng.standard_normal((n_seq, Hq, D)).astype(np.float32) for _ in range(steps)]
    kd = [rng.standard_normal((n_seq, Hkv, D)).astype(np.float32) for _ in range(steps)]
    vd = [rng.standard_normal((n_seq, Hkv, D)).astype(np.float32) for _ in range(steps)]
    dq = [torch.from_numpy(x).cuda() for x in qd]
    dk = [torch.from_numpy(x).cuda() for x in kd]
    dv = [torch.from_numpy(x).cuda() for x in vd]
    od = [torch.zeros((n_seq, Hq, D), dtype=torch.float32, device="cuda") for _ in range(steps)]
    torch.cuda.synchronize()
    print(f"serve: {steps} decode steps, each on a stream released and destroyed after it",
          flush=True)
    for step in range(steps):
        st = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(st)) == 0
        sv.begin_step(prefill=[], decode=[(sid, 1) for sid in ids], stream=st.value)
        sv.decode(0, dq[step], dk[step], dv[step], od[step], scale, stream=st.value)
        sv.release_stream(st.value)
        assert hip.hipStreamDestroy(st) == 0
    torch.cuda.synchronize()
    ctx.sync()
    for step in range(steps):
        got = od[step].cpu().numpy()
        for b, sid in enumerate(ids):
            m.append(sid, 0, kd[step][b:b + 1], vd[step][b:b + 1])
            want = m.attend(sid, 0, ctx_len + step + 1, qd[step][b], scale)
            assert_close(got[b].reshape(-1), want, what=f"step {step} id {sid}")
    sv.close()
