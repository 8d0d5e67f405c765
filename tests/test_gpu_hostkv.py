"""Pools whose pages live in pinned host memory (RKV_PAGES_HOST), the
reference's host-KV tier (research/host-kv/README.md:1-24: fetch a host KV
block once, stage it, serve every query row of the block from that one
fetch).  The same kernels run on the mapped host pages, except that the
decode stages K through LDS with V (three-stage ring) instead of loading it
into registers: every byte they store must equal the HBM pool's, prefill
outputs must equal the HBM pool's bit for bit, and every output must match
the oracle's flash_decode_reference (attention.rs:148-165) at the parity
bars of test_gpu_parity.py."""
import numpy as np
import pytest

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


def _attend(rko, kb, vb, Hq, Hkv, D, length, q, scale):
    """flash_decode_reference over the first `length` gathered rows;
    kb/vb: uint8 [Hkv][L][row bytes]."""
    kw = rko.rows_to_words(np.ascontiguousarray(kb[:, :length]))
    vw = rko.rows_to_words(np.ascontiguousarray(vb[:, :length]))
    p = rko.fd_params(Hq, Hkv, length, 1024, D)
    return rko.flash_decode_reference(p, kw, vw, (q * np.float32(scale)).reshape(-1))


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens", [
    (16, 2, 256, 64, [300, 77, 1000]),
    (8, 2, 128, 16, [129, 40, 513]),
])
def test_host_pool_matches_device_pool(rkv, rko, ctx, Hq, Hkv, D, PT, lens):
    torch = __import__("torch")
    rng = np.random.default_rng(D + PT)
    B = len(lens)
    W = max(lens) // PT + 2
    pools = [rkv.Pool(ctx, 1, Hkv, D, PT, B * W + 4, B, W, seed=9, page_memory=m)
             for m in (rkv.PAGES_DEVICE, rkv.PAGES_HOST)]
    rows = [rng.standard_normal((L, Hkv, D)).astype(np.float32) for L in lens]
    for pool in pools:
        for s, L in enumerate(lens):
            pool.alloc.reserve(s, L)
        pool.sync_tables()
        for s, r in enumerate(rows):
            kv = torch.from_numpy(r).cuda()
            pool.append(0, torch.full((len(r),), s, dtype=torch.int32, device="cuda"),
                        torch.arange(len(r), dtype=torch.int32, device="cuda"), kv, kv * 0.5)
    ctx.sync()
    rb = rkv.row_bytes(D)
    # stored bytes: equal across placements and to the oracle's encoder
    kbytes, vbytes = [], []
    for s, L in enumerate(lens):
        got = []
        for pool in pools:
            k = torch.empty(Hkv * L * rb, dtype=torch.uint8, device="cuda")
            v = torch.empty_like(k)
            pool.gather(0, s, 0, k)
            pool.gather(0, s, 1, v)
            ctx.sync()
            got.append((k.cpu().numpy().reshape(Hkv, L, rb), v.cpu().numpy().reshape(Hkv, L, rb)))
        assert np.array_equal(got[0][0], got[1][0]) and np.array_equal(got[0][1], got[1][1])
        for h in range(Hkv):
            want = rko.q8_encode(rows[s][:, h, :].reshape(-1)).reshape(L, rb)
            assert np.array_equal(got[1][0][h], want), f"seq {s} head {h}: host-pool K bytes"
        kbytes.append(got[1][0])
        vbytes.append(got[1][1])
    scale = 1.0 / np.sqrt(D)
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    for q_len in (1, 2, 4):
        q = rng.standard_normal((B, q_len, Hq, D)).astype(np.float32)
        qd = torch.from_numpy(q).cuda()
        outs = []
        for pool in pools:
            o = torch.empty(q.shape, dtype=torch.float32, device="cuda")
            a = rkv.decode_args(qd, o, sid, scale, W * PT, q_len=q_len)
            ws = torch.empty(max(rkv.decode_workspace_bytes(pool.geometry, a), 4),
                             dtype=torch.uint8, device="cuda")
            pool.decode(0, rkv.decode_args(qd, o, sid, scale, W * PT, q_len=q_len, workspace=ws))
            ctx.sync()
            outs.append(o.cpu().numpy())
        # the ring depth changes the partition plan, so the pools agree to the bars
        assert_close(outs[1], outs[0], what=f"q_len {q_len}: host pool vs HBM pool")
        for b, L in enumerate(lens):
            for j in range(q_len):
                want = _attend(rko, kbytes[b], vbytes[b], Hq, Hkv, D, L - q_len + j + 1,
                               q[b, j], scale)
                assert_close(outs[1][b, j].reshape(-1), want,
                             what=f"host pool q_len {q_len} seq {b} row {j}")
    # chunked prefill over the host pages: the last 70 rows of every sequence
    n = [min(70, L) for L in lens]
    qp = rng.standard_normal((sum(n), Hq, D)).astype(np.float32)
    qpd = torch.from_numpy(qp).cuda()
    outs = []
    for pool in pools:
        o = torch.empty(qp.shape, dtype=torch.float32, device="cuda")
        pool.prefill(0, rkv.prefill_args(list(range(B)), [L - k for L, k in zip(lens, n)], n,
                                         qpd, o, scale))
        ctx.sync()
        outs.append(o.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]), "prefill: host pool differs from HBM pool"
    off = 0
    for b, (L, k) in enumerate(zip(lens, n)):
        for j in (0, k - 1):
            want = _attend(rko, kbytes[b], vbytes[b], Hq, Hkv, D, L - k + j + 1, qp[off + j], scale)
            assert_close(outs[1][off + j].reshape(-1), want, what=f"host pool prefill seq {b} row {j}")
        off += k
    # a bf16 query with the workspace each pool asks for: the HBM pool's also
    # holds every tile widened once, the host pool's only the split partials
    qb = qpd.to(torch.bfloat16)
    qb_h = qb.float().cpu().numpy()
    cols = (list(range(B)), [L - k for L, k in zip(lens, n)], n)
    need = [pool.prefill_workspace_bytes(rkv.prefill_args(*cols, qb, torch.zeros_like(qpd), scale))
            for pool in pools]
    partials = [pool.prefill_workspace_bytes(rkv.prefill_args(*cols, qpd, torch.zeros_like(qpd),
                                                              scale)) for pool in pools]
    assert need[0] > partials[0] and need[1] == partials[1], (need, partials)
    outs = []
    for pool, nb in zip(pools, need):
        o = torch.empty(qp.shape, dtype=torch.float32, device="cuda")
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        pool.prefill(0, rkv.prefill_args(*cols, qb, o, scale, workspace=ws))
        ctx.sync()
        outs.append(o.cpu().numpy())
    assert_close(outs[1], outs[0], what="bf16 q prefill: host pool vs HBM pool")
    off = 0
    for b, (L, k) in enumerate(zip(lens, n)):
        for j in (0, k - 1):
            want = _attend(rko, kbytes[b], vbytes[b], Hq, Hkv, D, L - k + j + 1, qb_h[off + j], scale)
            assert_close(outs[1][off + j].reshape(-1), want,
                         what=f"host pool bf16 q prefill seq {b} row {j}")
        off += k
    for pool in pools:
        pool.close()


def test_host_serve_steps_match_device(rkv, ctx):
    """The serving adapter on host pages: a short script of steps (prefill,
    fork of a cached prefix, decode, rollback, finish) gives the HBM
    adapter's prefill outputs bit for bit and its decode outputs to the
    parity bars (the HBM adapter is checked against the oracle in
    test_gpu_serve.py)."""
    torch = __import__("torch")
    D, Hkv, Hq, PT, layers = 128, 2, 8, 16, 2
    svs = [rkv.Serve(ctx, layers, Hkv, D, PT, num_pages=80, max_seqs=4, max_pages_per_seq=40,
                     q_heads=Hq, max_decode=4, max_prefill_rows=256, seed=3, page_memory=m)
           for m in (rkv.PAGES_DEVICE, rkv.PAGES_HOST)]
    rng = np.random.default_rng(5)
    script = [([(1, 200), (2, 33)], [], None), ([(3, 20, 160, 1)], [1, 2], None),
              ([], [1, 2, 3], ("truncate", 3, 170)), ([], [1, 3], ("finish", 2)),
              ([(4, 50)], [1, 3], None)]
    for step, (pre, dec, act) in enumerate(script):
        n_pf = sum(e[1] for e in pre)
        data = [[torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda()
                 for shape in ((n_pf, Hq, D), (n_pf, Hkv, D), (n_pf, Hkv, D),
                               (len(dec), Hq, D), (len(dec), Hkv, D), (len(dec), Hkv, D))]
                for _ in range(layers)]
        outs = []
        for sv in svs:
            sv.begin_step(prefill=pre, decode=[(sid, 1) for sid in dec])
            got = []
            for layer in range(layers):
                qp, kp, vp, qd, kd, vd = data[layer]
                op = torch.zeros((max(n_pf, 1), Hq, D), device="cuda")
                od = torch.zeros((max(len(dec), 1), Hq, D), device="cuda")
                if n_pf:
                    sv.prefill(layer, qp, kp, vp, op, 0.09)
                if dec:
                    sv.decode(layer, qd, kd, vd, od, 0.09)
                got += [op, od]
            ctx.sync()
            outs.append([t.cpu().numpy() for t in got])
            if act and act[0] == "truncate":
                sv.truncate(act[1], act[2])
            elif act:
                sv.finish(act[1])
        for i, (a, b) in enumerate(zip(*outs)):
            if i % 2 == 0:
                assert np.array_equal(a, b), f"step {step}: host-page prefill differs"
            elif dec:
                assert_close(b, a, what=f"step {step} layer {i // 2}: host-page decode")
    for sv in svs:
        sv.close()


def test_host_pool_r4kv_spill_and_restore(rkv, ctx):
    """R4KV pages (r4kv/src/page.rs:101-252) from a host-memory pool: the
    spilled page equals the HBM pool's byte for byte, and restoring it into
    another sequence of the host pool reproduces the spilled rows (gathered
    bytes equal)."""
    torch = __import__("torch")
    Hkv, D, PT, layers = 2, 256, 64, 2
    lens = [260, 90]
    W = 8
    rng = np.random.default_rng(17)
    data = [[(rng.standard_normal((L, Hkv, D)).astype(np.float32),
              rng.standard_normal((L, Hkv, D)).astype(np.float32)) for L in lens]
            for _ in range(layers)]
    pools = []
    for mem in (rkv.PAGES_DEVICE, rkv.PAGES_HOST):
        pool = rkv.Pool(ctx, layers, Hkv, D, PT, 24, 4, W, seed=5, page_memory=mem)
        for s, L in enumerate(lens):
            pool.alloc.reserve(s, L)
        pool.sync_tables()
        for layer in range(layers):
            for s, L in enumerate(lens):
                k, v = (torch.from_numpy(x).cuda() for x in data[layer][s])
                pool.append(layer, torch.full((L,), s, dtype=torch.int32, device="cuda"),
                            torch.arange(L, dtype=torch.int32, device="cuda"), k, v)
        pools.append(pool)
    ctx.sync()
    t0, count = 64, 130
    hdr = rkv.R4kvHeader(prefix_digest=0x1234ABCD5678EF01, token_start=0, token_count=0,
                         pos_start=t0, layer_lo=0, layer_hi=0, k_fmt=0, v_fmt=0, epoch=3,
                         generation=9, payload_len=0, sketch_offset=0, flags=2)
    pages = []
    for pool in pools:
        n = pool.r4kv_page_bytes(count, 0, layers - 1)
        staging = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
        page = torch.zeros(n, dtype=torch.uint8).pin_memory()
        pool.spill(0, t0, count, 0, layers - 1, hdr, staging, page)
        ctx.sync()
        pages.append(page.numpy().tobytes())
    assert pages[0] == pages[1], "host-pool R4KV page differs from the HBM pool's"
    host = pools[1]
    host.alloc.reserve(2, t0 + count)
    host.sync_tables()
    exp = rkv.R4kvExpect(prefix_digest=0x1234ABCD5678EF01, token_start=t0, pos_start=t0,
                         layer_lo=0, layer_hi=layers - 1, k_fmt=1, v_fmt=1, check_generation=1,
                         generation_min=9, generation_max=9)
    staging = torch.zeros(len(pages[1]) + 64, dtype=torch.uint8, device="cuda")
    host.restore(2, pages[1], exp, staging)
    ctx.sync()
    rb = rkv.row_bytes(D)
    for layer in range(layers):
        for kind in (0, 1):
            a = torch.empty(Hkv * (t0 + count) * rb, dtype=torch.uint8, device="cuda")
            b = torch.empty(Hkv * lens[0] * rb, dtype=torch.uint8, device="cuda")
            host.gather(layer, 2, kind, a)
            host.gather(layer, 0, kind, b)
            ctx.sync()
            got = a.cpu().numpy().reshape(Hkv, t0 + count, rb)[:, t0:]
            want = b.cpu().numpy().reshape(Hkv, lens[0], rb)[:, t0:t0 + count]
            assert np.array_equal(got, want), f"layer {layer} kind {kind}: restored rows"
    for pool in pools:
        pool.close()
