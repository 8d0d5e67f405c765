"""Chunked prefill attention on the GPU against the oracle, through the C ABI.

The reference's prefill (BatchStepModel::prefill_batch, adapter.rs:31-60)
folds the one-token step over the chunk, so row i of a chunk after ctx
cached tokens must equal flash_decode_reference over the first ctx+i+1 rows
(attention.rs:148-165).  The oracle's paged decode with q_len = chunk rows
and length ctx+chunk computes exactly that per row (row j attends
len - q_len + j + 1 positions).  Bars as in test_gpu_parity.py: max-abs
2e-3 and relative 1e-3 over each entry's output."""
import numpy as np
import pytest

from tests.test_gpu_parity import (ATOL, RTOL, Scene, _as_u8, _bind_ctx,  # noqa: F401
                                   assert_close, outlier_q)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _oracle(rko, sc, seq, ctx, n, q, scale):
    lens = np.array(sc.lens, np.int32).copy()
    lens[seq] = ctx + n
    return rko.paged_decode(sc.lay, sc.pages, sc.bt, lens, np.array([seq], np.int32),
                            q[None], scale, 1024)[0]


def _run(rkv, rko, ctx_h, sc, entries, Hq, scale, q_bf16=False, out_bf16=False, seed=0,
         segment_tokens=None, q_outliers=False):
    """entries: (seq, ctx, n) with ctx + n <= the sequence's length.
    segment_tokens: None runs without a workspace (no split); otherwise the
    call gets the workspace rkv_prefill_workspace_bytes asks for."""
    torch = _torch()
    rng = np.random.default_rng(seed)
    D = sc.D
    rows = [n for _, _, n in entries]
    total = max(sum(rows), 1)
    q = outlier_q(rng, (total, Hq, D)) if q_outliers else \
        rng.standard_normal((total, Hq, D)).astype(np.float32)
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    qd = torch.from_numpy(q).cuda()
    if q_bf16:
        qd = qd.to(torch.bfloat16)
    out = torch.full((total, Hq, D), float("nan"), device="cuda",
                     dtype=torch.bfloat16 if out_bf16 else torch.float32)
    ent = ([s for s, _, _ in entries], [c for _, c, _ in entries], rows, qd, out, scale)
    a = rkv.prefill_args(*ent)
    if segment_tokens is not None:
        a = rkv.prefill_args(*ent, segment_tokens=segment_tokens)
        nb = rkv.prefill_workspace_bytes(sc.g, a)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        a = rkv.prefill_args(*ent, segment_tokens=segment_tokens, workspace=ws)
        _run.last_ws_bytes = nb
    rkv.prefill_q8(ctx_h, sc.g, sc.pages_d, sc.bt_d, len(sc.lens), a)
    ctx_h.sync()
    got = out.float().cpu().numpy()
    off = 0
    for s, c, n in entries:
        if n:
            want = _oracle(rko, sc, s, c, n, q[off:off + n], scale)
            g = got[off:off + n]
            if out_bf16:
                # the f32 result rounded once to bf16 (half an ulp = 2^-9 relative)
                assert float((np.abs(g - want) - np.abs(want) * 2.0 ** -8).max()) <= ATOL
                assert np.linalg.norm(g - want) / np.linalg.norm(want) <= RTOL + 2.0 ** -8
            else:
                assert_close(g, want, what=f"seq {s} ctx {c} rows {n}")
        off += n
    return got


@pytest.mark.parametrize("Hq,Hkv,D,PT,entries,q_bf16,out_bf16,outliers", [
    # G = 8 (16 chunk tokens per row block): chunk from empty, mid-page, a
    # block-sized chunk, one row, a long context
    (16, 2, 256, 64, [(0, 40), (300, 17), (129, 128), (64, 1), (1000, 70)], True, False, 0.01),
    # config 1 geometry (G = 4, 16-token pages: half-tile pages)
    (8, 2, 128, 16, [(0, 33), (200, 100), (31, 2)], False, False, 0.0),
    (8, 2, 128, 32, [(5, 64), (77, 45)], False, True, 0.0),
    # G = 1 (128 tokens per block) and G = 16 (8 tokens per block)
    (16, 16, 128, 64, [(10, 150), (0, 7)], True, False, 0.0),
    (32, 2, 128, 128, [(250, 23), (0, 9)], True, False, 0.01),
    # bf16 q (the f16 QK) on 16-token pages, D = 128 and 256
    (8, 2, 128, 16, [(0, 33), (200, 100), (31, 2)], True, True, 0.0),
    (16, 2, 256, 16, [(0, 40), (90, 33), (517, 16)], True, False, 0.01),
    # the reference's 24 q / 4 kv heads (G = 6, which does not divide 128:
    # 21 chunk tokens per row block, rows 126 and 127 dead) on 32-token pages
    (24, 4, 256, 32, [(0, 40), (300, 21), (129, 128), (64, 1), (1000, 70)], True, False, 0.01),
    (24, 4, 256, 32, [(0, 43), (200, 100), (31, 2)], False, False, 0.0),
    # G = 3 (42 tokens per block) and G = 12 (10 tokens per block)
    (12, 4, 128, 32, [(7, 130), (500, 42)], True, False, 0.0),
    (24, 2, 256, 64, [(100, 95), (0, 11)], True, True, 0.0),
])
def test_prefill_parity(rkv, rko, ctx, Hq, Hkv, D, PT, entries, q_bf16, out_bf16, outliers):
    lens = [c + n + extra for (c, n), extra in zip(entries, [3, 0, 5, 0, 2])]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=len(entries) + D, outliers=outliers,
               src_bf16=q_bf16)
    ent = [(i, c, n) for i, (c, n) in enumerate(entries)]
    _run(rkv, rko, ctx, sc, ent, Hq, 1.0 / np.sqrt(D), q_bf16, out_bf16, seed=D + PT)


@pytest.mark.parametrize("Hq,Hkv,D,PT,entries,q_bf16", [
    (16, 2, 256, 64, [(0, 40), (300, 17), (129, 128), (1000, 70)], True),
    (8, 2, 128, 16, [(0, 33), (200, 100), (31, 2)], False),
    (32, 2, 128, 128, [(250, 23), (0, 9)], True),
])
def test_prefill_outlier_query(rkv, rko, ctx, Hq, Hkv, D, PT, entries, q_bf16):
    """Prefill rows whose queries carry x32 and x100 outlier channels, split
    and unsplit, against the oracle's f32 q."""
    lens = [c + n + 1 for c, n in entries]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=7 + D + PT, outliers=0.01, src_bf16=True)
    ent = [(i, c, n) for i, (c, n) in enumerate(entries)]
    _run(rkv, rko, ctx, sc, ent, Hq, 1.0 / np.sqrt(D), q_bf16, seed=D, q_outliers=True)
    _run(rkv, rko, ctx, sc, ent, Hq, 1.0 / np.sqrt(D), q_bf16, seed=D, q_outliers=True,
         segment_tokens=128)


@pytest.mark.parametrize("Hq,Hkv,D,PT,entries,seg,out_bf16", [
    # forced segments: 128 tokens (two pages), so every long row block has
    # segments its early rows cannot see (fully masked partials)
    (16, 2, 256, 64, [(1000, 70), (0, 40), (300, 17), (129, 128)], 128, False),
    # half-tile pages, 32-token segments: the 64-segment cap raises the length
    (8, 2, 128, 16, [(0, 300), (2500, 33), (31, 2)], 32, True),
    # 256-token pages (segment rounded up to a page), G = 1 and G = 16
    (16, 16, 128, 256, [(700, 150), (0, 7)], 100, False),
    (32, 2, 128, 64, [(1500, 23), (0, 9)], 512, True),
    # the reference's 24 q / 4 kv heads on 32-token pages
    (24, 4, 256, 32, [(1000, 70), (0, 40), (300, 21)], 96, False),
])
def test_prefill_split_parity(rkv, rko, ctx, Hq, Hkv, D, PT, entries, seg, out_bf16):
    """Row blocks' causal ranges split into segments whose partials the
    combine merges: the same rows as the unsplit launch, at the same bars."""
    lens = [c + n + 1 for c, n in entries]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=len(entries) + PT)
    ent = [(i, c, n) for i, (c, n) in enumerate(entries)]
    _run(rkv, rko, ctx, sc, ent, Hq, 1.0 / np.sqrt(D), out_bf16=out_bf16, seed=PT,
         segment_tokens=seg)
    assert _run.last_ws_bytes > 0


def test_prefill_automatic_split(rkv, rko, ctx):
    """One long-context chunk has too few row blocks to fill the chip: with
    a workspace the launch splits by itself (workspace_bytes > 0) and the
    rows match the oracle; without one it runs unsplit, to the same rows;
    segment_tokens < 0 never splits; an explicit split that does not fit its
    workspace is refused."""
    torch = _torch()
    Hq, Hkv, D, PT = 16, 2, 128, 64
    c, n = 6000, 64
    sc = Scene(rkv, rko, Hkv, D, PT, [c + n], seed=11)
    got = _run(rkv, rko, ctx, sc, [(0, c, n)], Hq, 0.088, seed=12, segment_tokens=0)
    assert _run.last_ws_bytes > 0
    unsplit = _run(rkv, rko, ctx, sc, [(0, c, n)], Hq, 0.088, seed=12)
    assert float(np.abs(got - unsplit).max()) <= 1e-5
    q = torch.zeros((n, Hq, D), device="cuda")
    out = torch.zeros_like(q)
    assert rkv.prefill_workspace_bytes(
        sc.g, rkv.prefill_args([0], [c], [n], q, out, 1.0, segment_tokens=-1)) == 0
    a = rkv.prefill_args([0], [c], [n], q, out, 1.0, segment_tokens=256)
    need = rkv.prefill_workspace_bytes(sc.g, a)
    assert need > 0
    small = torch.empty(need - 256, dtype=torch.uint8, device="cuda")
    with pytest.raises(rkv.RkvError) as e:
        rkv.prefill_q8(ctx, sc.g, sc.pages_d, sc.bt_d, 1,
                       rkv.prefill_args([0], [c], [n], q, out, 1.0, segment_tokens=256,
                                        workspace=small))
    assert e.value.status == rkv.ERR_INVALID_ARG
    ctx.sync()


def test_prefill_entries_share_a_sequence(rkv, rko, ctx):
    """Two entries of one call read the same sequence at different chunk
    boundaries, entries with zero rows are skipped, and q_offsets may leave
    gaps: rows outside every entry stay untouched."""
    torch = _torch()
    Hq, Hkv, D, PT = 16, 2, 256, 64
    sc = Scene(rkv, rko, Hkv, D, PT, [500, 90], seed=3)
    rng = np.random.default_rng(4)
    total = 120
    q = rng.standard_normal((total, Hq, D)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    out = torch.full((total, Hq, D), 7.0, device="cuda")
    ent = [(0, 100, 30), (1, 0, 0), (0, 400, 50), (1, 60, 30)]
    offs = [0, 30, 35, 90]
    a = rkv.prefill_args([e[0] for e in ent], [e[1] for e in ent], [e[2] for e in ent], qd, out,
                         0.0625, q_offsets=offs)
    rkv.prefill_q8(ctx, sc.g, sc.pages_d, sc.bt_d, 2, a)
    ctx.sync()
    got = out.cpu().numpy()
    for (s, c, n), o in zip(ent, offs):
        if n:
            want = _oracle(rko, sc, s, c, n, q[o:o + n], 0.0625)
            assert_close(got[o:o + n], want, what=f"seq {s} ctx {c}")
    assert np.all(got[30:35] == 7.0) and np.all(got[85:90] == 7.0)


def test_prefill_rejects_bad_arguments(rkv, rko, ctx):
    torch = _torch()
    Hkv, D, PT = 2, 128, 16
    sc = Scene(rkv, rko, Hkv, D, PT, [40], seed=5)
    q = torch.zeros((8, 8, D), device="cuda")
    out = torch.zeros_like(q)

    def call(seq_ids, ctxs, rows, qq=q, oo=out, offs=None):
        a = rkv.prefill_args(seq_ids, ctxs, rows, qq, oo, 1.0, q_offsets=offs)
        rkv.prefill_q8(ctx, sc.g, sc.pages_d, sc.bt_d, 1, a)

    cases = [
        (([1], [0], [4]), rkv.ERR_INVALID_ARG),            # seq outside the table
        (([0], [-1], [4]), rkv.ERR_INVALID_ARG),           # negative ctx
        (([0], [0], [9]), rkv.ERR_INVALID_ARG),            # rows beyond q/out
        (([0], [41], [8]), rkv.ERR_UNSUPPORTED),           # beyond the table row (48 tokens)
    ]
    for args, status in cases:
        with pytest.raises(rkv.RkvError) as e:
            call(*args)
        assert e.value.status == status, (args, e.value)
    with pytest.raises(rkv.RkvError) as e:
        call([0], [0], [4], offs=[6])                      # offset + rows > total rows
    assert e.value.status == rkv.ERR_INVALID_ARG
    qbig = torch.zeros((8, 2 * 130, D), device="cuda")     # 130 q heads per kv head
    with pytest.raises(rkv.RkvError) as e:
        call([0], [0], [4], qq=qbig, oo=torch.zeros_like(qbig))
    assert e.value.status == rkv.ERR_UNSUPPORTED
    many = rkv.PREFILL_MAX_SEQS + 1
    with pytest.raises(rkv.RkvError) as e:
        call([0] * many, [0] * many, [0] * many)
    assert e.value.status == rkv.ERR_INVALID_ARG
    ctx.sync()


def test_pool_chunked_prefill_then_decode(rkv, rko, ctx):
    """A 300-token prompt through the pool in chunks of 128, 128 and 44
    (reserve, sync, append, prefill per chunk), on two layers; every chunk's
    rows equal the oracle, and the prompt's last row equals the pool decode
    of the same query at length 300."""
    torch = _torch()
    Hkv, D, PT, Hq, layers = 2, 256, 64, 16, 2
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, 32, 2, 8, seed=7)
    rng = np.random.default_rng(8)
    prompt = rng.standard_normal((300, Hkv, D)).astype(np.float32)
    q = rng.standard_normal((300, Hq, D)).astype(np.float32)
    outs = {layer: np.zeros((300, Hq, D), np.float32) for layer in range(layers)}
    done = 0
    for n in (128, 128, 44):
        pool.alloc.reserve(0, done + n)
        pool.sync_tables()
        for layer in range(layers):
            kd = torch.from_numpy(prompt[done:done + n] * (layer + 1)).cuda()
            pool.append(layer, torch.zeros(n, dtype=torch.int32, device="cuda"),
                        torch.arange(done, done + n, dtype=torch.int32, device="cuda"), kd, kd)
            qd = torch.from_numpy(q[done:done + n]).cuda()
            out = torch.empty_like(qd)
            pool.prefill(layer, rkv.prefill_args([0], [done], [n], qd, out, 0.0625))
            ctx.sync()
            outs[layer][done:done + n] = out.cpu().numpy()
        done += n
    with pytest.raises(rkv.RkvError):
        pool.prefill(0, rkv.prefill_args([0], [250], [51], torch.zeros((51, Hq, D), device="cuda"),
                                         torch.zeros((51, Hq, D), device="cuda"), 1.0))
    tables, lens = pool.alloc.export()
    lay = rko.layout(Hkv, D, PT, 32)
    pb = rkv.page_bytes(pool.geometry)
    for layer in range(layers):
        pages = _as_u8(pool.layer_pages(layer), 32 * pb).cpu().numpy()
        want = rko.paged_decode(lay, pages, tables, lens, np.array([0], np.int32), q[None],
                                0.0625, 1024)[0]
        assert_close(outs[layer], want, what=f"layer {layer} prompt")
    # the last prompt row through the decode kernel
    qd = torch.from_numpy(q[299:300][None]).cuda()
    o = torch.empty_like(qd)
    sid = torch.zeros(1, dtype=torch.int32, device="cuda")
    a = rkv.decode_args(qd, o, sid, 0.0625, 8 * PT)
    ws = torch.zeros(max(rkv.decode_workspace_bytes(pool.geometry, a), 4), dtype=torch.uint8,
                     device="cuda")
    a = rkv.decode_args(qd, o, sid, 0.0625, 8 * PT, workspace=ws)
    pool.decode(layers - 1, a)
    ctx.sync()
    assert_close(o.cpu().numpy()[0, 0], outs[layers - 1][299], what="decode vs prefill row")
    pool.close()


@pytest.mark.parametrize("Hq,Hkv,D,PT", [
    (16, 2, 256, 64),
    # 16-token pages: the widening pass looks up each 16-token half's page;
    # the ranges of entries 1 and 2 end inside the first half of their last
    # tile, whose second half then has no page
    (16, 2, 256, 16),
    (8, 2, 128, 16),
    # the reference's 24 q / 4 kv heads on 32-token pages
    (24, 4, 256, 32),
])
def test_prefill_widened_once_matches_per_block(rkv, rko, ctx, Hq, Hkv, D, PT):
    """A bf16 query with the full workspace widens each tile once into it;
    a workspace that holds only the split partials (what an f32 query asks
    for) and no workspace at all widen per row block instead.  All three
    give the oracle's rows, and the split runs agree to 1e-5."""
    torch = _torch()
    print(f"widened once Hq={Hq} Hkv={Hkv} D={D} PT={PT}", flush=True)
    # causal ranges 830 (ends in the second 16-token half of its last tile),
    # 97 and 45 (end in the first half)
    entries = [(0, 700, 130), (1, 33, 64), (2, 0, 45)]
    sc = Scene(rkv, rko, Hkv, D, PT, [c + n for _, c, n in entries], seed=21)
    rng = np.random.default_rng(22)
    total = sum(n for _, _, n in entries)
    q = rko.bf16_to_f32(rko.f32_to_bf16(
        outlier_q(rng, (total, Hq, D)))).reshape(total, Hq, D)
    qd = torch.from_numpy(q).cuda().to(torch.bfloat16)
    cols = ([s for s, _, _ in entries], [c for _, c, _ in entries], [n for _, _, n in entries])
    scale = 1.0 / np.sqrt(D)
    q32 = torch.zeros((total, Hq, D), device="cuda")
    partials = rkv.prefill_workspace_bytes(
        sc.g, rkv.prefill_args(*cols, q32, torch.zeros_like(q32), scale))
    full = rkv.prefill_workspace_bytes(
        sc.g, rkv.prefill_args(*cols, qd, torch.zeros_like(q32), scale))
    assert full >= partials + 3 * Hkv * 132 * D  # at least one widened tile per entry
    outs = {}
    for name, nb in (("full", full), ("partials", partials), ("none", None)):
        out = torch.full((total, Hq, D), float("nan"), device="cuda")
        ws = None if not nb else torch.empty(nb, dtype=torch.uint8, device="cuda")
        a = rkv.prefill_args(*cols, qd, out, scale, segment_tokens=0 if ws is not None else -1,
                             workspace=ws)
        rkv.prefill_q8(ctx, sc.g, sc.pages_d, sc.bt_d, len(entries), a)
        ctx.sync()
        outs[name] = out.cpu().numpy()
    off = 0
    for s, c, n in entries:
        want = _oracle(rko, sc, s, c, n, q[off:off + n], scale)
        for name, got in outs.items():
            assert_close(got[off:off + n], want, what=f"{name}: seq {s} ctx {c} rows {n}")
        off += n
    if partials:
        assert float(np.abs(outs["full"] - outs["partials"]).max()) <= 1e-5
