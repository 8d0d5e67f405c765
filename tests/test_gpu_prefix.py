"""Prefix sharing on the device: forked sequences read their parent's pages,
copy-on-write copies run inside the stream-ordered table sync, and every
sequence's bytes and attention equal the oracle over its own rows.

Bars as in test_gpu_parity.py: page bytes bit-exact; attention max-abs 2e-3
and relative 1e-3 against flash_decode_reference (attention.rs:148-165) over
the sequence's rows."""
import numpy as np
import pytest

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _append(pool, layer, seq, start, rows):
    torch = _torch()
    n = rows.shape[0]
    kd = torch.from_numpy(rows * (layer + 1)).cuda()
    pool.append(layer, torch.full((n,), seq, dtype=torch.int32, device="cuda"),
                torch.arange(start, start + n, dtype=torch.int32, device="cuda"), kd, kd)


def _gathered(rkv, ctx, pool, layer, seq, length, D, Hkv):
    torch = _torch()
    out = torch.empty(max(Hkv * length * rkv.row_bytes(D), 1), dtype=torch.uint8, device="cuda")
    pool.gather(layer, seq, 0, out)
    ctx.sync()
    return out.cpu().numpy()[:Hkv * length * rkv.row_bytes(D)].reshape(Hkv, length, -1)


def _encoded(rko, rows):
    L, Hkv, _ = rows.shape
    return np.stack([rko.q8_encode(rows[:, h, :].reshape(-1)).reshape(L, -1) for h in range(Hkv)])


def test_fork_copy_on_write_pool(rkv, rko, ctx):
    """Seq 0 holds a 70-row prompt; seqs 1-3 fork it at 70 (inside a page), 64
    (a page boundary) and 50 (inside an earlier page) and all four grow in
    one window (two copies queued).  In the next window seq 4 forks seq 0
    inside its last page and grows, seq 0 is freed while that copy is queued
    and seq 5 takes the freed page.  Each sequence's bytes on both layers
    equal the encoding of its own rows, and decode over the shared pages
    equals the oracle."""
    torch = _torch()
    Hkv, D, PT, Hq = 2, 128, 16, 8
    layers = 2
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, 64, 6, 16, seed=9)
    a = pool.alloc
    rng = np.random.default_rng(31)
    prompt = rng.standard_normal((70, Hkv, D)).astype(np.float32)
    a.reserve(0, 70)
    pool.sync_tables()
    for layer in range(layers):
        _append(pool, layer, 0, 0, prompt)
    forks = {1: 70, 2: 64, 3: 50}
    for s, n in forks.items():
        a.fork(0, s, n)
    shared = a.block_table(0)
    assert a.page_refs(shared[0]) == 4 and a.page_refs(shared[4]) == 2
    rows = {s: prompt[:n].copy() for s, n in forks.items()}
    rows[0] = prompt.copy()
    grow = {0: 5, 1: 9, 2: 20, 3: 3}
    extra = {s: rng.standard_normal((g, Hkv, D)).astype(np.float32) for s, g in grow.items()}
    for s, g in grow.items():
        a.reserve(s, len(rows[s]) + g)
    pool.sync_tables()
    for layer in range(layers):
        for s, g in grow.items():
            _append(pool, layer, s, len(rows[s]), extra[s])
    for s in grow:
        rows[s] = np.concatenate([rows[s], extra[s]])
    # seq 4 forks seq 0 inside seq 0's own (copied) last page and grows, so a
    # copy reading that page is queued; seq 0 then leaves, its last page goes
    # back to the free list and seq 5 takes it as a fresh page in the same
    # window: the copy must read the page before seq 5's rows overwrite it
    a.fork(0, 4, 75)
    a.reserve(4, 80)
    last0 = a.block_table(0)[4]
    a.free(0)
    assert a.page_refs(last0) == 0
    a.reserve(5, 40)
    assert a.block_table(5)[0] == last0
    pool.sync_tables()
    tail4 = rng.standard_normal((5, Hkv, D)).astype(np.float32)
    rows5 = rng.standard_normal((40, Hkv, D)).astype(np.float32)
    for layer in range(layers):
        _append(pool, layer, 4, 75, tail4)
        _append(pool, layer, 5, 0, rows5)
    rows[4] = np.concatenate([rows[0][:75], tail4])
    rows[5] = rows5
    del rows[0]
    ctx.sync()
    for layer in range(layers):
        for s, r in rows.items():
            got = _gathered(rkv, ctx, pool, layer, s, len(r), D, Hkv)
            assert np.array_equal(got, _encoded(rko, r * (layer + 1))), (layer, s)
    # pages shared where the forks left them shared
    t1, t2, t3, t4 = (a.block_table(s) for s in (1, 2, 3, 4))
    assert t1[:4] == t2[:4] and t1[:3] == t3[:3] and t1[:4] == t4[:4]
    assert t1[4] != t4[4]
    # decode over the shared pages, every sequence at once
    seqs = sorted(rows)
    q = rng.standard_normal((len(seqs), 1, Hq, D)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    o = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    sid = torch.tensor(seqs, dtype=torch.int32, device="cuda")
    args = rkv.decode_args(qd, o, sid, 0.125, 16 * PT)
    ws = torch.zeros(max(rkv.decode_workspace_bytes(pool.geometry, args), 4), dtype=torch.uint8,
                     device="cuda")
    args = rkv.decode_args(qd, o, sid, 0.125, 16 * PT, workspace=ws)
    for layer in range(layers):
        pool.decode(layer, args)
        ctx.sync()
        got = o.cpu().numpy()
        for i, s in enumerate(seqs):
            enc = _encoded(rko, rows[s] * (layer + 1))
            p = rko.fd_params(Hq, Hkv, len(rows[s]), 1024, D)
            w = rko.rows_to_words(enc)
            want = rko.flash_decode_reference(p, w, w, (q[i, 0] * np.float32(0.125)).reshape(-1))
            assert_close(got[i, 0].reshape(-1), want, what=f"layer {layer} seq {s}")
    pool.close()


def test_fork_decode_pages64(rkv, rko, ctx):
    """64-token pages, head_dim 256 (the K-in-registers decode): seq 0 holds
    300 rows; seq 1 forks it at 256 (a page boundary) and seq 2 at 200
    (inside page 3, copied on write); all three grow.  The decode over shared
    and private pages equals the oracle for every sequence."""
    torch = _torch()
    Hkv, D, PT, Hq = 2, 256, 64, 16
    pool = rkv.Pool(ctx, 1, Hkv, D, PT, 40, 3, 8, seed=4)
    a = pool.alloc
    rng = np.random.default_rng(8)
    prompt = rng.standard_normal((300, Hkv, D)).astype(np.float32)
    a.reserve(0, 300)
    pool.sync_tables()
    _append(pool, 0, 0, 0, prompt)
    a.fork(0, 1, 256)
    a.fork(0, 2, 200)
    rows = {0: prompt, 1: prompt[:256], 2: prompt[:200]}
    grow = {0: 40, 1: 100, 2: 70}
    extra = {s: rng.standard_normal((g, Hkv, D)).astype(np.float32) for s, g in grow.items()}
    for s, g in grow.items():
        a.reserve(s, len(rows[s]) + g)
    pool.sync_tables()
    for s, g in grow.items():
        _append(pool, 0, s, len(rows[s]), extra[s])
        rows[s] = np.concatenate([rows[s], extra[s]])
    ctx.sync()
    t0, t1, t2 = (a.block_table(s) for s in range(3))
    assert t0[:4] == t1[:4] and t0[:3] == t2[:3] and t0[3] != t2[3]
    seqs = [0, 1, 2]
    q = rng.standard_normal((3, 1, Hq, D)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    o = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    sid = torch.tensor(seqs, dtype=torch.int32, device="cuda")
    for part in (0, 64):
        args = rkv.decode_args(qd, o, sid, 0.0625, 8 * PT, partition_tokens=part)
        ws = torch.zeros(max(rkv.decode_workspace_bytes(pool.geometry, args), 4),
                         dtype=torch.uint8, device="cuda")
        args = rkv.decode_args(qd, o, sid, 0.0625, 8 * PT, partition_tokens=part, workspace=ws)
        pool.decode(0, args)
        ctx.sync()
        got = o.cpu().numpy()
        for i, s in enumerate(seqs):
            enc = _encoded(rko, rows[s])
            p = rko.fd_params(Hq, Hkv, len(rows[s]), 1024, D)
            w = rko.rows_to_words(enc)
            want = rko.flash_decode_reference(p, w, w, (q[i, 0] * np.float32(0.0625)).reshape(-1))
            assert_close(got[i, 0].reshape(-1), want, what=f"partition {part} seq {s}")
    pool.close()


def test_copy_pages_entry_point(rkv, ctx):
    """rkv_copy_pages over 3 layer arrays with a gap between them: every pair
    copied in every layer, out-of-range pairs skipped, nothing else touched."""
    torch = _torch()
    Hkv, D, PT, npages, layers = 2, 256, 64, 12, 3
    g = rkv.geometry(Hkv, D, PT, npages)
    pb = rkv.page_bytes(g)
    stride = npages * pb + 4096
    gen = torch.Generator().manual_seed(5)
    host = torch.randint(0, 256, (layers * stride,), dtype=torch.uint8, generator=gen)
    dev = host.cuda()
    pairs = np.array([[0, 5], [3, 7], [11, 2], [4, 40], [-1, 6]], np.int32)
    pd = torch.from_numpy(pairs.reshape(-1)).cuda()
    rkv.copy_pages(ctx, g, dev, stride, layers, pd, len(pairs))
    ctx.sync()
    want = host.numpy().copy()
    for layer in range(layers):
        base = layer * stride
        for src, dst in pairs:
            if 0 <= src < npages and 0 <= dst < npages:
                want[base + dst * pb:base + (dst + 1) * pb] = \
                    host.numpy()[base + src * pb:base + (src + 1) * pb]
    assert np.array_equal(dev.cpu().numpy(), want)
