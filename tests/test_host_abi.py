"""CPU-side checks of the C-ABI library: it loads, exports every function
include/rkv.h declares, rejects bad arguments with the documented statuses,
and its host page allocator keeps its invariants.  No kernel is launched."""
import ctypes as C

import numpy as np
import pytest


def test_library_exports_header(rkv):
    L = rkv.lib()
    declared = rkv.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(L, s)]
    assert missing == []
    assert rkv.lib().rkv_version().decode().startswith("rkv")


def test_row_and_page_bytes(rkv):
    assert rkv.row_bytes(256) == 272  # attention.rs:21
    assert rkv.row_bytes(128) == 136
    g = rkv.geometry(2, 256, 64, 10)
    assert rkv.page_bytes(g) == 2 * 2 * 64 * 272
    g = rkv.geometry(2, 128, 16, 10)
    assert rkv.page_bytes(g) == 2 * 2 * 16 * 136


@pytest.mark.parametrize("kv,d,pt,n,status", [
    (2, 64, 64, 10, -4), (2, 256, 48, 10, -4), (2, 256, 8, 10, -4), (0, 256, 64, 10, -1),
    (2, 256, 64, 0, -1)])
def test_geometry_rejected(rkv, kv, d, pt, n, status):
    with pytest.raises(rkv.RkvError) as e:
        rkv.geometry(kv, d, pt, n)
    assert e.value.status == status


def test_no_device_fails_loudly(rkv):
    import torch
    if torch.cuda.is_available():
        pytest.skip("host has a GPU")
    with pytest.raises(rkv.RkvError) as e:
        rkv.Ctx(0)
    assert e.value.status == rkv.ERR_DEVICE


def _invariants(a, num_pages, max_seqs):
    tables, lens = a.export()
    owned = []
    for s in range(max_seqs):
        n = (lens[s] + a_pt[0] - 1) // a_pt[0]
        row = tables[s]
        assert np.all(row[:n] >= 0) and np.all(row[n:] == -1)
        owned.extend(row[:n].tolist())
    assert len(owned) == len(set(owned)), "a page is owned twice"
    assert len(owned) + a.free_pages() == num_pages


a_pt = [16]


def test_allocator_properties(rkv):
    rng = np.random.default_rng(0)
    num_pages, PT, S, W = 200, 16, 12, 40
    a_pt[0] = PT
    a = rkv.Allocator(num_pages, PT, S, W, seed=7)
    lens = np.zeros(S, np.int64)
    for step in range(2000):
        s = int(rng.integers(S))
        op = rng.integers(3)
        if op == 0:
            new = int(lens[s] + rng.integers(0, 100))
            need = (new + PT - 1) // PT
            free_before = a.free_pages()
            held = (lens[s] + PT - 1) // PT
            try:
                a.reserve(s, new)
                lens[s] = new
            except rkv.RkvError as e:
                if need > W:
                    assert e.status == rkv.ERR_CAPACITY
                else:
                    assert e.status == rkv.ERR_OUT_OF_PAGES
                    assert need - held > free_before
                assert a.free_pages() == free_before  # all-or-nothing
        elif op == 1:
            new = int(rng.integers(0, lens[s] + 1))
            a.truncate(s, new)
            lens[s] = new
        else:
            a.free(s)
            lens[s] = 0
        assert a.seq_len(s) == lens[s]
        if step % 50 == 0:
            _invariants(a, num_pages, S)
    _invariants(a, num_pages, S)


def test_allocator_seeded_and_rollback(rkv):
    a = rkv.Allocator(64, 16, 4, 16, seed=3)
    b = rkv.Allocator(64, 16, 4, 16, seed=3)
    c = rkv.Allocator(64, 16, 4, 16, seed=4)
    for x in (a, b, c):
        x.reserve(0, 100)
    assert a.block_table(0) == b.block_table(0)
    assert a.block_table(0) != c.block_table(0)
    # the first pages are a shuffled (non-sequential) run
    assert a.block_table(0) != sorted(a.block_table(0))
    # rollback returns whole pages; re-growing reuses them in the same order
    before = a.block_table(0)
    a.truncate(0, 33)
    assert a.block_table(0) == before[:3]
    a.reserve(0, 100)
    assert a.block_table(0) == before


def test_allocator_errors(rkv):
    a = rkv.Allocator(8, 16, 2, 4, seed=0)
    with pytest.raises(rkv.RkvError) as e:
        a.reserve(2, 10)
    assert e.value.status == rkv.ERR_INVALID_ARG
    with pytest.raises(rkv.RkvError) as e:
        a.reserve(0, 65)
    assert e.value.status == rkv.ERR_CAPACITY
    a.reserve(0, 64)
    a.reserve(1, 64)
    with pytest.raises(rkv.RkvError) as e:
        a.truncate(1, 65)
    assert e.value.status == rkv.ERR_INVALID_ARG
    a.free(1)
    with pytest.raises(rkv.RkvError) as e:
        a.reserve(0, 30)  # shrinking through reserve is refused
    assert e.value.status == rkv.ERR_INVALID_ARG
    assert "rkv_seq_reserve" in rkv.lib().rkv_last_error().decode()


def test_allocator_pair_batches(rkv):
    """rkv_seq_reserve_n / rkv_seq_truncate_n apply their pairs in order,
    exactly as the single calls would, and stop at the first failing pair
    (which the error names), leaving the pairs before it applied."""
    rng = np.random.default_rng(7)
    one = rkv.Allocator(96, 16, 6, 16, seed=5)
    many = rkv.Allocator(96, 16, 6, 16, seed=5)
    lens = np.zeros(6, np.int64)
    for _ in range(40):
        seqs = rng.permutation(6)[: rng.integers(0, 7)].astype(np.int32)
        grow = rng.random() < 0.6
        new = np.array([lens[q] + rng.integers(0, 40) if grow else rng.integers(0, lens[q] + 1)
                        for q in seqs], np.int32)
        if grow and (sum(-(-int(x) // 16) for x in np.maximum(new, lens[seqs]))
                     + sum(-(-int(lens[q]) // 16) for q in range(6) if q not in seqs)) > 96:
            continue
        for q, x in zip(seqs, new):
            (one.reserve if grow else one.truncate)(int(q), int(x))
        assert (many.reserve_n if grow else many.truncate_n)(seqs, new) == len(seqs)
        lens[seqs] = new
        for q in range(6):
            assert one.block_table(q) == many.block_table(q)
            assert one.seq_len(q) == many.seq_len(q) == lens[q]
    # a failing pair stops the batch: earlier pairs applied, later ones not
    a = rkv.Allocator(8, 16, 3, 4, seed=0)
    seqs = np.array([0, 1, 2], np.int32)
    new = np.array([20, 99, 5], np.int32)  # 99 tokens need 7 pages > max_pages_per_seq 4
    done = C.c_int32(-1)
    L = rkv.lib()
    st = L.rkv_seq_reserve_n(a.h, 3, seqs.ctypes.data_as(rkv.I32P), new.ctypes.data_as(rkv.I32P),
                             C.byref(done))
    assert st == rkv.ERR_CAPACITY and done.value == 1
    msg = L.rkv_last_error().decode()
    assert "rkv_seq_reserve_n" in msg and "pair 1" in msg and "rkv_seq_reserve" in msg
    assert (a.seq_len(0), a.seq_len(1), a.seq_len(2)) == (20, 0, 0)
    assert L.rkv_seq_truncate_n(a.h, 0, None, None, None) == rkv.OK
    assert L.rkv_seq_truncate_n(a.h, 2, None, None, None) == rkv.ERR_INVALID_ARG
    assert L.rkv_seq_truncate_n(None, 1, seqs.ctypes.data_as(rkv.I32P), new.ctypes.data_as(rkv.I32P),
                                None) == rkv.ERR_INVALID_ARG


def _ws(rkv, g, B, L, q_heads, q_len=1, pt=0):
    a = rkv.DecodeArgs(B, None, None, rkv.BF16, q_len, q_heads, 1.0, None, rkv.F32, pt, L, None, 0,
                       None, None)
    return rkv.decode_workspace_bytes(g, a)


@pytest.mark.parametrize("kv_heads,q_heads,D,PT,max_decode,max_len", [
    (8, 32, 128, 16, 8, 16384),   # the advisor's case: 3..7 rows refused before
    (8, 64, 128, 16, 4, 8192),
    (2, 16, 256, 64, 64, 65536),
    (2, 16, 256, 64, 16, 262144),
    (1, 1, 128, 32, 40, 4096),
])
def test_decode_workspace_monotone(rkv, kv_heads, q_heads, D, PT, max_decode, max_len):
    """A workspace sized for the largest call (max_decode entries of the
    longest length) holds every smaller call: the serving adapter allocates it
    once (rkv_serve_create)."""
    g = rkv.geometry(kv_heads, D, PT, 1 << 20)
    top = _ws(rkv, g, max_decode, max_len, q_heads)
    lens = sorted({1, PT, 256, 257, 1000, 4096, 4097, max_len // 3, max_len - 1, max_len})
    prev_b = 0
    for B in range(1, max_decode + 1):
        prev_l = 0
        for L in lens:
            if L > max_len:
                continue
            w = _ws(rkv, g, B, L, q_heads)
            assert w <= top, (B, L, w, top)
            assert w >= prev_l, ("not monotone in length", B, L)
            prev_l = w
        w_top = _ws(rkv, g, B, max_len, q_heads)
        assert w_top >= prev_b, ("not monotone in batch", B)
        prev_b = w_top
