"""Prefix sharing on the host: reference-counted pages, fork, copy-on-write.

The allocator is host code with no reference counterpart to compare bytes
against (har-kv/src/graph.rs:447-533 shares prefix pages only logically), so
it is pinned by a model of the device: a page store that the queued copies
and the appended rows act on exactly as the pool's sync and append kernels
would.  Copies are applied in a random order, which fails if two queued
copies depend on each other.  No kernel is launched here."""
import random

import numpy as np
import pytest


PT = 16


def _check_refs(a, num_pages, max_seqs):
    tables, lens = a.export()
    named = {}
    for s in range(max_seqs):
        n = (int(lens[s]) + PT - 1) // PT
        row = tables[s]
        assert np.all(row[:n] >= 0) and np.all(row[n:] == -1), (s, row, lens[s])
        for p in row[:n].tolist():
            named[p] = named.get(p, 0) + 1
    for p in range(num_pages):
        assert a.page_refs(p) == named.get(p, 0), p
    assert a.free_pages() == num_pages - len(named)
    # shared pages form a prefix of every table
    for s in range(max_seqs):
        n = (int(lens[s]) + PT - 1) // PT
        shared = [named[p] > 1 for p in tables[s][:n].tolist()]
        assert shared == sorted(shared, reverse=True), (s, shared)
    return tables, lens


class _Device:
    """Page store acted on by queued copies and row writes."""

    def __init__(self, num_pages):
        self.store = [[None] * PT for _ in range(num_pages)]

    def sync(self, a, rng, writes):
        pairs = a.take_copies()
        dsts = [d for _, d in pairs]
        assert len(dsts) == len(set(dsts))
        assert not set(dsts) & {s for s, _ in pairs}, "a queued copy reads another's target"
        rng.shuffle(pairs)
        for src, dst in pairs:
            self.store[dst] = list(self.store[src])
        tables, _ = a.export()
        for seq, pos, val in writes:
            self.store[tables[seq][pos // PT]][pos % PT] = val
        return len(pairs)

    def view(self, a, seq, length):
        tables, _ = a.export()
        return [self.store[tables[seq][i // PT]][i % PT] for i in range(length)]


@pytest.mark.parametrize("seed", range(6))
def test_fork_cow_random_windows(rkv, seed):
    rng = random.Random(seed)
    num_pages, max_seqs, width = 48, 6, 8
    a = rkv.Allocator(num_pages, PT, max_seqs, width, seed=seed)
    dev = _Device(num_pages)
    content = [[] for _ in range(max_seqs)]   # logical rows per sequence
    written = [0] * max_seqs                   # rows on the device
    counter = [0]

    def fresh():
        counter[0] += 1
        return counter[0]

    forks = cows = 0
    for window in range(80):
        writes = []
        for _ in range(rng.randint(1, 5)):
            s = rng.randrange(max_seqs)
            op = rng.random()
            n = len(content[s])
            if op < 0.4:
                new = min(width * PT, n + rng.choice([1, 3, 7, 16, 20]))
                before = a.free_pages()
                try:
                    a.reserve(s, new)
                except rkv.RkvError as e:
                    assert e.status == rkv.ERR_OUT_OF_PAGES
                    assert a.free_pages() == before
                    continue
                for pos in range(n, new):
                    v = fresh()
                    content[s].append(v)
                    writes.append((s, pos, v))
            elif op < 0.55:
                new = rng.randint(0, n)
                a.truncate(s, new)
                del content[s][new:]
                writes = [w for w in writes if not (w[0] == s and w[1] >= new)]
                written[s] = min(written[s], new)
            elif op < 0.67:
                a.free(s)
                content[s] = []
                writes = [w for w in writes if w[0] != s]
                written[s] = 0
            else:
                empty = [d for d in range(max_seqs) if d != s and not content[d]]
                if not empty or written[s] == 0:
                    continue
                dst = rng.choice(empty)
                length = rng.randint(0, written[s])
                a.fork(s, dst, length)
                content[dst] = list(content[s][:length])
                written[dst] = length
                forks += 1
        _, lens = _check_refs(a, num_pages, max_seqs)
        cows += dev.sync(a, rng, writes)
        for s in range(max_seqs):
            assert lens[s] == len(content[s])
            written[s] = len(content[s])
            assert dev.view(a, s, len(content[s])) == content[s], (window, s)
    print(f"seed {seed}: {forks} forks, {cows} copies")
    assert forks > 5 and cows > 0


def test_copy_source_freed_and_reused(rkv):
    """A page a queued copy still reads is never a copy target in the same window."""
    num_pages = 8
    a = rkv.Allocator(num_pages, PT, 4, 4, seed=1)
    dev = _Device(num_pages)
    rng = random.Random(0)
    a.reserve(0, 20)                           # A: 2 pages, last one partial
    dev.sync(a, rng, [(0, i, ("A", i)) for i in range(20)])
    a.reserve(2, 20)                           # E
    dev.sync(a, rng, [(2, i, ("E", i)) for i in range(20)])
    a.fork(0, 1, 20)                           # B shares A's pages
    a_last = a.block_table(0)[1]
    a.reserve(1, 21)                           # B: copy of A's last page queued
    a.free(0)                                  # A's last page is free but still a copy source
    assert a.page_refs(a_last) == 0
    a.fork(2, 3, 20)
    a.reserve(3, 21)                           # F: its copy target must not be A's old page
    pairs = a.take_copies()
    assert len(pairs) == 2
    assert pairs[1][1] != a_last
    for src, dst in reversed(pairs):
        dev.store[dst] = list(dev.store[src])
    tables, _ = a.export()
    dev.store[tables[1][1]][4] = ("B", 20)
    dev.store[tables[3][1]][4] = ("F", 20)
    assert dev.view(a, 1, 21) == [("A", i) for i in range(20)] + [("B", 20)]
    assert dev.view(a, 3, 21) == [("E", i) for i in range(20)] + [("F", 20)]


def test_queued_copy_into_freed_page_is_dropped(rkv):
    a = rkv.Allocator(8, PT, 3, 4, seed=2)
    a.reserve(0, 20)
    a.take_copies()
    a.fork(0, 1, 20)
    a.reserve(1, 22)
    a.free(1)
    assert a.take_copies() == []
    assert a.page_refs(a.block_table(0)[1]) == 1


def test_copy_of_a_queued_copy_reads_its_source(rkv):
    """B copies A's page; D forks B before the sync and grows: D's copy reads A's page."""
    a = rkv.Allocator(8, PT, 4, 4, seed=3)
    a.reserve(0, 20)
    a.take_copies()
    a.fork(0, 1, 20)
    a.reserve(1, 21)
    a.fork(1, 2, 18)
    a.reserve(2, 19)
    pairs = a.take_copies()
    src_page = a.block_table(0)[1]
    assert [p[0] for p in pairs] == [src_page, src_page]
    assert len({p[1] for p in pairs}) == 2


def test_fork_errors(rkv):
    a = rkv.Allocator(8, PT, 3, 4, seed=4)
    a.reserve(0, 20)
    for args in [(0, 0, 5), (0, 1, 21), (0, 1, -1), (0, 5, 3), (-1, 1, 0)]:
        with pytest.raises(rkv.RkvError) as e:
            a.fork(*args)
        assert e.value.status == rkv.ERR_INVALID_ARG
    a.reserve(1, 3)
    with pytest.raises(rkv.RkvError):
        a.fork(0, 1, 5)                        # dst not empty
    a.fork(0, 2, 0)                            # an empty fork holds no page
    assert a.block_table(2) == [] and a.seq_len(2) == 0


def test_full_page_fork_needs_no_copy(rkv):
    a = rkv.Allocator(8, PT, 3, 4, seed=5)
    a.reserve(0, 32)
    a.take_copies()
    a.fork(0, 1, 32)
    a.reserve(1, 40)                           # next page is fresh: nothing to copy
    a.reserve(0, 33)
    assert a.take_copies() == []
    assert a.block_table(1)[:2] == a.block_table(0)[:2]
    assert a.block_table(1)[2] != a.block_table(0)[2]


def test_page_generation_counts_reuse(rkv):
    """A page's generation counts the times it left the free list: the pages a
    sequence frees come back (top of the list first) one generation later,
    and a fork shares pages without a new generation."""
    a = rkv.Allocator(6, PT, 3, 4, seed=3)
    assert all(a.page_generation(p) == 0 for p in range(6))
    a.reserve(0, 3 * PT)
    first = a.block_table(0)
    assert [a.page_generation(p) for p in first] == [1, 1, 1]
    a.fork(0, 1, 2 * PT)
    assert [a.page_generation(p) for p in a.block_table(1)] == [1, 1]
    a.free(0)
    a.free(1)
    a.reserve(2, 4 * PT)
    again = a.block_table(2)
    assert sorted(again[:3]) == sorted(first)
    assert all(a.page_generation(p) == 2 for p in first)
    assert a.page_generation(again[3]) == 1
    with pytest.raises(rkv.RkvError):
        a.page_generation(6)
