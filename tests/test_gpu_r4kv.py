"""R4KV spill/restore on the GPU: the device CRC32C and the page bytes
against the oracle (crc32c.rs, page.rs pack_page over the oracle's gather of
the same pool pages), the restore path's fail-closed gates, and round
trips through host memory.  Bit-exact throughout."""
import numpy as np
import pytest

from tests.test_gpu_parity import _as_u8

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


@pytest.mark.parametrize("n", [0, 1, 9, 15, 16, 17, 1000, 65535, 65536, 65537, 3 * 65536 + 5,
                               (1 << 22) + 13])
def test_device_crc32c(rkv, rko, ctx, n):
    torch = _torch()
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, n + 16, dtype=np.uint8)
    d = torch.from_numpy(data).cuda()
    out = torch.full((4,), -1, dtype=torch.int32, device="cuda")
    rkv.crc32c(ctx, d, n, out)
    ctx.sync()
    got = int(out[0].item()) & 0xFFFFFFFF
    assert got == rko.crc32c(data[:n].tobytes()), n


def test_device_crc32c_known_vector(rkv, ctx):
    torch = _torch()
    d = torch.tensor(list(b"123456789") + [0] * 7, dtype=torch.uint8, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    rkv.crc32c(ctx, d, 9, out)
    ctx.sync()
    assert int(out[0].item()) & 0xFFFFFFFF == 0xE3069283  # crc32c.rs:40


def _filled_pool(rkv, ctx, layers, Hkv, D, PT, lens, seed):
    torch = _torch()
    W = max((L + PT - 1) // PT for L in lens) + 2
    num = sum((L + PT - 1) // PT for L in lens) * 2 + 8
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, num, len(lens) + 2, W, seed=seed)
    rng = np.random.default_rng(seed)
    for s, L in enumerate(lens):
        pool.alloc.reserve(s, L)
    pool.sync_tables()
    for layer in range(layers):
        for s, L in enumerate(lens):
            k = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32)).cuda()
            v = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32)).cuda()
            pool.append(layer, torch.full((L,), s, dtype=torch.int32, device="cuda"),
                        torch.arange(L, dtype=torch.int32, device="cuda"), k, v)
    ctx.sync()
    return pool


def _oracle_body(rkv, rko, pool, seq, t0, count, lo, hi):
    """Payload body from the oracle's gather of the pool's own pages."""
    g = pool.geometry
    lay = rko.layout(g.kv_heads, g.head_dim, g.page_tokens, g.num_pages)
    pb = rkv.page_bytes(g)
    tables, lens = pool.alloc.export()
    parts = []
    for layer in range(lo, hi + 1):
        pages = _as_u8(pool.layer_pages(layer), g.num_pages * pb).cpu().numpy()
        for kind in (0, 1):
            rows = rko.paged_gather(lay, pages, tables[seq], int(lens[seq]), kind)
            parts.append(rows[:, t0:t0 + count, :].reshape(-1))
    return np.concatenate(parts).tobytes() if parts else b""


def _identity(rkv, **kw):
    f = dict(prefix_digest=0x1234ABCD5678EF01, token_start=0, token_count=0, pos_start=37,
             layer_lo=0, layer_hi=0, k_fmt=0, v_fmt=0, epoch=3, generation=9, payload_len=0,
             sketch_offset=0, flags=2)
    f.update(kw)
    return rkv.R4kvHeader(**f)


@pytest.mark.parametrize("D,PT", [(256, 64), (128, 16)])
def test_spill_bytes_match_oracle(rkv, rko, ctx, D, PT):
    torch = _torch()
    Hkv, layers = 2, 3
    pool = _filled_pool(rkv, ctx, layers, Hkv, D, PT, [300, 77], seed=D + PT)
    t0, count, lo, hi = 37, 150, 1, 2
    n = pool.r4kv_page_bytes(count, lo, hi)
    assert n == 96 + (hi - lo + 1) * 2 * Hkv * count * (D // 32 * 34) + 4
    staging = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    host = torch.zeros(n, dtype=torch.uint8).pin_memory()
    pool.spill(0, t0, count, lo, hi, _identity(rkv), staging, host)
    ctx.sync()
    body = _oracle_body(rkv, rko, pool, 0, t0, count, lo, hi)
    hdr = rko.r4kv_header(prefix_digest=0x1234ABCD5678EF01, token_start=t0, token_count=count,
                          pos_start=37, layer_lo=lo, layer_hi=hi, k_fmt=1, v_fmt=1, epoch=3,
                          generation=9, payload_len=len(body), sketch_offset=0, flags=2)
    want = rko.r4kv_pack_page(hdr, body)
    got = host.numpy().tobytes()
    assert got == want
    assert staging[:n].cpu().numpy().tobytes() == want
    pool.close()


def test_restore_round_trip_and_refusals(rkv, rko, ctx):
    """Spill a range of seq 0, restore it into seq 2 (reserved, other pages),
    and check its rows; a corrupted payload or a wrong identity is refused
    and leaves the pages untouched."""
    torch = _torch()
    Hkv, D, PT, layers = 2, 256, 64, 2
    pool = _filled_pool(rkv, ctx, layers, Hkv, D, PT, [260, 90], seed=4)
    t0, count = 64, 130
    n = pool.r4kv_page_bytes(count, 0, layers - 1)
    staging = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    page = torch.zeros(n, dtype=torch.uint8).pin_memory()
    pool.spill(0, t0, count, 0, layers - 1, _identity(rkv, pos_start=t0), staging, page)
    ctx.sync()
    page_bytes = page.numpy().tobytes()
    pool.alloc.reserve(2, t0 + count)
    pool.sync_tables()
    exp = rkv.R4kvExpect(prefix_digest=0x1234ABCD5678EF01, token_start=t0, pos_start=t0,
                         layer_lo=0, layer_hi=layers - 1, k_fmt=1, v_fmt=1, check_generation=1,
                         generation_min=9, generation_max=9)
    g = pool.geometry
    pb = rkv.page_bytes(g)

    def snapshot():
        return [_as_u8(pool.layer_pages(l), g.num_pages * pb).cpu().numpy().copy()
                for l in range(layers)]

    before = snapshot()
    bad = bytearray(page_bytes)
    bad[96 + 1000] ^= 0x40
    with pytest.raises(rkv.R4kvRefused) as e:
        pool.restore(2, bytes(bad), exp, staging)
    assert e.value.refusal == rkv.R4KV_PAYLOAD_CHECKSUM
    wrong = rkv.R4kvExpect(**{k: getattr(exp, k) for k, _ in exp._fields_})
    wrong.prefix_digest ^= 1
    with pytest.raises(rkv.R4kvRefused) as e:
        pool.restore(2, page_bytes, wrong, staging)
    assert e.value.refusal == rkv.R4KV_PREFIX
    wrong = rkv.R4kvExpect(**{k: getattr(exp, k) for k, _ in exp._fields_})
    wrong.generation_min = 10
    wrong.generation_max = 12
    with pytest.raises(rkv.R4kvRefused) as e:
        pool.restore(2, page_bytes, wrong, staging)
    assert e.value.refusal == rkv.R4KV_GENERATION
    ctx.sync()
    after = snapshot()
    assert all(np.array_equal(a, b) for a, b in zip(before, after)), "a refused page wrote pages"
    pool.restore(2, page_bytes, exp, staging)
    ctx.sync()
    want = _oracle_body(rkv, rko, pool, 0, t0, count, 0, layers - 1)
    got = _oracle_body(rkv, rko, pool, 2, t0, count, 0, layers - 1)
    assert got == want
    # the restored rows attend like the originals: spill seq 2's range again
    again = torch.zeros(n, dtype=torch.uint8, device="cuda")
    pool.spill(2, t0, count, 0, layers - 1, _identity(rkv, pos_start=t0), staging, again)
    ctx.sync()
    assert again.cpu().numpy().tobytes() == page_bytes
    pool.close()


@pytest.mark.parametrize("D,PT,t0,count", [(256, 64, 37, 150), (128, 16, 5, 40), (256, 32, 33, 1)])
def test_restore_partial_tiles_keep_neighbours(rkv, rko, ctx, D, PT, t0, count):
    """A range that starts and ends inside page tiles: restoring seq 0's rows
    into seq 1 replaces exactly [t0, t0+count) of seq 1 on every layer and
    leaves its other rows (same tiles included) byte-identical."""
    torch = _torch()
    Hkv, layers = 2, 2
    pool = _filled_pool(rkv, ctx, layers, Hkv, D, PT, [300, 300], seed=PT + t0)
    n = pool.r4kv_page_bytes(count, 0, layers - 1)
    staging = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    page = torch.zeros(n, dtype=torch.uint8).pin_memory()
    pool.spill(0, t0, count, 0, layers - 1, _identity(rkv, pos_start=t0), staging, page)
    ctx.sync()
    before = _oracle_body(rkv, rko, pool, 1, 0, 300, 0, layers - 1)
    src = _oracle_body(rkv, rko, pool, 0, 0, 300, 0, layers - 1)
    exp = rkv.R4kvExpect(prefix_digest=0x1234ABCD5678EF01, token_start=t0, pos_start=t0,
                         layer_lo=0, layer_hi=layers - 1, k_fmt=-1, v_fmt=-1, check_generation=0,
                         generation_min=0, generation_max=0)
    pool.restore(1, page.numpy().tobytes(), exp, staging)
    ctx.sync()
    after = _oracle_body(rkv, rko, pool, 1, 0, 300, 0, layers - 1)
    rb = D // 32 * 34
    shape = (layers, 2, Hkv, 300, rb)
    b = np.frombuffer(before, np.uint8).reshape(shape)
    a = np.frombuffer(after, np.uint8).reshape(shape)
    s = np.frombuffer(src, np.uint8).reshape(shape)
    assert np.array_equal(a[:, :, :, t0:t0 + count], s[:, :, :, t0:t0 + count])
    assert np.array_equal(a[:, :, :, :t0], b[:, :, :, :t0])
    assert np.array_equal(a[:, :, :, t0 + count:], b[:, :, :, t0 + count:])
    pool.close()
