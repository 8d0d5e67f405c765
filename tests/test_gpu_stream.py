"""The streaming-read ceiling helper (rkv_stream_read): the vector mode reads
every byte exactly once (the xor of all 32-bit words, against numpy), over
block counts that split the buffer unevenly or leave blocks idle; the
LDS-DMA mode runs; bad arguments are refused before any launch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n16,blocks", [(1, 1), (1, 7), (1000, 3), (65536 + 5, 256),
                                        ((1 << 20) + 37, 2048)])
def test_vector_mode_reads_every_word_once(rkv, ctx, n16, blocks):
    import torch
    rng = np.random.default_rng(n16 + blocks)
    words = rng.integers(0, 1 << 32, 4 * n16, dtype=np.uint32)
    d = torch.from_numpy(words.view(np.int32).copy()).cuda()
    out = torch.full((1,), 12345, dtype=torch.int32, device="cuda")
    rkv.stream_read(ctx, d, 0, blocks, out)
    ctx.sync()
    assert (int(out.item()) & 0xFFFFFFFF) == int(np.bitwise_xor.reduce(words))


def test_dma_mode_runs_and_bad_args_are_refused(rkv, ctx):
    import torch
    blocks = 64
    d = torch.zeros(blocks * rkv.STREAM_DMA_UNIT * 2, dtype=torch.uint8, device="cuda")
    rkv.stream_read(ctx, d, 1, blocks)
    ctx.sync()
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    for mode, nb, nbytes in [(1, blocks, d.numel() - 16),  # not a multiple of blocks * unit
                             (0, blocks, 24),                # not a multiple of 16
                             (2, blocks, 1024),              # unknown mode
                             (0, 0, 1024)]:                  # no blocks
        with pytest.raises(rkv.RkvError):
            rkv.stream_read(ctx, d, mode, nb, out, nbytes=nbytes)
    ctx.sync()


def test_tile_order_read_runs_and_bad_args_are_refused(rkv, ctx):
    """rkv_stream_read_tiles walks a pool's pages through its block tables
    in the decode's tile order; it writes nothing, reports no fault, and
    refuses shapes it does not cover."""
    import torch
    for D, PT in [(256, 64), (128, 32), (256, 256)]:
        print(f"tile-order read D={D} page {PT}", flush=True)
        Hkv, B, L = 2, 3, 4096
        npg = L // PT
        num_pages = B * npg + 5
        g = rkv.geometry(Hkv, D, PT, num_pages)
        pages = torch.zeros(num_pages * rkv.page_bytes(g), dtype=torch.uint8, device="cuda")
        perm = np.random.default_rng(D + PT).permutation(num_pages)[:B * npg]
        bt = torch.from_numpy(perm.reshape(B, npg).astype(np.int32)).cuda()
        bt[1, 3] = num_pages + 7  # outside the pool: read as page 0
        before = pages.clone()
        rkv.stream_read_tiles(ctx, g, pages, bt, npg, B, L, min(64 * PT, 1024))
        # partitions of whole tiles that start inside pages (the decode's
        # lengths in 32-token steps): 96 tokens, and 63 pages plus a tile
        for part in (96, 63 * PT + 32):
            if part < L and part % PT:
                rkv.stream_read_tiles(ctx, g, pages, bt, npg, B, L, part)
        ctx.sync()
        assert torch.equal(pages, before)
    # refusals, on 32-token pages (128 per sequence)
    PT = 32
    npg = L // PT
    g = rkv.geometry(Hkv, 128, PT, B * npg + 5)
    pages = torch.zeros(g.num_pages * rkv.page_bytes(g), dtype=torch.uint8, device="cuda")
    bt = torch.from_numpy(np.arange(B * npg, dtype=np.int32).reshape(B, npg)).cuda()
    rkv.stream_read_tiles(ctx, g, pages, bt, npg, B, L, 64 * PT)  # 64 pages: accepted
    for bt_stride, n, L, part in [(npg, B, L + 16, 1024),   # not a multiple of 32
                                  (npg, B, L, 48),          # not a multiple of 32
                                  (npg, B, L, 64 * PT + 32),  # the first partition spans 65 pages
                                  (npg - 1, B, L, 1024),     # rows too short
                                  (npg, 0, L, 1024)]:        # no sequences
        with pytest.raises(rkv.RkvError):
            rkv.stream_read_tiles(ctx, g, pages, bt, bt_stride, n, L, part)
    g16 = rkv.geometry(Hkv, 256, 16, num_pages)
    with pytest.raises(rkv.RkvError):  # 16-token pages are not covered
        rkv.stream_read_tiles(ctx, g16, pages, bt, npg, B, L, 256)
    ctx.sync()
