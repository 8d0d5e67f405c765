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
