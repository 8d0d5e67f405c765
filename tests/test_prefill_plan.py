"""Host-side plan of the prefill's split-K (no GPU): rkv_prefill_workspace_bytes
runs the same plan rkv_prefill_q8 launches, so its byte counts pin how many
segments each entry's causal range gets.  Workspace = (m, l) rows padded to
256 bytes + o rows, P = sum over split entries of rows * q_heads * nseg.
Launch shapes follow bench.py --config 7 (Hq=16, Hkv=2, D=256, page 64)."""
import pytest


def _ws_bytes(P, D=256):
    return (P * 8 + 255) // 256 * 256 + P * D * 4


@pytest.fixture(scope="module")
def plan(rkv):
    torch = pytest.importorskip("torch")
    g = rkv.Geometry(2, 256, 64, 1 << 20)

    def bytes_for(ctxs, rows, seg=0, Hq=16):
        q = torch.empty((max(sum(rows), 1), Hq, 256))
        a = rkv.prefill_args(list(range(len(rows))), ctxs, rows, q, q, 1.0, segment_tokens=seg)
        return rkv.prefill_workspace_bytes(g, a)
    return bytes_for


def test_balanced_launches_stay_unsplit(plan):
    assert plan([8192] * 8, [512] * 8) == 0          # config 7: two units per CU already
    assert plan([16384] * 2, [1024] * 2) == 0        # 256 equal units on 256 CUs
    assert plan([0], [4096]) == 0                     # 512 units
    assert plan([32768], [512], seg=-1) == 0          # never split


def test_few_row_blocks_split(plan):
    # one 512-row chunk after 32768 tokens: 64 units -> 4 segments a block (256 units)
    assert plan([32768], [512]) == _ws_bytes(512 * 16 * 4)
    # three such chunks after 16384 tokens: 192 units -> 4 segments (768 units, 3 per CU)
    assert plan([16384] * 3, [512] * 3) == _ws_bytes(3 * 512 * 16 * 4)


def test_one_long_range_among_short_ones_splits(plan):
    # a serving step's lognormal contexts: only the long entry is cut
    ctxs = [65536, 10180, 10143, 6878, 5370, 2694, 1238, 544]
    assert plan(ctxs, [512] * 8) == _ws_bytes(512 * 16 * 4)


def test_explicit_segments(plan):
    # 128-token segments: ceil(1070 / 128) = 9 segments for the first entry;
    # the second (40 tokens) stays whole
    assert plan([1000, 0], [70, 40], seg=128) == _ws_bytes(70 * 16 * 9)
    # rounded up to the page (64) and capped at 64 segments: 2533 tokens in
    # 32-token segments become ceil(2533 / 64) = 40 segments of 64
    assert plan([2500], [33], seg=32) == _ws_bytes(33 * 16 * 40)
