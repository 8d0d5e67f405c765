"""Softmax scales of either sign and zero, and all-zero query rows, on the
GPU against the oracle.

The kernels store a query row times the sign of the softmax scale (as int8
planes or, for a bf16 query, times a power of two in f16) and keep a
positive multiplier per row, |scale| times the row's own scale and at
least FLT_MIN: the softmax takes the maximum of the unscaled scores, scales
it once, and forms every exponent as one fma of an unscaled score.  The
oracle applies the scale to q in f32 before the reference's loop
(attention.rs:148-165 takes q as given), so a negative scale reverses the
order of the scores and a zero scale (or a zero query row) makes the
softmax uniform over the visible positions.  Every QK form is covered: the
8-row three-plane query, the 16-row f16 QK, the 32-row verify with a bf16
query (head dimension split over two waves) and with an f32 query, 16-token
pages, and the prefill with both query types, with and without the
widen-once workspace.  Bars as in test_gpu_parity.py."""
import math

import numpy as np
import pytest

from tests.test_gpu_parity import Scene, _bind_ctx, _run_decode, assert_close  # noqa: F401
from tests.test_gpu_prefill import _run as _run_prefill

pytestmark = pytest.mark.gpu

SIGNS = [-1.0, 0.0]


@pytest.mark.parametrize("sign", SIGNS)
@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_len,q_bf16", [
    (16, 2, 256, 64, [3000, 700], 1, False),   # 8 rows, int8 query planes
    (32, 2, 128, 64, [2000, 333], 1, True),    # 16 rows, f16 QK
    (16, 2, 256, 64, [1500, 900], 4, True),    # verify, split head dimension
    (16, 2, 256, 64, [1500, 900], 4, False),   # verify, f32 query
    (8, 2, 128, 16, [1000, 77], 1, False),     # 16-token pages
])
def test_decode_scale_sign(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_len, q_bf16, sign):
    print(f"scale sign {sign} Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens} q_len={q_len} "
          f"bf16={q_bf16}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=3 * D + PT + q_len, outliers=0.01, src_bf16=True)
    rng = np.random.default_rng(Hq + D + q_len + 7)
    q = rng.standard_normal((len(lens), q_len, Hq, D)).astype(np.float32)
    # all-zero rows: the first head of the first entry, the last head of the
    # last entry's last draft
    q[0, 0, 1, :] = 0.0
    q[-1, -1, Hq - 1, :] = 0.0
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = sign / math.sqrt(D)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=q_bf16, q_len=q_len)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, scale, pt)
    assert np.all(np.isfinite(got))
    assert_close(got, want, what=f"scale={scale:+.4f} rows={q_len * Hq // Hkv} pt={pt}")
    if sign == 0.0:
        # uniform softmax: the zero-scale output does not depend on q
        assert_close(got[0, 0, 0], got[0, 0, 1], atol=1e-5, rtol=1e-5, what="zero scale rows")


@pytest.mark.parametrize("sign", SIGNS)
@pytest.mark.parametrize("Hq,Hkv,D,PT,entries,q_bf16,segment", [
    (16, 2, 256, 64, [(0, 40), (300, 17), (1000, 70)], True, None),
    (16, 2, 256, 64, [(0, 40), (300, 17), (1000, 70)], True, 0),   # widen-once workspace
    (8, 2, 128, 16, [(200, 100), (0, 33)], False, None),
])
def test_prefill_scale_sign(rkv, rko, ctx, Hq, Hkv, D, PT, entries, q_bf16, segment, sign):
    print(f"prefill scale sign {sign} Hq={Hq} D={D} PT={PT} entries={entries} bf16={q_bf16} "
          f"segment={segment}", flush=True)
    lens = [c + n + 1 for c, n in entries]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=11 + D + PT, outliers=0.01, src_bf16=True)
    ent = [(i, c, n) for i, (c, n) in enumerate(entries)]
    _run_prefill(rkv, rko, ctx, sc, ent, Hq, sign / math.sqrt(D), q_bf16, seed=D + 1,
                 segment_tokens=segment)
