"""Attention over V of any magnitude, on the GPU against the oracle.

The PV weights are f16 products of p and the V scale (two terms).  V rows of
small magnitude (|v| ~ 1e-3, scales ~ 1e-5) would put those products in the
f16 subnormal range, where the reference's f32 dequantization
(attention.rs:79-112, 169-215) keeps full precision; the kernels scale each
tile's V scales by a power of two first (Decoder::scale_v).  Every PV form
is covered: the 8-row decode, the 16-row bf16-query decode, the 32-row
verify with a bf16 query (head dimension split over two waves) and with an
f32 query, 16-token pages, the prefill with both query types, all-zero V,
and partitions whose V magnitude rises or falls by 2^18 partway through
(the scale exponent then changes mid-partition).  Bars as in
test_gpu_parity.py."""
import math

import numpy as np
import pytest

from tests.test_gpu_parity import Scene, _bind_ctx, _run_decode, assert_close  # noqa: F401
from tests.test_gpu_prefill import _run as _run_prefill

pytestmark = pytest.mark.gpu


def _rise(pos):
    return np.where(pos < 2000, 1e-4, 30.0)


def _fall(pos):
    return np.where(pos < 2000, 30.0, 1e-4)


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_len,q_bf16,v_mul,part", [
    (16, 2, 256, 64, [3000, 700], 1, False, 1e-3, 0),    # 8 rows, int8 query planes
    (16, 2, 256, 64, [3000, 700], 1, False, 1e-5, 0),
    (32, 2, 128, 64, [2000, 333], 1, True, 1e-3, 0),     # 16 rows, f16 QK
    (16, 2, 256, 64, [1500, 900], 4, True, 1e-3, 0),     # verify, split head dimension
    (16, 2, 256, 64, [1500, 900], 4, False, 1e-4, 0),    # verify, f32 query
    (8, 2, 128, 16, [1000, 77], 1, False, 1e-3, 0),      # 16-token pages
    (16, 2, 256, 16, [1200, 50], 4, True, 1e-3, 0),      # 16-token pages, bf16 verify
    (16, 2, 256, 64, [700, 33], 1, False, 0.0, 0),       # all-zero V
    (16, 2, 256, 64, [4000], 1, False, _rise, 4096),     # one partition, V rises
    (16, 2, 256, 64, [4000], 1, False, _fall, 4096),     # one partition, V falls
    (16, 2, 256, 64, [4000, 2100], 4, True, _rise, 4096),
])
def test_decode_v_magnitudes(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_len, q_bf16, v_mul, part):
    name = getattr(v_mul, "__name__", v_mul)
    print(f"v range Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens} q_len={q_len} v={name}",
          flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=D + PT + q_len, outliers=0.01, src_bf16=True,
               v_mul=v_mul)
    rng = np.random.default_rng(Hq + D + q_len)
    q = rng.standard_normal((len(lens), q_len, Hq, D)).astype(np.float32)
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / math.sqrt(D)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=q_bf16, q_len=q_len,
                          partition_tokens=part)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, scale, pt)
    assert_close(got, want, what=f"v={name} rows={q_len * Hq // Hkv} pt={pt}")


@pytest.mark.parametrize("Hq,Hkv,D,PT,entries,q_bf16,v_mul", [
    (16, 2, 256, 64, [(0, 40), (300, 17), (1000, 70)], True, 1e-3),
    (8, 2, 128, 16, [(200, 100), (0, 33)], False, 1e-5),
    (16, 2, 256, 64, [(3900, 64)], True, _rise),
    (16, 2, 256, 64, [(3900, 64)], False, _fall),
])
def test_prefill_v_magnitudes(rkv, rko, ctx, Hq, Hkv, D, PT, entries, q_bf16, v_mul):
    name = getattr(v_mul, "__name__", v_mul)
    print(f"prefill v range Hq={Hq} D={D} PT={PT} entries={entries} v={name}", flush=True)
    lens = [c + n + 1 for c, n in entries]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=5 + D + PT, outliers=0.01, src_bf16=True,
               v_mul=v_mul)
    ent = [(i, c, n) for i, (c, n) in enumerate(entries)]
    _run_prefill(rkv, rko, ctx, sc, ent, Hq, 1.0 / np.sqrt(D), q_bf16, seed=D)
