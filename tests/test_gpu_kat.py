"""The r4kv KAT lane (repro/r4kv/storage/sanitized_receipt.json:29-34, generated
by tools/repro-harness/src/main.rs:97-175) through the device quantizer.

The receipt's source vector (seeded_float(i), i < 4096; its sha256 is pinned
in tests/test_oracle_kat.py) shifted to positive = |x| + 0.125 is appended as
16 rows of 256 values by rkv_append_q8 with the canonical rule, gathered back
in the reference row layout, and then:
  - the page bytes equal the oracle's Q8_0 encoder (r4kv/src/quant.rs:45-90)
    byte for byte, for K and V;
  - decoding those device bytes reproduces the receipt's BASE-Q8 numbers
    exactly: max-abs, rel-rms (quant.rs:27-32, 228-245) and the positive-proxy
    forward KL (main.rs:192-204).
"""
import json
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kat.json")


def _f32(x) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def test_r4kv_kat_lane_through_device_quantizer(rkv, rko, ctx):
    import torch
    want = json.load(open(GOLDEN))["r4kv_receipt"]["BASE-Q8"]
    src = np.array([rko.seeded_float(i) for i in range(4096)], np.float32)
    pos = (np.abs(src) + np.float32(0.125)).astype(np.float32)
    D, PT, rows = 256, 64, 4096 // 256
    g = rkv.geometry(1, D, PT, 2)
    pages = torch.zeros(2 * rkv.page_bytes(g), dtype=torch.uint8, device="cuda")
    bt = torch.tensor([1], dtype=torch.int32, device="cuda")  # the second page of the pool
    x = torch.from_numpy(pos.reshape(rows, 1, D)).cuda()
    rkv.append_q8(ctx, g, pages, bt[None], torch.zeros(rows, dtype=torch.int32, device="cuda"),
                  torch.arange(rows, dtype=torch.int32, device="cuda"), x, x, rule=0)
    ref_bytes = rko.q8_encode(pos)
    for kind in (0, 1):
        out = torch.empty(rows * rkv.row_bytes(D), dtype=torch.uint8, device="cuda")
        rkv.gather_q8(ctx, g, pages, bt, rows, kind, out)
        ctx.sync()
        dev_bytes = out.cpu().numpy()
        assert np.array_equal(dev_bytes, ref_bytes), f"kind {kind}: device bytes differ"
        dec = rko.q8_decode(dev_bytes, pos.size)
        # the receipt's sums run in f64 in element order (quant.rs:228-245)
        err = (pos - dec).astype(np.float32).astype(np.float64)
        max_abs = float(np.float32(np.max(np.abs(err))))
        se = sr = 0.0
        for e, r in zip(err.tolist(), pos.astype(np.float64).tolist()):
            se += e * e
            sr += r * r
        rel = _f32((se / sr) ** 0.5)
        kl = rko.normalized_kl(pos, dec)
        print(f"[KAT kind {kind}] max_abs={max_abs!r} rel_rms={rel!r} kl={kl!r}", flush=True)
        assert max_abs == want["value_roundtrip_max_abs_error"]
        assert rel == _f32(want["value_roundtrip_rel_rms"])
        assert kl == want["positive_proxy_forward_kl"]
