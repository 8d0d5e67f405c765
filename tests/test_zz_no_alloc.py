"""rkv_decode_q8_noalloc: the split-K decode with its partials in the
library's static device scratch (no allocation, no workspace argument),
against rkv_decode_q8 with a caller workspace, through the C ABI.  Results
are compared bit for bit: both calls run the same kernels on the same
workspace layout."""
import math

import numpy as np
import pytest

from tests.test_gpu_parity import Scene, _bind_ctx  # noqa: F401

pytestmark = pytest.mark.gpu


def _pair(rkv, ctx, sc, B, Hq, q_len, max_len, seed, partition_tokens=0):
    import torch
    D = sc.D
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    q = torch.randn((B, q_len, Hq, D), generator=gen, device="cuda").to(torch.bfloat16)
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    out_ws = torch.full((B, q_len, Hq, D), float("nan"), device="cuda")
    out_na = torch.full((B, q_len, Hq, D), float("nan"), device="cuda")
    a = rkv.decode_args(q, out_ws, sid, 1.0 / math.sqrt(D), max_len, q_len=q_len,
                        partition_tokens=partition_tokens)
    nbytes = rkv.decode_workspace_bytes(sc.g, a)
    assert 0 < nbytes <= rkv.DECODE_SCRATCH_BYTES, nbytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    a = rkv.decode_args(q, out_ws, sid, 1.0 / math.sqrt(D), max_len, q_len=q_len,
                        partition_tokens=partition_tokens, workspace=ws)
    rkv.decode_q8(ctx, sc.g, sc.pages_d, sc.bt_d, sc.lens_d, a)
    b = rkv.decode_args(q, out_na, sid, 1.0 / math.sqrt(D), max_len, q_len=q_len,
                        partition_tokens=partition_tokens)
    rkv.decode_q8_noalloc(ctx, sc.g, sc.pages_d, sc.bt_d, sc.lens_d, b)
    ctx.sync()
    return out_ws.cpu().numpy(), out_na.cpu().numpy()


def test_decode_noalloc_matches_workspace_decode(rkv, rko, ctx):
    """Two calls in a row, the second on a smaller input (fewer entries,
    shorter sequences, other partitions): each equals rkv_decode_q8 bit for
    bit.  Then a call whose partials exceed the scratch is refused."""
    import torch
    Hq, Hkv, D, PT = 16, 2, 256, 64
    lens = [9000, 4100, 7000, 300, 12000, 64, 2500, 5000]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=31, src_bf16=True)
    ws, na = _pair(rkv, ctx, sc, len(lens), Hq, 1, max(lens), seed=1)
    print(f"noalloc call 1: B={len(lens)} max_len={max(lens)} equal={np.array_equal(ws, na)}", flush=True)
    assert np.all(np.isfinite(na)) and np.array_equal(ws, na)
    # second call, smaller: 3 entries, q_len 2 (16 rows per kv head), an
    # explicit partition length, reading what the first call left behind
    ws, na = _pair(rkv, ctx, sc, 3, Hq, 2, max(lens[:3]), seed=2, partition_tokens=512)
    print(f"noalloc call 2: B=3 q_len=2 equal={np.array_equal(ws, na)}", flush=True)
    assert np.all(np.isfinite(na)) and np.array_equal(ws, na)
    # partials past the static scratch: refused before any launch
    B, L = 64, 32768
    q = torch.zeros((B, 1, Hq, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((B, 1, Hq, D), device="cuda")
    sid = torch.zeros(B, dtype=torch.int32, device="cuda")
    a = rkv.decode_args(q, out, sid, 1.0, L, partition_tokens=256)
    assert rkv.decode_workspace_bytes(sc.g, a) > rkv.DECODE_SCRATCH_BYTES
    with pytest.raises(rkv.RkvError) as e:
        rkv.decode_q8_noalloc(ctx, sc.g, sc.pages_d, sc.bt_d, sc.lens_d, a)
    assert e.value.status == rkv.ERR_INVALID_ARG and "static scratch" in str(e.value)
