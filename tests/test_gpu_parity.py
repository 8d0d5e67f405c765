"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars:
  - page bytes, scales and block-table gathers: bit-exact;
  - attention outputs: max |gpu - oracle| <= 2e-3 and
    ||gpu - oracle||_2 / ||oracle||_2 <= 1e-3 over the output tensor.
The oracle decodes with the reference's chunked loop (attention.rs:169-215)
using chunk = the kernel's partition length; q is prescaled by `scale` in f32
(the reference itself applies no scale).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    den = float(np.linalg.norm(want))
    rel = float(np.linalg.norm(got - want)) / den if den > 0 else float(np.linalg.norm(got))
    print(f"[{what}] max_abs={err:.3e} rel={rel:.3e}", flush=True)
    assert err <= atol, f"{what}: max abs err {err:.3e} > {atol}"
    assert rel <= rtol, f"{what}: rel err {rel:.3e} > {rtol}"


def _torch():
    import torch
    return torch


class Scene:
    """A shuffled page pool holding B sequences of the given lengths."""

    def __init__(self, rkv, rko, Hkv, D, PT, lens, seed=0, slack=1.1, outliers=0.0,
                 src_bf16=False, rule=0, extra_rows=None, v_mul=None):
        torch = _torch()
        rng = np.random.default_rng(seed)
        self.Hkv, self.D, self.PT = Hkv, D, PT
        self.lens = np.asarray(lens, np.int32)
        B = len(lens)
        npg = [(int(L) + PT - 1) // PT for L in lens]
        self.W = max(max(npg), 1)
        self.num_pages = max(int(math.ceil(sum(npg) * slack)) + 1, 2)
        perm = rng.permutation(self.num_pages).astype(np.int32)
        self.bt = np.full((B, self.W), -1, np.int32)
        o = 0
        for b in range(B):
            self.bt[b, :npg[b]] = perm[o:o + npg[b]]
            o += npg[b]
        self.g = rkv.geometry(Hkv, D, PT, self.num_pages)
        self.lay = rko.layout(Hkv, D, PT, self.num_pages)
        n = int(self.lens.sum())
        k = rng.standard_normal((n, Hkv, D)).astype(np.float32)
        v = rng.standard_normal((n, Hkv, D)).astype(np.float32)
        if outliers:
            nch = max(1, int(math.ceil(outliers * D)))
            for h in range(Hkv):
                ch = rng.choice(D, nch, replace=False)
                k[:, h, ch] *= 8
                v[:, h, ch] *= 8
        if v_mul is not None:
            # V magnitude: a factor, or a function of each row's position
            pos = np.concatenate([np.arange(L) for L in lens]) if n else np.zeros(0, np.int64)
            m = v_mul(pos) if callable(v_mul) else np.full(n, v_mul)
            v *= np.asarray(m, np.float32)[:, None, None]
        if src_bf16:
            k = rko.bf16_to_f32(rko.f32_to_bf16(k)).reshape(k.shape)
            v = rko.bf16_to_f32(rko.f32_to_bf16(v)).reshape(v.shape)
        self.k, self.v = k, v
        self.seq_ids = np.repeat(np.arange(B, dtype=np.int32), self.lens)
        self.pos = np.concatenate([np.arange(L, dtype=np.int32) for L in lens]) if n else \
            np.zeros(0, np.int32)
        # device
        dev = "cuda"
        pb = rkv.page_bytes(self.g)
        self.pages_d = torch.zeros(self.num_pages * pb, dtype=torch.uint8, device=dev)
        self.bt_d = torch.from_numpy(self.bt).to(dev)
        self.lens_d = torch.from_numpy(self.lens).to(dev)
        if n:
            sd = torch.from_numpy(self.seq_ids).to(dev)
            pd = torch.from_numpy(self.pos).to(dev)
            if src_bf16:
                kd = torch.from_numpy(k).to(dev).to(torch.bfloat16)
                vd = torch.from_numpy(v).to(dev).to(torch.bfloat16)
            else:
                kd = torch.from_numpy(k).to(dev)
                vd = torch.from_numpy(v).to(dev)
            rkv.append_q8(self.ctx_holder[0], self.g, self.pages_d, self.bt_d, sd, pd, kd, vd,
                          rule=rule)
        # oracle
        self.pages = np.zeros(self.num_pages * pb, np.uint8)
        if n:
            rko.paged_append(self.lay, self.pages, self.bt, self.seq_ids, self.pos, k, v, rule)

    ctx_holder = [None]


@pytest.fixture(autouse=True)
def _bind_ctx(ctx):
    Scene.ctx_holder[0] = ctx
    yield


def _run_decode(rkv, ctx, sc, q_np, scale, q_bf16=False, q_len=1, partition_tokens=0,
                out_bf16=False, seq_ids=None):
    torch = _torch()
    B = q_np.shape[0] if seq_ids is None else len(seq_ids)
    sid = np.arange(B, dtype=np.int32) if seq_ids is None else np.asarray(seq_ids, np.int32)
    qd = torch.from_numpy(q_np).cuda()
    if q_bf16:
        qd = qd.to(torch.bfloat16)
    out = torch.empty(q_np.shape, dtype=torch.bfloat16 if out_bf16 else torch.float32, device="cuda")
    sid_d = torch.from_numpy(sid).cuda()
    a = rkv.decode_args(qd, out, sid_d, scale, int(sc.lens.max()) if len(sc.lens) else 0,
                        q_len=q_len, partition_tokens=partition_tokens)
    ws_bytes = rkv.decode_workspace_bytes(sc.g, a)
    ws = torch.zeros(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    a = rkv.decode_args(qd, out, sid_d, scale, int(sc.lens.max()) if len(sc.lens) else 0,
                        q_len=q_len, partition_tokens=partition_tokens, workspace=ws)
    # the oracle's chunk: the explicit partition, else any (the online softmax
    # is chunk-invariant up to rounding)
    pt = rkv.decode_partition_tokens(sc.g, a) or 1024
    rkv.decode_q8(ctx, sc.g, sc.pages_d, sc.bt_d, sc.lens_d, a)
    ctx.sync()
    return out.float().cpu().numpy(), pt


# ---- binary16 encoders ---------------------------------------------------------

def test_f16_encoders_bitexact(rkv, rko, ctx):
    torch = _torch()
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2 ** 32, 60000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    # scales d = amax/127 span small positive values: sample them densely
    d = (rng.uniform(0, 1, 60000) * 2.0 ** rng.integers(-40, 18, 60000)).astype(np.float32)
    edges = []
    for k in range(-26, 17):
        base = np.float32(2.0 ** k)
        edges += [base, np.float32(base * (2 - 2.0 ** -11)), np.float32(base * (2 - 2.0 ** -12)),
                  np.float32(base * (1 + 2.0 ** -11)), np.nextafter(base, np.float32(0))]
    edges += [0.0, -0.0, np.inf, -np.inf, np.nan, 65504, 65520, 65519.99]
    x = np.concatenate([x, d, -d[:1000], np.array(edges, np.float32)]).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    L = rko.lib()
    for rule, fn in ((0, L.rko_f32_to_f16), (1, L.rko_f32_to_f16_harserve)):
        out = torch.empty(x.size, dtype=torch.int16, device="cuda")
        rkv.f32_to_f16(ctx, xd, out, rule)
        ctx.sync()
        got = out.cpu().numpy().view(np.uint16)
        want = np.array([fn(float(v)) for v in x], np.uint16)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"rule {rule}: {bad.size} mismatches, first x={x[bad[:3]]}"


# ---- append / gather / import ----------------------------------------------------

@pytest.mark.parametrize("D,PT,rule,bf16", [
    (128, 16, 0, False), (256, 64, 0, True), (256, 64, 1, False), (256, 32, 0, False),
    (128, 256, 1, True), (256, 16, 0, False)])
def test_append_bitexact(rkv, rko, ctx, D, PT, rule, bf16):
    print(f"append D={D} PT={PT} rule={rule} bf16={bf16}", flush=True)
    sc = Scene(rkv, rko, 2, D, PT, [3 * PT + 7, 1, 2 * PT], seed=D + PT + rule, outliers=0.01,
               src_bf16=bf16, rule=rule)
    ctx.sync()
    assert np.array_equal(sc.pages_d.cpu().numpy(), sc.pages), "page bytes differ"
    torch = _torch()
    for b, L in enumerate(sc.lens):
        for kind, src in ((0, sc.k), (1, sc.v)):
            out = torch.empty(2 * int(L) * rkv.row_bytes(D), dtype=torch.uint8, device="cuda")
            rkv.gather_q8(ctx, sc.g, sc.pages_d, sc.bt_d[b], int(L), kind, out)
            ctx.sync()
            got = out.cpu().numpy().reshape(2, L, -1)
            rows = src[sc.seq_ids == b]
            for h in range(2):
                want = rko.q8_quantize(rows[:, h, :].reshape(-1), rule).reshape(L, -1)
                assert np.array_equal(got[h], want), f"seq {b} kind {kind} head {h}"


@pytest.mark.parametrize("D,PT,order,big", [
    (256, 64, "chunks", False), (256, 64, "shuffled", False), (128, 16, "interleaved", False),
    (256, 32, "bad_rows", False), (128, 128, "chunks", False), (256, 16, "shuffled", False),
    # >= 32768 rows x 2 kv heads: the 32-row workgroups
    (256, 64, "shuffled", True), (128, 32, "chunks", True)])
def test_append_row_orders(rkv, rko, ctx, D, PT, order, big):
    """The append kernel quantizes 8 or 32 input rows per workgroup and
    writes 4 aligned consecutive slots of a page with one store: the page
    bytes equal the oracle's for rows in any order -- chunks starting
    mid-tile, shuffled rows, two sequences interleaved row by row, and
    invalid rows inside a group (reported, nothing written for them)."""
    torch = _torch()
    Hkv = 2
    rng = np.random.default_rng(D + PT + len(order) + big)
    lens = [20000, 13000, 5003] if big else [700, 413, 97]
    npg = [(L + PT - 1) // PT for L in lens]
    num_pages = sum(npg) + 5
    perm = rng.permutation(num_pages).astype(np.int32)
    W = max(npg)
    bt = np.full((3, W), -1, np.int32)
    o = 0
    for b in range(3):
        bt[b, :npg[b]] = perm[o:o + npg[b]]
        o += npg[b]
    sid = np.concatenate([np.full(L, b, np.int32) for b, L in enumerate(lens)])
    pos = np.concatenate([np.arange(L, dtype=np.int32) for L in lens])
    if order == "chunks":      # prefill-like chunks starting at unaligned positions
        L0, L1 = lens[0], lens[1]
        cuts = sorted({0, 13, 77, 300, 301, L0, L0 + 5, L0 + L1, len(sid)})
        idx = np.concatenate([np.arange(cuts[i], cuts[i + 1]) for i in rng.permutation(len(cuts) - 1)])
    elif order == "interleaved":
        a, b2 = np.arange(0, 413), np.arange(700, 700 + 413)
        idx = np.concatenate([np.stack([a, b2], 1).reshape(-1), np.arange(413, 700),
                              np.arange(1113, len(sid))])
    else:
        idx = rng.permutation(len(sid)) if order == "shuffled" else np.arange(len(sid))
    sid, pos = sid[idx], pos[idx]
    k = rng.standard_normal((len(sid), Hkv, D)).astype(np.float32)
    v = rng.standard_normal((len(sid), Hkv, D)).astype(np.float32)
    bad = np.zeros(len(sid), bool)
    if order == "bad_rows":    # a bad sequence id, a position past the table, a -1 page
        bad[[5, 40, 41]] = True
        sid[5] = 7
        pos[40] = W * PT + 3
        pos[41] = -1
        bt[2, npg[2] - 1] = -1
        bad |= (sid == 2) & (pos // PT == npg[2] - 1)
    g = rkv.geometry(Hkv, D, PT, num_pages)
    lay = rko.layout(Hkv, D, PT, num_pages)
    want = np.zeros(num_pages * rkv.page_bytes(g), np.uint8)
    rko.paged_append(lay, want, bt, sid[~bad], pos[~bad], k[~bad], v[~bad], 0)
    pages = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    rkv.append_q8(ctx, g, pages, torch.from_numpy(bt).cuda(), torch.from_numpy(sid).cuda(),
                  torch.from_numpy(pos).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    if bad.any():
        with pytest.raises(rkv.RkvError) as e:
            ctx.sync()
        assert e.value.status == rkv.ERR_BAD_BLOCK_TABLE
    ctx.sync()
    got = pages.cpu().numpy()
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} page bytes differ"


def test_append_special_values(rkv, rko, ctx):
    """Zero blocks, huge (f16-overflowing scale), tiny (subnormal scale), inf and
    NaN inputs quantize identically on both sides, for both rules."""
    torch = _torch()
    D, PT, Hkv = 256, 64, 1
    rng = np.random.default_rng(5)
    rows = rng.standard_normal((6, Hkv, D)).astype(np.float32)
    rows[0, 0, :32] = 0
    rows[1, 0, :] *= np.float32(3e6)
    rows[2, 0, :] *= np.float32(1e-9)
    rows[3, 0, 5] = np.inf
    rows[4, 0, 40] = np.nan
    rows[5, 0, 64:96] = np.float32(2.0 ** -5 * (2 - 2.0 ** -12) * 127)  # carry window
    for rule in (0, 1):
        g = rkv.geometry(Hkv, D, PT, 2)
        lay = rko.layout(Hkv, D, PT, 2)
        bt = np.array([[1]], np.int32)
        pages = np.zeros(2 * rkv.page_bytes(g), np.uint8)
        sid = np.zeros(6, np.int32)
        pos = np.arange(6, dtype=np.int32)
        rko.paged_append(lay, pages, bt, sid, pos, rows, rows, rule)
        pd = torch.zeros(pages.size, dtype=torch.uint8, device="cuda")
        rkv.append_q8(ctx, g, pd, torch.from_numpy(bt).cuda(), torch.from_numpy(sid).cuda(),
                      torch.from_numpy(pos).cuda(), torch.from_numpy(rows).cuda(),
                      torch.from_numpy(rows).cuda(), rule=rule)
        ctx.sync()
        assert np.array_equal(pd.cpu().numpy(), pages), f"rule {rule}"


@pytest.mark.parametrize("D,src_bf16", [(128, False), (256, True)])
def test_append_special_values_large_launch(rkv, rko, ctx, D, src_bf16):
    """The same special blocks through a launch of 8192 rows x 8 kv heads, which
    takes the 32-row tiles with one lane per 32-value block (a small launch
    takes 8-row tiles with four lanes per block): zero, huge, tiny, inf and
    NaN blocks, the f16 carry window, and exact ties k + 0.5 (amax 127, so
    d = 1 and v * (1/d) = v) that round half away from zero.  Page bytes
    equal the oracle's for both rules."""
    torch = _torch()
    PT, Hkv, L = 64, 8, 8192
    NB = D // 32
    rng = np.random.default_rng(D + 3)
    rows = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    blocks = rows.reshape(L, Hkv, NB, 32)
    kinds = rng.integers(0, 7, (L, Hkv, NB))
    pick = rng.random((L, Hkv, NB)) < 0.05  # about 5% of the blocks are special
    ties = (rng.integers(-127, 127, 32) + 0.5).astype(np.float32)
    ties[0] = 127.0  # amax 127: d = 1 exactly
    for t in range(7):
        sel = pick & (kinds == t)
        if t == 0:
            blocks[sel] = 0.0
        elif t == 1:
            blocks[sel] *= np.float32(3e6)
        elif t == 2:
            blocks[sel] *= np.float32(1e-9)
        elif t == 3:
            blocks[sel, 5] = np.inf
        elif t == 4:
            blocks[sel, 17] = np.nan
        elif t == 5:
            blocks[sel] = np.float32(2.0 ** -5 * (2 - 2.0 ** -12) * 127)
        else:
            blocks[sel] = ties
    if src_bf16:
        src = torch.from_numpy(rows).to(torch.bfloat16)
        rows = src.float().numpy()  # the values the kernel reads
    else:
        src = torch.from_numpy(rows)
    npg = L // PT
    bt = rng.permutation(npg + 3)[:npg].astype(np.int32)[None, :]
    sid = np.zeros(L, np.int32)
    pos = np.arange(L, dtype=np.int32)
    sd = src.cuda()
    for rule in (0, 1):
        g = rkv.geometry(Hkv, D, PT, npg + 3)
        lay = rko.layout(Hkv, D, PT, npg + 3)
        want = np.zeros((npg + 3) * rkv.page_bytes(g), np.uint8)
        rko.paged_append(lay, want, bt, sid, pos, rows, rows, rule)
        pd = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
        rkv.append_q8(ctx, g, pd, torch.from_numpy(bt).cuda(), torch.from_numpy(sid).cuda(),
                      torch.from_numpy(pos).cuda(), sd, sd, rule=rule)
        ctx.sync()
        got = pd.cpu().numpy()
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"rule {rule}: {bad.size} bytes differ, first at {bad[:4]}"


@pytest.mark.parametrize("D,PT", [(128, 16), (256, 64), (256, 32)])
def test_import_gather_roundtrip(rkv, rko, ctx, D, PT):
    torch = _torch()
    rng = np.random.default_rng(D * PT)
    L, Hkv = 5 * PT + 3, 2
    npg = (L + PT - 1) // PT
    g = rkv.geometry(Hkv, D, PT, npg + 4)
    bt = rng.permutation(npg + 4)[:npg].astype(np.int32)
    rows = rng.integers(0, 256, (Hkv, L, rkv.row_bytes(D)), dtype=np.uint8)
    pages = torch.zeros((npg + 4) * rkv.page_bytes(g), dtype=torch.uint8, device="cuda")
    btd = torch.from_numpy(bt).cuda()
    rd = torch.from_numpy(rows).cuda()
    for kind in (0, 1):
        rkv.import_q8(ctx, g, pages, btd, L, kind, rd)
        out = torch.empty_like(rd)
        rkv.gather_q8(ctx, g, pages, btd, L, kind, out)
        ctx.sync()
        assert np.array_equal(out.cpu().numpy(), rows)
    # the oracle reads the same page bytes back the same way
    lay = rko.layout(Hkv, D, PT, npg + 4)
    got = rko.paged_gather(lay, pages.cpu().numpy(), bt, L, 1)
    assert np.array_equal(got, rows)


# ---- decode ------------------------------------------------------------------------

def test_config1_decode(rkv, rko, ctx):
    """1 sequence, Hq 8 / Hkv 2, D 128, 16-token pages, 2048
    context, f32 K/V and q ~ N(0,1), scale 1/sqrt(128), seeded permutation."""
    sc = Scene(rkv, rko, 2, 128, 16, [2048], seed=0)
    rng = np.random.default_rng(100)
    q = rng.standard_normal((1, 1, 8, 128)).astype(np.float32)
    scale = 1.0 / math.sqrt(128)
    for pt_req in (0, 256, 1024):
        got, pt = _run_decode(rkv, ctx, sc, q, scale, partition_tokens=pt_req)
        want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(1, dtype=np.int32),
                                q, scale, pt)
        assert_close(got, want, what=f"config1 pt={pt}")


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_bf16,out_bf16", [
    (16, 2, 256, 64, [4100, 700, 33, 1, 2000], True, False),
    (16, 2, 256, 32, [1500, 31, 64], True, False),
    (8, 4, 256, 64, [1024, 999], False, False),
    (4, 4, 128, 16, [517, 64, 1], False, True),
    (32, 2, 128, 128, [3000], True, False),
    # a few tokens each: the outlier channels (|v| up to ~30) are averaged
    # over almost nothing, so every weight's rounding shows
    (16, 2, 256, 64, [2, 3, 5, 9, 17, 40], True, False),
    # the reference's own geometry: FlashDecodeParams::default() 24 q / 4 kv
    # heads (attention.rs:134-137), KVGeometry::qwen36_27b D 256 with
    # 32-token pages (har-kv/src/geometry.rs:39-59): 6 rows per kv head
    (24, 4, 256, 32, [3000, 517, 33, 1, 1200], True, False),
    (24, 4, 256, 32, [2100, 64, 7], False, False),
    (24, 4, 256, 32, [900, 31], True, True),
])
def test_decode_parity(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_bf16, out_bf16):
    print(f"decode Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=Hq + D + PT, outliers=0.01, src_bf16=True)
    rng = np.random.default_rng(7)
    q = rng.standard_normal((len(lens), 1, Hq, D)).astype(np.float32)
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / math.sqrt(D)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=q_bf16, out_bf16=out_bf16)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, scale, pt)
    if out_bf16:
        # the f32 result rounded once to bf16 (half an ulp = 2^-9 relative)
        err = np.abs(got - want) - np.abs(want) * 2.0 ** -8
        assert float(err.max()) <= ATOL
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= RTOL + 2.0 ** -8
    else:
        assert_close(got, want, what=f"decode pt={pt}")


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens", [
    (16, 2, 256, 64, [1, 5000, 300, 0, 17000, 64, 2047]),
    (8, 2, 128, 16, list(np.random.default_rng(5).integers(0, 3000, 150))),
    (8, 4, 128, 32, list(np.random.default_rng(6).integers(0, 200, 300))),
])
def test_decode_ragged_device_partitions(rkv, rko, ctx, Hq, Hkv, D, PT, lens):
    """Partition length chosen on the device (partition_tokens = 0) over ragged
    batches -- zero lengths, more than 64 and more than 256 entries (the
    lengths the scan keeps in registers and those it reloads) -- equals the
    oracle."""
    print(f"ragged Hq={Hq} Hkv={Hkv} D={D} PT={PT} B={len(lens)}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=len(lens), src_bf16=True)
    rng = np.random.default_rng(12)
    q = rng.standard_normal((len(lens), 1, Hq, D)).astype(np.float32)
    got, pt = _run_decode(rkv, ctx, sc, q, 1.0 / math.sqrt(D))
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, 1.0 / math.sqrt(D), pt)
    assert_close(got, want, what="ragged")


def outlier_q(rng, shape):
    """q ~ N(0,1) whose every head carries ceil(1% of D) channels scaled x32
    and one more channel scaled x100: queries after RoPE concentrate their
    energy in a few channels, so a row's largest |q| is 30-100x its typical
    element."""
    q = rng.standard_normal(shape).astype(np.float32)
    H, D = shape[-2], shape[-1]
    n32 = max(1, int(math.ceil(0.01 * D)))
    for h in range(H):
        ch = rng.choice(D, n32 + 1, replace=False)
        q[..., h, ch[:n32]] *= 32.0
        q[..., h, ch[n32]] *= 100.0
    return q


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_bf16,q_len", [
    # 8 rows per kv head: the 16x16x64 QK (8 rows x 2 block parities)
    (16, 2, 256, 64, [4100, 700, 33, 1, 2000], True, 1),
    (16, 2, 256, 64, [3000, 9, 1500], False, 1),
    (8, 2, 128, 16, [700, 3, 2048], False, 1),
    # 16 rows: the 16x16x32 QK on one wave
    (32, 2, 256, 64, [2500, 40, 1000], True, 1),
    (16, 2, 128, 32, [1200, 64], True, 2),
    # 32 rows: the two-wave causal verify
    (16, 2, 256, 64, [1504, 74, 37], True, 4),
    # the reference's 24 q / 4 kv heads on 32-token pages: 6 rows (q_len 1),
    # 12 rows (q_len 2), 18 and 24 rows (the two-wave verify, q_len 3 and 4)
    (24, 4, 256, 32, [2500, 40, 999], True, 1),
    (24, 4, 256, 32, [1700, 5, 640], False, 1),
    (24, 4, 256, 32, [1800, 65], True, 2),
    (24, 4, 256, 32, [1300, 77, 5], False, 2),
    (24, 4, 256, 32, [1100, 300, 40], True, 3),
    (24, 4, 256, 32, [1504, 74, 37], True, 4),
    (24, 4, 256, 32, [900, 33], False, 4),
])
def test_decode_outlier_query(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_bf16, q_len):
    """Queries with outlier channels (x32 and x100) against the reference's
    f32 q (attention.rs:186-192), at the same bars: the query's int8 planes
    must resolve the small elements of a row next to its outliers."""
    print(f"outlier q Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens} q_len={q_len}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=3 * Hq + D + q_len, outliers=0.01, src_bf16=True)
    rng = np.random.default_rng(D + Hq + q_len)
    q = outlier_q(rng, (len(lens), q_len, Hq, D))
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / math.sqrt(D)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=q_bf16, q_len=q_len)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, scale, pt)
    assert_close(got, want, what=f"outlier q rows={q_len * Hq // Hkv} pt={pt}")


def test_smoke_mirror(rkv, rko, ctx):
    """har-serve-vulkan-attn-smoke.rs:41-185 with its inputs (lcg K/V, har-serve
    quantizer, seq_len 1024, 8 q heads / 4 kv heads, no scale), through the
    flash_decode_q8.comp drop-in entry point; the smoke passes at max-abs <= 1e-3."""
    torch = _torch()
    S, Hq, Hkv, D = 1024, 8, 4, 256
    rb = rko.row_bytes(D)
    k = np.empty((Hkv, S, rb), np.uint8)
    v = np.empty_like(k)
    for h in range(Hkv):
        for p in range(S):
            k[h, p] = rko.q8_quantize_harserve(rko.lcg_values(D, 1000 + (h * S + p) * 31))
            v[h, p] = rko.q8_quantize_harserve(rko.lcg_values(D, 2000 + (h * S + p) * 17))
    kw, vw = rko.rows_to_words(k), rko.rows_to_words(v)
    query = rko.lcg_values(Hq * D, 3000)
    p = rko.fd_params(Hq, Hkv, S, 1024, D)
    want = rko.flash_decode_reference(p, kw, vw, query)
    rp = rkv.FlashDecodeParams(Hq, Hkv, S, 1024, D)
    scratch = torch.empty(rkv.flash_decode_scratch_bytes(rp), dtype=torch.uint8, device="cuda")
    out = torch.empty(Hq * D, dtype=torch.float32, device="cuda")
    rkv.flash_decode_q8(ctx, rp, torch.from_numpy(kw.view(np.int32)).cuda(),
                        torch.from_numpy(vw.view(np.int32)).cuda(), torch.from_numpy(query).cuda(),
                        out, scratch)
    ctx.sync()
    got = out.cpu().numpy()
    assert float(np.max(np.abs(got - want))) <= 1e-3
    assert_close(got, want, what="smoke")


def test_splitk_partials_and_combine(rkv, rko, ctx):
    """Per-partition (m, l, o) equal the oracle's per-chunk partials
    (attention.rs:182-204); the combine reproduces attention.rs:205-212."""
    torch = _torch()
    Hq, Hkv, D, PT = 8, 2, 256, 64
    sc = Scene(rkv, rko, Hkv, D, PT, [1000, 260], seed=3)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, 1, Hq, D)).astype(np.float32)
    scale = 1.0 / 16
    part = 256
    n_parts = 4
    qd = torch.from_numpy(q).cuda()
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    sid = torch.arange(2, dtype=torch.int32, device="cuda")
    a = rkv.decode_args(qd, out, sid, scale, 1000, partition_tokens=part)
    ml = torch.full((2, Hq, n_parts, 2), float("nan"), device="cuda")
    o = torch.full((2, Hq, n_parts, D), float("nan"), device="cuda")
    rkv.decode_q8_partials(ctx, sc.g, sc.pages_d, sc.bt_d, sc.lens_d, a, ml, o)
    ctx.sync()
    mln, on = ml.cpu().numpy(), o.cpu().numpy()
    log2e = 1.0 / math.log(2.0)
    for b, L in enumerate(sc.lens):
        kr = rko.paged_gather(sc.lay, sc.pages, sc.bt[b], int(L), 0)
        vr = rko.paged_gather(sc.lay, sc.pages, sc.bt[b], int(L), 1)
        kw, vw = rko.rows_to_words(kr), rko.rows_to_words(vr)
        for h in range(Hq):
            kvh = h // (Hq // Hkv)
            off = kvh * int(L) * rko.row_bytes(D) // 4
            p = rko.fd_params(Hq, Hkv, int(L), part, D)
            qs = (q[b, 0, h] * np.float32(scale)).astype(np.float32)
            cm, lc, oc = rko.flash_decode_partials(p, kw[off:], vw[off:], qs, 0)
            np_b = len(cm)
            assert np_b == (int(L) + part - 1) // part
            # (m, l) are relative to a reference max the kernel may keep up to
            # 2^4 below the true one; their log-sum-exp m + log2(l) is invariant
            m_k, l_k = mln[b, h, :np_b, 0], mln[b, h, :np_b, 1]
            assert np.all(m_k <= cm * log2e + 1e-3) and np.all(m_k >= cm * log2e - 4.0 - 1e-3)
            assert np.allclose(m_k + np.log2(l_k), cm * log2e + np.log2(lc), atol=2e-3)
            # o normalised by the partition's weight mass
            for i in range(np_b):
                assert_close(on[b, h, i] / l_k[i], oc[i] / lc[i], what=f"partial b{b} h{h} p{i}")
    comb = torch.empty_like(out)
    rkv.splitk_combine(ctx, ml, o, 2, Hq, n_parts, D, sid, sc.lens_d, part, comb)
    direct, _ = _run_decode(rkv, ctx, sc, q, scale, partition_tokens=part)
    ctx.sync()
    # rkv_decode_q8 merges the same partials with its own (online) combine
    assert np.allclose(comb.cpu().numpy(), direct, rtol=1e-5, atol=1e-7)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(2, dtype=np.int32), q,
                            scale, part)
    assert_close(direct, want, what="combine")


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_len,part,out_bf16", [
    # D = 128, device-chosen partitions
    (16, 2, 128, 64, [700, 33, 1], 4, 0, False),
    # 16-token pages, bf16 out
    (16, 2, 256, 16, [300, 40], 4, 0, True),
    # 24 rows per kv head (8 dead rows in the second wave's n-tile); every
    # length <= 256: one partition, direct (normalized) output
    (16, 2, 256, 64, [200, 100, 7], 3, 0, False),
    # explicit partitions, bf16 out
    (32, 4, 256, 32, [900, 129], 4, 512, True),
    # the reference's 24 q / 4 kv heads: 24 rows (8 dead rows in the second
    # wave's n-tile), device-chosen and explicit partitions
    (24, 4, 256, 32, [1100, 129, 3], 4, 0, False),
    (24, 4, 256, 32, [700, 300], 4, 256, True),
])
def test_verify_bf16_query_shapes(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_len, part, out_bf16):
    """17..32 rows per kv head with a bf16 query: the two waves split the head
    dimension (f16 QK on widened K codes, partial scores and p exchanged
    through LDS).  Against the oracle, across head sizes, page sizes, dead
    rows, the direct output and the split-K partials."""
    print(f"verify bf16 Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens} q_len={q_len} part={part}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=5 * D + PT + q_len, src_bf16=True, outliers=0.01)
    rng = np.random.default_rng(D + q_len + PT)
    q = outlier_q(rng, (len(lens), q_len, Hq, D))
    q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / math.sqrt(D)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=True, q_len=q_len, partition_tokens=part,
                          out_bf16=out_bf16)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, scale, pt)
    if out_bf16:
        # the f32 result rounded once to bf16 (half an ulp = 2^-9 relative)
        err = np.abs(got - want) - np.abs(want) * 2.0 ** -8
        assert float(err.max()) <= ATOL
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= RTOL + 2.0 ** -8
    else:
        assert_close(got, want, what="verify bf16 q")


def test_verify_causal(rkv, rko, ctx):
    """q_len=4 causal verify: draft row j attends positions [0, ctx+j]; equal to
    the oracle and to single-row decodes of length ctx+j+1 (attention.rs:169-215)."""
    torch = _torch()
    Hq, Hkv, D, PT, ctx_len, ql = 16, 2, 256, 64, 1500, 4
    lens = [ctx_len + ql, 70 + ql, 33]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=21, src_bf16=True)
    rng = np.random.default_rng(4)
    q = rng.standard_normal((3, ql, Hq, D)).astype(np.float32)
    q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / 16
    # one explicit partition length for the verify and the single-row decodes:
    # the f16 rounding of p depends on each partition's reference max
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=True, q_len=ql, partition_tokens=512)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(3, dtype=np.int32), q,
                            scale, pt)
    assert_close(got, want, what=f"verify pt={pt}")
    # row j == a decode over the first len-ql+j+1 positions
    for j in range(ql):
        lens_j = torch.from_numpy(sc.lens - ql + j + 1).cuda()
        qj = torch.from_numpy(np.ascontiguousarray(q[:, j:j + 1])).cuda().to(torch.bfloat16)
        out = torch.empty(qj.shape, dtype=torch.float32, device="cuda")
        sid = torch.arange(3, dtype=torch.int32, device="cuda")
        a = rkv.decode_args(qj, out, sid, scale, int(sc.lens.max()), partition_tokens=pt)
        ws = torch.zeros(max(rkv.decode_workspace_bytes(sc.g, a), 4), dtype=torch.uint8, device="cuda")
        a = rkv.decode_args(qj, out, sid, scale, int(sc.lens.max()), partition_tokens=pt, workspace=ws)
        rkv.decode_q8(ctx, sc.g, sc.pages_d, sc.bt_d, lens_j, a)
        ctx.sync()
        assert_close(got[:, j:j + 1], out.cpu().numpy(), atol=1e-5, rtol=1e-5, what=f"row {j}")


def test_decode_edge_lengths(rkv, rko, ctx):
    """len 0 -> zeros (flash_decode_q8.comp:144-148); len 1 -> dequant(V_0);
    lengths around tile and partition boundaries."""
    Hq, Hkv, D, PT = 8, 2, 128, 32
    lens = [0, 1, 31, 32, 33, 255, 256, 257]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=2)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((len(lens), 1, Hq, D)).astype(np.float32)
    got, pt = _run_decode(rkv, ctx, sc, q, 0.1, partition_tokens=64)
    assert pt == 64
    assert np.all(got[0] == 0.0)
    v0 = rko.paged_gather(sc.lay, sc.pages, sc.bt[1], 1, 1)
    for h in range(Hq):
        want = rko.q8_decode(v0[h // 4, 0], D)
        assert_close(got[1, 0, h], want, atol=1e-3, rtol=1e-3, what="len1")
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(len(lens), dtype=np.int32),
                            q, 0.1, pt)
    want[0] = 0.0
    assert_close(got, want, what="edges")


def test_bad_block_table_is_reported(rkv, rko, ctx):
    """An out-of-pool page id never leaves the pool on the device and makes the
    next rkv_ctx_sync fail with RKV_ERR_BAD_BLOCK_TABLE."""
    torch = _torch()
    sc = Scene(rkv, rko, 2, 128, 16, [100], seed=1)
    ctx.sync()
    bad = sc.bt.copy()
    bad[0, 3] = sc.num_pages + 5
    sc.bt_d = torch.from_numpy(bad).cuda()
    q = np.ones((1, 1, 4, 128), np.float32)
    with pytest.raises(rkv.RkvError) as e:
        _run_decode(rkv, ctx, sc, q, 1.0)
    assert e.value.status == rkv.ERR_BAD_BLOCK_TABLE
    ctx.sync()  # the fault word was cleared
    k = torch.zeros((1, 2, 128), device="cuda")
    bad[0, 0] = -1
    with pytest.raises(rkv.RkvError) as e:
        rkv.append_q8(ctx, sc.g, sc.pages_d, torch.from_numpy(bad).cuda(),
                      torch.zeros(1, dtype=torch.int32, device="cuda"),
                      torch.zeros(1, dtype=torch.int32, device="cuda"), k, k)
        ctx.sync()
    assert e.value.status == rkv.ERR_BAD_BLOCK_TABLE


def test_pool_api_and_rollback(rkv, rko, ctx):
    """Operator-level API: allocator-driven pool, append, decode, gather; a
    speculative rollback (truncate) followed by re-append gives the same bytes
    as appending the accepted rows directly."""
    torch = _torch()
    Hkv, D, PT, Hq = 2, 256, 64, 16
    pool = rkv.Pool(ctx, 2, Hkv, D, PT, 64, 4, 16, seed=5)
    rng = np.random.default_rng(12)
    L0 = 200
    pool.alloc.reserve(0, L0)
    pool.alloc.reserve(1, 90)
    pool.sync_tables()
    rows0 = rng.standard_normal((L0, Hkv, D)).astype(np.float32)
    rows1 = rng.standard_normal((90, Hkv, D)).astype(np.float32)
    for layer in (0, 1):
        for s, rows in ((0, rows0), (1, rows1)):
            n = rows.shape[0]
            pool.append(layer, torch.full((n,), s, dtype=torch.int32, device="cuda"),
                        torch.arange(n, dtype=torch.int32, device="cuda"),
                        torch.from_numpy(rows * (layer + 1)).cuda(),
                        torch.from_numpy(rows * (layer + 1)).cuda())
    # speculative: append 4 draft rows to seq 0, accept 1, roll back the rest
    draft = rng.standard_normal((4, Hkv, D)).astype(np.float32)
    pool.alloc.reserve(0, L0 + 4)
    pool.sync_tables()
    pool.append(0, torch.zeros(4, dtype=torch.int32, device="cuda"),
                torch.arange(L0, L0 + 4, dtype=torch.int32, device="cuda"),
                torch.from_numpy(draft).cuda(), torch.from_numpy(draft).cuda())
    pool.alloc.truncate(0, L0 + 1)
    nxt = rng.standard_normal((1, Hkv, D)).astype(np.float32)
    pool.alloc.reserve(0, L0 + 2)
    pool.sync_tables()
    pool.append(0, torch.zeros(1, dtype=torch.int32, device="cuda"),
                torch.full((1,), L0 + 1, dtype=torch.int32, device="cuda"),
                torch.from_numpy(nxt).cuda(), torch.from_numpy(nxt).cuda())
    ctx.sync()
    accepted = np.concatenate([rows0, draft[:1], nxt])
    out = torch.empty(Hkv * (L0 + 2) * rkv.row_bytes(D), dtype=torch.uint8, device="cuda")
    pool.gather(0, 0, 0, out)
    ctx.sync()
    got = out.cpu().numpy().reshape(Hkv, L0 + 2, -1)
    for h in range(Hkv):
        assert np.array_equal(got[h], rko.q8_encode(accepted[:, h, :].reshape(-1)).reshape(L0 + 2, -1))
    # decode through the pool equals the oracle over the gathered rows
    q = rng.standard_normal((2, 1, Hq, D)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    o = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    sid = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    a = rkv.decode_args(qd, o, sid, 1 / 16, 16 * PT, partition_tokens=256)
    ws = torch.zeros(max(rkv.decode_workspace_bytes(pool.geometry, a), 4), dtype=torch.uint8,
                     device="cuda")
    a = rkv.decode_args(qd, o, sid, 1 / 16, 16 * PT, partition_tokens=256, workspace=ws)
    pool.decode(0, a)
    ctx.sync()
    tables, lens = pool.alloc.export()
    pages0 = _as_u8(pool.layer_pages(0), 64 * rkv.page_bytes(pool.geometry)).clone()
    lay = rko.layout(Hkv, D, PT, 64)
    want = rko.paged_decode(lay, pages0.cpu().numpy(), tables, lens, np.array([0, 1], np.int32), q,
                            1 / 16, 256)
    assert_close(o.cpu().numpy(), want, what="pool decode")
    pool.close()


def test_workspace_reuse_repeated_calls(rkv, rko, ctx):
    """rkv_decode_q8 through one workspace that starts as NaN garbage, three
    calls with the lengths changing in between (shorter sequences leave stale
    partials of earlier calls behind): every call equals the per-entry path
    (partials + rkv_splitk_combine) to rounding and the oracle within tolerance."""
    torch = _torch()
    Hq, Hkv, D, PT = 16, 2, 256, 64
    sc = Scene(rkv, rko, Hkv, D, PT, [3000, 1000, 64, 2500], seed=31, src_bf16=True)
    rng = np.random.default_rng(3)
    q = torch.from_numpy(rng.standard_normal((4, 1, Hq, D)).astype(np.float32)).cuda().to(torch.bfloat16)
    sid = torch.arange(4, dtype=torch.int32, device="cuda")
    part = 512
    out = torch.empty((4, 1, Hq, D), dtype=torch.float32, device="cuda")
    a = rkv.decode_args(q, out, sid, 1 / 16, 3000, partition_tokens=part)
    ws = torch.full((rkv.decode_workspace_bytes(sc.g, a),), 0xFF, dtype=torch.uint8, device="cuda")
    a = rkv.decode_args(q, out, sid, 1 / 16, 3000, partition_tokens=part, workspace=ws)
    n_parts = (3000 + part - 1) // part
    for call, lens in enumerate(([3000, 1000, 64, 2500], [2999, 1, 64, 2048], [3000, 1000, 0, 513])):
        lens_d = torch.tensor(lens, dtype=torch.int32, device="cuda")
        rkv.decode_q8(ctx, sc.g, sc.pages_d, sc.bt_d, lens_d, a)
        ml = torch.empty((4, Hq, n_parts, 2), device="cuda")
        o = torch.empty((4, Hq, n_parts, D), device="cuda")
        rkv.decode_q8_partials(ctx, sc.g, sc.pages_d, sc.bt_d, lens_d, a, ml, o)
        ref = torch.empty_like(out)
        rkv.splitk_combine(ctx, ml, o, 4, Hq, n_parts, D, sid, lens_d, part, ref)
        ctx.sync()
        got = out.cpu().numpy()
        assert np.allclose(got, ref.cpu().numpy(), rtol=1e-5, atol=1e-7), f"call {call}"
        want = rko.paged_decode(sc.lay, sc.pages, sc.bt, np.array(lens, np.int32),
                                np.arange(4, dtype=np.int32), q.float().cpu().numpy(), 1 / 16, 256)
        assert_close(got, want, what=f"call {call}")


def _last_rows(sc, b, q_len):
    """The scene's source rows of sequence b at positions len-q_len .. len-1."""
    start = int(np.sum(sc.lens[:b])) + int(sc.lens[b]) - q_len
    return sc.k[start:start + q_len], sc.v[start:start + q_len]


@pytest.mark.parametrize("Hq,Hkv,D,PT,lens,q_len,part,rule,src_bf16", [
    # rows in a partition's first tile (len 1), second tile (len 64) and later
    (16, 2, 256, 64, [3000, 1000, 64, 2500, 1], 1, 512, 0, True),
    (16, 4, 128, 16, [514, 300, 4, 1030], 4, 512, 0, True),
    # straddling partitions (2049), tiles 0+1 (33), tile 1 only (40)
    (8, 2, 256, 32, [2049, 33, 40], 2, 1024, 1, True),
    # 16 rows per kv head with K codes in registers; f32 source rows
    (16, 4, 128, 32, [514, 300, 4, 1030, 35], 4, 512, 0, False),
    # device-chosen partitions (the last partition takes a one-tile remainder)
    (16, 2, 256, 64, [4097, 66, 300, 12000], 1, 0, 1, False),
    # the reference's 24 q / 4 kv heads on 32-token pages: 6, 12 and 24 rows
    (24, 4, 256, 32, [2049, 33, 40, 700], 1, 0, 0, True),
    (24, 4, 256, 32, [1030, 64, 5], 2, 512, 1, True),
    (24, 4, 256, 32, [2049, 33, 40], 4, 1024, 0, True),
])
def test_append_in_decode(rkv, rko, ctx, Hq, Hkv, D, PT, lens, q_len, part, rule, src_bf16):
    """The decode launch's own append (rkv_decode_args.append) writes the same
    bytes as rkv_append_q8 -- also for draft rows that straddle a partition
    boundary and for rows in a partition's first or second tile -- and its
    output equals append-then-decode bit for bit (and the oracle within
    tolerance)."""
    torch = _torch()
    print(f"append-in-decode Hq={Hq} Hkv={Hkv} D={D} PT={PT} lens={lens} q_len={q_len} "
          f"part={part} bf16={src_bf16}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=40 + D + q_len, src_bf16=src_bf16, rule=rule)
    B = len(lens)
    # the pages the fused path starts from hold junk at the rows it appends
    fused = sc.pages_d.clone()
    rng = np.random.default_rng(8)
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    rows_sid = torch.repeat_interleave(sid, q_len)
    pos = torch.from_numpy(np.concatenate([np.arange(L - q_len, L) for L in lens]).astype(np.int32)).cuda()
    junk = torch.from_numpy(rng.standard_normal((B * q_len, Hkv, D)).astype(np.float32) * 5).cuda()
    rkv.append_q8(ctx, sc.g, fused, sc.bt_d, rows_sid, pos, junk, -junk)
    kn = np.concatenate([_last_rows(sc, b, q_len)[0] for b in range(B)])
    vn = np.concatenate([_last_rows(sc, b, q_len)[1] for b in range(B)])
    src_dt = torch.bfloat16 if src_bf16 else torch.float32
    kd = torch.from_numpy(kn).cuda().to(src_dt)
    vd = torch.from_numpy(vn).cuda().to(src_dt)
    q = rng.standard_normal((B, q_len, Hq, D)).astype(np.float32)
    q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    qd = torch.from_numpy(q).cuda().to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    outs = []
    for pages, app in ((sc.pages_d, None), (fused, rkv.append_args(rows_sid, pos, kd, vd, rule=rule))):
        out = torch.empty((B, q_len, Hq, D), dtype=torch.float32, device="cuda")
        a = rkv.decode_args(qd, out, sid, scale, max(lens), q_len=q_len, partition_tokens=part)
        ws = torch.empty(max(rkv.decode_workspace_bytes(sc.g, a), 4), dtype=torch.uint8, device="cuda")
        a = rkv.decode_args(qd, out, sid, scale, max(lens), q_len=q_len, partition_tokens=part,
                            workspace=ws, append=app)
        rkv.decode_q8(ctx, sc.g, pages, sc.bt_d, sc.lens_d, a)
        ctx.sync()
        outs.append(out.cpu().numpy())
    assert torch.equal(fused, sc.pages_d), "pages written by the decode's append differ"
    assert np.array_equal(outs[0], outs[1])
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(B, dtype=np.int32), q,
                            scale, part or 1024)
    assert_close(outs[1], want, what="append-in-decode")


def test_append_in_decode_bad_rows_are_reported(rkv, rko, ctx):
    """A row whose sequence is not its batch entry's (fault bit 4) or whose
    position is at or past the sequence length (fault bit 2) is reported by
    rkv_ctx_sync and writes nothing."""
    torch = _torch()
    Hq, Hkv, D, PT = 8, 2, 128, 32
    sc = Scene(rkv, rko, Hkv, D, PT, [100, 200], seed=9)
    sid = torch.arange(2, dtype=torch.int32, device="cuda")
    q = torch.randn((2, 1, Hq, D), device="cuda")
    rows = torch.randn((2, Hkv, D), device="cuda")
    for rows_sid, pos, bit in (([1, 1], [50, 60], 4), ([0, 1], [100, 60], 2)):
        pages = sc.pages_d.clone()
        out = torch.empty_like(q)
        app = rkv.append_args(torch.tensor(rows_sid, dtype=torch.int32, device="cuda"),
                              torch.tensor(pos, dtype=torch.int32, device="cuda"), rows, rows)
        a = rkv.decode_args(q, out, sid, 0.1, 200, partition_tokens=64)
        ws = torch.empty(rkv.decode_workspace_bytes(sc.g, a), dtype=torch.uint8, device="cuda")
        a = rkv.decode_args(q, out, sid, 0.1, 200, partition_tokens=64, workspace=ws, append=app)
        rkv.decode_q8(ctx, sc.g, pages, sc.bt_d, sc.lens_d, a)
        with pytest.raises(rkv.RkvError) as ei:
            ctx.sync()
        assert ei.value.status == rkv.ERR_BAD_BLOCK_TABLE and f"0x{bit:x}" in str(ei.value)
        # only the valid row of the pair was written
        valid = [i for i in range(2) if not (rows_sid[i] != i or pos[i] >= sc.lens[i])]
        ref = sc.pages_d.clone()
        if valid:
            rkv.append_q8(ctx, sc.g, ref, sc.bt_d, torch.tensor([rows_sid[i] for i in valid], dtype=torch.int32, device="cuda"),
                          torch.tensor([pos[i] for i in valid], dtype=torch.int32, device="cuda"),
                          rows[valid], rows[valid])
        ctx.sync()
        assert torch.equal(pages, ref)


def test_pool_async_table_updates(rkv, rko, ctx):
    """Allocator edits uploaded by rkv_pool_sync_tables are stream-ordered: six
    steps of grow (crossing page boundaries), append-in-decode and rollback are
    queued with no host synchronisation in between (so both pinned staging
    buffers are reused while earlier uploads may still be pending), and every
    step's output equals the oracle over that step's pages and lengths."""
    torch = _torch()
    Hkv, D, PT, Hq, B = 2, 128, 16, 8, 3
    pool = rkv.Pool(ctx, 1, Hkv, D, PT, 96, B, 40, seed=3)
    rng = np.random.default_rng(21)
    lens = [30, 47, 5]
    for s, L in enumerate(lens):
        pool.alloc.reserve(s, L)
    pool.sync_tables()
    base = [rng.standard_normal((L, Hkv, D)).astype(np.float32) for L in lens]
    for s, rows in enumerate(base):
        pool.append(0, torch.full((len(rows),), s, dtype=torch.int32, device="cuda"),
                    torch.arange(len(rows), dtype=torch.int32, device="cuda"),
                    torch.from_numpy(rows).cuda(), torch.from_numpy(rows).cuda())
    ctx.sync()
    stream = torch.cuda.current_stream()
    sid = torch.arange(B, dtype=torch.int32, device="cuda")
    history = []  # per step: rows of each sequence after the step, q, out
    rows_now = [r.copy() for r in base]
    outs = []
    for step in range(6):
        grow = [int(x) for x in rng.integers(1, 4, B)]  # 1..3 draft rows, q_len = 1 row decoded
        new_rows = [rng.standard_normal((1, Hkv, D)).astype(np.float32) for _ in range(B)]
        for s in range(B):
            pool.alloc.reserve(s, len(rows_now[s]) + 1)
            rows_now[s] = np.concatenate([rows_now[s], new_rows[s]])
        pool.sync_tables(stream)
        q = torch.from_numpy(rng.standard_normal((B, 1, Hq, D)).astype(np.float32)).cuda()
        out = torch.empty_like(q)
        kn = torch.from_numpy(np.concatenate(new_rows)).cuda()
        pos = torch.tensor([len(r) - 1 for r in rows_now], dtype=torch.int32, device="cuda")
        app = rkv.append_args(sid, pos, kn, kn)
        a = rkv.decode_args(q, out, sid, 0.125, 40 * PT, partition_tokens=64)
        ws = torch.empty(rkv.decode_workspace_bytes(pool.geometry, a), dtype=torch.uint8, device="cuda")
        a = rkv.decode_args(q, out, sid, 0.125, 40 * PT, partition_tokens=64, workspace=ws, append=app)
        pool.decode(0, a, stream=stream)
        outs.append((out, q, a, ws, app, kn, pos))
        history.append([r.copy() for r in rows_now])
        # roll back a seeded number of the rows (keeps at least the base rows)
        for s in range(B):
            keep = max(len(base[s]), len(rows_now[s]) - int(rng.integers(0, 2)) * grow[s])
            pool.alloc.truncate(s, keep)
            rows_now[s] = rows_now[s][:keep]
    ctx.sync()
    scale = np.float32(0.125)
    for step, (out, q, *_rest) in enumerate(outs):
        got = out.cpu().numpy()
        qn = q.cpu().numpy()
        for s in range(B):
            rows = history[step][s]
            kq = np.stack([rko.q8_encode(rows[t, h]) for t in range(len(rows)) for h in range(Hkv)])
            kq = kq.reshape(len(rows), Hkv, -1).transpose(1, 0, 2).copy()
            p = rko.fd_params(Hq, Hkv, len(rows), 64, D)
            want = rko.flash_decode_reference(p, rko.rows_to_words(kq), rko.rows_to_words(kq),
                                              (qn[s, 0] * scale).astype(np.float32).reshape(-1))
            assert_close(got[s, 0].reshape(-1), want, what=f"step {step} seq {s}")
    pool.close()


def test_continuous_batching_steps(rkv, rko, ctx):
    """Config 4's flow at a small size on 2 layer pools with 16-token pages:
    per step some sequences finish (pages freed, restart empty), two append a
    40-row prefill chunk, the rest decode one token appended inside the decode
    launch; one stream-ordered table upload per step, no host sync until the
    end.  Every (step, layer) decode output equals the oracle over that
    layer's rows at that step."""
    torch = _torch()
    Hkv, D, PT, Hq, S, layers = 2, 128, 16, 8, 8, 2
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, 400, S, 48, seed=11)
    rng = np.random.default_rng(31)
    rows = [[np.zeros((0, Hkv, D), np.float32) for _ in range(S)] for _ in range(layers)]

    def append(layer, seqs, starts, new, stream=None):
        sid = np.concatenate([np.full(len(x), s, np.int32) for s, x in zip(seqs, new)])
        pos = np.concatenate([np.arange(st, st + len(x), dtype=np.int32) for st, x in zip(starts, new)])
        kv = np.concatenate(new)
        pool.append(layer, torch.from_numpy(sid).cuda(), torch.from_numpy(pos).cuda(),
                    torch.from_numpy(kv).cuda(), torch.from_numpy(kv).cuda(), stream=stream)

    lens = [int(x) for x in rng.integers(5, 200, S)]
    for s in range(S):
        pool.alloc.reserve(s, lens[s])
    pool.sync_tables()
    for layer in range(layers):
        new = [rng.standard_normal((lens[s], Hkv, D)).astype(np.float32) for s in range(S)]
        append(layer, range(S), [0] * S, new)
        for s in range(S):
            rows[layer][s] = new[s]
    ctx.sync()
    stream = torch.cuda.current_stream()
    keep = []  # device inputs of queued launches
    checks = []
    for step in range(4):
        for s in range(S):
            if rng.random() < 0.25:
                pool.alloc.free(s)
                lens[s] = 0
                for layer in range(layers):
                    rows[layer][s] = rows[layer][s][:0]
        pf = [(2 * step) % S, (2 * step + 1) % S]
        dset = [s for s in range(S) if s not in pf]
        for s in pf:
            pool.alloc.reserve(s, lens[s] + 40)
        for s in dset:
            pool.alloc.reserve(s, lens[s] + 1)
        pool.sync_tables(stream)
        sid = torch.tensor(dset, dtype=torch.int32, device="cuda")
        pos = torch.tensor([lens[s] for s in dset], dtype=torch.int32, device="cuda")
        for layer in range(layers):
            chunk = [rng.standard_normal((40, Hkv, D)).astype(np.float32) for _ in pf]
            append(layer, pf, [lens[s] for s in pf], chunk, stream)
            new = rng.standard_normal((len(dset), Hkv, D)).astype(np.float32)
            kn = torch.from_numpy(new).cuda()
            q = torch.from_numpy(rng.standard_normal((len(dset), 1, Hq, D)).astype(np.float32)).cuda()
            out = torch.empty_like(q)
            app = rkv.append_args(sid, pos, kn, kn)
            a = rkv.decode_args(q, out, sid, 0.1, 48 * PT)
            ws = torch.empty(rkv.decode_workspace_bytes(pool.geometry, a), dtype=torch.uint8, device="cuda")
            a = rkv.decode_args(q, out, sid, 0.1, 48 * PT, workspace=ws, append=app)
            pool.decode(layer, a, stream=stream)
            keep.append((kn, q, ws, app, a))
            for i, s in enumerate(pf):
                rows[layer][s] = np.concatenate([rows[layer][s], chunk[i]])
            for i, s in enumerate(dset):
                rows[layer][s] = np.concatenate([rows[layer][s], new[i:i + 1]])
            checks.append((step, layer, out, q,
                           {s: rows[layer][s].copy() for s in dset}, list(dset)))
        for s in pf:
            lens[s] += 40
        for s in dset:
            lens[s] += 1
    ctx.sync()
    for step, layer, out, q, snap, dset in checks:
        got = out.cpu().numpy()
        qn = q.cpu().numpy()
        for i, s in enumerate(dset):
            r = snap[s]
            kq = np.stack([rko.q8_encode(r[t, h]) for t in range(len(r)) for h in range(Hkv)])
            kq = kq.reshape(len(r), Hkv, -1).transpose(1, 0, 2).copy()
            p = rko.fd_params(Hq, Hkv, len(r), 1024, D)
            want = rko.flash_decode_reference(p, rko.rows_to_words(kq), rko.rows_to_words(kq),
                                              (qn[i, 0] * np.float32(0.1)).astype(np.float32).reshape(-1))
            assert_close(got[i, 0].reshape(-1), want, what=f"step {step} layer {layer} seq {s}")
    pool.close()


def _as_u8(ptr, n):
    """A uint8 torch view of n bytes of device memory owned by the pool."""
    torch = _torch()

    class _Holder:
        __cuda_array_interface__ = {"shape": (n,), "typestr": "|u1", "data": (ptr, False),
                                    "version": 3}
    return torch.as_tensor(_Holder(), device="cuda")
