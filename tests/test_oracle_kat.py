"""Pins the CPU oracle (oracle/rkv_oracle.c) to the reference's own known
answers and unit-test assertions before it is used to check the kernels.

Reference sources restated by the oracle:
  har/crates/r4kv/src/{quant.rs,f16.rs}, har/crates/har-serve/src/{attention.rs,q4k.rs},
  tools/repro-harness/src/main.rs.
"""
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kat.json")


@pytest.fixture(scope="module")
def kat():
    with open(GOLDEN) as f:
        return json.load(f)


def _f32(x) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


# ---- r4kv KAT lane (repro/r4kv/storage/sanitized_receipt.json) -----------------

def _kat_source(rko):
    return np.array([rko.seeded_float(i) for i in range(4096)], np.float32)


def test_kat_source_vector_sha256(rko, kat):
    src = _kat_source(rko)
    digest = hashlib.sha256(src.astype("<f4").tobytes()).hexdigest()
    assert digest == kat["r4kv_receipt"]["source_vector_sha256"]


def test_kat_base_q8_roundtrip(rko, kat):
    src = _kat_source(rko)
    pos = (np.abs(src) + np.float32(0.125)).astype(np.float32)
    dec, st, rel = rko.roundtrip_stats(pos, 1)
    want = kat["r4kv_receipt"]["BASE-Q8"]
    # exact: the receipt prints the f32 values the Rust code computed
    assert st.max_abs_err == want["value_roundtrip_max_abs_error"]
    assert rel == _f32(want["value_roundtrip_rel_rms"])
    assert rko.normalized_kl(pos, dec) == want["positive_proxy_forward_kl"]


def test_kat_f16_roundtrip(rko, kat):
    src = _kat_source(rko)
    pos = (np.abs(src) + np.float32(0.125)).astype(np.float32)
    dec, st, rel = rko.roundtrip_stats(pos, 0)
    want = kat["r4kv_receipt"]["REF-A_f16f16"]
    assert st.max_abs_err == want["value_roundtrip_max_abs_error"]
    assert rel == _f32(want["value_roundtrip_rel_rms"])
    assert rko.normalized_kl(pos, dec) == want["positive_proxy_forward_kl"]


def test_kat_wire_sizes(rko, kat):
    x = rko.lcg_values(1024, 7)
    assert rko.q8_encode(x).size == kat["wire"]["q8_row_bytes_1024"]
    assert rko.q8_encode(x[:32]).size == kat["wire"]["q8_group_bytes"]


# ---- f16 encoders (r4kv f16.rs:92-145, attention.rs:289-296) -------------------

def _parse(tok: str) -> np.float32:
    if tok.endswith("-") or tok.endswith("+"):
        base = np.float32(float(tok[:-1]))
        delta = np.float32(2.0 ** -30)
        return np.float32(base - delta) if tok.endswith("-") else np.float32(base + delta)
    return np.float32(float(tok))


def test_f16_exact_values(rko, kat):
    L = rko.lib()
    for tok, bits in kat["f16_exact"]["pairs"]:
        assert L.rko_f32_to_f16(float(_parse(tok))) == bits, tok
    # decoder side of the same tests
    assert L.rko_f16_to_f32(0x7C00) == math.inf
    assert L.rko_f16_to_f32(0x3C00) == 1.0
    assert L.rko_f16_to_f32(6) == 6.0 * 2.0 ** -24


def test_f16_roundtrip_small_set(rko):
    L = rko.lib()
    for i in range(-20, 21):  # f16.rs:115-122
        v = i * 0.25
        assert abs(L.rko_f16_to_f32(L.rko_f32_to_f16(v)) - v) < 1e-6
    for d in (3.0, 0.57, 1.0 / 31.0, 9.0):  # f16.rs:137-145
        back = L.rko_f16_to_f32(L.rko_f32_to_f16(d))
        assert abs(back - _f32(d)) <= _f32(d) * 5e-4 + 1e-9


def test_f16_matches_numpy_rtne(rko):
    """r4kv's encoder is IEEE round-to-nearest-even: numpy's float16 cast is an
    independent implementation of the same rounding."""
    L = rko.lib()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    got = np.array([L.rko_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_decoders_exhaustive(rko):
    """Both binary16 decoders (f16.rs:4-25, q4k.rs:22-50) against numpy's
    float16 -> float32 widening over all 65536 bit patterns."""
    L = rko.lib()
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    a = np.array([L.rko_f16_to_f32(int(b)) for b in bits], np.float32)
    h = np.array([L.rko_f16_to_f32_harserve(int(b) & 0xFF, int(b) >> 8) for b in bits], np.float32)
    nan = np.isnan(want)
    for got in (a, h):
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_matches_torch(rko):
    """The bf16 rounding used to make bf16 test inputs is torch's (RTNE)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 2 ** 32, 50000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    got = rko.f32_to_bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got.reshape(-1), want)
    L = rko.lib()
    assert all(L.rko_f32_to_bf16(float(v)) == w for v, w in zip(x[:5000], want[:5000]))


def test_harserve_f16_roundtrip(rko):
    """attention.rs:289-296: |v - f16(v)| < 1e-3 for the listed values."""
    L = rko.lib()
    for v in (1.0, -1.0, 0.5, math.pi, 0.0, 127.0, -0.25):
        bits = L.rko_f32_to_f16_harserve(v)
        back = L.rko_f16_to_f32_harserve(bits & 0xFF, bits >> 8)
        assert abs(_f32(v) - back) < 1e-3


def _harserve_int(v: np.float32) -> int:
    """Integer-form reading of attention.rs:45-76 (independent of the oracle's
    f64 transcription): exp = unbiased exponent, mantissa rounded half away
    from zero on the dropped 13 bits, carry dropped by `& 0x3ff`."""
    u = int(np.array(v, np.float32).view(np.uint32))
    sign = (u >> 16) & 0x8000
    e = (u >> 23) & 0xFF
    frac = u & 0x7FFFFF
    if u & 0x7FFFFFFF == 0:
        return sign
    if e == 0xFF:
        return 0x7E00 if frac else sign | 0x7C00
    if e == 0:
        return sign
    ex = e - 127
    if ex < -14:
        if sign:
            return 0x8000
        m = frac | 0x800000
        sh = -1 - ex
        return (m + (1 << (sh - 1))) >> sh if sh < 40 else 0
    if ex > 15:
        return sign | 0x7C00
    mant = 0 if sign else ((frac + 0x1000) >> 13)
    return sign | ((ex + 15) << 10) | (mant & 0x3FF)


def test_harserve_f16_integer_form(rko):
    L = rko.lib()
    rng = np.random.default_rng(2)
    # dense over the exponent range a scale can take, both signs, plus edges
    vals = [np.float32(x) for x in (rng.uniform(-1, 1, 20000) * 2.0 ** rng.integers(-30, 20, 20000))]
    edges = [np.float32(2.0 ** k * (2 - 2.0 ** -11)) for k in range(-20, 17)]
    edges += [np.float32(np.nextafter(np.float32(x), np.float32(0))) for x in edges]
    edges += [np.float32(0.0), np.float32(-0.0), np.float32(np.inf), np.float32(-np.inf),
              np.float32(65504), np.float32(65520), np.float32(2.0 ** -24), np.float32(2.0 ** -25),
              np.float32(3 * 2.0 ** -26)]
    for v in vals + edges:
        assert L.rko_f32_to_f16_harserve(float(v)) == _harserve_int(v), v


def test_harserve_drops_mantissa_carry(rko):
    """A scale in [2^e(2-2^-11), 2^(e+1)) encodes as 2^e under attention.rs's
    encoder but as 2^(e+1) under r4kv's (the defect the canonical rule fixes)."""
    L = rko.lib()
    v = float(np.float32(2.0 ** -5 * (2 - 2.0 ** -12)))
    assert L.rko_f16_to_f32(L.rko_f32_to_f16_harserve(v)) == 2.0 ** -5
    assert L.rko_f16_to_f32(L.rko_f32_to_f16(v)) == 2.0 ** -4


# ---- Q8 codecs ------------------------------------------------------------------

def test_q8_roundtrip_is_close(rko):
    """attention.rs:279-287."""
    x = rko.lcg_values(256, 11)
    y = rko.q8_dequant_row(rko.q8_quantize_harserve(x), 256)
    assert np.all(np.abs(x - y) < 0.02)


def test_q8_canonical_closed_form(rko):
    """quant.rs:45-90 recomputed in numpy: d = amax/127, q = round(v*(1/d))."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(32 * 500).astype(np.float32)
    x[::97] *= 8  # outliers
    x[32:64] = 0  # zero block
    enc = rko.q8_encode(x).reshape(-1, 34)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1) / d).astype(np.float32)
    prod = (blocks * inv[:, None]).astype(np.float32)
    # round half away from zero, evaluated exactly in f64
    qx = np.clip(np.sign(prod) * np.floor(np.abs(prod.astype(np.float64)) + 0.5), -127, 127)
    assert np.array_equal(enc[:, 2:].view(np.int8), qx.astype(np.int8))
    assert np.array_equal(enc[:, :2].copy().view("<u2")[:, 0], d.astype(np.float16).view(np.uint16))


def test_q8_canonical_vs_harserve_count(rko):
    """The two reference rules agree except in the dropped-carry windows and rare
    v/d vs v*(1/d) rounding flips; count them on N(0,1) data (D=256 rows)."""
    x = rko.normal_f32(256 * 2048, 5)
    a = rko.q8_encode(x).reshape(-1, 34)
    b = rko.q8_quantize_harserve(x).reshape(-1, 34)
    scale_diff = np.any(a[:, :2] != b[:, :2], axis=1).mean()
    code_diff = np.any(a[:, 2:] != b[:, 2:], axis=1).mean()
    assert scale_diff < 0.01  # ~1/2048 of blocks hit the carry window
    assert code_diff < 0.05


# ---- flash decode (attention.rs tests and closed forms) -----------------------------

def _kv_cache(rko, p, seed):
    """attention.rs:257-273 (kv_cache test helper)."""
    rb = rko.row_bytes(p.head_dim)
    k = np.empty((p.kv_heads, p.seq_len, rb), np.uint8)
    v = np.empty_like(k)
    for h in range(p.kv_heads):
        for pos in range(p.seq_len):
            k[h, pos] = rko.q8_quantize_harserve(
                rko.lcg_values(p.head_dim, seed + (h * p.seq_len + pos) * 31 + 7))
            v[h, pos] = rko.q8_quantize_harserve(
                rko.lcg_values(p.head_dim, seed + (h * p.seq_len + pos) * 17 + 3))
    return rko.rows_to_words(k), rko.rows_to_words(v)


def test_online_matches_bruteforce(rko):
    """attention.rs:298-318."""
    p = rko.fd_params(4, 2, 513, 128)
    kw, vw = _kv_cache(rko, p, 5)
    q = rko.lcg_values(p.q_heads * 256, 9)
    for qh in range(p.q_heads):
        kvh = qh // (p.q_heads // p.kv_heads)
        qq = q[qh * 256:(qh + 1) * 256]
        _, l, o = rko.flash_decode_online(p, kw, vw, qq, kvh)
        bf = rko.flash_decode_bruteforce(p, kw, vw, qq, kvh)
        assert np.all(np.abs(o / l - bf) < 1e-5)


def test_reference_many_equals_reference(rko):
    """The multi-threaded timing helper runs the same per-head loop: bit-equal
    to flash_decode_reference for every sequence."""
    p = rko.fd_params(8, 2, 300, 128, 256)
    ks, vs, qs = [], [], []
    for s in range(3):
        kw, vw = _kv_cache(rko, p, 50 + s)
        ks.append(kw)
        vs.append(vw)
        qs.append(rko.lcg_values(8 * 256, 90 + s).reshape(8, 256))
    got = rko.flash_decode_reference_many(p, ks, vs, np.stack(qs), threads=4)
    for s in range(3):
        want = rko.flash_decode_reference(p, ks[s], vs[s], qs[s].reshape(-1))
        assert np.array_equal(got[s].reshape(-1), want)


def test_gqa_mapping_uses_shared_kv_head(rko):
    """attention.rs:320-342."""
    p = rko.fd_params(4, 2, 64, 32)
    kw, vw = _kv_cache(rko, p, 3)
    q = rko.lcg_values(p.q_heads * 256, 4)
    _, l0, o0 = rko.flash_decode_online(p, kw, vw, q[:256], 0)
    _, l1, o1 = rko.flash_decode_online(p, kw, vw, q[:256], 0)
    assert np.all(np.abs(o0 / l0 - o1 / l1) < 1e-6)


def test_reference_vs_f64_truth(rko):
    p = rko.fd_params(8, 2, 300, 64, 128)
    kw, vw = _kv_cache(rko, p, 1)
    q = rko.lcg_values(p.q_heads * 128, 2) * np.float32(4)
    out = rko.flash_decode_reference(p, kw, vw, q).reshape(8, 128)
    rows = 300 * rko.row_bytes(128) // 4
    for qh in range(8):
        kvh = qh // 4
        t = rko.attention_f64(300, 128, kw[kvh * rows:], vw[kvh * rows:], q[qh * 128:(qh + 1) * 128])
        assert np.max(np.abs(out[qh] - t)) < 1e-5


def test_closed_forms(rko):
    D = 256
    rb = rko.row_bytes(D)
    # seq_len == 1 -> out == dequant(V_0) exactly
    k = rko.q8_quantize_harserve(rko.lcg_values(D, 1))
    v = rko.q8_quantize_harserve(rko.lcg_values(D, 2))
    p = rko.fd_params(1, 1, 1, 1024, D)
    out = rko.flash_decode_reference(p, rko.rows_to_words(k), rko.rows_to_words(v), rko.lcg_values(D, 3))
    assert np.array_equal(out, rko.q8_dequant_row(v, D))
    # identical K rows -> uniform weights -> mean of V
    n = 64
    krow = np.tile(k, n)
    vrows = np.concatenate([rko.q8_quantize_harserve(rko.lcg_values(D, 10 + i)) for i in range(n)])
    p = rko.fd_params(1, 1, n, 1024, D)
    out = rko.flash_decode_reference(p, rko.rows_to_words(krow), rko.rows_to_words(vrows),
                                     rko.lcg_values(D, 4))
    mean = np.mean([rko.q8_dequant_row(vrows[i * rb:(i + 1) * rb], D) for i in range(n)], axis=0)
    assert np.max(np.abs(out - mean)) < 1e-6
    # one dominating score -> that V row
    q = np.zeros(D, np.float32)
    kk = np.zeros((n, rb), np.uint8)
    for i in range(n):
        kk[i] = rko.q8_quantize_harserve(np.zeros(D, np.float32))
    kk[17] = rko.q8_quantize_harserve(np.full(D, 1.0, np.float32))
    q[:] = 10.0
    out = rko.flash_decode_reference(p, rko.rows_to_words(kk), rko.rows_to_words(vrows), q)
    assert np.array_equal(out, rko.q8_dequant_row(vrows[17 * rb:18 * rb], D))


def test_partials_then_combine_equals_online(rko):
    """Split-K identity: per-chunk partials (attention.rs:182-204) merged with
    the combine of :205-212 reproduce flash_decode_online exactly."""
    p = rko.fd_params(2, 1, 700, 128, 128)
    kw, vw = _kv_cache(rko, p, 8)
    q = rko.lcg_values(128, 9)
    m, l, o = rko.flash_decode_online(p, kw, vw, q, 0)
    cm, lc, oc = rko.flash_decode_partials(p, kw, vw, q, 0)
    assert len(cm) == 6
    out, m2, l2 = rko.lse_combine(cm, lc, oc)
    assert m2 == m and l2 == l
    assert np.array_equal(out, o / l)


# ---- paged layout in the oracle ----------------------------------------------------

@pytest.mark.parametrize("D,PT", [(128, 16), (256, 64), (256, 32), (128, 128)])
def test_oracle_paged_roundtrip(rko, D, PT):
    """gather(append(rows)) == the rows quantized in token order, for a shuffled
    block table (the bitwise invariant the kernels are held to)."""
    rng = np.random.default_rng(D + PT)
    Hkv, L = 2, 3 * PT + 5
    npg = (L + PT - 1) // PT
    num_pages = npg + 7
    lay = rko.layout(Hkv, D, PT, num_pages)
    pages = np.zeros(num_pages * rko.page_bytes(lay), np.uint8)
    bt = rng.permutation(num_pages)[:npg].astype(np.int32)[None, :]
    k = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    rko.paged_append(lay, pages, bt, np.zeros(L, np.int32), np.arange(L, dtype=np.int32), k, v, 0)
    for kind, src in ((0, k), (1, v)):
        got = rko.paged_gather(lay, pages, bt[0], L, kind)
        for h in range(Hkv):
            want = rko.q8_encode(src[:, h, :].reshape(-1)).reshape(L, -1)
            assert np.array_equal(got[h], want)


def test_har_kv_geometry_bytes(rko, kat):
    """Q8 page bytes reproduce har-kv's 262144-token total (lib.rs:53-65)."""
    g = kat["har_kv_geometry"]
    lay = rko.layout(4, 256, 64, g["tokens"] // 64)
    assert rko.page_bytes(lay) // 64 // 2 == g["q8_row_bytes"]  # per token, K or V
    assert rko.page_bytes(lay) * (g["tokens"] // 64) * 16 == g["total_bytes"]


def _lcg_state(seed: int, n: int) -> int:
    """State of q4k.rs:109-120's LCG after n steps, in closed form (the
    skip-ahead of an affine recurrence): s_n = a^n s_0 + c (a^n - 1)/(a - 1)
    mod 2^64.  (a - 1) is even, so the geometric sum is taken exactly from
    a^n mod 2^64 (a - 1) instead of by a modular inverse."""
    a, c, m = 6364136223846793005, 1442695040888963407, 1 << 64
    an = pow(a, n, m * (a - 1))
    geo = (an - 1) // (a - 1)
    return (an % m * seed + c * geo) % m


@pytest.mark.parametrize("seed", [0, 1, 3000, 1000 + (3 * 1024 + 1023) * 31, 2**64 - 1])
def test_lcg_values_closed_form(rko, seed):
    """rko_lcg_values (the smoke's K/V and query generator) against the
    LCG's closed-form state at sampled indices up to 10^6: value i is
    ((s_{i+1} >> 40) / 2^24) - 0.5, exact in f32."""
    n = 1_000_000 if seed in (0, 3000) else 4096
    got = rko.lcg_values(n, seed)
    for i in sorted({0, 1, 2, 17, 1023, n // 3, n - 2, n - 1}):
        s = _lcg_state(seed, i + 1)
        want = np.float32(np.float32(s >> 40) / np.float32(1 << 24)) - np.float32(0.5)
        assert got[i] == want, (seed, i, float(got[i]), float(want))
    assert np.all(got >= -0.5) and np.all(got < 0.5)
