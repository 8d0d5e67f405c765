"""R4KV page container on the host: the oracle's CRC32C and header bytes
pinned against the reference's known answers, and the library's host
functions (header encode/decode, restore gate, unpack) against the oracle
and the reference's own unit tests (har/crates/r4kv/src/page.rs:262-373,
crc32c.rs:33-52).  No kernel is launched."""
import random

import numpy as np
import pytest


def _crc32c_bitwise(data: bytes) -> int:
    """Textbook bit-at-a-time CRC32C (Castagnoli, reflected), independent of
    any table."""
    c = 0xFFFFFFFF
    for b in data:
        c ^= b
        for _ in range(8):
            c = (c >> 1) ^ (0x82F63B78 if c & 1 else 0)
    return c ^ 0xFFFFFFFF


def test_crc32c_known_vectors(rko, rkv):
    # crc32c.rs:37-42
    for data, want in [(b"", 0x00000000), (b"123456789", 0xE3069283),
                       (b"hello world", 0xC99465AA)]:
        assert rko.crc32c(data) == want
        assert rkv.crc32c_host(data) == want
        assert _crc32c_bitwise(data) == want


def test_crc32c_matches_bitwise_and_detects_flips(rko, rkv):
    rng = random.Random(3)
    for n in [1, 2, 3, 7, 64, 255, 1000, 4099]:
        data = bytes(rng.randrange(256) for _ in range(n))
        want = _crc32c_bitwise(data)
        assert rko.crc32c(data) == want and rkv.crc32c_host(data) == want
    d = bytearray([7] * 512)                      # crc32c.rs:45-52
    base = rko.crc32c(bytes(d))
    d[123] ^= 0x10
    assert rko.crc32c(bytes(d)) != base


def _sample_header(rko):
    # page.rs:264-279
    return dict(prefix_digest=0xDEADBEEF12345678, token_start=4096, token_count=512,
                pos_start=4096, layer_lo=3, layer_hi=63, k_fmt=2, v_fmt=3, epoch=7,
                generation=42, payload_len=1024, sketch_offset=96 + 1024, flags=0)


def test_header_bytes_layout(rko, rkv):
    """Field offsets of PageHeader::to_bytes (page.rs:100-126), byte by byte."""
    f = _sample_header(rko)
    b = rko.r4kv_header_bytes(rko.r4kv_header(**f))
    assert b[0:4] == (0x52344B56).to_bytes(4, "little") and b[4:6] == (1).to_bytes(2, "little")
    assert b[6:8] == (0).to_bytes(2, "little")
    assert b[8:16] == f["prefix_digest"].to_bytes(8, "little")
    assert b[16:20] == (4096).to_bytes(4, "little") and b[20:24] == (512).to_bytes(4, "little")
    assert b[24:28] == (4096).to_bytes(4, "little")
    assert b[28:30] == (3).to_bytes(2, "little") and b[30:32] == (63).to_bytes(2, "little")
    assert b[32] == 2 and b[33] == 3
    assert b[34:38] == (7).to_bytes(4, "little") and b[38:42] == (42).to_bytes(4, "little")
    assert b[42:50] == (1024).to_bytes(8, "little") and b[50:54] == (1120).to_bytes(4, "little")
    assert b[54:92] == bytes(38)
    assert b[92:96] == _crc32c_bitwise(b[:92]).to_bytes(4, "little")
    assert rkv.r4kv_header_encode(rkv.R4kvHeader(**f)) == b


def test_header_encode_matches_oracle_random(rko, rkv):
    rng = random.Random(9)
    for _ in range(200):
        f = dict(prefix_digest=rng.getrandbits(64), token_start=rng.getrandbits(32),
                 token_count=rng.getrandbits(32), pos_start=rng.getrandbits(32),
                 layer_lo=rng.getrandbits(16), layer_hi=rng.getrandbits(16),
                 k_fmt=rng.randrange(5), v_fmt=rng.randrange(5), epoch=rng.getrandbits(32),
                 generation=rng.getrandbits(32), payload_len=rng.getrandbits(64),
                 sketch_offset=rng.getrandbits(32), flags=rng.getrandbits(16))
        b = rkv.r4kv_header_encode(rkv.R4kvHeader(**f))
        assert b == rko.r4kv_header_bytes(rko.r4kv_header(**f))
        back = rkv.r4kv_header_decode(b)
        assert {k: getattr(back, k) for k in f} == f


def _refusal(rkv, fn, *args):
    with pytest.raises(rkv.R4kvRefused) as e:
        fn(*args)
    assert e.value.status == rkv.ERR_REFUSED
    return e.value.refusal


def test_header_roundtrip_and_checksum_gate(rko, rkv):
    # page.rs:283-296, plus the magic / version / format gates of from_bytes
    f = _sample_header(rko)
    b = bytearray(rkv.r4kv_header_encode(rkv.R4kvHeader(**f)))
    assert len(b) == 96
    back = rkv.r4kv_header_decode(bytes(b))
    assert {k: getattr(back, k) for k in f} == f
    bad = bytearray(b)
    bad[20] ^= 0x01
    assert _refusal(rkv, rkv.r4kv_header_decode, bytes(bad)) == rkv.R4KV_HEADER_CHECKSUM
    bad = bytearray(b)
    bad[0] ^= 0xFF
    assert _refusal(rkv, rkv.r4kv_header_decode, bytes(bad)) == rkv.R4KV_BAD_MAGIC
    bad = bytearray(b)
    bad[4] = 2
    assert _refusal(rkv, rkv.r4kv_header_decode, bytes(bad)) == rkv.R4KV_BAD_VERSION
    g = dict(f, k_fmt=5)  # an id from_u8 refuses (lib.rs:33-42), with a valid header CRC
    raw = rko.r4kv_header_bytes(rko.r4kv_header(**g))
    assert _refusal(rkv, rkv.r4kv_header_decode, raw) == rkv.R4KV_FORMAT


def test_page_roundtrip_with_payload_crc(rko, rkv):
    # page.rs:298-316
    f = _sample_header(rko)
    body = bytes((i * 31 % 251) for i in range(1024))
    f["payload_len"] = len(body)
    page = rko.r4kv_pack_page(rko.r4kv_header(**f), body)
    h, b2 = rkv.r4kv_unpack_host(page)
    assert {k: getattr(h, k) for k in f} == f and b2 == body
    bad = bytearray(page)
    bad[len(bad) - 10] ^= 0xFF
    assert _refusal(rkv, rkv.r4kv_unpack_host, bytes(bad)) == rkv.R4KV_PAYLOAD_CHECKSUM
    assert _refusal(rkv, rkv.r4kv_unpack_host, page[:99]) == rkv.R4KV_LENGTH
    assert _refusal(rkv, rkv.r4kv_unpack_host, page[:-1]) == rkv.R4KV_LENGTH


def test_restore_gate_fails_closed_on_every_axis(rko, rkv):
    # page.rs:318-373, plus the format and generation axes of check_restore
    f = _sample_header(rko)
    h = rkv.R4kvHeader(**f)

    def exp(**kw):
        base = dict(prefix_digest=f["prefix_digest"], token_start=4096, pos_start=4096, layer_lo=3,
                    layer_hi=63, k_fmt=-1, v_fmt=-1, check_generation=0, generation_min=0,
                    generation_max=0)
        base.update(kw)
        return rkv.R4kvExpect(**base)

    rkv.r4kv_check_restore(h, exp(), 1024)
    cases = [
        (dict(), 1000, rkv.R4KV_LENGTH),
        (dict(prefix_digest=1), 1024, rkv.R4KV_PREFIX),
        (dict(token_start=999), 1024, rkv.R4KV_TOKEN_RANGE),
        (dict(pos_start=1), 1024, rkv.R4KV_POS),
        (dict(layer_hi=99), 1024, rkv.R4KV_LAYER_RANGE),
        (dict(layer_lo=2), 1024, rkv.R4KV_LAYER_RANGE),
        (dict(v_fmt=0), 1024, rkv.R4KV_FORMAT),
        (dict(k_fmt=1), 1024, rkv.R4KV_FORMAT),
        (dict(check_generation=1, generation_min=41, generation_max=41), 1024, rkv.R4KV_GENERATION),
    ]
    for kw, n, why in cases:
        assert _refusal(rkv, rkv.r4kv_check_restore, h, exp(**kw), n) == why, kw
    # a narrower wanted layer range and a matching generation predicate pass
    rkv.r4kv_check_restore(h, exp(layer_lo=10, layer_hi=20, check_generation=1, generation_min=40,
                                  generation_max=42, k_fmt=2, v_fmt=3), 1024)
