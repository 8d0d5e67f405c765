"""ctypes binding of the CPU oracle (oracle/rkv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product path (remora-lab_amd/) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def _stale() -> bool:
    if not os.path.exists(_SO):
        return True
    so = os.path.getmtime(_SO)
    return any(os.path.getmtime(os.path.join(_HERE, f)) > so
               for f in ("rkv_oracle.c", "rkv_oracle.h", "Makefile"))


def lib():
    global _lib
    if _lib is None:
        if _stale():
            build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


class FdParams(C.Structure):
    _fields_ = [("q_heads", C.c_int32), ("kv_heads", C.c_int32), ("seq_len", C.c_int32),
                ("chunk", C.c_int32), ("head_dim", C.c_int32)]


class Layout(C.Structure):
    _fields_ = [("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("page_tokens", C.c_int32), ("num_pages", C.c_int32)]


class GroupStats(C.Structure):
    _fields_ = [("max_abs_err", C.c_float), ("sum_sq_err", C.c_double),
                ("sum_sq_ref", C.c_double)]


P = C.c_void_p


class R4kvHeader(C.Structure):
    _fields_ = [("prefix_digest", C.c_uint64), ("token_start", C.c_uint32),
                ("token_count", C.c_uint32), ("pos_start", C.c_uint32), ("layer_lo", C.c_uint16),
                ("layer_hi", C.c_uint16), ("k_fmt", C.c_uint8), ("v_fmt", C.c_uint8),
                ("epoch", C.c_uint32), ("generation", C.c_uint32), ("payload_len", C.c_uint64),
                ("sketch_offset", C.c_uint32), ("flags", C.c_uint16)]


def _declare(L):
    sig = {
        "rko_crc32c": (C.c_uint32, [P, C.c_size_t]),
        "rko_r4kv_header_bytes": (None, [P, P]),
        "rko_r4kv_pack_page": (None, [P, P, C.c_size_t, P]),
        "rko_splitmix64": (C.c_uint64, [C.c_uint64]),
        "rko_seeded_float": (C.c_float, [C.c_uint64]),
        "rko_lcg_values": (None, [P, C.c_size_t, C.c_uint64]),
        "rko_normal_f32": (None, [P, C.c_size_t, C.c_uint64]),
        "rko_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "rko_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "rko_f16_to_f32": (C.c_float, [C.c_uint16]),
        "rko_f16_to_f32_harserve": (C.c_float, [C.c_uint8, C.c_uint8]),
        "rko_f32_to_f16": (C.c_uint16, [C.c_float]),
        "rko_f32_to_f16_harserve": (C.c_uint16, [C.c_float]),
        "rko_q8_encode": (C.c_float, [P, C.c_size_t, P]),
        "rko_q8_quantize_harserve": (None, [P, C.c_size_t, P]),
        "rko_q8_decode": (None, [P, C.c_size_t, P]),
        "rko_q8_dequant_row": (None, [P, C.c_size_t, P]),
        "rko_roundtrip_stats": (None, [P, C.c_size_t, C.c_int, P, C.POINTER(GroupStats)]),
        "rko_rel_rms": (C.c_float, [C.POINTER(GroupStats)]),
        "rko_normalized_kl": (C.c_double, [P, P, C.c_size_t]),
        "rko_q8_kv_value": (C.c_float, [P, C.c_size_t, C.c_size_t]),
        "rko_row_to_words": (None, [P, C.c_size_t, P]),
        "rko_flash_decode_online": (None, [C.POINTER(FdParams), P, P, P, C.c_int32, P, P, P]),
        "rko_flash_decode_reference": (None, [C.POINTER(FdParams), P, P, P, P]),
        "rko_flash_decode_reference_many": (None, [C.POINTER(FdParams), C.c_int32, P, P, P, P,
                                                   C.c_int32]),
        "rko_flash_decode_bruteforce": (None, [C.POINTER(FdParams), P, P, P, C.c_int32, P]),
        "rko_flash_decode_partials": (C.c_int32, [C.POINTER(FdParams), P, P, P, C.c_int32, P, P, P]),
        "rko_lse_combine": (None, [C.c_int32, C.c_int32, P, P, P, P, P, P]),
        "rko_attention_f64": (None, [C.c_int32, C.c_int32, P, P, P, P]),
        "rko_region_bytes": (C.c_size_t, [C.POINTER(Layout)]),
        "rko_page_bytes": (C.c_size_t, [C.POINTER(Layout)]),
        "rko_code_offset": (C.c_size_t, [C.POINTER(Layout), C.c_int, C.c_int32, C.c_int32]),
        "rko_scale_offset": (C.c_size_t, [C.POINTER(Layout), C.c_int32, C.c_int32]),
        "rko_paged_append": (C.c_int32, [C.POINTER(Layout), P, P, C.c_int32, P, P, C.c_int32, P, P, C.c_int]),
        "rko_paged_gather": (C.c_int32, [C.POINTER(Layout), P, P, C.c_int32, C.c_int, P]),
        "rko_paged_decode": (C.c_int32, [C.POINTER(Layout), P, P, C.c_int32, P, P, C.c_int32,
                                         C.c_int32, C.c_int32, P, C.c_float, C.c_int32, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(P)


# ---- generators -------------------------------------------------------------

def lcg_values(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().rko_lcg_values(_p(out), count, seed)
    return out


def normal_f32(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().rko_normal_f32(_p(out), count, seed)
    return out


def seeded_float(i: int) -> float:
    return lib().rko_seeded_float(i)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """RTNE f32 -> bf16 bits (uint16), vectorised in numpy."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- codecs -----------------------------------------------------------------

def q8_encode(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, np.float32)
    out = np.empty(src.size // 32 * 34, np.uint8)
    lib().rko_q8_encode(_p(src), src.size, _p(out))
    return out


def q8_quantize_harserve(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, np.float32)
    out = np.empty(src.size // 32 * 34, np.uint8)
    lib().rko_q8_quantize_harserve(_p(src), src.size, _p(out))
    return out


def q8_quantize(src: np.ndarray, rule: int) -> np.ndarray:
    return q8_encode(src) if rule == 0 else q8_quantize_harserve(src)


def q8_decode(enc: np.ndarray, n: int) -> np.ndarray:
    enc = np.ascontiguousarray(enc, np.uint8)
    out = np.empty(n, np.float32)
    lib().rko_q8_decode(_p(enc), n, _p(out))
    return out


def q8_dequant_row(row: np.ndarray, n: int) -> np.ndarray:
    row = np.ascontiguousarray(row, np.uint8)
    out = np.empty(n, np.float32)
    lib().rko_q8_dequant_row(_p(row), n, _p(out))
    return out


def roundtrip_stats(src: np.ndarray, fmt: int):
    src = np.ascontiguousarray(src, np.float32)
    dec = np.empty_like(src)
    st = GroupStats()
    lib().rko_roundtrip_stats(_p(src), src.size, fmt, _p(dec), C.byref(st))
    return dec, st, lib().rko_rel_rms(C.byref(st))


def normalized_kl(ref: np.ndarray, cand: np.ndarray) -> float:
    ref = np.ascontiguousarray(ref, np.float32)
    cand = np.ascontiguousarray(cand, np.float32)
    return lib().rko_normalized_kl(_p(ref), _p(cand), ref.size)


def row_bytes(head_dim: int) -> int:
    return head_dim // 32 * 34


def rows_to_words(rows: np.ndarray) -> np.ndarray:
    rows = np.ascontiguousarray(rows, np.uint8)
    return rows.reshape(-1).view("<u4").copy()


# ---- reference flash decode ----------------------------------------------

def fd_params(q_heads, kv_heads, seq_len, chunk, head_dim=256) -> FdParams:
    return FdParams(q_heads, kv_heads, seq_len, chunk, head_dim)


def flash_decode_reference(p: FdParams, k_words, v_words, query) -> np.ndarray:
    query = np.ascontiguousarray(query, np.float32)
    out = np.empty(p.q_heads * p.head_dim, np.float32)
    lib().rko_flash_decode_reference(C.byref(p), _p(k_words), _p(v_words), _p(query), _p(out))
    return out


def flash_decode_reference_many(p: FdParams, k_words: list, v_words: list, queries,
                                threads: int) -> np.ndarray:
    """flash_decode_reference over len(k_words) sequences of p.seq_len tokens
    on `threads` OpenMP threads; queries [n][q_heads][D] -> out [n][q_heads][D]."""
    n = len(k_words)
    queries = np.ascontiguousarray(queries, np.float32)
    ks = [np.ascontiguousarray(k, np.uint32) for k in k_words]
    vs = [np.ascontiguousarray(v, np.uint32) for v in v_words]
    kp = (P * n)(*[_p(k) for k in ks])
    vp = (P * n)(*[_p(v) for v in vs])
    out = np.empty((n, p.q_heads, p.head_dim), np.float32)
    lib().rko_flash_decode_reference_many(C.byref(p), n, kp, vp, _p(queries), _p(out), threads)
    return out


def flash_decode_online(p: FdParams, k_words, v_words, q, kvh):
    q = np.ascontiguousarray(q, np.float32)
    o = np.empty(p.head_dim, np.float32)
    m = C.c_float()
    l = C.c_float()
    lib().rko_flash_decode_online(C.byref(p), _p(k_words), _p(v_words), _p(q), kvh,
                                  C.byref(m), C.byref(l), _p(o))
    return m.value, l.value, o


def flash_decode_bruteforce(p: FdParams, k_words, v_words, q, kvh) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    o = np.empty(p.head_dim, np.float32)
    lib().rko_flash_decode_bruteforce(C.byref(p), _p(k_words), _p(v_words), _p(q), kvh, _p(o))
    return o


def flash_decode_partials(p: FdParams, k_words, v_words, q, kvh):
    q = np.ascontiguousarray(q, np.float32)
    nmax = (p.seq_len + p.chunk - 1) // p.chunk
    cm = np.empty(max(nmax, 1), np.float32)
    lc = np.empty(max(nmax, 1), np.float32)
    oc = np.empty((max(nmax, 1), p.head_dim), np.float32)
    n = lib().rko_flash_decode_partials(C.byref(p), _p(k_words), _p(v_words), _p(q), kvh,
                                        _p(cm), _p(lc), _p(oc))
    return cm[:n], lc[:n], oc[:n]


def lse_combine(cm, lc, oc):
    cm = np.ascontiguousarray(cm, np.float32)
    lc = np.ascontiguousarray(lc, np.float32)
    oc = np.ascontiguousarray(oc, np.float32)
    d = oc.shape[-1]
    out = np.empty(d, np.float32)
    m = C.c_float()
    l = C.c_float()
    lib().rko_lse_combine(len(cm), d, _p(cm), _p(lc), _p(oc), _p(out), C.byref(m), C.byref(l))
    return out, m.value, l.value


def attention_f64(seq_len, head_dim, k_words, v_words, q) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty(head_dim, np.float64)
    lib().rko_attention_f64(seq_len, head_dim, _p(k_words), _p(v_words), _p(q), _p(out))
    return out


# ---- paged layout -----------------------------------------------------------

def layout(kv_heads, head_dim, page_tokens, num_pages) -> Layout:
    return Layout(kv_heads, head_dim, page_tokens, num_pages)


def page_bytes(L: Layout) -> int:
    return lib().rko_page_bytes(C.byref(L))


def paged_append(L: Layout, pages: np.ndarray, block_tables: np.ndarray, seq_ids, positions,
                 k_src: np.ndarray, v_src: np.ndarray, rule: int = 0) -> None:
    bt = np.ascontiguousarray(block_tables, np.int32)
    sid = np.ascontiguousarray(seq_ids, np.int32)
    pos = np.ascontiguousarray(positions, np.int32)
    k = np.ascontiguousarray(k_src, np.float32)
    v = np.ascontiguousarray(v_src, np.float32)
    rc = lib().rko_paged_append(C.byref(L), _p(pages), _p(bt), bt.shape[-1], _p(sid), _p(pos),
                                len(sid), _p(k), _p(v), rule)
    if rc != 0:
        raise ValueError(f"oracle paged_append failed rc={rc}")


def paged_gather(L: Layout, pages: np.ndarray, block_table: np.ndarray, length: int,
                 kind: int) -> np.ndarray:
    bt = np.ascontiguousarray(block_table, np.int32)
    out = np.empty(L.kv_heads * length * row_bytes(L.head_dim), np.uint8)
    rc = lib().rko_paged_gather(C.byref(L), _p(pages), _p(bt), length, kind, _p(out))
    if rc != 0:
        raise ValueError(f"oracle paged_gather failed rc={rc}")
    return out.reshape(L.kv_heads, length, row_bytes(L.head_dim))


def paged_decode(L: Layout, pages, block_tables, seq_lens, seq_ids, q: np.ndarray,
                 scale: float, chunk: int) -> np.ndarray:
    """q: [B][q_len][q_heads][D] f32.  Returns the same shape."""
    q = np.ascontiguousarray(q, np.float32)
    B, q_len, q_heads, D = q.shape
    bt = np.ascontiguousarray(block_tables, np.int32)
    sl = np.ascontiguousarray(seq_lens, np.int32)
    sid = np.ascontiguousarray(seq_ids, np.int32)
    out = np.empty_like(q)
    rc = lib().rko_paged_decode(C.byref(L), _p(pages), _p(bt), bt.shape[-1], _p(sl), _p(sid), B,
                                q_len, q_heads, _p(q), scale, chunk, _p(out))
    if rc != 0:
        raise ValueError(f"oracle paged_decode failed rc={rc}")
    return out


def crc32c(data) -> int:
    b = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else \
        np.ascontiguousarray(data, np.uint8).reshape(-1)
    return int(lib().rko_crc32c(_p(b) if b.size else None, b.size))


def r4kv_header(**fields) -> R4kvHeader:
    return R4kvHeader(**fields)


def r4kv_header_bytes(h: R4kvHeader) -> bytes:
    out = np.zeros(96, np.uint8)
    lib().rko_r4kv_header_bytes(C.byref(h), _p(out))
    return out.tobytes()


def r4kv_pack_page(h: R4kvHeader, body) -> bytes:
    b = np.ascontiguousarray(np.frombuffer(bytes(body), np.uint8) if not isinstance(body, np.ndarray)
                             else body, np.uint8).reshape(-1)
    out = np.zeros(96 + b.size + 4, np.uint8)
    lib().rko_r4kv_pack_page(C.byref(h), _p(b) if b.size else None, b.size, _p(out))
    return out.tobytes()

