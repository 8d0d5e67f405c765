"""Python binding of librkv.so, the C ABI in include/rkv.h.

The paged Q8_0 KV-cache hot path runs entirely in the HIP kernels behind that
ABI; this module only forwards device pointers (torch tensors on a ROCm
device) and turns non-zero statuses into RkvError, mirroring the reference's
fail-closed HarError convention (har/crates/har-vulkan/src/lib.rs:17-56).
There is no CPU fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librkv.so")
HEADER = os.path.join(HERE, "..", "include", "rkv.h")

OK = 0
ERR_INVALID_ARG = -1
ERR_OUT_OF_PAGES = -2
ERR_BAD_BLOCK_TABLE = -3
ERR_UNSUPPORTED = -4
ERR_DEVICE = -5
ERR_CAPACITY = -6
ERR_REFUSED = -7

F32, BF16 = 0, 1
Q8_CANONICAL, Q8_HARSERVE = 0, 1
K, V = 0, 1

_STATUS_NAMES = {0: "OK", -1: "INVALID_ARG", -2: "OUT_OF_PAGES", -3: "BAD_BLOCK_TABLE",
                 -4: "UNSUPPORTED", -5: "DEVICE", -6: "CAPACITY", -7: "REFUSED"}

# R4KV refusal reasons (RestoreError, r4kv/src/page.rs:63-76) and formats
R4KV_ACCEPTED, R4KV_BAD_MAGIC, R4KV_BAD_VERSION, R4KV_HEADER_CHECKSUM = 0, 1, 2, 3
R4KV_PAYLOAD_CHECKSUM, R4KV_LENGTH, R4KV_PREFIX, R4KV_TOKEN_RANGE = 4, 5, 6, 7
R4KV_POS, R4KV_LAYER_RANGE, R4KV_FORMAT, R4KV_GENERATION = 8, 9, 10, 11
FMT_F16, FMT_Q8, FMT_Q6, FMT_Q4, FMT_Q3 = 0, 1, 2, 3, 4


class RkvError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


P = C.c_void_p
I32P = C.POINTER(C.c_int32)


class Geometry(C.Structure):
    _fields_ = [("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("page_tokens", C.c_int32),
                ("num_pages", C.c_int32)]


class AllocDesc(C.Structure):
    _fields_ = [("num_pages", C.c_int32), ("page_tokens", C.c_int32), ("max_seqs", C.c_int32),
                ("max_pages_per_seq", C.c_int32), ("free_list_seed", C.c_uint64)]


class AppendArgs(C.Structure):
    _fields_ = [("n_rows", C.c_int32), ("seq_ids", P), ("positions", P), ("k_src", P),
                ("v_src", P), ("src_dtype", C.c_int32), ("rule", C.c_int32)]


class DecodeArgs(C.Structure):
    _fields_ = [("batch", C.c_int32), ("seq_ids", P), ("q", P), ("q_dtype", C.c_int32),
                ("q_len", C.c_int32), ("q_heads", C.c_int32), ("scale", C.c_float),
                ("out", P), ("out_dtype", C.c_int32), ("partition_tokens", C.c_int32),
                ("max_seq_len", C.c_int32), ("workspace", P), ("workspace_bytes", C.c_size_t),
                ("append", C.POINTER(AppendArgs)), ("split_event", P)]


class PrefillArgs(C.Structure):
    _fields_ = [("n_seqs", C.c_int32), ("seq_ids", I32P), ("ctx_lens", I32P), ("q_rows", I32P),
                ("q_offsets", I32P), ("total_rows", C.c_int32), ("q", P), ("q_dtype", C.c_int32),
                ("q_heads", C.c_int32), ("scale", C.c_float), ("out", P), ("out_dtype", C.c_int32),
                ("segment_tokens", C.c_int32), ("workspace", P), ("workspace_bytes", C.c_size_t)]


PREFILL_MAX_SEQS = 64


class R4kvHeader(C.Structure):
    _fields_ = [("prefix_digest", C.c_uint64), ("token_start", C.c_uint32),
                ("token_count", C.c_uint32), ("pos_start", C.c_uint32), ("layer_lo", C.c_uint16),
                ("layer_hi", C.c_uint16), ("k_fmt", C.c_uint8), ("v_fmt", C.c_uint8),
                ("epoch", C.c_uint32), ("generation", C.c_uint32), ("payload_len", C.c_uint64),
                ("sketch_offset", C.c_uint32), ("flags", C.c_uint16)]


class R4kvExpect(C.Structure):
    _fields_ = [("prefix_digest", C.c_uint64), ("token_start", C.c_uint32),
                ("pos_start", C.c_uint32), ("layer_lo", C.c_uint16), ("layer_hi", C.c_uint16),
                ("k_fmt", C.c_int32), ("v_fmt", C.c_int32), ("check_generation", C.c_int32),
                ("generation_min", C.c_uint32), ("generation_max", C.c_uint32)]


class FlashDecodeParams(C.Structure):
    _fields_ = [("q_heads", C.c_int32), ("kv_heads", C.c_int32), ("seq_len", C.c_int32),
                ("chunk", C.c_int32), ("head_dim", C.c_int32)]


class ServeDesc(C.Structure):
    _fields_ = [("layers", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("page_tokens", C.c_int32), ("num_pages", C.c_int32), ("max_seqs", C.c_int32),
                ("max_pages_per_seq", C.c_int32), ("q_heads", C.c_int32),
                ("max_decode", C.c_int32), ("max_prefill_rows", C.c_int32), ("rule", C.c_int32),
                ("free_list_seed", C.c_uint64), ("page_memory", C.c_int32)]


class ServeEntry(C.Structure):
    _fields_ = [("id", C.c_uint64), ("tokens", C.c_int32), ("fork_len", C.c_int32),
                ("parent", C.c_uint64)]


class PageLocation(C.Structure):
    _fields_ = [("page", C.c_int32), ("offset", C.c_uint64), ("length", C.c_uint64),
                ("layer_stride", C.c_uint64), ("generation", C.c_uint64),
                ("first_slot", C.c_int32), ("slots", C.c_int32)]


class PoolDesc(C.Structure):
    _fields_ = [("layers", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("page_tokens", C.c_int32), ("num_pages", C.c_int32), ("max_seqs", C.c_int32),
                ("max_pages_per_seq", C.c_int32), ("free_list_seed", C.c_uint64),
                ("page_memory", C.c_int32)]


PAGES_DEVICE, PAGES_HOST = 0, 1


_SIGS = {
    "rkv_last_error": (C.c_char_p, []),
    "rkv_version": (C.c_char_p, []),
    "rkv_ctx_create": (C.c_int32, [C.c_int32, C.POINTER(P)]),
    "rkv_ctx_destroy": (C.c_int32, [P]),
    "rkv_ctx_sync": (C.c_int32, [P, P]),
    "rkv_geometry_check": (C.c_int32, [C.POINTER(Geometry)]),
    "rkv_page_bytes": (C.c_size_t, [C.POINTER(Geometry)]),
    "rkv_row_bytes": (C.c_size_t, [C.c_int32]),
    "rkv_alloc_create": (C.c_int32, [C.POINTER(AllocDesc), C.POINTER(P)]),
    "rkv_alloc_destroy": (C.c_int32, [P]),
    "rkv_seq_reserve": (C.c_int32, [P, C.c_int32, C.c_int32]),
    "rkv_seq_truncate": (C.c_int32, [P, C.c_int32, C.c_int32]),
    "rkv_seq_reserve_n": (C.c_int32, [P, C.c_int32, I32P, I32P, I32P]),
    "rkv_seq_truncate_n": (C.c_int32, [P, C.c_int32, I32P, I32P, I32P]),
    "rkv_seq_free": (C.c_int32, [P, C.c_int32]),
    "rkv_seq_len": (C.c_int32, [P, C.c_int32, I32P]),
    "rkv_block_table_get": (C.c_int32, [P, C.c_int32, I32P, C.c_int32, I32P]),
    "rkv_alloc_free_pages": (C.c_int32, [P, I32P]),
    "rkv_alloc_export": (C.c_int32, [P, P, P]),
    "rkv_seq_fork": (C.c_int32, [P, C.c_int32, C.c_int32, C.c_int32]),
    "rkv_page_refs": (C.c_int32, [P, C.c_int32, I32P]),
    "rkv_alloc_take_copies": (C.c_int32, [P, P, C.c_int32, I32P]),
    "rkv_copy_pages": (C.c_int32, [P, C.POINTER(Geometry), P, C.c_int64, C.c_int32, P,
                                   C.c_int32, P]),
    "rkv_append_q8": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, C.c_int32,
                                  C.POINTER(AppendArgs), P]),
    "rkv_decode_q8": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, P, C.c_int32,
                                  C.POINTER(DecodeArgs), P]),
    "rkv_decode_q8_noalloc": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, P, C.c_int32,
                                          C.POINTER(DecodeArgs), P]),
    "rkv_decode_workspace_bytes": (C.c_size_t, [C.POINTER(Geometry), C.POINTER(DecodeArgs)]),
    "rkv_prefill_workspace_bytes": (C.c_size_t, [C.POINTER(Geometry), C.POINTER(PrefillArgs)]),
    "rkv_pool_prefill_workspace_bytes": (C.c_size_t, [P, C.POINTER(PrefillArgs)]),
    "rkv_decode_partition_tokens": (C.c_int32, [C.POINTER(Geometry), C.POINTER(DecodeArgs)]),
    "rkv_decode_q8_partials": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, P,
                                           C.c_int32, C.POINTER(DecodeArgs), P, P, P]),
    "rkv_splitk_combine": (C.c_int32, [P, P, P, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                       P, P, C.c_int32, C.c_int32, P, C.c_int32, P]),
    "rkv_gather_q8": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, C.c_int32, P, P]),
    "rkv_import_q8": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, C.c_int32, P, P]),
    "rkv_f32_to_f16": (C.c_int32, [P, P, P, C.c_int64, C.c_int32, P]),
    "rkv_flash_decode_scratch_bytes": (C.c_size_t, [C.POINTER(FlashDecodeParams)]),
    "rkv_flash_decode_q8": (C.c_int32, [P, C.POINTER(FlashDecodeParams), P, P, P, P, P, P]),
    "rkv_pool_create": (C.c_int32, [P, C.POINTER(PoolDesc), C.POINTER(P)]),
    "rkv_pool_destroy": (C.c_int32, [P]),
    "rkv_pool_release_stream": (C.c_int32, [P, P]),
    "rkv_pool_allocator": (P, [P]),
    "rkv_pool_sync_tables": (C.c_int32, [P, P]),
    "rkv_pool_layer_pages": (P, [P, C.c_int32]),
    "rkv_pool_block_tables": (P, [P]),
    "rkv_pool_seq_lens": (P, [P]),
    "rkv_pool_append": (C.c_int32, [P, C.c_int32, C.POINTER(AppendArgs), P]),
    "rkv_pool_decode": (C.c_int32, [P, C.c_int32, C.POINTER(DecodeArgs), P]),
    "rkv_pool_gather": (C.c_int32, [P, C.c_int32, C.c_int32, C.c_int32, P, P]),
    "rkv_prefill_q8": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, C.c_int32,
                                   C.POINTER(PrefillArgs), P]),
    "rkv_pool_prefill": (C.c_int32, [P, C.c_int32, C.POINTER(PrefillArgs), P]),
    "rkv_crc32c_host": (C.c_uint32, [P, C.c_size_t]),
    "rkv_crc32c": (C.c_int32, [P, P, C.c_uint64, P, P]),
    "rkv_r4kv_header_encode": (C.c_int32, [C.POINTER(R4kvHeader), P]),
    "rkv_r4kv_header_decode": (C.c_int32, [P, C.POINTER(R4kvHeader), I32P]),
    "rkv_r4kv_check_restore": (C.c_int32, [C.POINTER(R4kvHeader), C.POINTER(R4kvExpect),
                                           C.c_uint64, I32P]),
    "rkv_r4kv_unpack_host": (C.c_int32, [P, C.c_size_t, C.POINTER(R4kvHeader),
                                         C.POINTER(P), I32P]),
    "rkv_r4kv_page_bytes": (C.c_size_t, [P, C.c_int32, C.c_int32, C.c_int32]),
    "rkv_pool_spill": (C.c_int32, [P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                   C.POINTER(R4kvHeader), P, C.c_size_t, P, C.c_size_t, P]),
    "rkv_pool_restore": (C.c_int32, [P, C.c_int32, P, C.c_size_t, C.POINTER(R4kvExpect), P,
                                     C.c_size_t, I32P, P]),
    "rkv_stream_read": (C.c_int32, [P, P, C.c_uint64, C.c_int32, C.c_int32, P, P]),
    "rkv_stream_read_tiles": (C.c_int32, [P, C.POINTER(Geometry), P, P, C.c_int32, C.c_int32,
                                          C.c_int32, C.c_int32, P]),
    "rkv_page_generation": (C.c_int32, [P, C.c_int32, C.POINTER(C.c_uint64)]),
    "rkv_serve_create": (C.c_int32, [P, C.POINTER(ServeDesc), C.POINTER(P)]),
    "rkv_serve_destroy": (C.c_int32, [P]),
    "rkv_serve_pool": (P, [P]),
    "rkv_serve_geometry": (C.c_int32, [P, C.POINTER(Geometry)]),
    "rkv_serve_begin_step": (C.c_int32, [P, C.POINTER(ServeEntry), C.c_int32,
                                         C.POINTER(ServeEntry), C.c_int32, P]),
    "rkv_serve_decode": (C.c_int32, [P, C.c_int32, P, P, P, C.c_int32, P, C.c_int32,
                                     C.c_float, P]),
    "rkv_serve_prefill": (C.c_int32, [P, C.c_int32, P, P, P, C.c_int32, P, C.c_int32,
                                      C.c_float, P]),
    "rkv_serve_truncate": (C.c_int32, [P, C.c_uint64, C.c_int32]),
    "rkv_serve_finish": (C.c_int32, [P, C.c_uint64]),
    "rkv_serve_seq_len": (C.c_int32, [P, C.c_uint64, I32P]),
    "rkv_serve_page_location": (C.c_int32, [P, C.c_uint64, C.c_int32, C.POINTER(PageLocation)]),
    "rkv_serve_seq_slot": (C.c_int32, [P, C.c_uint64, I32P]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/rkv.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(rkv_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load librkv.so; raise if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise RkvError(status, lib().rkv_last_error().decode())


def _ptr(t) -> P:
    """Device pointer of a torch tensor (or an int address, or None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return P(t)
    return P(t.data_ptr())


def _stream(s) -> P:
    if s is None:
        import torch
        return P(torch.cuda.current_stream().cuda_stream)
    if isinstance(s, int):
        return P(s)
    return P(s.cuda_stream)


class Ctx:
    """Device context (replaces har-vulkan Device::open + Queue)."""

    def __init__(self, device: int = 0):
        h = P()
        check(lib().rkv_ctx_create(device, C.byref(h)))
        self.h = h
        self.device = device

    def sync(self, stream=None) -> None:
        check(lib().rkv_ctx_sync(self.h, _stream(stream)))

    def close(self) -> None:
        if self.h:
            lib().rkv_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def geometry(kv_heads: int, head_dim: int, page_tokens: int, num_pages: int) -> Geometry:
    g = Geometry(kv_heads, head_dim, page_tokens, num_pages)
    check(lib().rkv_geometry_check(C.byref(g)))
    return g


def page_bytes(g: Geometry) -> int:
    return lib().rkv_page_bytes(C.byref(g))


def row_bytes(head_dim: int) -> int:
    return lib().rkv_row_bytes(head_dim)


class Allocator:
    """Host page allocator + block tables (rkv_alloc_*)."""

    def __init__(self, num_pages, page_tokens, max_seqs, max_pages_per_seq, seed=0, handle=None):
        self.owned = handle is None
        if handle is None:
            h = P()
            d = AllocDesc(num_pages, page_tokens, max_seqs, max_pages_per_seq, seed)
            check(lib().rkv_alloc_create(C.byref(d), C.byref(h)))
            handle = h
        self.h = handle
        self.num_pages = num_pages
        self.max_seqs = max_seqs
        self.max_pages_per_seq = max_pages_per_seq

    def reserve(self, seq: int, new_len: int) -> None:
        check(lib().rkv_seq_reserve(self.h, seq, new_len))

    def truncate(self, seq: int, new_len: int) -> None:
        check(lib().rkv_seq_truncate(self.h, seq, new_len))

    def _apply_n(self, fn, seqs, new_lens) -> int:
        import numpy as np
        s = np.ascontiguousarray(seqs, dtype=np.int32)
        n = np.ascontiguousarray(new_lens, dtype=np.int32)
        if s.shape != n.shape or s.ndim != 1:
            raise ValueError("seqs and new_lens must be 1-D and of one length")
        done = C.c_int32(0)
        st = fn(self.h, int(s.size), s.ctypes.data_as(I32P), n.ctypes.data_as(I32P), C.byref(done))
        check(st)
        return done.value

    def reserve_n(self, seqs, new_lens) -> int:
        """rkv_seq_reserve_n: every (seq, new_len) pair in order, stopping at
        the first failure (raised; the pairs before it have taken effect)."""
        return self._apply_n(lib().rkv_seq_reserve_n, seqs, new_lens)

    def truncate_n(self, seqs, new_lens) -> int:
        """rkv_seq_truncate_n: as reserve_n, rolling back."""
        return self._apply_n(lib().rkv_seq_truncate_n, seqs, new_lens)

    def free(self, seq: int) -> None:
        check(lib().rkv_seq_free(self.h, seq))

    def fork(self, src: int, dst: int, length: int) -> None:
        """Share src's first `length` tokens with the empty sequence dst."""
        check(lib().rkv_seq_fork(self.h, src, dst, length))

    def page_generation(self, page: int) -> int:
        n = C.c_uint64()
        check(lib().rkv_page_generation(self.h, page, C.byref(n)))
        return n.value

    def page_refs(self, page: int) -> int:
        n = C.c_int32()
        check(lib().rkv_page_refs(self.h, page, C.byref(n)))
        return n.value

    def take_copies(self) -> list[tuple[int, int]]:
        """Queued copy-on-write copies as (src, dst) pairs; clears the queue."""
        buf = (C.c_int32 * (2 * self.num_pages))()
        n = C.c_int32()
        check(lib().rkv_alloc_take_copies(self.h, buf, self.num_pages, C.byref(n)))
        return [(buf[2 * i], buf[2 * i + 1]) for i in range(n.value)]

    def seq_len(self, seq: int) -> int:
        n = C.c_int32()
        check(lib().rkv_seq_len(self.h, seq, C.byref(n)))
        return n.value

    def block_table(self, seq: int) -> list[int]:
        buf = (C.c_int32 * self.max_pages_per_seq)()
        n = C.c_int32()
        check(lib().rkv_block_table_get(self.h, seq, buf, self.max_pages_per_seq, C.byref(n)))
        return list(buf[: n.value])

    def free_pages(self) -> int:
        n = C.c_int32()
        check(lib().rkv_alloc_free_pages(self.h, C.byref(n)))
        return n.value

    def export(self):
        import numpy as np
        tables = np.empty((self.max_seqs, self.max_pages_per_seq), np.int32)
        lens = np.empty(self.max_seqs, np.int32)
        check(lib().rkv_alloc_export(self.h, tables.ctypes.data_as(P), lens.ctypes.data_as(P)))
        return tables, lens

    def close(self) -> None:
        if self.owned and self.h:
            lib().rkv_alloc_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- kernel-level operations (torch tensors on the device) -------------------

def append_q8(ctx: Ctx, g: Geometry, pages, block_tables, seq_ids, positions, k_src, v_src,
              rule: int = Q8_CANONICAL, stream=None) -> None:
    import torch
    bt_stride = block_tables.shape[-1]
    n_seqs = block_tables.shape[0]
    dtype = BF16 if k_src.dtype == torch.bfloat16 else F32
    a = AppendArgs(seq_ids.numel(), _ptr(seq_ids), _ptr(positions), _ptr(k_src), _ptr(v_src),
                   dtype, rule)
    check(lib().rkv_append_q8(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables), bt_stride,
                              n_seqs, C.byref(a), _stream(stream)))


def append_args(seq_ids, positions, k_src, v_src, rule=Q8_CANONICAL) -> AppendArgs:
    """Rows [n][kv_heads][head_dim] (f32 or bf16) for rkv_append_q8 or for the
    `append` of a decode."""
    import torch
    a = AppendArgs(seq_ids.numel(), _ptr(seq_ids), _ptr(positions), _ptr(k_src), _ptr(v_src),
                   BF16 if k_src.dtype == torch.bfloat16 else F32, rule)
    a._refs = (seq_ids, positions, k_src, v_src)
    return a


def decode_args(q, out, seq_ids, scale, max_seq_len, q_len=1, partition_tokens=0,
                workspace=None, append: AppendArgs | None = None, split_event=None) -> DecodeArgs:
    """`append` (optional): rows [batch*q_len] the decode launch appends
    before attending over them.  `split_event` (optional): a hipEvent_t handle
    (int) recorded between the decode and the combine kernel."""
    import torch
    B = seq_ids.numel()
    q_heads = q.shape[-2]
    a = DecodeArgs(B, _ptr(seq_ids), _ptr(q), BF16 if q.dtype == torch.bfloat16 else F32,
                   q_len, q_heads, scale, _ptr(out),
                   BF16 if out.dtype == torch.bfloat16 else F32, partition_tokens,
                   max_seq_len, _ptr(workspace),
                   0 if workspace is None else workspace.numel() * workspace.element_size(),
                   C.pointer(append) if append is not None else None,
                   P(split_event) if split_event else None)
    a._refs = (q, out, seq_ids, workspace, append)  # the struct holds raw pointers
    return a


def prefill_args(seq_ids, ctx_lens, q_rows, q, out, scale, q_offsets=None, segment_tokens=0,
                 workspace=None) -> PrefillArgs:
    """Host entry table (lists of ints) + device q/out [total_rows][q_heads][D].
    q_offsets defaults to the running sum of q_rows.  segment_tokens and the
    device tensor `workspace` control the split of row blocks' causal ranges
    (0 with a workspace: automatic; > 0: that segment length; < 0: never)."""
    import torch
    n = len(seq_ids)
    if q_offsets is None:
        q_offsets, o = [], 0
        for r in q_rows:
            q_offsets.append(o)
            o += int(r)
    arr = [(C.c_int32 * max(n, 1))(*[int(v) for v in x]) for x in (seq_ids, ctx_lens, q_rows, q_offsets)]
    a = PrefillArgs(n, *[C.cast(x, I32P) for x in arr], q.shape[0], _ptr(q),
                    BF16 if q.dtype == torch.bfloat16 else F32, q.shape[1], scale, _ptr(out),
                    BF16 if out.dtype == torch.bfloat16 else F32, int(segment_tokens),
                    _ptr(workspace) if workspace is not None else None,
                    workspace.numel() * workspace.element_size() if workspace is not None else 0)
    a._refs = (q, out, arr, workspace)  # the struct holds raw pointers
    return a


def prefill_workspace_bytes(g: Geometry, a: PrefillArgs) -> int:
    return lib().rkv_prefill_workspace_bytes(C.byref(g), C.byref(a))


def prefill_q8(ctx: Ctx, g: Geometry, pages, block_tables, n_seqs: int, a: PrefillArgs,
               stream=None) -> None:
    check(lib().rkv_prefill_q8(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables),
                               block_tables.shape[1], n_seqs, C.byref(a), _stream(stream)))


def _host_buf(data):
    import numpy as np
    b = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not hasattr(data, "dtype")
                             else data, np.uint8).reshape(-1)
    return b, (b.ctypes.data_as(P) if b.size else None)


def crc32c_host(data) -> int:
    b, ptr = _host_buf(data)
    return int(lib().rkv_crc32c_host(ptr, b.size))


def crc32c(ctx: Ctx, data, n: int, out, stream=None) -> None:
    """CRC32C of n bytes of a device tensor into the int32 device tensor `out`."""
    check(lib().rkv_crc32c(ctx.h, _ptr(data), n, _ptr(out), _stream(stream)))


STREAM_DMA_UNIT = 16384


def stream_read(ctx: Ctx, data, mode: int, blocks: int, out=None, nbytes=None, stream=None) -> None:
    """Read the device tensor `data` once (the streaming-read ceiling):
    mode 0 vector loads, xor of its 32-bit words into the int32 device
    tensor `out`; mode 1 LDS-DMA copies (out unused)."""
    n = data.numel() * data.element_size() if nbytes is None else nbytes
    check(lib().rkv_stream_read(ctx.h, _ptr(data), n, mode, blocks,
                                _ptr(out) if out is not None else None, _stream(stream)))


def stream_read_tiles(ctx: Ctx, g: Geometry, pages, block_tables, bt_stride: int, n_seqs: int,
                      seq_tokens: int, partition_tokens: int, stream=None) -> None:
    """The decode's tile order over a pool's pages, for its read rate
    (rkv_stream_read_tiles); reads and discards."""
    check(lib().rkv_stream_read_tiles(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables), bt_stride,
                                      n_seqs, seq_tokens, partition_tokens, _stream(stream)))


class R4kvRefused(RkvError):
    def __init__(self, status, message, refusal):
        super().__init__(status, message)
        self.refusal = refusal


def _check_refusal(status: int, refusal) -> None:
    if status == ERR_REFUSED:
        raise R4kvRefused(status, lib().rkv_last_error().decode(), refusal.value)
    check(status)


def r4kv_header_encode(h: R4kvHeader) -> bytes:
    import numpy as np
    out = np.zeros(96, np.uint8)
    check(lib().rkv_r4kv_header_encode(C.byref(h), out.ctypes.data_as(P)))
    return out.tobytes()


def r4kv_header_decode(data) -> R4kvHeader:
    b, ptr = _host_buf(data)
    h = R4kvHeader()
    why = C.c_int32()
    _check_refusal(lib().rkv_r4kv_header_decode(ptr, C.byref(h), C.byref(why)), why)
    return h


def r4kv_check_restore(h: R4kvHeader, e: R4kvExpect, payload_body_len: int) -> None:
    why = C.c_int32()
    _check_refusal(lib().rkv_r4kv_check_restore(C.byref(h), C.byref(e), payload_body_len,
                                                C.byref(why)), why)


def r4kv_unpack_host(page):
    """(header, body bytes) of a page held in host memory; raises R4kvRefused."""
    b, ptr = _host_buf(page)
    h = R4kvHeader()
    body = P()
    why = C.c_int32()
    _check_refusal(lib().rkv_r4kv_unpack_host(ptr, b.size, C.byref(h), C.byref(body),
                                              C.byref(why)), why)
    return h, bytes(b[96:96 + h.payload_len])


def decode_workspace_bytes(g: Geometry, a: DecodeArgs) -> int:
    return lib().rkv_decode_workspace_bytes(C.byref(g), C.byref(a))


def decode_partition_tokens(g: Geometry, a: DecodeArgs) -> int:
    return lib().rkv_decode_partition_tokens(C.byref(g), C.byref(a))


def decode_q8(ctx: Ctx, g: Geometry, pages, block_tables, seq_lens, a: DecodeArgs,
              stream=None) -> None:
    check(lib().rkv_decode_q8(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables),
                              block_tables.shape[-1], _ptr(seq_lens), seq_lens.numel(),
                              C.byref(a), _stream(stream)))


DECODE_SCRATCH_BYTES = 64 << 20  # RKV_DECODE_SCRATCH_BYTES


def decode_q8_noalloc(ctx: Ctx, g: Geometry, pages, block_tables, seq_lens, a: DecodeArgs,
                      stream=None) -> None:
    """rkv_decode_q8 with the partials in the library's static device
    scratch: a.workspace is ignored and nothing is allocated."""
    check(lib().rkv_decode_q8_noalloc(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables),
                                      block_tables.shape[-1], _ptr(seq_lens), seq_lens.numel(),
                                      C.byref(a), _stream(stream)))


def decode_q8_partials(ctx: Ctx, g: Geometry, pages, block_tables, seq_lens, a: DecodeArgs,
                       ml, o, stream=None) -> None:
    check(lib().rkv_decode_q8_partials(ctx.h, C.byref(g), _ptr(pages), _ptr(block_tables),
                                       block_tables.shape[-1], _ptr(seq_lens), seq_lens.numel(),
                                       C.byref(a), _ptr(ml), _ptr(o), _stream(stream)))


def splitk_combine(ctx: Ctx, ml, o, batch, rows, n_parts, head_dim, seq_ids, seq_lens,
                   partition_tokens, out, stream=None) -> None:
    import torch
    check(lib().rkv_splitk_combine(ctx.h, _ptr(ml), _ptr(o), batch, rows, n_parts, head_dim,
                                   _ptr(seq_ids), _ptr(seq_lens), seq_lens.numel(),
                                   partition_tokens, _ptr(out),
                                   BF16 if out.dtype == torch.bfloat16 else F32,
                                   _stream(stream)))


def gather_q8(ctx: Ctx, g: Geometry, pages, block_table, length: int, kind: int, out,
              stream=None) -> None:
    check(lib().rkv_gather_q8(ctx.h, C.byref(g), _ptr(pages), _ptr(block_table), length, kind,
                              _ptr(out), _stream(stream)))


def import_q8(ctx: Ctx, g: Geometry, pages, block_table, length: int, kind: int, rows,
              stream=None) -> None:
    check(lib().rkv_import_q8(ctx.h, C.byref(g), _ptr(pages), _ptr(block_table), length, kind,
                              _ptr(rows), _stream(stream)))


def copy_pages(ctx: Ctx, g: Geometry, pages, layer_stride: int, layers: int, pairs,
               n_pairs: int, stream=None) -> None:
    """Page dst := page src per (src, dst) pair of the int32 device tensor `pairs`."""
    check(lib().rkv_copy_pages(ctx.h, C.byref(g), _ptr(pages), layer_stride, layers,
                               _ptr(pairs), n_pairs, _stream(stream)))


def f32_to_f16(ctx: Ctx, x, out, rule: int, stream=None) -> None:
    check(lib().rkv_f32_to_f16(ctx.h, _ptr(x), _ptr(out), x.numel(), rule, _stream(stream)))


def flash_decode_scratch_bytes(p: FlashDecodeParams) -> int:
    return lib().rkv_flash_decode_scratch_bytes(C.byref(p))


def flash_decode_q8(ctx: Ctx, p: FlashDecodeParams, k_words, v_words, query, out, scratch,
                    stream=None) -> None:
    check(lib().rkv_flash_decode_q8(ctx.h, C.byref(p), _ptr(k_words), _ptr(v_words),
                                    _ptr(query), _ptr(out), _ptr(scratch), _stream(stream)))


class Pool:
    """Device pages for `layers` layers + allocator + device block tables."""

    def __init__(self, ctx: Ctx, layers, kv_heads, head_dim, page_tokens, num_pages, max_seqs,
                 max_pages_per_seq, seed=0, page_memory=0):
        self.ctx = ctx
        d = PoolDesc(layers, kv_heads, head_dim, page_tokens, num_pages, max_seqs,
                     max_pages_per_seq, seed, page_memory)
        h = P()
        check(lib().rkv_pool_create(ctx.h, C.byref(d), C.byref(h)))
        self.h = h
        self.desc = d
        self.geometry = Geometry(kv_heads, head_dim, page_tokens, num_pages)
        self.alloc = Allocator(num_pages, page_tokens, max_seqs, max_pages_per_seq,
                               handle=P(lib().rkv_pool_allocator(h)))

    def sync_tables(self, stream=None) -> None:
        check(lib().rkv_pool_sync_tables(self.h, _stream(stream)))

    def release_stream(self, stream) -> None:
        """Let the pool forget `stream` (before the caller destroys it)."""
        check(lib().rkv_pool_release_stream(self.h, _stream(stream)))

    def layer_pages(self, layer: int) -> int:
        return lib().rkv_pool_layer_pages(self.h, layer)

    def block_tables_ptr(self) -> int:
        return lib().rkv_pool_block_tables(self.h)

    def seq_lens_ptr(self) -> int:
        return lib().rkv_pool_seq_lens(self.h)

    def append(self, layer, seq_ids, positions, k_src, v_src, rule=Q8_CANONICAL,
               stream=None) -> None:
        import torch
        dtype = BF16 if k_src.dtype == torch.bfloat16 else F32
        a = AppendArgs(seq_ids.numel(), _ptr(seq_ids), _ptr(positions), _ptr(k_src),
                       _ptr(v_src), dtype, rule)
        check(lib().rkv_pool_append(self.h, layer, C.byref(a), _stream(stream)))

    def decode(self, layer, a: DecodeArgs, stream=None) -> None:
        check(lib().rkv_pool_decode(self.h, layer, C.byref(a), _stream(stream)))

    def prefill(self, layer, a: PrefillArgs, stream=None) -> None:
        check(lib().rkv_pool_prefill(self.h, layer, C.byref(a), _stream(stream)))

    def prefill_workspace_bytes(self, a: PrefillArgs) -> int:
        return lib().rkv_pool_prefill_workspace_bytes(self.h, C.byref(a))

    def r4kv_page_bytes(self, token_count, layer_lo, layer_hi) -> int:
        return lib().rkv_r4kv_page_bytes(self.h, token_count, layer_lo, layer_hi)

    def spill(self, seq, token_start, token_count, layer_lo, layer_hi, identity: R4kvHeader,
              staging, dst, stream=None) -> None:
        """R4KV page of the range into `staging` (device tensor), copied to
        `dst` (a host or device tensor, or staging itself)."""
        check(lib().rkv_pool_spill(self.h, seq, token_start, token_count, layer_lo, layer_hi,
                                   C.byref(identity), _ptr(staging),
                                   staging.numel() * staging.element_size(), _ptr(dst),
                                   dst.numel() * dst.element_size(), _stream(stream)))

    def restore(self, seq, page, expect: R4kvExpect, staging, stream=None) -> None:
        """Restore a page held in host memory (bytes / numpy / CPU tensor);
        raises R4kvRefused with .refusal set when a fail-closed check fails."""
        import numpy as np
        if hasattr(page, "numpy"):
            page = page.numpy()
        b, ptr = _host_buf(page)
        why = C.c_int32()
        st = lib().rkv_pool_restore(self.h, seq, ptr, b.size, C.byref(expect), _ptr(staging),
                                    staging.numel() * staging.element_size(), C.byref(why),
                                    _stream(stream))
        _check_refusal(st, why)

    def gather(self, layer, seq, kind, out, stream=None) -> None:
        check(lib().rkv_pool_gather(self.h, layer, seq, kind, _ptr(out), _stream(stream)))

    def close(self) -> None:
        if self.h:
            self.alloc.h = None
            lib().rkv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _entries(items):
    """ServeEntry array from (id, tokens) or (id, tokens, fork_len, parent) tuples."""
    arr = (ServeEntry * max(len(items), 1))()
    for i, it in enumerate(items):
        sid, tokens, fork_len, parent = (tuple(it) + (0, 0))[:4]
        arr[i] = ServeEntry(sid, tokens, fork_len, parent)
    return arr


class Serve:
    """Serving adapter (rkv_serve_*): one pool for all layers, sequences named
    by the scheduler's SequenceId, per-step prefill chunks and decode rows."""

    def __init__(self, ctx: Ctx, layers, kv_heads, head_dim, page_tokens, num_pages, max_seqs,
                 max_pages_per_seq, q_heads, max_decode, max_prefill_rows, rule=Q8_CANONICAL,
                 seed=0, page_memory=0):
        self.ctx = ctx
        d = ServeDesc(layers, kv_heads, head_dim, page_tokens, num_pages, max_seqs,
                      max_pages_per_seq, q_heads, max_decode, max_prefill_rows, rule, seed,
                      page_memory)
        h = P()
        check(lib().rkv_serve_create(ctx.h, C.byref(d), C.byref(h)))
        self.h = h
        self.desc = d
        # the pool's own geometry: scheduler pages below 16 tokens share
        # 32-token pool pages
        self.geometry = Geometry()
        check(lib().rkv_serve_geometry(h, C.byref(self.geometry)))
        self.pool_h = P(lib().rkv_serve_pool(h))
        per = self.geometry.page_tokens // page_tokens
        self.alloc = Allocator(self.geometry.num_pages, self.geometry.page_tokens, max_seqs,
                               (max_pages_per_seq + per - 1) // per,
                               handle=P(lib().rkv_pool_allocator(self.pool_h)))

    def begin_step(self, prefill=(), decode=(), stream=None) -> None:
        """prefill / decode: (id, tokens[, fork_len, parent]) per sequence."""
        pe, de = _entries(list(prefill)), _entries(list(decode))
        check(lib().rkv_serve_begin_step(self.h, pe, len(prefill), de, len(decode),
                                         _stream(stream)))

    def decode(self, layer, q, k, v, out, scale, stream=None) -> None:
        import torch
        check(lib().rkv_serve_decode(self.h, layer, _ptr(q), _ptr(k), _ptr(v),
                                     BF16 if q.dtype == torch.bfloat16 else F32, _ptr(out),
                                     BF16 if out.dtype == torch.bfloat16 else F32, scale,
                                     _stream(stream)))

    def prefill(self, layer, q, k, v, out, scale, stream=None) -> None:
        import torch
        check(lib().rkv_serve_prefill(self.h, layer, _ptr(q), _ptr(k), _ptr(v),
                                      BF16 if q.dtype == torch.bfloat16 else F32, _ptr(out),
                                      BF16 if out.dtype == torch.bfloat16 else F32, scale,
                                      _stream(stream)))

    def truncate(self, sid: int, length: int) -> None:
        check(lib().rkv_serve_truncate(self.h, sid, length))

    def finish(self, sid: int) -> None:
        check(lib().rkv_serve_finish(self.h, sid))

    def seq_len(self, sid: int) -> int:
        n = C.c_int32()
        check(lib().rkv_serve_seq_len(self.h, sid, C.byref(n)))
        return n.value

    def slot(self, sid: int) -> int:
        """The pool sequence of a live id (for pool-level calls on it)."""
        n = C.c_int32()
        check(lib().rkv_serve_seq_slot(self.h, sid, C.byref(n)))
        return n.value

    def pool_append(self, layer, slots, positions, k, v, stream=None) -> None:
        """rkv_pool_append on the adapter's pool: rows of pool sequences `slots`."""
        import torch
        a = AppendArgs(slots.numel(), _ptr(slots), _ptr(positions), _ptr(k), _ptr(v),
                       BF16 if k.dtype == torch.bfloat16 else F32, Q8_CANONICAL)
        check(lib().rkv_pool_append(self.pool_h, layer, C.byref(a), _stream(stream)))

    def sync_tables(self, stream=None) -> None:
        check(lib().rkv_pool_sync_tables(self.pool_h, _stream(stream)))

    def release_stream(self, stream) -> None:
        """Let the adapter's pool forget `stream` (before the caller destroys it)."""
        check(lib().rkv_pool_release_stream(self.pool_h, _stream(stream)))

    def page_location(self, sid: int, ordinal: int) -> PageLocation:
        loc = PageLocation()
        check(lib().rkv_serve_page_location(self.h, sid, ordinal, C.byref(loc)))
        return loc

    def layer_pages(self, layer: int) -> int:
        return lib().rkv_pool_layer_pages(self.pool_h, layer)

    def gather(self, layer, sid_slot, kind, out, stream=None) -> None:
        check(lib().rkv_pool_gather(self.pool_h, layer, sid_slot, kind, _ptr(out),
                                    _stream(stream)))

    def close(self) -> None:
        if self.h:
            self.alloc.h = None
            lib().rkv_serve_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
