// rkv_runtime.cpp -- host side of the C ABI in include/rkv.h: errors,
// device context, page allocator + block tables, pool, argument checking
// and kernel dispatch.  No entry point computes on the CPU: every data
// operation is a HIP kernel, and a missing device is an error.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "../../include/rkv.h"
#include "rkv_crc32c.h"
#include "rkv_host.h"
#include "rkv_launch.h"

using rkv::Geo;
using rkv::host::fail;
using rkv::host::hip_fail;
using rkv::host::use_device;

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace rkv {
namespace host {

// Mirrors HarError{operation, message} (har-vulkan/src/lib.rs:19-56): the
// status says what kind of failure, the message says where and why.
rkv_status fail(rkv_status code, const char *op, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = std::string(op) + ": " + buf;
  return code;
}

rkv_status hip_fail(const char *op, hipError_t e) {
  return fail(RKV_ERR_DEVICE, op, "%s (%s)", hipGetErrorString(e), hipGetErrorName(e));
}

}  // namespace host
}  // namespace rkv

namespace {

uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

bool pow2(int32_t v) { return v > 0 && (v & (v - 1)) == 0; }

rkv_status check_geometry(const rkv_kv_geometry *g, const char *op) {
  if (!g) return fail(RKV_ERR_INVALID_ARG, op, "geometry is NULL");
  if (g->kv_heads < 1 || g->kv_heads > 64)
    return fail(RKV_ERR_INVALID_ARG, op, "kv_heads=%d outside [1, 64]", g->kv_heads);
  if (g->head_dim != 128 && g->head_dim != 256)
    return fail(RKV_ERR_UNSUPPORTED, op, "head_dim=%d (built: 128, 256)", g->head_dim);
  if (!pow2(g->page_tokens) || g->page_tokens < 16 || g->page_tokens > 256)
    return fail(RKV_ERR_UNSUPPORTED, op, "page_tokens=%d (built: 16, 32, 64, 128, 256)",
                g->page_tokens);
  if (g->num_pages < 1) return fail(RKV_ERR_INVALID_ARG, op, "num_pages=%d", g->num_pages);
  return RKV_OK;
}

Geo to_geo(const rkv_kv_geometry *g) {
  return Geo{g->kv_heads, g->head_dim, g->page_tokens, g->num_pages};
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

}  // namespace

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
struct rkv_ctx {
  int32_t device = 0;
  int32_t *d_fault = nullptr;  // device fault word (rkv::FAULT_* bits)
  void *scratch = nullptr;     // this device's static decode scratch (rkv_scratch.hip)
};

namespace rkv {
namespace host {
rkv_status use_device(rkv_ctx *ctx, const char *op) {
  if (!ctx) return fail(RKV_ERR_INVALID_ARG, op, "ctx is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(op, e);
  return RKV_OK;
}
}  // namespace host
}  // namespace rkv

extern "C" {

const char *rkv_last_error(void) { return g_last_error.c_str(); }
const char *rkv_version(void) { return "rkv 0.1 (gfx950)"; }

rkv_status rkv_ctx_create(int32_t device, rkv_ctx **out) {
  const char *op = "rkv_ctx_create";
  if (!out) return fail(RKV_ERR_INVALID_ARG, op, "out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(RKV_ERR_DEVICE, op, "no HIP device (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(RKV_ERR_INVALID_ARG, op, "device %d of %d", device, n);
  if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(op, e);
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return hip_fail(op, e);
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(RKV_ERR_UNSUPPORTED, op, "device %d is %s; kernels are built for gfx950", device,
                prop.gcnArchName);
  // The decode's partition plan, the prefill's dispatch simulation and the
  // workspace sizes that follow from them are sized for the whole chip (256
  // CUs in 8 XCDs) whatever the device reports: a part with fewer CUs (a
  // partition mode) runs the same launches in more rounds, correct and
  // slower.  The workspace queries take no context, so the plans cannot
  // follow the device.
  // the static decode scratch of rkv_decode_q8_noalloc, resolved once per
  // device with the device current
  void *scratch = nullptr;
  if ((e = rkv::scratch_address(device, &scratch)) != hipSuccess) return hip_fail(op, e);
  rkv_ctx *c = new rkv_ctx;
  c->device = device;
  c->scratch = scratch;
  if ((e = hipMalloc(&c->d_fault, sizeof(int32_t))) != hipSuccess) {
    delete c;
    return hip_fail(op, e);
  }
  if ((e = hipMemset(c->d_fault, 0, sizeof(int32_t))) != hipSuccess) {
    (void)hipFree(c->d_fault);
    delete c;
    return hip_fail(op, e);
  }
  *out = c;
  return RKV_OK;
}

rkv_status rkv_ctx_destroy(rkv_ctx *ctx) {
  if (!ctx) return RKV_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipFree(ctx->d_fault);
  delete ctx;
  return RKV_OK;
}

rkv_status rkv_ctx_sync(rkv_ctx *ctx, void *stream) {
  const char *op = "rkv_ctx_sync";
  if (rkv_status s = use_device(ctx, op)) return s;
  hipError_t e = hipStreamSynchronize(as_stream(stream));
  if (e != hipSuccess) return hip_fail(op, e);
  int32_t fault = 0;
  if ((e = hipMemcpy(&fault, ctx->d_fault, sizeof fault, hipMemcpyDeviceToHost)) != hipSuccess)
    return hip_fail(op, e);
  if (fault) {
    if ((e = hipMemset(ctx->d_fault, 0, sizeof(int32_t))) != hipSuccess) return hip_fail(op, e);
    return fail(RKV_ERR_BAD_BLOCK_TABLE, op,
                "device reported fault bits 0x%x (1: page id outside the pool, 2: position "
                "beyond the block-table row, 4: sequence id outside the table)",
                fault);
  }
  return RKV_OK;
}

// ---------------------------------------------------------------------------
// geometry
// ---------------------------------------------------------------------------
rkv_status rkv_geometry_check(const rkv_kv_geometry *g) {
  return check_geometry(g, "rkv_geometry_check");
}
size_t rkv_page_bytes(const rkv_kv_geometry *g) {
  if (!g || check_geometry(g, "rkv_page_bytes") != RKV_OK) return 0;
  return (size_t)rkv::page_bytes(to_geo(g));
}
size_t rkv_row_bytes(int32_t head_dim) {
  return head_dim > 0 && head_dim % 32 == 0 ? (size_t)head_dim / 32 * 34 : 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// page allocator
// ---------------------------------------------------------------------------
struct rkv_alloc {
  rkv_alloc_desc d{};
  std::vector<int32_t> free_list;  // top of the stack = back
  std::vector<int32_t> tables;     // [max_seqs][max_pages_per_seq], -1 = none
  std::vector<int32_t> lens;       // [max_seqs]
  std::vector<int32_t> held;       // pages held per sequence
  std::vector<uint8_t> dirty;      // table row changed since the last upload (lengths always go)
  std::vector<int32_t> refs;       // [num_pages] block-table entries naming the page, 0 = free
  std::vector<uint64_t> gen;       // [num_pages] times the page left the free list
  // Copy-on-write copies queued since the last take, as (src, dst) pairs;
  // copy_src[dst] = src while the pair is queued (else -1) and copy_reads[p]
  // counts queued pairs that read p.  A page a queued pair reads is never
  // chosen as a copy destination, so queued copies are independent of each
  // other and run in any order.
  std::vector<int32_t> copies;
  std::vector<int32_t> copy_src;
  std::vector<int32_t> copy_reads;
};

namespace {
rkv_status check_seq(const rkv_alloc *a, int32_t seq, const char *op) {
  if (!a) return fail(RKV_ERR_INVALID_ARG, op, "allocator is NULL");
  if (seq < 0 || seq >= a->d.max_seqs)
    return fail(RKV_ERR_INVALID_ARG, op, "seq %d outside [0, %d)", seq, a->d.max_seqs);
  return RKV_OK;
}
int32_t pages_for(const rkv_alloc *a, int64_t len) {
  return (int32_t)((len + a->d.page_tokens - 1) / a->d.page_tokens);
}
// Drop one block-table reference to `page`; the last one returns it to the
// free list and cancels a queued copy into it (nothing reads it any more).
void release_page(rkv_alloc *a, int32_t page) {
  if (--a->refs[page] > 0) return;
  a->free_list.push_back(page);
  if (a->copy_src[page] < 0) return;
  --a->copy_reads[a->copy_src[page]];
  a->copy_src[page] = -1;
  for (size_t i = 0; i < a->copies.size(); i += 2) {
    if (a->copies[i + 1] == page) {
      a->copies.erase(a->copies.begin() + (std::ptrdiff_t)i, a->copies.begin() + (std::ptrdiff_t)i + 2);
      break;
    }
  }
}
// Index in the free list of the topmost page no queued copy reads, or -1.
int32_t copy_target_index(const rkv_alloc *a) {
  for (int32_t i = (int32_t)a->free_list.size() - 1; i >= 0; --i)
    if (a->copy_reads[a->free_list[i]] == 0) return i;
  return -1;
}
int32_t take_page(rkv_alloc *a) {
  const int32_t page = a->free_list.back();
  a->free_list.pop_back();
  a->refs[page] = 1;
  ++a->gen[page];
  return page;
}
}  // namespace

extern "C" {

rkv_status rkv_alloc_create(const rkv_alloc_desc *desc, rkv_alloc **out) {
  const char *op = "rkv_alloc_create";
  if (!desc || !out) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  *out = nullptr;
  if (desc->num_pages < 1 || desc->max_seqs < 1 || desc->max_pages_per_seq < 1)
    return fail(RKV_ERR_INVALID_ARG, op, "num_pages=%d max_seqs=%d max_pages_per_seq=%d",
                desc->num_pages, desc->max_seqs, desc->max_pages_per_seq);
  if (!pow2(desc->page_tokens) || desc->page_tokens < 16 || desc->page_tokens > 256)
    return fail(RKV_ERR_UNSUPPORTED, op, "page_tokens=%d", desc->page_tokens);
  if ((int64_t)desc->max_seqs * desc->max_pages_per_seq > (int64_t)1 << 31)
    return fail(RKV_ERR_INVALID_ARG, op, "block table too large");
  rkv_alloc *a = new rkv_alloc;
  a->d = *desc;
  // Seeded Fisher-Yates permutation of [0, num_pages): pages are handed out
  // from the back, so the first sequence gets a shuffled page run.
  a->free_list.resize(desc->num_pages);
  for (int32_t i = 0; i < desc->num_pages; ++i) a->free_list[i] = i;
  uint64_t st = desc->free_list_seed;
  for (int32_t i = desc->num_pages - 1; i > 0; --i) {
    st = splitmix64(st);
    int32_t j = (int32_t)(st % (uint64_t)(i + 1));
    std::swap(a->free_list[i], a->free_list[j]);
  }
  a->tables.assign((size_t)desc->max_seqs * desc->max_pages_per_seq, -1);
  a->lens.assign(desc->max_seqs, 0);
  a->held.assign(desc->max_seqs, 0);
  a->dirty.assign(desc->max_seqs, 1);
  a->refs.assign(desc->num_pages, 0);
  a->gen.assign(desc->num_pages, 0);
  a->copy_src.assign(desc->num_pages, -1);
  a->copy_reads.assign(desc->num_pages, 0);
  *out = a;
  return RKV_OK;
}

rkv_status rkv_alloc_destroy(rkv_alloc *a) {
  delete a;
  return RKV_OK;
}

rkv_status rkv_seq_reserve(rkv_alloc *a, int32_t seq, int32_t new_len) {
  const char *op = "rkv_seq_reserve";
  if (rkv_status s = check_seq(a, seq, op)) return s;
  if (new_len < a->lens[seq])
    return fail(RKV_ERR_INVALID_ARG, op, "seq %d: new_len %d < length %d (use rkv_seq_truncate)",
                seq, new_len, a->lens[seq]);
  const int32_t need = pages_for(a, new_len);
  if (need > a->d.max_pages_per_seq)
    return fail(RKV_ERR_CAPACITY, op, "seq %d: %d tokens need %d pages > max_pages_per_seq %d",
                seq, new_len, need, a->d.max_pages_per_seq);
  int32_t *row = &a->tables[(size_t)seq * a->d.max_pages_per_seq];
  const int32_t len = a->lens[seq];
  // Growing into a partly filled last page that other tables also name:
  // this sequence gets a private copy of it first (copy-on-write).
  const int32_t last = len / a->d.page_tokens;
  const bool cow = new_len > len && len % a->d.page_tokens != 0 && a->refs[row[last]] > 1;
  const int32_t extra = need - a->held[seq] + (cow ? 1 : 0);
  if (extra > (int32_t)a->free_list.size())
    return fail(RKV_ERR_OUT_OF_PAGES, op, "seq %d needs %d more pages, %zu free", seq, extra,
                a->free_list.size());
  if (cow) {
    const int32_t at = copy_target_index(a);
    if (at < 0)
      return fail(RKV_ERR_OUT_OF_PAGES, op,
                  "seq %d: every free page is still read by a queued copy; sync first", seq);
    std::swap(a->free_list[at], a->free_list.back());
    const int32_t shared = row[last];
    // A queued copy into `shared` has not run yet and no device write can
    // reach `shared` before it does, so the new copy reads the same source.
    const int32_t src = a->copy_src[shared] >= 0 ? a->copy_src[shared] : shared;
    const int32_t page = take_page(a);
    --a->refs[shared];
    row[last] = page;
    a->copies.push_back(src);
    a->copies.push_back(page);
    a->copy_src[page] = src;
    ++a->copy_reads[src];
    a->dirty[seq] = 1;
  }
  for (int32_t i = a->held[seq]; i < need; ++i) row[i] = take_page(a);
  if (need > a->held[seq]) a->dirty[seq] = 1;
  a->held[seq] = std::max(a->held[seq], need);
  a->lens[seq] = new_len;
  return RKV_OK;
}

rkv_status rkv_seq_truncate(rkv_alloc *a, int32_t seq, int32_t new_len) {
  const char *op = "rkv_seq_truncate";
  if (rkv_status s = check_seq(a, seq, op)) return s;
  if (new_len < 0 || new_len > a->lens[seq])
    return fail(RKV_ERR_INVALID_ARG, op, "seq %d: new_len %d outside [0, %d]", seq, new_len,
                a->lens[seq]);
  const int32_t keep = pages_for(a, new_len);
  int32_t *row = &a->tables[(size_t)seq * a->d.max_pages_per_seq];
  // return pages last-first so a re-grow gets the same pages back
  for (int32_t i = a->held[seq] - 1; i >= keep; --i) {
    release_page(a, row[i]);
    row[i] = -1;
  }
  if (keep < a->held[seq]) a->dirty[seq] = 1;
  a->held[seq] = std::min(a->held[seq], keep);
  a->lens[seq] = new_len;
  return RKV_OK;
}

rkv_status rkv_seq_free(rkv_alloc *a, int32_t seq) { return rkv_seq_truncate(a, seq, 0); }

// The _n forms: each pair through the single form, in order, stopping at
// the first failure (whose message names the pair).
static rkv_status seq_apply_n(rkv_alloc *a, int32_t n, const int32_t *seqs, const int32_t *new_lens,
                              int32_t *done, const char *op,
                              rkv_status (*one)(rkv_alloc *, int32_t, int32_t)) {
  if (done) *done = 0;
  if (!a) return fail(RKV_ERR_INVALID_ARG, op, "allocator is NULL");
  if (n < 0) return fail(RKV_ERR_INVALID_ARG, op, "n=%d", n);
  if (n > 0 && (!seqs || !new_lens)) return fail(RKV_ERR_INVALID_ARG, op, "seqs or new_lens is NULL");
  for (int32_t i = 0; i < n; ++i) {
    if (rkv_status st = one(a, seqs[i], new_lens[i])) {
      const std::string inner = g_last_error;
      return fail(st, op, "pair %d (seq %d, new_len %d): %s", i, seqs[i], new_lens[i], inner.c_str());
    }
    if (done) *done = i + 1;
  }
  return RKV_OK;
}

rkv_status rkv_seq_reserve_n(rkv_alloc *a, int32_t n, const int32_t *seqs, const int32_t *new_lens,
                             int32_t *done) {
  return seq_apply_n(a, n, seqs, new_lens, done, "rkv_seq_reserve_n", rkv_seq_reserve);
}

rkv_status rkv_seq_truncate_n(rkv_alloc *a, int32_t n, const int32_t *seqs, const int32_t *new_lens,
                              int32_t *done) {
  return seq_apply_n(a, n, seqs, new_lens, done, "rkv_seq_truncate_n", rkv_seq_truncate);
}

rkv_status rkv_seq_fork(rkv_alloc *a, int32_t src, int32_t dst, int32_t len) {
  const char *op = "rkv_seq_fork";
  if (rkv_status s = check_seq(a, src, op)) return s;
  if (rkv_status s = check_seq(a, dst, op)) return s;
  if (src == dst) return fail(RKV_ERR_INVALID_ARG, op, "src and dst are both seq %d", src);
  if (a->held[dst] != 0 || a->lens[dst] != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "dst seq %d is not empty (length %d)", dst, a->lens[dst]);
  if (len < 0 || len > a->lens[src])
    return fail(RKV_ERR_INVALID_ARG, op, "len %d outside [0, %d] of seq %d", len, a->lens[src],
                src);
  const int32_t n = pages_for(a, len);
  const int32_t *from = &a->tables[(size_t)src * a->d.max_pages_per_seq];
  int32_t *to = &a->tables[(size_t)dst * a->d.max_pages_per_seq];
  for (int32_t i = 0; i < n; ++i) {
    to[i] = from[i];
    ++a->refs[from[i]];
  }
  a->held[dst] = n;
  a->lens[dst] = len;
  a->dirty[dst] = 1;
  return RKV_OK;
}

rkv_status rkv_page_refs(const rkv_alloc *a, int32_t page, int32_t *refs) {
  const char *op = "rkv_page_refs";
  if (!a || !refs) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  if (page < 0 || page >= a->d.num_pages)
    return fail(RKV_ERR_INVALID_ARG, op, "page %d outside [0, %d)", page, a->d.num_pages);
  *refs = a->refs[page];
  return RKV_OK;
}

rkv_status rkv_page_generation(const rkv_alloc *a, int32_t page, uint64_t *gen) {
  const char *op = "rkv_page_generation";
  if (!a || !gen) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  if (page < 0 || page >= a->d.num_pages)
    return fail(RKV_ERR_INVALID_ARG, op, "page %d outside [0, %d)", page, a->d.num_pages);
  *gen = a->gen[page];
  return RKV_OK;
}

rkv_status rkv_alloc_take_copies(rkv_alloc *a, int32_t *pairs, int32_t cap, int32_t *n) {
  const char *op = "rkv_alloc_take_copies";
  if (!a || !n) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  const int32_t count = (int32_t)(a->copies.size() / 2);
  *n = count;
  if (count == 0) return RKV_OK;
  if (!pairs || cap < count)
    return fail(RKV_ERR_INVALID_ARG, op, "cap %d < %d queued copies", cap, count);
  std::memcpy(pairs, a->copies.data(), sizeof(int32_t) * a->copies.size());
  for (int32_t i = 0; i < count; ++i) {
    a->copy_src[a->copies[2 * i + 1]] = -1;
    a->copy_reads[a->copies[2 * i]] = 0;
  }
  a->copies.clear();
  return RKV_OK;
}

rkv_status rkv_seq_len(const rkv_alloc *a, int32_t seq, int32_t *len) {
  const char *op = "rkv_seq_len";
  if (rkv_status s = check_seq(a, seq, op)) return s;
  if (!len) return fail(RKV_ERR_INVALID_ARG, op, "len is NULL");
  *len = a->lens[seq];
  return RKV_OK;
}

rkv_status rkv_block_table_get(const rkv_alloc *a, int32_t seq, int32_t *out, int32_t cap,
                               int32_t *n) {
  const char *op = "rkv_block_table_get";
  if (rkv_status s = check_seq(a, seq, op)) return s;
  if (!n) return fail(RKV_ERR_INVALID_ARG, op, "n is NULL");
  *n = a->held[seq];
  if (cap < a->held[seq])
    return fail(RKV_ERR_INVALID_ARG, op, "cap %d < %d pages", cap, a->held[seq]);
  if (a->held[seq] > 0 && !out) return fail(RKV_ERR_INVALID_ARG, op, "out is NULL");
  std::memcpy(out, &a->tables[(size_t)seq * a->d.max_pages_per_seq],
              sizeof(int32_t) * (size_t)a->held[seq]);
  return RKV_OK;
}

rkv_status rkv_alloc_free_pages(const rkv_alloc *a, int32_t *n) {
  if (!a || !n) return fail(RKV_ERR_INVALID_ARG, "rkv_alloc_free_pages", "NULL argument");
  *n = (int32_t)a->free_list.size();
  return RKV_OK;
}

rkv_status rkv_alloc_export(const rkv_alloc *a, int32_t *tables, int32_t *lens) {
  if (!a || !tables || !lens) return fail(RKV_ERR_INVALID_ARG, "rkv_alloc_export", "NULL argument");
  std::memcpy(tables, a->tables.data(), sizeof(int32_t) * a->tables.size());
  std::memcpy(lens, a->lens.data(), sizeof(int32_t) * a->lens.size());
  return RKV_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// kernel-level operations
// ---------------------------------------------------------------------------
namespace {

int32_t decode_stages();

rkv_status check_decode(const rkv_kv_geometry *g, const rkv_decode_args *a, const char *op) {
  if (rkv_status s = check_geometry(g, op)) return s;
  if (!a) return fail(RKV_ERR_INVALID_ARG, op, "args is NULL");
  if (a->batch < 0) return fail(RKV_ERR_INVALID_ARG, op, "batch=%d", a->batch);
  if (a->q_heads < 1 || a->q_heads % g->kv_heads != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "q_heads=%d is not a multiple of kv_heads=%d",
                a->q_heads, g->kv_heads);
  if (a->q_len < 1 || a->q_len > 4) return fail(RKV_ERR_UNSUPPORTED, op, "q_len=%d (1..4)", a->q_len);
  const int32_t R = a->q_len * (a->q_heads / g->kv_heads);
  if (R > 32)
    return fail(RKV_ERR_UNSUPPORTED, op, "q_len*q_heads/kv_heads=%d rows per kv head (<= 32)", R);
  if (a->q_dtype != RKV_F32 && a->q_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "q_dtype=%d", a->q_dtype);
  if (a->out_dtype != RKV_F32 && a->out_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "out_dtype=%d", a->out_dtype);
  if (!(std::isfinite(a->scale))) return fail(RKV_ERR_INVALID_ARG, op, "scale is not finite");
  // partitions start on page (and 32-token tile) boundaries and span at most
  // 64 pages: the kernel keeps one page id per lane
  const int32_t unit = std::max<int32_t>(32, g->page_tokens);
  if (a->partition_tokens < 0 || a->partition_tokens % unit != 0 ||
      a->partition_tokens > 64 * g->page_tokens)
    return fail(RKV_ERR_INVALID_ARG, op,
                "partition_tokens=%d must be a multiple of %d and <= 64*page_tokens (%d)",
                a->partition_tokens, unit, 64 * g->page_tokens);
  if (a->max_seq_len < 0) return fail(RKV_ERR_INVALID_ARG, op, "max_seq_len=%d", a->max_seq_len);
  if (a->batch > 0 && (!a->seq_ids || !a->q || !a->out))
    return fail(RKV_ERR_INVALID_ARG, op, "NULL seq_ids/q/out");
  if (a->batch > 65535) return fail(RKV_ERR_INVALID_ARG, op, "batch=%d > 65535", a->batch);
  if (const rkv_append_args *ap = a->append) {
    if (ap->n_rows != a->batch * a->q_len)
      return fail(RKV_ERR_INVALID_ARG, op, "append n_rows=%d != batch*q_len=%d", ap->n_rows,
                  a->batch * a->q_len);
    if (ap->src_dtype != RKV_F32 && ap->src_dtype != RKV_BF16)
      return fail(RKV_ERR_UNSUPPORTED, op, "append src_dtype=%d", ap->src_dtype);
    if (ap->rule != RKV_Q8_CANONICAL && ap->rule != RKV_Q8_HARSERVE)
      return fail(RKV_ERR_INVALID_ARG, op, "append rule=%d", ap->rule);
    if (ap->n_rows > 0 && (!ap->seq_ids || !ap->positions || !ap->k_src || !ap->v_src))
      return fail(RKV_ERR_INVALID_ARG, op, "NULL append seq_ids/positions/k_src/v_src");
  }
  return RKV_OK;
}

// LDS ring depth of the decode kernel.  2 stages (one tile in flight per
// workgroup, four workgroups per CU) is the default: measured at the
// headline shape it beats 3 stages (two tiles in flight, but only three
// workgroups per CU, so one SIMD idles).  RKV_DECODE_STAGES=3 selects the
// deeper ring for measurement.
int32_t decode_stages() {
  static const int32_t v = [] {
    const char *e = std::getenv("RKV_DECODE_STAGES");
    return (e && std::atoi(e) == 3) ? 3 : 2;
  }();
  return v;
}

// Partition plan of a decode launch (rkv::DecodeLaunch fields).  Explicit
// partition_tokens fix the length; 0 leaves it to the kernel, which picks the
// smallest whole number of 32-token tiles, at least 256 tokens and at most
// 64 pages, whose partition count over the batch's actual lengths fills one
// round of resident workgroups (target = resident slots / kv_heads).  Tile
// granularity (not page) keeps the longest partition short: config 2's
// ragged batch gets 11-tile partitions where whole 64-token pages gave 12.
struct Plan {
  int32_t pt = 0;  // explicit length, 0 = chosen on the device
  int32_t unit = 0, kmin = 0, kmax = 0, target = 0;
  int32_t max_len = 0;
  int32_t n_wg = 0;     // grid.x: upper bound of the batch's partition count
  int32_t n_parts = 0;  // explicit: ceil(max_len / pt)
  bool direct = false;  // one partition covers every sequence: no partials
  int32_t stages = 2;   // LDS ring depth of the launch
};

Plan plan_of(const rkv_kv_geometry *g, const rkv_decode_args *a, int32_t stages) {
  Plan pl;
  pl.stages = stages;
  pl.unit = 32;
  pl.kmin = 256 / pl.unit;
  pl.kmax = 64 * g->page_tokens / pl.unit;
  pl.max_len = std::max<int32_t>(a->max_seq_len, 1);
  const int32_t rows = a->q_len * (a->q_heads / std::max(g->kv_heads, 1));
  const int64_t slots = (int64_t)rkv::kComputeUnits *
                        rkv::decode_wgs_per_cu(g->head_dim, rows, stages);
  pl.target = (int32_t)std::max<int64_t>(1, slots / g->kv_heads);
  const int64_t B = std::max<int32_t>(a->batch, 0);
  if (a->partition_tokens > 0) {
    pl.pt = a->partition_tokens;
    pl.n_parts = (pl.max_len + pl.pt - 1) / pl.pt;
    pl.n_wg = (int32_t)std::min<int64_t>(B * pl.n_parts, INT32_MAX);
    pl.direct = pl.n_parts == 1;
  } else {
    const int64_t pmax = (int64_t)pl.kmax * pl.unit;
    pl.n_wg = (int32_t)std::min<int64_t>(
        std::max<int64_t>(pl.target, B * ((pl.max_len + pmax - 1) / pmax)), INT32_MAX);
    pl.direct = pl.max_len <= pl.kmin * pl.unit;
  }
  return pl;
}

int32_t batch_rows_per_kv(const rkv_kv_geometry *g, const rkv_decode_args *a) {
  return a->q_len * (a->q_heads / g->kv_heads);
}

// Flat workspace of rkv_decode_q8, each part 256-byte aligned:
//   header   int32 [1 + 2*batch]: partition length; first partition and
//            partition count of every entry (written by the decode)
//   partials f32 (m, l) then o of every (kv head, partition, row)
// Everything is written before it is read in the same call, so the
// workspace needs no initialisation.  Every part grows with batch and
// max_seq_len: a workspace sized for the largest call of a serving loop
// holds every smaller one.
size_t align256(size_t n) { return (n + 255) / 256 * 256; }
struct WsLayout {
  size_t hdr = 0, ml = 0, o = 0, total = 0;
  int32_t combine_slices = 1;
};
WsLayout ws_layout(const rkv_kv_geometry *g, const rkv_decode_args *a, const Plan &pl) {
  WsLayout w;
  const size_t B = (size_t)std::max<int32_t>(a->batch, 0);
  const size_t out_rows = B * a->q_len * a->q_heads;
  const size_t prows = (size_t)g->kv_heads * pl.n_wg * batch_rows_per_kv(g, a);
  // partitions of one entry: ceil(max_len / shortest partition), and with a
  // device-chosen length no more than the target minus one per other entry
  // (or the count at the longest length, where the search stops)
  const int64_t shortest = pl.pt > 0 ? pl.pt : (int64_t)pl.kmin * pl.unit;
  int64_t n_entry = (pl.max_len + shortest - 1) / shortest;
  if (pl.pt == 0) {
    const int64_t longest = (int64_t)pl.kmax * pl.unit;
    const int64_t by_target = (int64_t)pl.target - std::max<int64_t>((int64_t)B - 1, 0);
    n_entry = std::min(n_entry, std::max(by_target, (pl.max_len + longest - 1) / longest));
  }
  n_entry = std::min<int64_t>(n_entry, pl.n_wg);
  // Combine blocks: (row, entry) times a power-of-two count of dimension
  // slices, enough for about 512 blocks when partition lists are long (at
  // most 16 partitions and 256 rows take one slice: one thread per dim).
  if (n_entry > 16 || out_rows < 256)
    while (out_rows * w.combine_slices < 512 && g->head_dim / w.combine_slices > 16)
      w.combine_slices *= 2;
  w.ml = align256(sizeof(int32_t) * (1 + 2 * B));
  w.o = w.ml + align256(sizeof(float) * 2 * prows);
  w.total = w.o + sizeof(float) * prows * g->head_dim;
  return w;
}
size_t ws_bytes(const rkv_kv_geometry *g, const rkv_decode_args *a, const Plan &pl) {
  return pl.direct ? 0 : ws_layout(g, a, pl).total;
}

rkv::DecodeLaunch make_decode(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                              const int32_t *bt, int32_t bt_stride, const int32_t *seq_lens,
                              int32_t n_seqs, const rkv_decode_args *a, const Plan &pl) {
  rkv::DecodeLaunch d{};
  d.g = to_geo(g);
  d.pages = static_cast<const uint8_t *>(pages);
  d.bt = bt;
  d.bt_stride = bt_stride;
  d.seq_lens = seq_lens;
  d.n_seqs = n_seqs;
  d.seq_ids = a->seq_ids;
  d.batch = a->batch;
  d.q = a->q;
  d.q_bf16 = a->q_dtype == RKV_BF16;
  d.q_len = a->q_len;
  d.q_heads = a->q_heads;
  d.scale_log2 = a->scale * 1.4426950408889634f;
  d.part_tokens = pl.pt;
  d.pt_unit = pl.unit;
  d.pt_kmin = pl.kmin;
  d.pt_kmax = pl.kmax;
  d.target_parts = pl.target;
  d.max_len = pl.max_len;
  d.n_wg = pl.n_wg;
  d.n_parts = pl.n_parts;
  d.out = a->out;
  d.out_bf16 = a->out_dtype == RKV_BF16;
  d.fault = ctx->d_fault;
  d.stages = pl.stages;
  if (const rkv_append_args *ap = a->append; ap && ap->n_rows > 0) {
    d.pages_w = static_cast<uint8_t *>(const_cast<void *>(pages));
    d.app_seq_ids = ap->seq_ids;
    d.app_pos = ap->positions;
    d.app_k = ap->k_src;
    d.app_v = ap->v_src;
    d.app_bf16 = ap->src_dtype == RKV_BF16;
    d.app_rule = ap->rule;
  }
  return d;
}

rkv_status check_tables(const void *pages, const int32_t *bt, int32_t bt_stride,
                        int32_t n_seqs, const char *op) {
  if (!pages || !bt) return fail(RKV_ERR_INVALID_ARG, op, "NULL pages/block_tables");
  if (bt_stride < 1 || n_seqs < 1)
    return fail(RKV_ERR_INVALID_ARG, op, "bt_stride=%d n_seqs=%d", bt_stride, n_seqs);
  return RKV_OK;
}

// Split-K plan of a prefill launch: segment length in tokens (0: no split)
// and the partial rows it writes, rows * q_heads * nseg summed over the
// entries with more than one segment.  An entry's segment count follows its
// longest row block (the last), ctx + rows tokens.
struct SegPlan {
  int32_t seg = 0;
  int64_t partial_rows = 0;
};

constexpr int32_t kPrefillMinSegment = 1024;  // tokens: 32 tiles a unit at least

int32_t segments_of(int64_t range, int32_t seg) {
  return seg > 0 && range > seg ? (int32_t)((range + seg - 1) / seg) : 1;
}

size_t prefill_ws_bytes(int64_t partial_rows, int32_t head_dim) {
  if (partial_rows <= 0) return 0;
  const size_t ml = ((size_t)partial_rows * 8 + 255) / 256 * 256;
  return ml + (size_t)partial_rows * head_dim * 4;
}

// Widened tile images (PrefillLaunch::pre) of a bf16-query prefill: one per
// (entry, kv head, 32-token tile of [0, ctx + rows)), after the partials at
// a 1 KiB boundary.
size_t prefill_pre_bytes(const rkv_kv_geometry *g, int32_t n, const int32_t *ctx_lens,
                         const int32_t *q_rows) {
  int64_t tiles = 0;
  for (int32_t e = 0; e < n; ++e) tiles += ((int64_t)ctx_lens[e] + q_rows[e] + 31) / 32;
  return (size_t)tiles * g->kv_heads * (size_t)rkv::prefill_tile_bytes(g->head_dim);
}
size_t prefill_pre_at(size_t partial_bytes) { return (partial_bytes + 1023) / 1024 * 1024; }

constexpr int64_t kUnitCost = 64;       // tokens: a unit's prologue and epilogue
constexpr int64_t kSplitUnitCost = 32;  // tokens: a split unit's partial rows
constexpr int64_t kMaxSimUnits = 16384; // units (times kv heads) a plan simulates at most

// Makespan, in tokens of causal range, of the launch's units in the
// kernel's list order (entries by `order`; an entry's units segment by
// segment, kv head by kv head, row blocks last first).  Unit j runs on XCD
// (j / xcd_chunk) % 8, on whichever of that XCD's CUs frees first.
// One prefill workgroup keeps a CU about as busy as two, so a CU's time is
// the sum of its units'.
int64_t simulate_prefill(const int32_t *ctx, const int32_t *rows, const int32_t *order, int32_t n,
                         int32_t tq, int32_t kv_heads, int64_t seg, int32_t xcd_chunk) {
  constexpr int kXcds = 8;
  constexpr int kCusPerXcd = rkv::kComputeUnits / kXcds;
  std::vector<int64_t> load(rkv::kComputeUnits, 0);  // kXcds min-heaps of kCusPerXcd
  const auto later = std::greater<int64_t>();
  int64_t j = 0;
  for (int32_t k = 0; k < n; ++k) {
    const int64_t c = ctx[order[k]], r = rows[order[k]];
    const int64_t nb = (r + tq - 1) / tq;
    const int32_t ns = segments_of(c + r, (int32_t)seg);
    for (int32_t sg = 0; sg < ns; ++sg)
      for (int32_t h = 0; h < kv_heads; ++h)
        for (int64_t b = nb - 1; b >= 0; --b, ++j) {
          const int64_t range = c + std::min<int64_t>(tq * (b + 1), r);
          const int64_t len = ns == 1 ? range : std::clamp<int64_t>(range - sg * seg, 0, seg);
          auto first = load.begin() + (j / xcd_chunk) % kXcds * kCusPerXcd;
          std::pop_heap(first, first + kCusPerXcd, later);
          first[kCusPerXcd - 1] += len + kUnitCost + (ns > 1 ? kSplitUnitCost : 0);
          std::push_heap(first, first + kCusPerXcd, later);
        }
  }
  return *std::max_element(load.begin(), load.end());
}

// The automatic split.  A launch whose units do not divide evenly over the
// CUs -- too few row blocks, or a few long causal ranges among short ones --
// ends when its longest units do; cutting every range longer than a segment
// into segments evens the CUs' loads.  Candidates: the longest range in k
// segments for a few k; the plan is memoized for the next call with the same
// entries (a serving step repeats them for every layer).
template <typename RowsFor>
SegPlan auto_segments(const rkv_kv_geometry *g, int32_t q_heads, int32_t tq, int32_t n,
                      const int32_t *ctx_lens, const int32_t *q_rows, size_t cap,
                      int32_t xcd_chunk, int64_t max_range, int64_t seg_floor, RowsFor rows_for) {
  SegPlan none;
  thread_local std::vector<int64_t> memo_key;
  thread_local SegPlan memo_plan;
  std::vector<int64_t> key = {tq, q_heads, g->kv_heads, g->page_tokens, g->head_dim,
                              (int64_t)std::min<size_t>(cap, INT64_MAX), xcd_chunk, n};
  for (int32_t e = 0; e < n; ++e) {
    key.push_back(ctx_lens[e]);
    key.push_back(q_rows[e]);
  }
  if (key == memo_key) return memo_plan;
  int32_t order[RKV_PREFILL_MAX_SEQS];
  int64_t units = 0;
  for (int32_t e = 0; e < n; ++e) {
    order[e] = e;
    if (ctx_lens[e] < 0 || q_rows[e] < 0) return none;  // refused by the caller
    units += ((int64_t)q_rows[e] + tq - 1) / tq;
  }
  std::stable_sort(order, order + n, [&](int32_t x, int32_t y) {
    return (int64_t)ctx_lens[x] + q_rows[x] > (int64_t)ctx_lens[y] + q_rows[y];
  });
  SegPlan best = none;
  if (units > 0 && units * g->kv_heads <= kMaxSimUnits / 4) {
    const int64_t unit = std::max<int32_t>(32, g->page_tokens);
    auto round_up = [&](int64_t t) { return (t + unit - 1) / unit * unit; };
    const int64_t base = simulate_prefill(ctx_lens, q_rows, order, n, tq, g->kv_heads, 0, xcd_chunk);
    int64_t best_t = base;
    int64_t last = -1;
    for (int64_t k : {2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64}) {
      const int64_t seg = std::max<int64_t>({round_up((max_range + k - 1) / k),
                                             round_up(kPrefillMinSegment), seg_floor});
      if (seg >= max_range || seg == last) continue;
      last = seg;
      int64_t su = 0;
      for (int32_t e = 0; e < n; ++e)
        su += ((int64_t)q_rows[e] + tq - 1) / tq *
              segments_of((int64_t)ctx_lens[e] + q_rows[e], (int32_t)seg);
      if (su * g->kv_heads > kMaxSimUnits) continue;
      const int64_t p = rows_for(seg);
      if (p == 0 || prefill_ws_bytes(p, g->head_dim) > cap) continue;
      const int64_t t = simulate_prefill(ctx_lens, q_rows, order, n, tq, g->kv_heads, seg, xcd_chunk);
      if (t < best_t) {
        best_t = t;
        best.seg = (int32_t)seg;
        best.partial_rows = p;
      }
    }
    if (best_t * 20 > base * 19) best = none;
  }
  memo_key = std::move(key);
  memo_plan = best;
  return best;
}

// cap: workspace bytes available to the automatic split.
SegPlan plan_segments(const rkv_kv_geometry *g, int32_t q_heads, int32_t tq, int32_t n,
                      const int32_t *ctx_lens, const int32_t *q_rows, int32_t request,
                      size_t cap, int32_t xcd_chunk) {
  SegPlan none;
  if (request < 0 || n <= 0) return none;
  const int64_t unit = std::max<int32_t>(32, g->page_tokens);
  auto round_up = [&](int64_t t) { return (t + unit - 1) / unit * unit; };
  int64_t max_range = 0;
  for (int32_t e = 0; e < n; ++e)
    max_range = std::max<int64_t>(max_range, (int64_t)ctx_lens[e] + q_rows[e]);
  auto rows_for = [&](int64_t seg) {
    int64_t p = 0;
    for (int32_t e = 0; e < n; ++e) {
      const int32_t ns = segments_of((int64_t)ctx_lens[e] + q_rows[e], (int32_t)seg);
      if (ns > 1) p += (int64_t)q_rows[e] * q_heads * ns;
    }
    return p;
  };
  const int64_t seg_floor = round_up((max_range + rkv::kPrefillMaxSegs - 1) / rkv::kPrefillMaxSegs);
  if (request > 0) {
    SegPlan pl;
    pl.seg = (int32_t)std::min<int64_t>(std::max(round_up(request), seg_floor), INT32_MAX);
    pl.partial_rows = rows_for(pl.seg);
    if (pl.partial_rows == 0) pl.seg = 0;
    return pl;
  }
  // automatic: simulate the launch for a few segment lengths and keep the
  // shortest makespan, if it beats the unsplit launch by a twentieth
  return auto_segments(g, q_heads, tq, n, ctx_lens, q_rows, cap, xcd_chunk, max_range, seg_floor,
                       rows_for);
}

// Arguments of a prefill call, and the launch's entry table (row blocks of
// kPrefillRows rows per kv head, in entry order, each in nseg units);
// xcd_chunk as in rkv::PrefillLaunch.
rkv_status make_prefill(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                        const int32_t *bt, int32_t bt_stride, int32_t n_seqs,
                        const rkv_prefill_args *a, const char *op, int32_t xcd_chunk,
                        bool widen_once, rkv::PrefillLaunch &pf) {
  if (rkv_status s = check_geometry(g, op)) return s;
  if (rkv_status s = check_tables(pages, bt, bt_stride, n_seqs, op)) return s;
  if (!a) return fail(RKV_ERR_INVALID_ARG, op, "args is NULL");
  if (a->n_seqs < 0 || a->n_seqs > RKV_PREFILL_MAX_SEQS)
    return fail(RKV_ERR_INVALID_ARG, op, "n_seqs=%d outside [0, %d]", a->n_seqs,
                RKV_PREFILL_MAX_SEQS);
  if (a->q_heads < 1 || a->q_heads % g->kv_heads != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "q_heads=%d is not a multiple of kv_heads=%d",
                a->q_heads, g->kv_heads);
  // a row block holds tq = floor(128 / G) chunk tokens times the G q heads
  // of its kv head; a group that does not divide 128 (the reference's
  // default 24 q / 4 kv heads, attention.rs:134-137, leaves 2 of the 128
  // rows) runs the rows past tq * G as dead rows, as a chunk's last block
  // runs those past its last token
  const int32_t G = a->q_heads / g->kv_heads;
  if (G > rkv::kPrefillRows)
    return fail(RKV_ERR_UNSUPPORTED, op, "q_heads/kv_heads=%d exceeds %d rows per block", G,
                rkv::kPrefillRows);
  if (a->q_dtype != RKV_F32 && a->q_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "q_dtype=%d", a->q_dtype);
  if (a->out_dtype != RKV_F32 && a->out_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "out_dtype=%d", a->out_dtype);
  if (!(std::isfinite(a->scale))) return fail(RKV_ERR_INVALID_ARG, op, "scale is not finite");
  if (a->total_rows < 0) return fail(RKV_ERR_INVALID_ARG, op, "total_rows=%d", a->total_rows);
  if (a->n_seqs > 0 && (!a->seq_ids || !a->ctx_lens || !a->q_rows || !a->q_offsets))
    return fail(RKV_ERR_INVALID_ARG, op, "NULL seq_ids/ctx_lens/q_rows/q_offsets");
  pf = rkv::PrefillLaunch{};
  pf.tq = rkv::kPrefillRows / G;
  pf.n_entries = a->n_seqs;
  // Longest first: a row block's time grows with its causal range, so the
  // entries go into the launch table by descending ctx + rows (and the
  // kernel takes each entry's later row blocks first), which keeps a long
  // entry dispatched last from setting the launch's end.  Outputs are
  // addressed per entry, so the order changes nothing else.
  int32_t order[RKV_PREFILL_MAX_SEQS];
  for (int32_t e = 0; e < a->n_seqs; ++e) order[e] = e;
  std::stable_sort(order, order + a->n_seqs, [&](int32_t x, int32_t y) {
    return (int64_t)a->ctx_lens[x] + a->q_rows[x] > (int64_t)a->ctx_lens[y] + a->q_rows[y];
  });
  if (a->workspace && reinterpret_cast<uintptr_t>(a->workspace) % 256 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "workspace is not 256-byte aligned");
  const SegPlan sp = plan_segments(g, a->q_heads, pf.tq, a->n_seqs, a->ctx_lens, a->q_rows,
                                   a->segment_tokens, a->workspace ? a->workspace_bytes : 0,
                                   xcd_chunk);
  const size_t ws_need = prefill_ws_bytes(sp.partial_rows, g->head_dim);
  if (ws_need > 0 && (!a->workspace || a->workspace_bytes < ws_need))
    return fail(RKV_ERR_INVALID_ARG, op, "segment_tokens=%d needs a %zu-byte workspace (have %zu)",
                a->segment_tokens, ws_need, a->workspace ? a->workspace_bytes : (size_t)0);
  int64_t blocks = 0, prow = 0;
  for (int32_t k = 0; k < a->n_seqs; ++k) {
    const int32_t e = order[k];
    const int32_t seq = a->seq_ids[e], c = a->ctx_lens[e], n = a->q_rows[e], off = a->q_offsets[e];
    if (seq < 0 || seq >= n_seqs)
      return fail(RKV_ERR_INVALID_ARG, op, "entry %d: seq %d outside [0, %d)", e, seq, n_seqs);
    if (c < 0 || n < 0 || off < 0 || (int64_t)off + n > a->total_rows)
      return fail(RKV_ERR_INVALID_ARG, op, "entry %d: ctx_len=%d q_rows=%d q_offset=%d total_rows=%d",
                  e, c, n, off, a->total_rows);
    const int64_t end = (int64_t)c + n;
    if (end > (int64_t)bt_stride * g->page_tokens ||
        (end + g->page_tokens - 1) / g->page_tokens > rkv::kPrefillMaxPages)
      return fail(RKV_ERR_UNSUPPORTED, op, "entry %d: %lld tokens exceed the table row (%d pages, "
                  "at most %d)", e, (long long)end, bt_stride, rkv::kPrefillMaxPages);
    pf.seq[k] = seq;
    pf.ctx[k] = c;
    pf.rows[k] = n;
    pf.qoff[k] = off;
    pf.nseg[k] = segments_of(end, sp.seg);
    pf.seg[k] = pf.nseg[k] > 1 ? sp.seg : 0;
    pf.wsoff[k] = pf.nseg[k] > 1 ? prow : 0;
    if (pf.nseg[k] > 1) prow += (int64_t)n * a->q_heads * pf.nseg[k];
    pf.first[k] = (int32_t)std::min<int64_t>(blocks, INT32_MAX);
    blocks += (int64_t)(n + pf.tq - 1) / pf.tq * pf.nseg[k];
  }
  if (ws_need > 0) {
    pf.ws_ml = static_cast<float *>(a->workspace);
    pf.ws_o = reinterpret_cast<float *>(static_cast<uint8_t *>(a->workspace) +
                                        ws_need - (size_t)prow * g->head_dim * 4);
  }
  // a bf16 query whose workspace also holds every tile widened: the widening
  // pass runs once per tile and the prefill copies the images; otherwise
  // each workgroup widens the tiles it reads.  Not for pages in host memory:
  // there the pass would read every page over the link before the prefill
  // starts (measured 1.30 ms against 0.73-0.77 for a 512-row chunk after
  // 32768 tokens), where the row blocks' reads overlap their compute.
  pf.pre = nullptr;
  if (widen_once && a->q_dtype == RKV_BF16 && a->workspace && a->n_seqs > 0) {
    const size_t at = prefill_pre_at(ws_need);
    const size_t need = prefill_pre_bytes(g, a->n_seqs, a->ctx_lens, a->q_rows);
    if (need > 0 && a->workspace_bytes >= at + need) {
      pf.pre = static_cast<uint8_t *>(a->workspace) + at;
      int64_t t = 0;
      for (int32_t k = 0; k < a->n_seqs; ++k) {
        pf.preoff[k] = t;
        t += ((int64_t)pf.ctx[k] + pf.rows[k] + 31) / 32 * g->kv_heads;
      }
      pf.preoff[a->n_seqs] = t;
      if (t > INT32_MAX) pf.pre = nullptr;  // one widening workgroup per image
    }
  }
  pf.first[a->n_seqs] = (int32_t)blocks;
  pf.xcd_chunk = xcd_chunk;
  if (blocks > 0 && (!a->q || !a->out)) return fail(RKV_ERR_INVALID_ARG, op, "NULL q/out");
  // the grid rounds units up to whole XCD chunk rounds (8 * xcd_chunk)
  if (blocks * g->kv_heads > INT32_MAX - 8 * (int64_t)xcd_chunk)
    return fail(RKV_ERR_INVALID_ARG, op, "too many row blocks");
  if (blocks > 0 && (int64_t)a->total_rows * a->q_heads > INT32_MAX)
    return fail(RKV_ERR_INVALID_ARG, op, "total_rows * q_heads exceeds 2^31");
  rkv::DecodeLaunch &d = pf.d;
  d.g = to_geo(g);
  d.pages = static_cast<const uint8_t *>(pages);
  d.bt = bt;
  d.bt_stride = bt_stride;
  d.n_seqs = n_seqs;
  d.q = a->q;
  d.q_bf16 = a->q_dtype == RKV_BF16;
  d.q_heads = a->q_heads;
  d.scale_log2 = a->scale * 1.4426950408889634f;
  d.out = a->out;
  d.out_bf16 = a->out_dtype == RKV_BF16;
  d.fault = ctx->d_fault;
  d.stages = 2;
  return RKV_OK;
}

rkv_status prefill_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                      const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                      const rkv_prefill_args *a, void *stream, int32_t xcd_chunk,
                      bool widen_once = true) {
  const char *op = "rkv_prefill_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  rkv::PrefillLaunch pf{};
  if (rkv_status s =
          make_prefill(ctx, g, pages, block_tables, bt_stride, n_seqs, a, op, xcd_chunk, widen_once, pf))
    return s;
  hipError_t e = rkv::launch_prefill(pf, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

}  // namespace

extern "C" {

rkv_status rkv_prefill_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                          const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                          const rkv_prefill_args *a, void *stream) {
  return prefill_q8(ctx, g, pages, block_tables, bt_stride, n_seqs, a, stream,
                    rkv::kPrefillXcdChunkHbm);
}

}  // extern "C"

namespace {
// Workspace of a prefill launched with this XCD chunk (the split plan's
// dispatch simulation depends on it), with room for the widened tiles when
// the launch would widen once (HBM pages and a bf16 query).
size_t prefill_ws_query(const rkv_kv_geometry *g, const rkv_prefill_args *a, int32_t xcd_chunk,
                        bool widen_once) {
  if (!g || !a || check_geometry(g, "rkv_prefill_workspace_bytes") != RKV_OK) return 0;
  if (a->n_seqs < 1 || a->n_seqs > RKV_PREFILL_MAX_SEQS || !a->ctx_lens || !a->q_rows) return 0;
  if (a->q_heads < 1 || a->q_heads % g->kv_heads != 0) return 0;
  const int32_t G = a->q_heads / g->kv_heads;
  if (G > rkv::kPrefillRows) return 0;
  for (int32_t e = 0; e < a->n_seqs; ++e)
    if (a->ctx_lens[e] < 0 || a->q_rows[e] < 0) return 0;
  const SegPlan sp = plan_segments(g, a->q_heads, rkv::kPrefillRows / G, a->n_seqs, a->ctx_lens,
                                   a->q_rows, a->segment_tokens, SIZE_MAX, xcd_chunk);
  const size_t partials = prefill_ws_bytes(sp.partial_rows, g->head_dim);
  if (a->q_dtype != RKV_BF16 || !widen_once) return partials;
  return prefill_pre_at(partials) + prefill_pre_bytes(g, a->n_seqs, a->ctx_lens, a->q_rows);
}
}  // namespace

extern "C" {

size_t rkv_prefill_workspace_bytes(const rkv_kv_geometry *g, const rkv_prefill_args *a) {
  return prefill_ws_query(g, a, rkv::kPrefillXcdChunkHbm, true);
}

rkv_status rkv_append_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                         const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                         const rkv_append_args *args, void *stream) {
  const char *op = "rkv_append_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_geometry(g, op)) return s;
  if (rkv_status s = check_tables(pages, block_tables, bt_stride, n_seqs, op)) return s;
  if (!args) return fail(RKV_ERR_INVALID_ARG, op, "args is NULL");
  if (args->n_rows < 0) return fail(RKV_ERR_INVALID_ARG, op, "n_rows=%d", args->n_rows);
  if (args->src_dtype != RKV_F32 && args->src_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "src_dtype=%d", args->src_dtype);
  if (args->rule != RKV_Q8_CANONICAL && args->rule != RKV_Q8_HARSERVE)
    return fail(RKV_ERR_INVALID_ARG, op, "rule=%d", args->rule);
  if (args->n_rows == 0) return RKV_OK;
  if (!args->seq_ids || !args->positions || !args->k_src || !args->v_src)
    return fail(RKV_ERR_INVALID_ARG, op, "NULL seq_ids/positions/k_src/v_src");
  rkv::AppendLaunch a{};
  a.g = to_geo(g);
  a.pages = static_cast<uint8_t *>(pages);
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.n_seqs = n_seqs;
  a.n_rows = args->n_rows;
  a.seq_ids = args->seq_ids;
  a.positions = args->positions;
  a.k_src = args->k_src;
  a.v_src = args->v_src;
  a.src_bf16 = args->src_dtype == RKV_BF16;
  a.rule = args->rule;
  a.fault = ctx->d_fault;
  hipError_t e = rkv::launch_append(a, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

int32_t rkv_decode_partition_tokens(const rkv_kv_geometry *g, const rkv_decode_args *a) {
  if (!g || !a) return 0;
  return a->partition_tokens > 0 ? a->partition_tokens : 0;
}

size_t rkv_decode_workspace_bytes(const rkv_kv_geometry *g, const rkv_decode_args *a) {
  if (!g || !a || check_geometry(g, "rkv_decode_workspace_bytes") != RKV_OK) return 0;
  if (a->q_heads < 1 || a->q_heads % g->kv_heads != 0 || a->q_len < 1) return 0;
  // enough for either ring depth (a pool in host memory launches 3 stages)
  return std::max(ws_bytes(g, a, plan_of(g, a, 2)), ws_bytes(g, a, plan_of(g, a, 3)));
}

}  // extern "C"

namespace {
// rkv_decode_q8 with an explicit LDS ring depth: 2 (the default, K codes in
// registers) or 3 (K codes staged in LDS with V, two tiles in flight).
rkv_status decode_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                     const int32_t *block_tables, int32_t bt_stride, const int32_t *seq_lens,
                     int32_t n_seqs, const rkv_decode_args *a, void *stream, int32_t stages) {
  const char *op = "rkv_decode_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_decode(g, a, op)) return s;
  if (rkv_status s = check_tables(pages, block_tables, bt_stride, n_seqs, op)) return s;
  if (!seq_lens) return fail(RKV_ERR_INVALID_ARG, op, "seq_lens is NULL");
  if (a->batch == 0) return RKV_OK;
  const Plan pl = plan_of(g, a, stages);
  rkv::DecodeLaunch d = make_decode(ctx, g, pages, block_tables, bt_stride, seq_lens, n_seqs, a, pl);
  hipStream_t hs = as_stream(stream);
  if (!pl.direct) {
    const size_t need = ws_bytes(g, a, pl);
    if (!a->workspace || a->workspace_bytes < need)
      return fail(RKV_ERR_INVALID_ARG, op, "workspace %zu bytes < %zu needed", a->workspace_bytes,
                  need);
    const WsLayout w = ws_layout(g, a, pl);
    uint8_t *base = static_cast<uint8_t *>(a->workspace);
    d.ws_hdr = reinterpret_cast<int32_t *>(base + w.hdr);
    d.ws_ml = reinterpret_cast<float *>(base + w.ml);
    d.ws_o = reinterpret_cast<float *>(base + w.o);
  }
  hipError_t e = rkv::launch_decode(d, hs);
  if (e != hipSuccess) return hip_fail(op, e);
  if (!pl.direct) {
    if (a->split_event && (e = hipEventRecord(static_cast<hipEvent_t>(a->split_event), hs)) != hipSuccess)
      return hip_fail(op, e);
    const WsLayout w = ws_layout(g, a, pl);
    rkv::FlatCombineLaunch c{d.ws_ml,       d.ws_o,       d.ws_hdr,          a->batch,
                             a->q_len,      a->q_heads,   g->kv_heads,       g->head_dim,
                             pl.n_wg,       w.combine_slices, a->out,        d.out_bf16};
    if ((e = rkv::launch_combine_flat(c, hs)) != hipSuccess) return hip_fail(op, e);
  }
  return RKV_OK;
}
}  // namespace

extern "C" {

rkv_status rkv_decode_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_lens, int32_t n_seqs, const rkv_decode_args *a,
                         void *stream) {
  return decode_q8(ctx, g, pages, block_tables, bt_stride, seq_lens, n_seqs, a, stream,
                   decode_stages());
}

rkv_status rkv_decode_q8_noalloc(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                                 const int32_t *block_tables, int32_t bt_stride,
                                 const int32_t *seq_lens, int32_t n_seqs,
                                 const rkv_decode_args *a, void *stream) {
  const char *op = "rkv_decode_q8_noalloc";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_decode(g, a, op)) return s;
  if (!ctx->scratch) return fail(RKV_ERR_DEVICE, op, "no static scratch on device %d", ctx->device);
  const size_t need = ws_bytes(g, a, plan_of(g, a, decode_stages()));
  if (need > rkv::kDecodeScratchBytes)
    return fail(RKV_ERR_INVALID_ARG, op,
                "the split-K partials need %zu bytes, more than the %zu-byte static scratch "
                "(fewer entries, shorter max_seq_len or longer partitions fit; rkv_decode_q8 "
                "takes a workspace of any size)", need, rkv::kDecodeScratchBytes);
  rkv_decode_args b = *a;
  b.workspace = ctx->scratch;
  b.workspace_bytes = rkv::kDecodeScratchBytes;
  return decode_q8(ctx, g, pages, block_tables, bt_stride, seq_lens, n_seqs, &b, stream,
                   decode_stages());
}

rkv_status rkv_decode_q8_partials(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                                  const int32_t *block_tables, int32_t bt_stride,
                                  const int32_t *seq_lens, int32_t n_seqs,
                                  const rkv_decode_args *a, float *ml, float *o, void *stream) {
  const char *op = "rkv_decode_q8_partials";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_decode(g, a, op)) return s;
  if (rkv_status s = check_tables(pages, block_tables, bt_stride, n_seqs, op)) return s;
  if (!seq_lens || !ml || !o) return fail(RKV_ERR_INVALID_ARG, op, "NULL seq_lens/ml/o");
  if (a->partition_tokens <= 0)
    return fail(RKV_ERR_INVALID_ARG, op, "needs an explicit partition_tokens (the [B][rows][n_parts] "
                                         "layout is sized by it)");
  if (a->batch == 0) return RKV_OK;
  const Plan pl = plan_of(g, a, decode_stages());
  rkv::DecodeLaunch d = make_decode(ctx, g, pages, block_tables, bt_stride, seq_lens, n_seqs, a, pl);
  d.ws_ml = ml;  // per-entry layout, written even for one partition
  d.ws_o = o;
  d.out = nullptr;
  hipError_t e = rkv::launch_decode(d, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_splitk_combine(rkv_ctx *ctx, const float *ml, const float *o, int32_t batch,
                              int32_t rows, int32_t n_parts, int32_t head_dim,
                              const int32_t *seq_ids, const int32_t *seq_lens, int32_t n_seqs,
                              int32_t partition_tokens, void *out, int32_t out_dtype,
                              void *stream) {
  const char *op = "rkv_splitk_combine";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (!ml || !o || !seq_ids || !seq_lens || !out)
    return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  if (batch < 0 || rows < 1 || n_parts < 1 || partition_tokens < 1)
    return fail(RKV_ERR_INVALID_ARG, op, "batch=%d rows=%d n_parts=%d partition_tokens=%d", batch,
                rows, n_parts, partition_tokens);
  if (head_dim < 1 || head_dim > 256)
    return fail(RKV_ERR_UNSUPPORTED, op, "head_dim=%d (<= 256)", head_dim);
  if (out_dtype != RKV_F32 && out_dtype != RKV_BF16)
    return fail(RKV_ERR_UNSUPPORTED, op, "out_dtype=%d", out_dtype);
  if (n_seqs < 1) return fail(RKV_ERR_INVALID_ARG, op, "n_seqs=%d", n_seqs);
  rkv::CombineLaunch c{ml, o, batch, rows, n_parts, head_dim, seq_ids, seq_lens, n_seqs,
                       partition_tokens, out, out_dtype == RKV_BF16};
  hipError_t e = rkv::launch_combine(c, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_gather_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                         const int32_t *block_table, int32_t len, int32_t kind, uint8_t *out,
                         void *stream) {
  const char *op = "rkv_gather_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_geometry(g, op)) return s;
  if (kind != RKV_K && kind != RKV_V) return fail(RKV_ERR_INVALID_ARG, op, "kind=%d", kind);
  if (len < 0) return fail(RKV_ERR_INVALID_ARG, op, "len=%d", len);
  if (len == 0) return RKV_OK;
  if (!pages || !block_table || !out) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  hipError_t e = rkv::launch_gather(to_geo(g), static_cast<const uint8_t *>(pages), block_table,
                                    len, kind, out, ctx->d_fault, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_import_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                         const int32_t *block_table, int32_t len, int32_t kind,
                         const uint8_t *rows, void *stream) {
  const char *op = "rkv_import_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_geometry(g, op)) return s;
  if (kind != RKV_K && kind != RKV_V) return fail(RKV_ERR_INVALID_ARG, op, "kind=%d", kind);
  if (len < 0) return fail(RKV_ERR_INVALID_ARG, op, "len=%d", len);
  if (len == 0) return RKV_OK;
  if (!pages || !block_table || !rows) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  hipError_t e = rkv::launch_import(to_geo(g), static_cast<uint8_t *>(pages), block_table, len,
                                    kind, rows, ctx->d_fault, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_copy_pages(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                          int64_t layer_stride_bytes, int32_t layers, const int32_t *pairs,
                          int32_t n_pairs, void *stream) {
  const char *op = "rkv_copy_pages";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_geometry(g, op)) return s;
  const int64_t pb = (int64_t)rkv::page_bytes(to_geo(g));
  if (layers < 1 || n_pairs < 0)
    return fail(RKV_ERR_INVALID_ARG, op, "layers=%d n_pairs=%d", layers, n_pairs);
  if (layers > 1 && layer_stride_bytes < pb * g->num_pages)
    return fail(RKV_ERR_INVALID_ARG, op, "layer stride %lld < %lld bytes of one layer's pages",
                (long long)layer_stride_bytes, (long long)(pb * g->num_pages));
  if (n_pairs == 0) return RKV_OK;
  if (!pages || !pairs) return fail(RKV_ERR_INVALID_ARG, op, "NULL pages or pairs");
  hipError_t e = rkv::launch_copy_pages(static_cast<uint8_t *>(pages), layer_stride_bytes, layers,
                                        g->num_pages, pairs, n_pairs, pb, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_f32_to_f16(rkv_ctx *ctx, const float *in, uint16_t *out, int64_t n, int32_t rule,
                          void *stream) {
  const char *op = "rkv_f32_to_f16";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (n < 0 || (n > 0 && (!in || !out))) return fail(RKV_ERR_INVALID_ARG, op, "bad buffer");
  if (rule != RKV_Q8_CANONICAL && rule != RKV_Q8_HARSERVE)
    return fail(RKV_ERR_INVALID_ARG, op, "rule=%d", rule);
  hipError_t e = rkv::launch_f32_to_f16(in, out, n, rule, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

// ---------------------------------------------------------------------------
// flash_decode_q8.comp drop-in: contiguous rows -> scratch pages -> decode
// ---------------------------------------------------------------------------
// Scratch layout: [pages][block table int32 ceil(seq_len/64)][seq_len int32]
// [seq_id int32], all 256-byte aligned.
namespace {
struct FdScratch {
  rkv_kv_geometry g;
  size_t pages_off, bt_off, len_off, sid_off, ws_off, total;
  int32_t n_pages;
};
FdScratch fd_scratch(const rkv_flash_decode_params *p) {
  FdScratch s{};
  s.g.kv_heads = p->kv_heads;
  s.g.head_dim = p->head_dim;
  s.g.page_tokens = 64;
  s.n_pages = std::max(1, (p->seq_len + 63) / 64);
  s.g.num_pages = s.n_pages;
  auto up = [](size_t v) { return (v + 255) / 256 * 256; };
  s.pages_off = 0;
  s.bt_off = up(s.pages_off + (size_t)s.n_pages * rkv::page_bytes(to_geo(&s.g)));
  s.len_off = up(s.bt_off + sizeof(int32_t) * s.n_pages);
  s.sid_off = up(s.len_off + sizeof(int32_t));
  s.ws_off = up(s.sid_off + sizeof(int32_t));
  s.total = s.ws_off;
  return s;
}
rkv_decode_args fd_args(const rkv_flash_decode_params *p, const FdScratch &s, uint8_t *base,
                        const float *query, float *out) {
  rkv_decode_args a{};
  a.batch = 1;
  a.seq_ids = reinterpret_cast<const int32_t *>(base + s.sid_off);
  a.q = query;
  a.q_dtype = RKV_F32;
  a.q_len = 1;
  a.q_heads = p->q_heads;
  a.scale = 1.0f;  // flash_decode_q8.comp applies no softmax scale
  a.out = out;
  a.out_dtype = RKV_F32;
  a.max_seq_len = p->seq_len;
  // one partition covers the sequence when it fits 64 pages; else split
  a.partition_tokens = 0;
  return a;
}
}  // namespace

size_t rkv_flash_decode_scratch_bytes(const rkv_flash_decode_params *p) {
  if (!p || p->seq_len < 0 || p->kv_heads < 1) return 0;
  FdScratch s = fd_scratch(p);
  rkv_decode_args a = fd_args(p, s, nullptr, nullptr, nullptr);
  return s.total + rkv_decode_workspace_bytes(&s.g, &a);
}

rkv_status rkv_flash_decode_q8(rkv_ctx *ctx, const rkv_flash_decode_params *p,
                               const uint32_t *k_words, const uint32_t *v_words,
                               const float *query, float *out, void *scratch, void *stream) {
  const char *op = "rkv_flash_decode_q8";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (!p || !query || !out || !scratch) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  // smoke :47-51 asserts the GQA divisibility
  if (p->kv_heads < 1 || p->q_heads % p->kv_heads != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "GQA requires q_heads %% kv_heads == 0 (%d, %d)",
                p->q_heads, p->kv_heads);
  if (p->seq_len < 0) return fail(RKV_ERR_INVALID_ARG, op, "seq_len=%d", p->seq_len);
  if (p->seq_len > 0 && (!k_words || !v_words)) return fail(RKV_ERR_INVALID_ARG, op, "NULL K/V");
  FdScratch s = fd_scratch(p);
  if (rkv_status st = check_geometry(&s.g, op)) return st;
  uint8_t *base = static_cast<uint8_t *>(scratch);
  hipStream_t hs = as_stream(stream);
  // identity block table, length and sequence id, written by a tiny upload
  std::vector<int32_t> bt(s.n_pages);
  for (int32_t i = 0; i < s.n_pages; ++i) bt[i] = i;
  const int32_t meta[2] = {p->seq_len, 0};
  hipError_t e;
  if ((e = hipMemcpyAsync(base + s.bt_off, bt.data(), sizeof(int32_t) * s.n_pages,
                          hipMemcpyHostToDevice, hs)) != hipSuccess)
    return hip_fail(op, e);
  if ((e = hipMemcpyAsync(base + s.len_off, &meta[0], sizeof(int32_t), hipMemcpyHostToDevice, hs)) !=
      hipSuccess)
    return hip_fail(op, e);
  if ((e = hipMemcpyAsync(base + s.sid_off, &meta[1], sizeof(int32_t), hipMemcpyHostToDevice, hs)) !=
      hipSuccess)
    return hip_fail(op, e);
  // the host copies above come from stack/vector memory: finish them first
  if ((e = hipStreamSynchronize(hs)) != hipSuccess) return hip_fail(op, e);
  const int32_t *dbt = reinterpret_cast<const int32_t *>(base + s.bt_off);
  if (p->seq_len > 0) {
    if (rkv_status st = rkv_import_q8(ctx, &s.g, base + s.pages_off, dbt, p->seq_len, RKV_K,
                                      reinterpret_cast<const uint8_t *>(k_words), stream))
      return st;
    if (rkv_status st = rkv_import_q8(ctx, &s.g, base + s.pages_off, dbt, p->seq_len, RKV_V,
                                      reinterpret_cast<const uint8_t *>(v_words), stream))
      return st;
  }
  rkv_decode_args a = fd_args(p, s, base, query, out);
  a.workspace = base + s.ws_off;
  a.workspace_bytes = rkv_decode_workspace_bytes(&s.g, &a);
  return rkv_decode_q8(ctx, &s.g, base + s.pages_off, dbt, s.n_pages,
                       reinterpret_cast<const int32_t *>(base + s.len_off), 1, &a, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// pool
// ---------------------------------------------------------------------------
struct rkv_pool {
  rkv_ctx *ctx = nullptr;
  rkv_pool_desc d{};
  rkv_kv_geometry g{};
  rkv_alloc *alloc = nullptr;
  uint8_t *pages = nullptr;  // layers * num_pages * page_bytes (device address)
  void *host_pages = nullptr;  // RKV_PAGES_HOST: the pinned allocation behind `pages`
  size_t layer_bytes = 0;
  int32_t *d_tables = nullptr;
  int32_t *d_lens = nullptr;
  // table uploads: two slots, each a pinned host staging buffer and a device
  // buffer of the packed size max_seqs * (W + 1) + max_seqs int32, followed
  // by room for num_pages queued copy-on-write pairs.  A slot is reused every
  // other sync, after the event recorded behind the last kernel that read its
  // device buffer, so syncs on different streams never overwrite a buffer
  // still in use.
  // table-sync staging: two pinned, coherent host buffers that the scatter
  // kernel reads in place (their device mappings d_stage), alternately; the
  // kernel's last block stores the sync's number to done[slot] (pinned,
  // coherent) once every block has read the buffer, and a sync waits for
  // that before it rewrites the slot.  scatter_count is the device counter
  // of the scatter blocks run so far, scatter_blocks the blocks launched.
  int32_t *h_stage[2] = {nullptr, nullptr};
  int32_t *d_stage[2] = {nullptr, nullptr};
  unsigned long long *done = nullptr, *d_done = nullptr;
  unsigned long long slot_sync[2] = {0, 0};  // the sync that last used each slot (0: none)
  unsigned long long *scatter_count = nullptr;
  unsigned long long scatter_blocks = 0;
  uint32_t n_syncs = 0;
  // R4KV page CRC: device result word and its pinned host copy
  uint32_t *d_crc = nullptr;
  uint32_t *h_crc = nullptr;
  // the stream of the pool's last call (see order_after_last)
  hipStream_t last_stream = nullptr;
  bool has_last = false;
  // rkv_pool_release_stream forgot last_stream: `handoff` already marks the
  // work queued on it (when handoff_set; a capturing stream has none)
  bool released = false;
  bool handoff_set = false;
  hipEvent_t handoff = nullptr;
};

namespace {
size_t stage_ints(const rkv_pool_desc &d) {
  return (size_t)d.max_seqs * (d.max_pages_per_seq + 1) + d.max_seqs + 2 * (size_t)d.num_pages;
}

// A pool's calls run in call order, whatever streams they are queued on.
// The device tables, lengths and pages are one state: a table sync rewrites
// the lengths while a decode queued earlier on another stream may still be
// reading them.  So a call on a stream other than the previous call's first
// makes its stream wait, on the device, for all the work queued so far on
// the previous one (an event recorded there; nothing waits on the host).
// Calls that stay on one stream pay nothing.  A graph capture on either
// stream is left alone: a capturing stream may neither wait on nor record for
// work outside its capture, and the stream the graph is launched on orders the
// captured calls when it runs.
// Wait until the scatter kernel of the sync that last used staging slot
// `slot` has read it (its completion word reached that sync's number).
// The wait spins on host memory; after two seconds it waits for the whole
// device once, and a word still short then (the kernel did not run: a
// device error) returns false instead of waiting on.
bool wait_stage(rkv_pool *p, int slot) {
  if (!p->done) return true;
  const unsigned long long want = p->slot_sync[slot];
  auto ready = [&] { return __atomic_load_n(&p->done[slot], __ATOMIC_ACQUIRE) >= want; };
  const auto t0 = std::chrono::steady_clock::now();
  while (!ready()) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2)) {
      (void)hipDeviceSynchronize();
      return ready();
    }
    std::this_thread::yield();
  }
  return true;
}

// A stream the caller released (rkv_pool_release_stream) is never touched
// again: its handoff event was recorded at the release.
rkv_status order_after_last(rkv_pool *p, hipStream_t hs, const char *op) {
  if (p->released) {
    hipStreamCaptureStatus now = hipStreamCaptureStatusNone;
    hipError_t e;
    if ((e = hipStreamIsCapturing(hs, &now)) != hipSuccess) return hip_fail(op, e);
    if (p->handoff_set && now == hipStreamCaptureStatusNone &&
        (e = hipStreamWaitEvent(hs, p->handoff, 0)) != hipSuccess)
      return hip_fail(op, e);
  } else if (p->has_last && p->last_stream != hs) {
    hipStreamCaptureStatus now = hipStreamCaptureStatusNone, before = hipStreamCaptureStatusNone;
    hipError_t e;
    if ((e = hipStreamIsCapturing(hs, &now)) != hipSuccess ||
        (e = hipStreamIsCapturing(p->last_stream, &before)) != hipSuccess)
      return hip_fail(op, e);
    if (now == hipStreamCaptureStatusNone && before == hipStreamCaptureStatusNone &&
        ((e = hipEventRecord(p->handoff, p->last_stream)) != hipSuccess ||
         (e = hipStreamWaitEvent(hs, p->handoff, 0)) != hipSuccess))
      return hip_fail(op, e);
  }
  p->last_stream = hs;
  p->has_last = true;
  p->released = false;
  return RKV_OK;
}
}  // namespace

extern "C" {

rkv_status rkv_pool_create(rkv_ctx *ctx, const rkv_pool_desc *desc, rkv_pool **out) {
  const char *op = "rkv_pool_create";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (!desc || !out) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  *out = nullptr;
  if (desc->layers < 1) return fail(RKV_ERR_INVALID_ARG, op, "layers=%d", desc->layers);
  if (desc->page_memory != RKV_PAGES_DEVICE && desc->page_memory != RKV_PAGES_HOST)
    return fail(RKV_ERR_INVALID_ARG, op, "page_memory=%d", desc->page_memory);
  rkv_kv_geometry g{desc->kv_heads, desc->head_dim, desc->page_tokens, desc->num_pages};
  if (rkv_status s = check_geometry(&g, op)) return s;
  rkv_alloc_desc ad{desc->num_pages, desc->page_tokens, desc->max_seqs, desc->max_pages_per_seq,
                    desc->free_list_seed};
  rkv_pool *p = new rkv_pool;
  p->ctx = ctx;
  p->d = *desc;
  p->g = g;
  if (rkv_status s = rkv_alloc_create(&ad, &p->alloc)) {
    delete p;
    return s;
  }
  p->layer_bytes = (size_t)desc->num_pages * rkv::page_bytes(to_geo(&g));
  hipError_t e;
  const size_t tbytes = sizeof(int32_t) * (size_t)desc->max_seqs * desc->max_pages_per_seq;
  const size_t sbytes = sizeof(int32_t) * stage_ints(*desc);
  const size_t all_pages = p->layer_bytes * desc->layers;
  if (desc->page_memory == RKV_PAGES_HOST) {
    // pinned, mapped for the device; non-coherent, so the device may cache
    // what it reads (the pages change only through this library's kernels)
    if ((e = hipHostMalloc(&p->host_pages, all_pages,
                           hipHostMallocMapped | hipHostMallocNonCoherent)) != hipSuccess ||
        (e = hipHostGetDevicePointer(reinterpret_cast<void **>(&p->pages), p->host_pages, 0)) !=
            hipSuccess) {
      rkv_status s = fail(RKV_ERR_DEVICE, op, "allocating %zu pinned host page bytes: %s",
                          all_pages, hipGetErrorString(e));
      rkv_pool_destroy(p);
      return s;
    }
    std::memset(p->host_pages, 0, all_pages);
  }
  if ((desc->page_memory == RKV_PAGES_DEVICE &&
       (e = hipMalloc(&p->pages, all_pages)) != hipSuccess) ||
      (e = hipMalloc(&p->d_tables, tbytes)) != hipSuccess ||
      (e = hipMalloc(&p->d_lens, sizeof(int32_t) * desc->max_seqs)) != hipSuccess ||
      (e = hipHostMalloc(&p->h_stage[0], sbytes, hipHostMallocMapped | hipHostMallocCoherent)) !=
          hipSuccess ||
      (e = hipHostMalloc(&p->h_stage[1], sbytes, hipHostMallocMapped | hipHostMallocCoherent)) !=
          hipSuccess ||
      (e = hipHostGetDevicePointer(reinterpret_cast<void **>(&p->d_stage[0]), p->h_stage[0], 0)) !=
          hipSuccess ||
      (e = hipHostGetDevicePointer(reinterpret_cast<void **>(&p->d_stage[1]), p->h_stage[1], 0)) !=
          hipSuccess ||
      (e = hipHostMalloc(&p->done, 2 * sizeof(unsigned long long),
                         hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess ||
      (e = hipHostGetDevicePointer(reinterpret_cast<void **>(&p->d_done), p->done, 0)) != hipSuccess ||
      (e = hipMalloc(&p->scatter_count, sizeof(unsigned long long))) != hipSuccess ||
      (e = hipMemset(p->scatter_count, 0, sizeof(unsigned long long))) != hipSuccess ||
      (e = hipEventCreateWithFlags(&p->handoff, hipEventDisableTiming)) != hipSuccess ||
      (e = hipMalloc(&p->d_crc, 256)) != hipSuccess ||
      (e = hipHostMalloc(&p->h_crc, 256, hipHostMallocDefault)) != hipSuccess) {
    rkv_status s = fail(RKV_ERR_DEVICE, op, "allocating %zu page bytes and tables: %s",
                        p->layer_bytes * desc->layers, hipGetErrorString(e));
    rkv_pool_destroy(p);
    return s;
  }
  p->done[0] = p->done[1] = 0;
  // zeroed pages: never-written slots hold finite codes and scales
  if (desc->page_memory == RKV_PAGES_DEVICE && (e = hipMemset(p->pages, 0, all_pages)) != hipSuccess) {
    rkv_pool_destroy(p);
    return hip_fail(op, e);
  }
  if (rkv_status s = rkv_pool_sync_tables(p, nullptr)) {
    rkv_pool_destroy(p);
    return s;
  }
  if ((e = hipStreamSynchronize(nullptr)) != hipSuccess) {
    rkv_pool_destroy(p);
    return hip_fail(op, e);
  }
  *out = p;
  return RKV_OK;
}

rkv_status rkv_pool_destroy(rkv_pool *p) {
  if (!p) return RKV_OK;
  if (p->ctx) (void)hipSetDevice(p->ctx->device);
  // the last syncs' scatter kernels may still be reading the staging buffers
  for (int i = 0; i < 2; ++i) (void)wait_stage(p, i);
  if (p->host_pages) (void)hipHostFree(p->host_pages);
  else (void)hipFree(p->pages);
  (void)hipFree(p->d_tables);
  (void)hipFree(p->d_lens);
  (void)hipFree(p->scatter_count);
  (void)hipFree(p->d_crc);
  if (p->h_crc) (void)hipHostFree(p->h_crc);
  if (p->done) (void)hipHostFree(p->done);
  for (int i = 0; i < 2; ++i)
    if (p->h_stage[i]) (void)hipHostFree(p->h_stage[i]);
  if (p->handoff) (void)hipEventDestroy(p->handoff);
  rkv_alloc_destroy(p->alloc);
  delete p;
  return RKV_OK;
}

rkv_status rkv_pool_release_stream(rkv_pool *pool, void *stream) {
  const char *op = "rkv_pool_release_stream";
  if (!pool) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (rkv_status s = use_device(pool->ctx, op)) return s;
  hipStream_t hs = as_stream(stream);
  if (pool->released || !pool->has_last || pool->last_stream != hs) return RKV_OK;
  hipStreamCaptureStatus now = hipStreamCaptureStatusNone;
  hipError_t e;
  if ((e = hipStreamIsCapturing(hs, &now)) != hipSuccess) return hip_fail(op, e);
  // a capturing stream's calls are ordered by the stream its graph runs on
  pool->handoff_set = now == hipStreamCaptureStatusNone;
  if (pool->handoff_set && (e = hipEventRecord(pool->handoff, hs)) != hipSuccess)
    return hip_fail(op, e);
  pool->released = true;
  return RKV_OK;
}

rkv_alloc *rkv_pool_allocator(rkv_pool *p) { return p ? p->alloc : nullptr; }

rkv_status rkv_pool_sync_tables(rkv_pool *p, void *stream) {
  const char *op = "rkv_pool_sync_tables";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (rkv_status s = use_device(p->ctx, op)) return s;
  // Stream-ordered upload: the changed rows, every length and the queued
  // copy-on-write pairs are packed into a pinned staging buffer, copied in
  // one transfer, then the page copies run and the rows are scattered on the
  // device, so launches queued after this call on `stream` see the new
  // tables and copied pages, and earlier ones the old.  Nothing here waits
  // for the device unless the staging slot's kernels from two syncs ago are
  // still pending.
  hipStream_t hs = as_stream(stream);
  {
    // the staging buffer is read in place when the kernel runs, so a graph
    // replay would upload the tables of the capture, not the current ones
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(hs, &cap);
    if (e != hipSuccess) return hip_fail(op, e);
    if (cap != hipStreamCaptureStatusNone)
      return fail(RKV_ERR_INVALID_ARG, op, "the stream is capturing a graph: table uploads carry "
                  "host state and run eagerly, before the captured launches");
  }
  if (rkv_status s = order_after_last(p, hs, op)) return s;
  rkv_alloc *a = p->alloc;
  const int32_t W = a->d.max_pages_per_seq;
  const int32_t S = a->d.max_seqs;
  const uint32_t slot = p->n_syncs & 1u;
  if (!wait_stage(p, (int)slot))
    return fail(RKV_ERR_DEVICE, op, "the table upload of sync %llu never ran (device error)",
                p->slot_sync[slot]);
  hipError_t e = hipSuccess;
  int32_t *h = p->h_stage[slot];
  int32_t n_rows = 0;
  for (int32_t s = 0; s < S; ++s) {
    if (!a->dirty[s]) continue;
    int32_t *rec = h + (size_t)n_rows * (W + 1);
    rec[0] = s;
    std::memcpy(rec + 1, &a->tables[(size_t)s * W], sizeof(int32_t) * W);
    a->dirty[s] = 0;
    ++n_rows;
  }
  std::memcpy(h + (size_t)n_rows * (W + 1), a->lens.data(), sizeof(int32_t) * S);
  const size_t pairs_at = (size_t)n_rows * (W + 1) + S;
  int32_t n_pairs = 0;
  if (rkv_status s = rkv_alloc_take_copies(a, h + pairs_at, a->d.num_pages, &n_pairs)) return s;
  // the kernels read the staging buffer in place (pinned, coherent): no
  // copy, and no event, in the stream; the copies run before the scatter,
  // so the scatter's completion word covers both
  const int32_t *d = p->d_stage[slot];
  ++p->n_syncs;
  if ((e = rkv::launch_copy_pages(p->pages, (int64_t)p->layer_bytes, p->d.layers, p->d.num_pages,
                                  d + pairs_at, n_pairs,
                                  (int64_t)rkv::page_bytes(to_geo(&p->g)), hs)) != hipSuccess)
    return hip_fail(op, e);
  const unsigned long long blocks = (unsigned long long)n_rows + 1;
  const unsigned long long seq = p->n_syncs;
  if ((e = rkv::launch_table_scatter(d, n_rows, W, S, p->d_tables, p->d_lens, p->scatter_count,
                                     p->scatter_blocks + blocks - 1, p->d_done + slot, seq, hs)) !=
      hipSuccess)
    return hip_fail(op, e);
  p->scatter_blocks += blocks;
  p->slot_sync[slot] = seq;
  return RKV_OK;
}

void *rkv_pool_layer_pages(rkv_pool *p, int32_t layer) {
  if (!p || layer < 0 || layer >= p->d.layers) return nullptr;
  return p->pages + (size_t)layer * p->layer_bytes;
}
const int32_t *rkv_pool_block_tables(rkv_pool *p) { return p ? p->d_tables : nullptr; }
const int32_t *rkv_pool_seq_lens(rkv_pool *p) { return p ? p->d_lens : nullptr; }

rkv_status rkv_pool_append(rkv_pool *p, int32_t layer, const rkv_append_args *args, void *stream) {
  const char *op = "rkv_pool_append";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (layer < 0 || layer >= p->d.layers) return fail(RKV_ERR_INVALID_ARG, op, "layer=%d", layer);
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = order_after_last(p, as_stream(stream), op)) return s;
  return rkv_append_q8(p->ctx, &p->g, rkv_pool_layer_pages(p, layer), p->d_tables,
                       p->d.max_pages_per_seq, p->d.max_seqs, args, stream);
}

rkv_status rkv_pool_decode(rkv_pool *p, int32_t layer, const rkv_decode_args *args, void *stream) {
  const char *op = "rkv_pool_decode";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (layer < 0 || layer >= p->d.layers) return fail(RKV_ERR_INVALID_ARG, op, "layer=%d", layer);
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = order_after_last(p, as_stream(stream), op)) return s;
  // pages in host memory: K staged through LDS with V (the register loads
  // of K read the host link at 87% of the LDS-DMA copies' rate)
  return decode_q8(p->ctx, &p->g, rkv_pool_layer_pages(p, layer), p->d_tables,
                   p->d.max_pages_per_seq, p->d_lens, p->d.max_seqs, args, stream,
                   p->d.page_memory == RKV_PAGES_HOST ? 3 : decode_stages());
}

rkv_status rkv_pool_prefill(rkv_pool *p, int32_t layer, const rkv_prefill_args *args,
                            void *stream) {
  const char *op = "rkv_pool_prefill";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (layer < 0 || layer >= p->d.layers) return fail(RKV_ERR_INVALID_ARG, op, "layer=%d", layer);
  if (args) {
    for (int32_t e = 0; e < args->n_seqs && args->seq_ids && args->ctx_lens && args->q_rows; ++e) {
      const int32_t seq = args->seq_ids[e];
      if (seq < 0 || seq >= p->d.max_seqs) continue;  // reported by the kernel-level check
      if ((int64_t)args->ctx_lens[e] + args->q_rows[e] > p->alloc->lens[seq])
        return fail(RKV_ERR_INVALID_ARG, op, "entry %d: ctx_len %d + q_rows %d > length %d of seq %d",
                    e, args->ctx_lens[e], args->q_rows[e], p->alloc->lens[seq], seq);
    }
  }
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = order_after_last(p, as_stream(stream), op)) return s;
  // pages behind the host link: the row blocks of one causal range share
  // one XCD's L2 (in HBM, chunks of 8 spread them over 4 XCDs)
  // (and no widening pass, which would read every page over the link first)
  const bool host = p->d.page_memory == RKV_PAGES_HOST;
  return prefill_q8(p->ctx, &p->g, rkv_pool_layer_pages(p, layer), p->d_tables,
                    p->d.max_pages_per_seq, p->d.max_seqs, args, stream,
                    host ? rkv::kPrefillXcdChunkHost : rkv::kPrefillXcdChunkHbm, !host);
}

size_t rkv_pool_prefill_workspace_bytes(const rkv_pool *p, const rkv_prefill_args *args) {
  if (!p) return 0;
  const bool host = p->d.page_memory == RKV_PAGES_HOST;
  return prefill_ws_query(&p->g, args, host ? rkv::kPrefillXcdChunkHost : rkv::kPrefillXcdChunkHbm,
                          !host);
}

rkv_status rkv_pool_gather(rkv_pool *p, int32_t layer, int32_t seq, int32_t kind, uint8_t *out,
                           void *stream) {
  const char *op = "rkv_pool_gather";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (layer < 0 || layer >= p->d.layers) return fail(RKV_ERR_INVALID_ARG, op, "layer=%d", layer);
  if (rkv_status s = check_seq(p->alloc, seq, op)) return s;
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = order_after_last(p, as_stream(stream), op)) return s;
  return rkv_gather_q8(p->ctx, &p->g, rkv_pool_layer_pages(p, layer),
                       p->d_tables + (size_t)seq * p->d.max_pages_per_seq, p->alloc->lens[seq],
                       kind, out, stream);
}


}  // extern "C"

// ---------------------------------------------------------------------------
// R4KV pages (r4kv/src/page.rs)
// ---------------------------------------------------------------------------
namespace {

void put16(uint8_t *b, int off, uint16_t v) {
  for (int i = 0; i < 2; ++i) b[off + i] = (uint8_t)(v >> (8 * i));
}
void put32(uint8_t *b, int off, uint32_t v) {
  for (int i = 0; i < 4; ++i) b[off + i] = (uint8_t)(v >> (8 * i));
}
void put64(uint8_t *b, int off, uint64_t v) {
  for (int i = 0; i < 8; ++i) b[off + i] = (uint8_t)(v >> (8 * i));
}
uint16_t get16(const uint8_t *b, int off) { return (uint16_t)(b[off] | (b[off + 1] << 8)); }
uint32_t get32(const uint8_t *b, int off) {
  uint32_t v = 0;
  for (int i = 0; i < 4; ++i) v |= (uint32_t)b[off + i] << (8 * i);
  return v;
}
uint64_t get64(const uint8_t *b, int off) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)b[off + i] << (8 * i);
  return v;
}

const char *refusal_name(int32_t r) {
  static const char *names[] = {"accepted", "BadMagic", "BadVersion", "HeaderChecksumMismatch",
                                "PayloadChecksumMismatch", "LengthMismatch", "PrefixMismatch",
                                "TokenRangeMismatch", "PosMismatch", "LayerRangeInsufficient",
                                "FormatRefused", "GenerationRejected"};
  return r >= 0 && r <= RKV_R4KV_GENERATION ? names[r] : "unknown";
}

rkv_status refuse(int32_t *refusal, int32_t why, const char *op, const char *detail) {
  if (refusal) *refusal = why;
  return fail(RKV_ERR_REFUSED, op, "%s (%s)", refusal_name(why), detail);
}

size_t spill_body_bytes(const rkv_pool *p, int64_t count, int32_t n_layers) {
  return (size_t)n_layers * 2 * (size_t)p->d.kv_heads * (size_t)count * rkv_row_bytes(p->d.head_dim);
}

}  // namespace

extern "C" {

uint32_t rkv_crc32c_host(const uint8_t *data, size_t n) {
  return data || n == 0 ? rkv::crc::crc32c(data, n) : 0u;
}

rkv_status rkv_crc32c(rkv_ctx *ctx, const void *data, uint64_t n, uint32_t *out, void *stream) {
  const char *op = "rkv_crc32c";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (!out || (n > 0 && !data)) return fail(RKV_ERR_INVALID_ARG, op, "NULL data/out");
  if (reinterpret_cast<uintptr_t>(data) % 16 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "data is not 16-byte aligned");
  if (n >= ((uint64_t)1 << rkv::crc::kShiftBits))
    return fail(RKV_ERR_UNSUPPORTED, op, "n=%llu bytes (< 2^40)", (unsigned long long)n);
  hipError_t e = rkv::launch_crc32c(static_cast<const uint8_t *>(data), (int64_t)n, out,
                                    as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_stream_read(rkv_ctx *ctx, const void *data, uint64_t bytes, int32_t mode,
                           int32_t blocks, uint32_t *out, void *stream) {
  const char *op = "rkv_stream_read";
  static_assert(RKV_STREAM_DMA_UNIT == 16384, "LDS-DMA round of the stream kernel");
  if (rkv_status s = use_device(ctx, op)) return s;
  if (mode != 0 && mode != 1) return fail(RKV_ERR_INVALID_ARG, op, "mode=%d", mode);
  if (blocks < 1 || blocks > (1 << 20)) return fail(RKV_ERR_INVALID_ARG, op, "blocks=%d", blocks);
  if (!data || (mode == 0 && !out)) return fail(RKV_ERR_INVALID_ARG, op, "NULL data/out");
  if (reinterpret_cast<uintptr_t>(data) % 16 != 0 || bytes % 16 != 0 || bytes == 0)
    return fail(RKV_ERR_INVALID_ARG, op, "data/bytes (%llu) not 16-byte aligned",
                (unsigned long long)bytes);
  if (mode == 1 && bytes % ((uint64_t)blocks * rkv::stream_read_dma_unit()) != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "bytes %llu not a multiple of blocks * %d",
                (unsigned long long)bytes, RKV_STREAM_DMA_UNIT);
  hipError_t e = rkv::launch_stream_read(static_cast<const uint8_t *>(data), (int64_t)bytes, mode,
                                         blocks, out, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_stream_read_tiles(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                                 const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                                 int32_t seq_tokens, int32_t partition_tokens, void *stream) {
  const char *op = "rkv_stream_read_tiles";
  if (rkv_status s = use_device(ctx, op)) return s;
  if (rkv_status s = check_geometry(g, op)) return s;
  if (g->page_tokens < 32) return fail(RKV_ERR_UNSUPPORTED, op, "page_tokens=%d < 32", g->page_tokens);
  if (!pages || !block_tables) return fail(RKV_ERR_INVALID_ARG, op, "NULL pages/block_tables");
  if (n_seqs < 1 || seq_tokens < 32 || seq_tokens % 32 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "n_seqs=%d seq_tokens=%d", n_seqs, seq_tokens);
  if (partition_tokens < 32 || partition_tokens % 32 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "partition_tokens=%d (a multiple of 32)", partition_tokens);
  // partitions start on 32-token tiles, inside a page when partition_tokens
  // is not a whole number of pages; each must span at most 64 pages (the
  // kernel holds one page id per lane), the decode's rule
  for (int64_t t0 = 0; t0 < seq_tokens; t0 += partition_tokens) {
    const int64_t t1 = std::min<int64_t>(seq_tokens, t0 + partition_tokens);
    if ((t1 - 1) / g->page_tokens - t0 / g->page_tokens + 1 > 64)
      return fail(RKV_ERR_INVALID_ARG, op,
                  "partition_tokens=%d: the partition at token %lld spans more than 64 pages of %d",
                  partition_tokens, (long long)t0, g->page_tokens);
  }
  if ((seq_tokens + g->page_tokens - 1) / g->page_tokens > bt_stride)
    return fail(RKV_ERR_INVALID_ARG, op, "seq_tokens=%d needs more pages than bt_stride=%d",
                seq_tokens, bt_stride);
  const int32_t parts = (seq_tokens + partition_tokens - 1) / partition_tokens;
  if ((int64_t)n_seqs * parts > INT32_MAX)
    return fail(RKV_ERR_INVALID_ARG, op, "n_seqs=%d x %d partitions", n_seqs, parts);
  rkv::TileStreamLaunch t{to_geo(g), static_cast<const uint8_t *>(pages), block_tables, bt_stride,
                          n_seqs, seq_tokens, partition_tokens, parts};
  hipError_t e = rkv::launch_stream_tiles(t, as_stream(stream));
  return e == hipSuccess ? RKV_OK : hip_fail(op, e);
}

rkv_status rkv_r4kv_header_encode(const rkv_r4kv_header *h, uint8_t out[RKV_R4KV_HEADER_BYTES]) {
  if (!h || !out) return fail(RKV_ERR_INVALID_ARG, "rkv_r4kv_header_encode", "NULL argument");
  std::memset(out, 0, RKV_R4KV_HEADER_BYTES);
  put32(out, 0, RKV_R4KV_MAGIC);
  put16(out, 4, RKV_R4KV_VERSION);
  put16(out, 6, h->flags);
  put64(out, 8, h->prefix_digest);
  put32(out, 16, h->token_start);
  put32(out, 20, h->token_count);
  put32(out, 24, h->pos_start);
  put16(out, 28, h->layer_lo);
  put16(out, 30, h->layer_hi);
  out[32] = h->k_fmt;
  out[33] = h->v_fmt;
  put32(out, 34, h->epoch);
  put32(out, 38, h->generation);
  put64(out, 42, h->payload_len);
  put32(out, 50, h->sketch_offset);
  put32(out, 92, rkv::crc::crc32c(out, 92));  // 54..92 reserved zeros
  return RKV_OK;
}

rkv_status rkv_r4kv_header_decode(const uint8_t in[RKV_R4KV_HEADER_BYTES], rkv_r4kv_header *h,
                                  int32_t *refusal) {
  const char *op = "rkv_r4kv_header_decode";
  if (refusal) *refusal = RKV_R4KV_ACCEPTED;
  if (!in || !h) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  if (get32(in, 0) != RKV_R4KV_MAGIC) return refuse(refusal, RKV_R4KV_BAD_MAGIC, op, "magic");
  if (get16(in, 4) != RKV_R4KV_VERSION) return refuse(refusal, RKV_R4KV_BAD_VERSION, op, "version");
  if (rkv::crc::crc32c(in, 92) != get32(in, 92))
    return refuse(refusal, RKV_R4KV_HEADER_CHECKSUM, op, "header CRC32C");
  if (in[32] > RKV_FMT_Q3) return refuse(refusal, RKV_R4KV_FORMAT, op, "k_fmt");
  if (in[33] > RKV_FMT_Q3) return refuse(refusal, RKV_R4KV_FORMAT, op, "v_fmt");
  h->flags = get16(in, 6);
  h->prefix_digest = get64(in, 8);
  h->token_start = get32(in, 16);
  h->token_count = get32(in, 20);
  h->pos_start = get32(in, 24);
  h->layer_lo = get16(in, 28);
  h->layer_hi = get16(in, 30);
  h->k_fmt = in[32];
  h->v_fmt = in[33];
  h->epoch = get32(in, 34);
  h->generation = get32(in, 38);
  h->payload_len = get64(in, 42);
  h->sketch_offset = get32(in, 50);
  return RKV_OK;
}

rkv_status rkv_r4kv_check_restore(const rkv_r4kv_header *h, const rkv_r4kv_expect *e,
                                  uint64_t payload_body_len, int32_t *refusal) {
  const char *op = "rkv_r4kv_check_restore";
  if (refusal) *refusal = RKV_R4KV_ACCEPTED;
  if (!h || !e) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  char msg[128];
  if (payload_body_len != h->payload_len) {
    std::snprintf(msg, sizeof msg, "declared %llu, actual %llu", (unsigned long long)h->payload_len,
                  (unsigned long long)payload_body_len);
    return refuse(refusal, RKV_R4KV_LENGTH, op, msg);
  }
  if (h->prefix_digest != e->prefix_digest) {
    std::snprintf(msg, sizeof msg, "want %016llx, got %016llx", (unsigned long long)e->prefix_digest,
                  (unsigned long long)h->prefix_digest);
    return refuse(refusal, RKV_R4KV_PREFIX, op, msg);
  }
  if (h->token_start != e->token_start) {
    std::snprintf(msg, sizeof msg, "want %u, got %u", e->token_start, h->token_start);
    return refuse(refusal, RKV_R4KV_TOKEN_RANGE, op, msg);
  }
  if (h->pos_start != e->pos_start) {
    std::snprintf(msg, sizeof msg, "want %u, got %u", e->pos_start, h->pos_start);
    return refuse(refusal, RKV_R4KV_POS, op, msg);
  }
  if (h->layer_lo > e->layer_lo || h->layer_hi < e->layer_hi) {
    std::snprintf(msg, sizeof msg, "want [%u, %u], got [%u, %u]", e->layer_lo, e->layer_hi,
                  h->layer_lo, h->layer_hi);
    return refuse(refusal, RKV_R4KV_LAYER_RANGE, op, msg);
  }
  if (e->k_fmt >= 0 && e->k_fmt != h->k_fmt) return refuse(refusal, RKV_R4KV_FORMAT, op, "k_fmt");
  if (e->v_fmt >= 0 && e->v_fmt != h->v_fmt) return refuse(refusal, RKV_R4KV_FORMAT, op, "v_fmt");
  if (e->check_generation && (h->generation < e->generation_min || h->generation > e->generation_max))
    return refuse(refusal, RKV_R4KV_GENERATION, op, "generation predicate");
  return RKV_OK;
}

rkv_status rkv_r4kv_unpack_host(const uint8_t *page, size_t len, rkv_r4kv_header *h,
                                const uint8_t **body, int32_t *refusal) {
  const char *op = "rkv_r4kv_unpack_host";
  if (refusal) *refusal = RKV_R4KV_ACCEPTED;
  if (!h || (len > 0 && !page)) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  if (len < RKV_R4KV_HEADER_BYTES + 4) return refuse(refusal, RKV_R4KV_LENGTH, op, "shorter than 100 bytes");
  if (rkv_status s = rkv_r4kv_header_decode(page, h, refusal)) return s;
  const size_t body_len = len - RKV_R4KV_HEADER_BYTES - 4;
  if (body_len != h->payload_len) return refuse(refusal, RKV_R4KV_LENGTH, op, "body length");
  const uint8_t *b = page + RKV_R4KV_HEADER_BYTES;
  if (rkv::crc::crc32c(b, body_len) != get32(b, (int)body_len))
    return refuse(refusal, RKV_R4KV_PAYLOAD_CHECKSUM, op, "payload CRC32C");
  if (body) *body = b;
  return RKV_OK;
}

size_t rkv_r4kv_page_bytes(const rkv_pool *p, int32_t token_count, int32_t layer_lo,
                           int32_t layer_hi) {
  if (!p || token_count < 0 || layer_lo < 0 || layer_hi < layer_lo || layer_hi >= p->d.layers)
    return 0;
  return RKV_R4KV_HEADER_BYTES + spill_body_bytes(p, token_count, layer_hi - layer_lo + 1) + 4;
}

rkv_status rkv_pool_spill(rkv_pool *p, int32_t seq, int32_t token_start, int32_t token_count,
                          int32_t layer_lo, int32_t layer_hi, const rkv_r4kv_header *identity,
                          void *staging, size_t staging_bytes, void *dst, size_t dst_bytes,
                          void *stream) {
  const char *op = "rkv_pool_spill";
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = check_seq(p->alloc, seq, op)) return s;
  if (!identity) return fail(RKV_ERR_INVALID_ARG, op, "identity is NULL");
  if (token_start < 0 || token_count < 0 ||
      (int64_t)token_start + token_count > p->alloc->lens[seq])
    return fail(RKV_ERR_INVALID_ARG, op, "tokens [%d, +%d) outside the %d of seq %d", token_start,
                token_count, p->alloc->lens[seq], seq);
  const size_t need = rkv_r4kv_page_bytes(p, token_count, layer_lo, layer_hi);
  if (need == 0) return fail(RKV_ERR_INVALID_ARG, op, "layers [%d, %d] of %d", layer_lo, layer_hi, p->d.layers);
  if (!staging || staging_bytes < need || !dst || dst_bytes < need)
    return fail(RKV_ERR_INVALID_ARG, op, "staging %zu / dst %zu bytes < %zu", staging_bytes,
                dst_bytes, need);
  if (reinterpret_cast<uintptr_t>(staging) % 16 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "staging is not 16-byte aligned");
  rkv_r4kv_header h = *identity;
  h.token_start = (uint32_t)token_start;
  h.token_count = (uint32_t)token_count;
  h.layer_lo = (uint16_t)layer_lo;
  h.layer_hi = (uint16_t)layer_hi;
  h.k_fmt = RKV_FMT_Q8;
  h.v_fmt = RKV_FMT_Q8;
  h.payload_len = need - RKV_R4KV_HEADER_BYTES - 4;
  h.sketch_offset = 0;
  h.flags = (uint16_t)(identity->flags & ~1u);  // no sketch
  rkv::R4kvLaunch r{};
  r.g = to_geo(&p->g);
  r.layer_stride = (int64_t)p->layer_bytes;
  r.layer_lo = layer_lo;
  r.n_layers = layer_hi - layer_lo + 1;
  r.t0 = token_start;
  r.count = token_count;
  rkv_r4kv_header_encode(&h, r.header);
  hipStream_t hs = as_stream(stream);
  if (rkv_status s = order_after_last(p, hs, op)) return s;
  hipError_t e = rkv::launch_r4kv_pack(r, p->pages, p->d_tables + (size_t)seq * p->d.max_pages_per_seq,
                                       static_cast<uint8_t *>(staging), p->d_crc, p->ctx->d_fault, hs);
  if (e != hipSuccess) return hip_fail(op, e);
  if (dst != staging && (e = hipMemcpyAsync(dst, staging, need, hipMemcpyDefault, hs)) != hipSuccess)
    return hip_fail(op, e);
  return RKV_OK;
}

rkv_status rkv_pool_restore(rkv_pool *p, int32_t seq, const uint8_t *page, size_t page_bytes,
                            const rkv_r4kv_expect *expect, void *staging, size_t staging_bytes,
                            int32_t *refusal, void *stream) {
  const char *op = "rkv_pool_restore";
  if (refusal) *refusal = RKV_R4KV_ACCEPTED;
  if (!p) return fail(RKV_ERR_INVALID_ARG, op, "pool is NULL");
  if (rkv_status s = use_device(p->ctx, op)) return s;
  if (rkv_status s = check_seq(p->alloc, seq, op)) return s;
  if (!page || !expect) return fail(RKV_ERR_INVALID_ARG, op, "NULL page/expect");
  // host gates first: nothing reaches the device unless these pass
  if (page_bytes < RKV_R4KV_HEADER_BYTES + 4) return refuse(refusal, RKV_R4KV_LENGTH, op, "shorter than 100 bytes");
  rkv_r4kv_header h;
  if (rkv_status s = rkv_r4kv_header_decode(page, &h, refusal)) return s;
  const size_t body_len = page_bytes - RKV_R4KV_HEADER_BYTES - 4;
  if (rkv_status s = rkv_r4kv_check_restore(&h, expect, body_len, refusal)) return s;
  if (h.k_fmt != RKV_FMT_Q8 || h.v_fmt != RKV_FMT_Q8)
    return fail(RKV_ERR_UNSUPPORTED, op, "k_fmt=%u v_fmt=%u (this pool holds Q8)", h.k_fmt, h.v_fmt);
  if (h.layer_hi >= p->d.layers || h.layer_lo > h.layer_hi)
    return fail(RKV_ERR_INVALID_ARG, op, "page layers [%u, %u] of %d", h.layer_lo, h.layer_hi, p->d.layers);
  if (body_len != spill_body_bytes(p, h.token_count, h.layer_hi - h.layer_lo + 1))
    return fail(RKV_ERR_INVALID_ARG, op, "body of %zu bytes does not match %u tokens x layers [%u, %u]",
                body_len, h.token_count, h.layer_lo, h.layer_hi);
  if ((int64_t)h.token_start + h.token_count > p->alloc->lens[seq])
    return fail(RKV_ERR_INVALID_ARG, op, "tokens [%u, +%u) outside the %d reserved for seq %d",
                h.token_start, h.token_count, p->alloc->lens[seq], seq);
  if (!staging || staging_bytes < body_len || reinterpret_cast<uintptr_t>(staging) % 16 != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "staging must be 16-byte aligned and hold %zu bytes", body_len);
  const uint32_t stored = get32(page, (int)(RKV_R4KV_HEADER_BYTES + body_len));
  hipStream_t hs = as_stream(stream);
  if (rkv_status s = order_after_last(p, hs, op)) return s;
  hipError_t e;
  if (body_len > 0 &&
      (e = hipMemcpyAsync(staging, page + RKV_R4KV_HEADER_BYTES, body_len, hipMemcpyHostToDevice, hs)) != hipSuccess)
    return hip_fail(op, e);
  if ((e = rkv::launch_crc32c(static_cast<const uint8_t *>(staging), (int64_t)body_len, p->d_crc, hs)) != hipSuccess ||
      (e = hipMemcpyAsync(p->h_crc, p->d_crc, 4, hipMemcpyDeviceToHost, hs)) != hipSuccess ||
      (e = hipStreamSynchronize(hs)) != hipSuccess)
    return hip_fail(op, e);
  if (*p->h_crc != stored) return refuse(refusal, RKV_R4KV_PAYLOAD_CHECKSUM, op, "payload CRC32C");
  rkv::R4kvLaunch r{};
  r.g = to_geo(&p->g);
  r.layer_stride = (int64_t)p->layer_bytes;
  r.layer_lo = h.layer_lo;
  r.n_layers = h.layer_hi - h.layer_lo + 1;
  r.t0 = (int32_t)h.token_start;
  r.count = (int32_t)h.token_count;
  if ((e = rkv::launch_r4kv_unpack(r, p->pages, p->d_tables + (size_t)seq * p->d.max_pages_per_seq,
                                   static_cast<const uint8_t *>(staging), p->ctx->d_fault, hs)) != hipSuccess)
    return hip_fail(op, e);
  return RKV_OK;
}

}  // extern "C"
