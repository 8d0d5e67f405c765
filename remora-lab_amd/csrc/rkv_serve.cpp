// rkv_serve.cpp -- serving adapter over a pool: the KV side of a
// BatchStepModel backend (har-serve/src/adapter.rs:28-72) as the serving
// scheduler drives it once per step (ServeScheduler::step,
// har-serve/src/scheduler.rs:603-960).
//
// The scheduler names sequences by SequenceId (scheduler.rs:122).  The
// adapter maps each live id to a pool sequence, grows it by the tokens the
// step consumes, and runs each layer's attention for the step's rows: the
// decode rows (batch_step, one token per sequence) through rkv_pool_decode
// with the rows' K/V appended inside the launch, the prefill chunks
// (prefill_batch) through rkv_pool_append + rkv_pool_prefill.  Page
// locations are the ExactHotQ8 representation's PhysicalPageLocation
// (har-kv/src/page.rs:100-115) of the KV page records the scheduler
// attaches every page_size consumed tokens (scheduler.rs:1045-1077).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/rkv.h"
#include "rkv_host.h"
#include "rkv_launch.h"

using rkv::host::fail;
using rkv::host::hip_fail;
using rkv::host::use_device;

struct rkv_serve {
  rkv_ctx *ctx = nullptr;
  rkv_serve_desc d{};
  rkv_pool *pool = nullptr;
  rkv_kv_geometry g{};  // the pool's physical geometry
  size_t page_bytes = 0;
  int32_t per_page = 1;  // the scheduler's pages (KV page records) per pool page
  int32_t row_pages = 0; // pool pages of a block-table row
  std::unordered_map<uint64_t, int32_t> slot_of;  // live SequenceId -> pool sequence
  std::vector<int32_t> free_slots;                 // unused pool sequences, a stack
  // the step begun last
  int32_t n_decode = 0;
  int32_t decode_max_len = 0;                  // longest decode sequence after its growth
  std::vector<int32_t> pf_seq, pf_ctx, pf_rows, pf_off;  // prefill entries (host)
  int32_t pf_total = 0;
  // device row layout of the step, packed as [decode seq ids][decode
  // positions][prefill row seq ids][prefill row positions] by the actual
  // counts, copied from pinned staging (two buffers, alternate steps)
  int32_t *d_meta = nullptr;
  int32_t *h_meta[2] = {nullptr, nullptr};
  hipEvent_t meta_done[2] = {nullptr, nullptr};
  uint32_t n_steps = 0;
  void *ws = nullptr;  // decode workspace for max_decode rows of the longest sequence
  size_t ws_bytes = 0;
  void *pf_ws = nullptr;  // prefill split-K partials (the automatic split fits itself in it)
  size_t pf_ws_bytes = 0;
};

namespace {

size_t meta_ints(const rkv_serve_desc &d) {
  return 2 * ((size_t)d.max_decode + (size_t)d.max_prefill_rows);
}

rkv_status live_slot(const rkv_serve *s, uint64_t id, const char *op, int32_t *slot) {
  if (!s) return fail(RKV_ERR_INVALID_ARG, op, "serve is NULL");
  auto it = s->slot_of.find(id);
  if (it == s->slot_of.end())
    return fail(RKV_ERR_INVALID_ARG, op, "sequence id %llu is not live", (unsigned long long)id);
  *slot = it->second;
  return RKV_OK;
}

}  // namespace

extern "C" {

rkv_status rkv_serve_create(rkv_ctx *ctx, const rkv_serve_desc *desc, rkv_serve **out) {
  const char *op = "rkv_serve_create";
  if (!desc || !out) return fail(RKV_ERR_INVALID_ARG, op, "NULL argument");
  *out = nullptr;
  if (rkv_status st = use_device(ctx, op)) return st;
  if (desc->kv_heads < 1 || desc->q_heads < 1 || desc->q_heads % desc->kv_heads != 0)
    return fail(RKV_ERR_INVALID_ARG, op, "q_heads=%d is not a multiple of kv_heads=%d",
                desc->q_heads, desc->kv_heads);
  if (desc->max_decode < 1 || desc->max_decode > desc->max_seqs || desc->max_prefill_rows < 0)
    return fail(RKV_ERR_INVALID_ARG, op, "max_decode=%d (max_seqs=%d) max_prefill_rows=%d",
                desc->max_decode, desc->max_seqs, desc->max_prefill_rows);
  if (desc->rule != RKV_Q8_CANONICAL && desc->rule != RKV_Q8_HARSERVE)
    return fail(RKV_ERR_INVALID_ARG, op, "rule=%d", desc->rule);
  // The scheduler's page (attach_page_if_boundary, scheduler.rs:1045-1077;
  // ServeConfig::default() page_size 8, :103-120) is a record of
  // page_tokens tokens.  Pool pages hold whole records: a record of 16
  // tokens or more is one pool page; smaller records (1, 2, 4, 8) share
  // 32-token pool pages, which the kernels read as one 32-token tile (the
  // page of KVGeometry::qwen36_27b, har-kv/src/geometry.rs:39-59).
  const int32_t lpt = desc->page_tokens;
  if (lpt < 1 || lpt > 256 || (lpt & (lpt - 1)) != 0)
    return fail(RKV_ERR_UNSUPPORTED, op, "page_tokens=%d (a power of two, 1..256)", lpt);
  if (desc->num_pages < 1 || desc->max_pages_per_seq < 1)
    return fail(RKV_ERR_INVALID_ARG, op, "num_pages=%d max_pages_per_seq=%d", desc->num_pages,
                desc->max_pages_per_seq);
  const int32_t ppt = lpt >= 16 ? lpt : 32;
  const int32_t per = ppt / lpt;
  rkv_pool_desc pd{desc->layers,
                   desc->kv_heads,
                   desc->head_dim,
                   ppt,
                   (int32_t)(((int64_t)desc->num_pages + per - 1) / per),
                   desc->max_seqs,
                   (int32_t)(((int64_t)desc->max_pages_per_seq + per - 1) / per),
                   desc->free_list_seed,
                   desc->page_memory};
  rkv_serve *s = new rkv_serve;
  s->ctx = ctx;
  s->d = *desc;
  s->per_page = per;
  s->row_pages = pd.max_pages_per_seq;
  s->g = rkv_kv_geometry{desc->kv_heads, desc->head_dim, ppt, pd.num_pages};
  if (rkv_status st = rkv_pool_create(ctx, &pd, &s->pool)) {
    delete s;
    return st;
  }
  s->page_bytes = rkv_page_bytes(&s->g);
  for (int32_t i = desc->max_seqs - 1; i >= 0; --i) s->free_slots.push_back(i);
  // decode workspace for the largest decode step: max_decode rows of the
  // longest sequence a block-table row holds
  rkv_decode_args a{};
  a.batch = desc->max_decode;
  a.q_len = 1;
  a.q_heads = desc->q_heads;
  a.max_seq_len = pd.max_pages_per_seq * ppt;
  s->ws_bytes = rkv_decode_workspace_bytes(&s->g, &a);
  // prefill partials: about two units of 128 rows per workgroup slot, which
  // the automatic split (about one unit per slot) fits in; layout (m, l)
  // rows padded to 256 bytes, then o rows
  const int64_t pf_rows = std::min<int64_t>(
      (int64_t)desc->max_prefill_rows * desc->q_heads * rkv::kPrefillMaxSegs,
      2LL * rkv::kComputeUnits * rkv::kPrefillWgsPerCu * rkv::kPrefillRows);
  s->pf_ws_bytes =
      pf_rows > 0 ? ((size_t)pf_rows * 8 + 255) / 256 * 256 + (size_t)pf_rows * desc->head_dim * 4 : 0;
  const size_t mbytes = sizeof(int32_t) * std::max<size_t>(meta_ints(*desc), 1);
  hipError_t e = hipSuccess;
  if ((s->ws_bytes > 0 && (e = hipMalloc(&s->ws, s->ws_bytes)) != hipSuccess) ||
      (s->pf_ws_bytes > 0 && (e = hipMalloc(&s->pf_ws, s->pf_ws_bytes)) != hipSuccess) ||
      (e = hipMalloc(&s->d_meta, mbytes)) != hipSuccess ||
      (e = hipHostMalloc(&s->h_meta[0], mbytes, hipHostMallocDefault)) != hipSuccess ||
      (e = hipHostMalloc(&s->h_meta[1], mbytes, hipHostMallocDefault)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&s->meta_done[0], hipEventDisableTiming)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&s->meta_done[1], hipEventDisableTiming)) != hipSuccess) {
    rkv_status st = hip_fail(op, e);
    rkv_serve_destroy(s);
    return st;
  }
  *out = s;
  return RKV_OK;
}

rkv_status rkv_serve_destroy(rkv_serve *s) {
  if (!s) return RKV_OK;
  (void)use_device(s->ctx, "rkv_serve_destroy");
  for (int i = 0; i < 2; ++i)
    if (s->meta_done[i]) (void)hipEventSynchronize(s->meta_done[i]);
  (void)hipFree(s->ws);
  (void)hipFree(s->pf_ws);
  (void)hipFree(s->d_meta);
  for (int i = 0; i < 2; ++i) {
    if (s->h_meta[i]) (void)hipHostFree(s->h_meta[i]);
    if (s->meta_done[i]) (void)hipEventDestroy(s->meta_done[i]);
  }
  rkv_pool_destroy(s->pool);
  delete s;
  return RKV_OK;
}

rkv_pool *rkv_serve_pool(rkv_serve *s) { return s ? s->pool : nullptr; }

rkv_status rkv_serve_begin_step(rkv_serve *s, const rkv_serve_entry *prefill, int32_t n_prefill,
                                const rkv_serve_entry *decode, int32_t n_decode, void *stream) {
  const char *op = "rkv_serve_begin_step";
  if (!s) return fail(RKV_ERR_INVALID_ARG, op, "serve is NULL");
  if (n_prefill < 0 || n_decode < 0 || n_decode > s->d.max_decode)
    return fail(RKV_ERR_INVALID_ARG, op, "n_prefill=%d n_decode=%d (max_decode %d)", n_prefill,
                n_decode, s->d.max_decode);
  if ((n_prefill > 0 && !prefill) || (n_decode > 0 && !decode))
    return fail(RKV_ERR_INVALID_ARG, op, "NULL entries");
  if (rkv_status st = use_device(s->ctx, op)) return st;
  rkv_alloc *a = rkv_pool_allocator(s->pool);

  // ---- checks first: nothing changes unless the whole step is accepted ----
  const int32_t n = n_prefill + n_decode;
  auto entry = [&](int32_t i) -> const rkv_serve_entry & {
    return i < n_prefill ? prefill[i] : decode[i - n_prefill];
  };
  std::unordered_set<uint64_t> seen;
  int64_t rows = 0;
  int32_t admits = 0;
  for (int32_t i = 0; i < n; ++i) {
    const rkv_serve_entry &en = entry(i);
    if (!seen.insert(en.id).second)
      return fail(RKV_ERR_INVALID_ARG, op, "sequence id %llu appears twice in the step",
                  (unsigned long long)en.id);
    if (i >= n_prefill ? en.tokens != 1 : en.tokens < 1)
      return fail(RKV_ERR_INVALID_ARG, op, "%s entry for id %llu consumes %d tokens",
                  i >= n_prefill ? "decode" : "prefill", (unsigned long long)en.id, en.tokens);
    if (i < n_prefill) rows += en.tokens;
    if (s->slot_of.count(en.id)) continue;
    ++admits;
    if (en.fork_len < 0) return fail(RKV_ERR_INVALID_ARG, op, "fork_len=%d", en.fork_len);
    if (en.fork_len > 0) {
      auto it = s->slot_of.find(en.parent);
      if (it == s->slot_of.end())
        return fail(RKV_ERR_INVALID_ARG, op, "fork parent %llu is not live",
                    (unsigned long long)en.parent);
      int32_t plen = 0;
      rkv_seq_len(a, it->second, &plen);
      if (en.fork_len > plen)
        return fail(RKV_ERR_INVALID_ARG, op, "fork_len %d > length %d of parent %llu", en.fork_len,
                    plen, (unsigned long long)en.parent);
    }
  }
  if (rows > s->d.max_prefill_rows)
    return fail(RKV_ERR_INVALID_ARG, op, "%lld prefill rows > max_prefill_rows %d",
                (long long)rows, s->d.max_prefill_rows);
  if (admits > (int32_t)s->free_slots.size())
    return fail(RKV_ERR_CAPACITY, op, "%d new sequences, %zu free of max_seqs %d", admits,
                s->free_slots.size(), s->d.max_seqs);

  // ---- admit and grow; undo everything on the first failure ----
  std::vector<int32_t> slot(n), ctx(n);
  std::vector<uint8_t> admitted(n, 0);
  int32_t done = 0;
  rkv_status st = RKV_OK;
  for (; done < n; ++done) {
    const rkv_serve_entry &en = entry(done);
    auto it = s->slot_of.find(en.id);
    if (it == s->slot_of.end()) {
      const int32_t sl = s->free_slots.back();
      if (en.fork_len > 0) st = rkv_seq_fork(a, s->slot_of.at(en.parent), sl, en.fork_len);
      if (st != RKV_OK) break;
      s->free_slots.pop_back();
      s->slot_of.emplace(en.id, sl);
      admitted[done] = 1;
      slot[done] = sl;
    } else {
      slot[done] = it->second;
    }
    rkv_seq_len(a, slot[done], &ctx[done]);
    if ((st = rkv_seq_reserve(a, slot[done], ctx[done] + en.tokens)) != RKV_OK) {
      if (admitted[done]) {  // undo this entry's admission too
        rkv_seq_free(a, slot[done]);
        s->slot_of.erase(en.id);
        s->free_slots.push_back(slot[done]);
      }
      break;
    }
  }
  if (st != RKV_OK) {
    const std::string why = rkv_last_error();
    for (int32_t i = done - 1; i >= 0; --i) {
      if (admitted[i]) {
        rkv_seq_free(a, slot[i]);
        s->slot_of.erase(entry(i).id);
        s->free_slots.push_back(slot[i]);
      } else {
        rkv_seq_truncate(a, slot[i], ctx[i]);
      }
    }
    return fail(st, op, "step refused, no sequence changed (%s)", why.c_str());
  }

  // ---- the step's layout ----
  s->n_decode = n_decode;
  s->decode_max_len = 0;
  s->pf_seq.assign(slot.begin(), slot.begin() + n_prefill);
  s->pf_ctx.assign(ctx.begin(), ctx.begin() + n_prefill);
  s->pf_rows.resize(n_prefill);
  s->pf_off.resize(n_prefill);
  s->pf_total = 0;
  for (int32_t i = 0; i < n_prefill; ++i) {
    s->pf_rows[i] = prefill[i].tokens;
    s->pf_off[i] = s->pf_total;
    s->pf_total += prefill[i].tokens;
  }
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if ((st = rkv_pool_sync_tables(s->pool, stream)) != RKV_OK) return st;
  const uint32_t buf = s->n_steps & 1u;
  hipError_t e = hipEventSynchronize(s->meta_done[buf]);
  if (e != hipSuccess) return hip_fail(op, e);
  int32_t *h = s->h_meta[buf];
  for (int32_t b = 0; b < n_decode; ++b) {
    h[b] = slot[n_prefill + b];
    h[n_decode + b] = ctx[n_prefill + b];
    s->decode_max_len = std::max(s->decode_max_len, ctx[n_prefill + b] + 1);
  }
  int32_t *rs = h + 2 * n_decode;
  int32_t *rp = rs + s->pf_total;
  for (int32_t i = 0; i < n_prefill; ++i)
    for (int32_t j = 0; j < s->pf_rows[i]; ++j) {
      rs[s->pf_off[i] + j] = s->pf_seq[i];
      rp[s->pf_off[i] + j] = s->pf_ctx[i] + j;
    }
  const size_t used = 2 * ((size_t)n_decode + (size_t)s->pf_total);
  if (used > 0 &&
      (e = hipMemcpyAsync(s->d_meta, h, sizeof(int32_t) * used, hipMemcpyHostToDevice, hs)) !=
          hipSuccess)
    return hip_fail(op, e);
  if ((e = hipEventRecord(s->meta_done[buf], hs)) != hipSuccess) return hip_fail(op, e);
  ++s->n_steps;
  return RKV_OK;
}

rkv_status rkv_serve_decode(rkv_serve *s, int32_t layer, const void *q, const void *k,
                            const void *v, int32_t dtype, void *out, int32_t out_dtype,
                            float scale, void *stream) {
  const char *op = "rkv_serve_decode";
  if (!s) return fail(RKV_ERR_INVALID_ARG, op, "serve is NULL");
  if (s->n_decode == 0) return RKV_OK;
  const int32_t nd = s->n_decode;
  rkv_append_args app{nd, s->d_meta, s->d_meta + nd, k, v, dtype, s->d.rule};
  rkv_decode_args a{};
  a.batch = nd;
  a.seq_ids = s->d_meta;
  a.q = q;
  a.q_dtype = dtype;
  a.q_len = 1;
  a.q_heads = s->d.q_heads;
  a.scale = scale;
  a.out = out;
  a.out_dtype = out_dtype;
  a.partition_tokens = 0;
  a.max_seq_len = s->decode_max_len;
  a.workspace = s->ws;
  a.workspace_bytes = s->ws_bytes;
  a.append = &app;
  return rkv_pool_decode(s->pool, layer, &a, stream);
}

rkv_status rkv_serve_prefill(rkv_serve *s, int32_t layer, const void *q, const void *k,
                             const void *v, int32_t dtype, void *out, int32_t out_dtype,
                             float scale, void *stream) {
  const char *op = "rkv_serve_prefill";
  if (!s) return fail(RKV_ERR_INVALID_ARG, op, "serve is NULL");
  if (s->pf_total == 0) return RKV_OK;
  int32_t *rs = s->d_meta + 2 * s->n_decode;
  rkv_append_args app{s->pf_total, rs, rs + s->pf_total, k, v, dtype, s->d.rule};
  if (rkv_status st = rkv_pool_append(s->pool, layer, &app, stream)) return st;
  const int32_t n = (int32_t)s->pf_seq.size();
  for (int32_t e0 = 0; e0 < n; e0 += RKV_PREFILL_MAX_SEQS) {
    rkv_prefill_args pa{};
    pa.n_seqs = std::min(RKV_PREFILL_MAX_SEQS, n - e0);
    pa.seq_ids = s->pf_seq.data() + e0;
    pa.ctx_lens = s->pf_ctx.data() + e0;
    pa.q_rows = s->pf_rows.data() + e0;
    pa.q_offsets = s->pf_off.data() + e0;
    pa.total_rows = s->pf_total;
    pa.q = q;
    pa.q_dtype = dtype;
    pa.q_heads = s->d.q_heads;
    pa.scale = scale;
    pa.out = out;
    pa.out_dtype = out_dtype;
    pa.workspace = s->pf_ws;
    pa.workspace_bytes = s->pf_ws_bytes;
    if (rkv_status st = rkv_pool_prefill(s->pool, layer, &pa, stream)) return st;
  }
  return RKV_OK;
}

rkv_status rkv_serve_truncate(rkv_serve *s, uint64_t id, int32_t len) {
  int32_t slot;
  if (rkv_status st = live_slot(s, id, "rkv_serve_truncate", &slot)) return st;
  return rkv_seq_truncate(rkv_pool_allocator(s->pool), slot, len);
}

rkv_status rkv_serve_finish(rkv_serve *s, uint64_t id) {
  int32_t slot;
  if (rkv_status st = live_slot(s, id, "rkv_serve_finish", &slot)) return st;
  if (rkv_status st = rkv_seq_free(rkv_pool_allocator(s->pool), slot)) return st;
  s->slot_of.erase(id);
  s->free_slots.push_back(slot);
  return RKV_OK;
}

rkv_status rkv_serve_seq_len(const rkv_serve *s, uint64_t id, int32_t *len) {
  int32_t slot;
  if (rkv_status st = live_slot(s, id, "rkv_serve_seq_len", &slot)) return st;
  if (!len) return fail(RKV_ERR_INVALID_ARG, "rkv_serve_seq_len", "len is NULL");
  return rkv_seq_len(rkv_pool_allocator(s->pool), slot, len);
}

rkv_status rkv_serve_seq_slot(const rkv_serve *s, uint64_t id, int32_t *slot) {
  if (!slot) return fail(RKV_ERR_INVALID_ARG, "rkv_serve_seq_slot", "slot is NULL");
  return live_slot(s, id, "rkv_serve_seq_slot", slot);
}

rkv_status rkv_serve_geometry(const rkv_serve *s, rkv_kv_geometry *out) {
  if (!s || !out) return fail(RKV_ERR_INVALID_ARG, "rkv_serve_geometry", "NULL argument");
  *out = s->g;
  return RKV_OK;
}

rkv_status rkv_serve_page_location(const rkv_serve *s, uint64_t id, int32_t ordinal,
                                   rkv_page_location *out) {
  const char *op = "rkv_serve_page_location";
  int32_t slot;
  if (rkv_status st = live_slot(s, id, op, &slot)) return st;
  if (!out) return fail(RKV_ERR_INVALID_ARG, op, "out is NULL");
  const rkv_alloc *a = rkv_pool_allocator(s->pool);
  int32_t len = 0;
  if (rkv_status st = rkv_seq_len(a, slot, &len)) return st;
  // records that hold at least one of the sequence's tokens
  const int32_t lpt = s->d.page_tokens;
  const int32_t records = (int32_t)(((int64_t)len + lpt - 1) / lpt);
  if (ordinal < 0 || ordinal >= records)
    return fail(RKV_ERR_INVALID_ARG, op, "page ordinal %d outside [0, %d) of id %llu", ordinal,
                records, (unsigned long long)id);
  std::vector<int32_t> row((size_t)s->row_pages);
  int32_t held = 0;
  if (rkv_status st = rkv_block_table_get(a, slot, row.data(), (int32_t)row.size(), &held))
    return st;
  const int32_t k = ordinal / s->per_page;
  if (k >= held)  // the allocator holds ceil(len / pool page) pages
    return fail(RKV_ERR_INVALID_ARG, op, "pool page %d of id %llu not held", k,
                (unsigned long long)id);
  out->page = row[k];
  out->offset = (uint64_t)row[k] * s->page_bytes;
  out->length = s->page_bytes;
  out->layer_stride = (uint64_t)s->g.num_pages * s->page_bytes;
  out->first_slot = (ordinal % s->per_page) * lpt;
  out->slots = lpt;
  return rkv_page_generation(a, row[k], &out->generation);
}

}  // extern "C"
