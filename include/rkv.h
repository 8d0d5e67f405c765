/*
 * rkv.h -- C ABI of the MI355X (gfx950) paged Q8_0 KV-cache hot path.
 *
 * Four device operations sit behind this boundary:
 *   - quantize-and-append of K/V rows into Q8_0 pages through block tables;
 *   - paged flash-decode (GQA, in-register dequant, online softmax,
 *     split-K partitions) and the causal multi-query verify variant;
 *   - the split-K log-sum-exp combine;
 *   - bit-exact export (gather) and import of pages in the reference's
 *     contiguous row layout.
 * plus the host-side page allocator and per-sequence block tables that
 * drive them.
 *
 * Reference interfaces replaced (paths under leoinfer/remora-lab):
 *   har/crates/har-serve/src/attention.rs:25-250   (Rust operator API)
 *   har/shaders/flash_decode_q8.comp:34-52          (kernel ABI)
 *   har/crates/har-vulkan/src/lib.rs:17-56, 236, 540-617, 1673-1777
 *                                                   (device/queue/error API)
 * The reference has no block table, page pool, split-K or verify kernel;
 * those entry points extend its API in the same style.
 *
 * Conventions (mirroring HarError / NativeRequired, har-vulkan/src/lib.rs:17-56,
 * har-runtime/src/policy.rs:18-48):
 *   - every call returns rkv_status; 0 is success;
 *   - failures never fall back to another implementation; the message of
 *     the last failure on the calling thread is rkv_last_error();
 *   - device pointers are plain pointers into device memory; streams are
 *     hipStream_t passed as void* (NULL = the legacy default stream);
 *   - calls on one pool are not thread-safe; kernels are enqueued
 *     asynchronously and device-side faults (bad block-table entries,
 *     positions beyond capacity) are reported by rkv_ctx_sync().
 */
#ifndef RKV_H
#define RKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t rkv_status;
enum {
  RKV_OK = 0,
  RKV_ERR_INVALID_ARG = -1,    /* HarError::argument (har-vulkan/src/lib.rs:547-552) */
  RKV_ERR_OUT_OF_PAGES = -2,   /* capacity exhausted (har-native-qwen3.rs:657-660) */
  RKV_ERR_BAD_BLOCK_TABLE = -3,/* page id / position outside the pool */
  RKV_ERR_UNSUPPORTED = -4,    /* head_dim, page size or dtype not built */
  RKV_ERR_DEVICE = -5,         /* HIP runtime error (HarError.result) */
  RKV_ERR_CAPACITY = -6,       /* sequence longer than its block-table row */
  RKV_ERR_REFUSED = -7         /* R4KV page refused by a fail-closed check
                                  (r4kv/src/page.rs RestoreError); the reason
                                  is an rkv_r4kv_refusal code */
};

enum { RKV_F32 = 0, RKV_BF16 = 1 };                 /* element types */
enum { RKV_Q8_CANONICAL = 0, RKV_Q8_HARSERVE = 1 }; /* quantization rules */
enum { RKV_K = 0, RKV_V = 1 };                      /* cache kinds */

/* ---- errors / version ------------------------------------------------------ */
/* Last error of the calling thread, "operation: message"; mirrors
 * HarError{operation,message} (har-vulkan/src/lib.rs:19-56). */
const char *rkv_last_error(void);
const char *rkv_version(void);

/* ---- device context ---------------------------------------------------------
 * Replaces Device::open + create_queue (har-vulkan/src/lib.rs:236, 618).
 * Holds the device index and a device-side fault word that kernels set when
 * they meet a bad block-table entry; rkv_ctx_sync() waits for `stream`,
 * reads and clears that word (ComputeTicket::wait, lib.rs:2154-2201). */
typedef struct rkv_ctx rkv_ctx;
rkv_status rkv_ctx_create(int32_t device, rkv_ctx **out);
rkv_status rkv_ctx_destroy(rkv_ctx *ctx);
rkv_status rkv_ctx_sync(rkv_ctx *ctx, void *stream);

/* ---- geometry of one layer's page pool ------------------------------------
 * kv_heads, head_dim (128 or 256; attention.rs:17 fixes 256), page_tokens
 * (16, 32, 64, 128 or 256), num_pages.  A Q8_0 row of head_dim values is
 * head_dim/32 blocks of [f16 scale][32 x int8] (attention.rs:17-21,
 * r4kv/src/quant.rs:1-12). */
typedef struct rkv_kv_geometry {
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;
  int32_t num_pages;
} rkv_kv_geometry;
rkv_status rkv_geometry_check(const rkv_kv_geometry *g);
/* Bytes of one page (all kv heads, K and V) and of the reference row
 * (head_dim/32*34; attention.rs:21, har-kv/src/geometry.rs:81-94). */
size_t rkv_page_bytes(const rkv_kv_geometry *g);
size_t rkv_row_bytes(int32_t head_dim);

/* ---- page allocator and block tables (host) --------------------------------
 * The reference has no physical page allocator (har-kv/src/page.rs:100-140
 * keeps PhysicalPageLocation = None).  Nearest
 * analogue: VramSlotTable::reserve (har-residency/src/manager.rs:110-157).
 * Pages come from a free list whose initial order is a seeded permutation
 * of [0, num_pages); freed pages return to the top of the list. */
typedef struct rkv_alloc_desc {
  int32_t num_pages;
  int32_t page_tokens;
  int32_t max_seqs;
  int32_t max_pages_per_seq;
  uint64_t free_list_seed;
} rkv_alloc_desc;
typedef struct rkv_alloc rkv_alloc;
rkv_status rkv_alloc_create(const rkv_alloc_desc *desc, rkv_alloc **out);
rkv_status rkv_alloc_destroy(rkv_alloc *a);
/* Grow `seq` to new_len tokens (new_len >= current length), taking whole
 * pages from the free list; all-or-nothing on RKV_ERR_OUT_OF_PAGES. */
rkv_status rkv_seq_reserve(rkv_alloc *a, int32_t seq, int32_t new_len);
/* Roll `seq` back to new_len tokens, returning pages past ceil(new_len /
 * page_tokens) (speculative rollback, har-execution/src/speculation.rs:55,172). */
rkv_status rkv_seq_truncate(rkv_alloc *a, int32_t seq, int32_t new_len);
rkv_status rkv_seq_free(rkv_alloc *a, int32_t seq);
/* rkv_seq_reserve / rkv_seq_truncate over n (seq, new_len) pairs (host
 * arrays), in order: one call where a serving step grows or rolls back every
 * running sequence.  Stops at the first failing pair and returns its status
 * (with that pair named in rkv_last_error); the pairs before it have taken
 * effect.  *done (may be NULL) = the number of pairs applied.  No
 * counterpart in the reference, whose scheduler records pages one sequence
 * at a time (har-serve/src/scheduler.rs:1045-1077); for callers where each
 * foreign call costs more than the allocator's work. */
rkv_status rkv_seq_reserve_n(rkv_alloc *a, int32_t n, const int32_t *seqs, const int32_t *new_lens,
                             int32_t *done);
rkv_status rkv_seq_truncate_n(rkv_alloc *a, int32_t n, const int32_t *seqs, const int32_t *new_lens,
                              int32_t *done);
rkv_status rkv_seq_len(const rkv_alloc *a, int32_t seq, int32_t *len);
rkv_status rkv_block_table_get(const rkv_alloc *a, int32_t seq, int32_t *out,
                               int32_t cap, int32_t *n);
rkv_status rkv_alloc_free_pages(const rkv_alloc *a, int32_t *n);
/* Copy the whole table [max_seqs][max_pages_per_seq] (-1 = no page) and the
 * lengths [max_seqs] to host buffers. */
rkv_status rkv_alloc_export(const rkv_alloc *a, int32_t *tables, int32_t *lens);

/* Prefix sharing.  The reference shares prefix pages logically: a lease
 * raises a page's reference_count and eviction refuses referenced pages
 * (har-kv/src/graph.rs:447-533).  Here the sharing is physical: every page
 * carries the number of block-table entries naming it and returns to the
 * free list when that drops to zero.
 *
 * rkv_seq_fork: the empty sequence `dst` takes the first
 * ceil(len/page_tokens) pages of `src` (0 <= len <= length of src) and has
 * length len.  Fork after src's rows below len are written (stream order).
 * Shared pages are read-only and always form a prefix of each table; rows
 * may be written only at positions a reserve added.  When a reserve grows a
 * sequence whose partly filled last page is shared, that sequence gets a
 * fresh page and a queued copy of the shared one (copy-on-write). */
rkv_status rkv_seq_fork(rkv_alloc *a, int32_t src, int32_t dst, int32_t len);
/* Block-table entries naming `page` (0 = free). */
rkv_status rkv_page_refs(const rkv_alloc *a, int32_t page, int32_t *refs);
/* Times `page` has left the free list (0 = never handed out): the
 * generation of a PhysicalPageLocation (har-kv/src/page.rs:100-105), which
 * tells a location recorded before the page was freed and reused from a
 * current one. */
rkv_status rkv_page_generation(const rkv_alloc *a, int32_t page, uint64_t *gen);
/* Move the queued copy-on-write copies, as (src, dst) page pairs, to
 * `pairs` (host, room for `cap` pairs); *n = number queued.  The copies are
 * independent of each other.  Run them (rkv_copy_pages) on the stream before
 * the next launch that reads or writes the pages.  A pool does this itself
 * in rkv_pool_sync_tables. */
rkv_status rkv_alloc_take_copies(rkv_alloc *a, int32_t *pairs, int32_t cap, int32_t *n);

/* ---- operation arguments -------------------------------------------------- */
typedef struct rkv_append_args {
  int32_t n_rows;
  const int32_t *seq_ids;   /* device [n_rows] */
  const int32_t *positions; /* device [n_rows], token index within the sequence */
  const void *k_src;        /* device [n_rows][kv_heads][head_dim] */
  const void *v_src;        /* device [n_rows][kv_heads][head_dim] */
  int32_t src_dtype;        /* RKV_F32 | RKV_BF16 */
  int32_t rule;             /* RKV_Q8_CANONICAL | RKV_Q8_HARSERVE */
} rkv_append_args;

typedef struct rkv_decode_args {
  int32_t batch;            /* B */
  const int32_t *seq_ids;   /* device [B] */
  const void *q;            /* device [B][q_len][q_heads][head_dim], 16-byte aligned */
  int32_t q_dtype;          /* RKV_F32 | RKV_BF16 */
  int32_t q_len;            /* 1 = decode; 2..4 = causal verify of draft rows */
  int32_t q_heads;          /* multiple of kv_heads (attention.rs:154-157) */
  float scale;              /* softmax scale on q.k (1.0 = attention.rs); any finite
                               value: negative reverses the score order, 0 gives a
                               uniform softmax over the visible positions */
  void *out;                /* device [B][q_len][q_heads][head_dim] */
  int32_t out_dtype;        /* RKV_F32 | RKV_BF16 */
  int32_t partition_tokens; /* split-K partition length: a multiple of max(32,
                               page_tokens), at most 64*page_tokens; 0 = chosen
                               per launch on the device from the batch's
                               lengths (the smallest such length, >= 256,
                               whose partitions fill one round of resident
                               workgroups) */
  int32_t max_seq_len;      /* >= every seq_lens[seq_ids[b]]; sizes the grid */
  void *workspace;          /* device scratch for the split-K partials, of
                               rkv_decode_workspace_bytes (may be NULL when one
                               partition covers every sequence) */
  size_t workspace_bytes;
  const rkv_append_args *append; /* optional (NULL = none): this step's K/V rows,
                               appended by the decode launch itself before it
                               attends over them.  n_rows = batch*q_len; row
                               b*q_len+j belongs to seq_ids[b] (else fault bit
                               4) at a position < its seq_lens entry (else
                               fault bit 2).  `pages` must then be writable.
                               Same bytes as rkv_append_q8 of the same rows,
                               one launch fewer per step (the reference step
                               quantizes, then dispatches the decode:
                               har-serve-vulkan-attn-smoke.rs:62-69, 149-161). */
  void *split_event;        /* optional hipEvent_t, recorded on the stream
                               between the decode kernel and the combine kernel
                               (per-kernel timing); NULL = none */
} rkv_decode_args;

/* Chunked prefill attention.  The reference's BatchStepModel::prefill_batch
 * (har-serve/src/adapter.rs:31-60) folds the one-token step over the chunk,
 * so query row i of entry e -- at position ctx_lens[e] + i of sequence
 * seq_ids[e] -- attends positions [0, ctx_lens[e] + i]: exactly the decode
 * of that length (attention.rs:148-165).  The chunk's own K/V rows must be
 * appended first (rkv_append_q8 / rkv_pool_append, same stream).  The entry
 * table is host memory and travels in the kernel arguments. */
#define RKV_PREFILL_MAX_SEQS 64
typedef struct rkv_prefill_args {
  int32_t n_seqs;           /* entries, 0..RKV_PREFILL_MAX_SEQS */
  const int32_t *seq_ids;   /* host [n_seqs] */
  const int32_t *ctx_lens;  /* host [n_seqs]: tokens cached before the chunk */
  const int32_t *q_rows;    /* host [n_seqs]: chunk tokens (query rows), >= 0 */
  const int32_t *q_offsets; /* host [n_seqs]: the entry's first row in q and out */
  int32_t total_rows;       /* rows of q and out */
  const void *q;            /* device [total_rows][q_heads][head_dim], 16-byte aligned */
  int32_t q_dtype;          /* RKV_F32 | RKV_BF16 */
  int32_t q_heads;          /* multiple of kv_heads, q_heads/kv_heads <= 128; a row
                               block takes floor(128/(q_heads/kv_heads)) chunk
                               tokens of all the kv head's q heads */
  float scale;              /* softmax scale on q.k (any finite value, as in the decode) */
  void *out;                /* device [total_rows][q_heads][head_dim] */
  int32_t out_dtype;        /* RKV_F32 | RKV_BF16 */
  /* Split-K over the causal range (a row block's range in segments, merged
   * by the decode's log-sum-exp combine).  0: split when the launch has
   * fewer row blocks than the device has workgroup slots and `workspace`
   * holds the partials; > 0: segments of this many tokens (rounded up to a
   * multiple of max(32, page_tokens), and to at most 64 segments); < 0:
   * never split. */
  int32_t segment_tokens;
  void *workspace;          /* device, 256-byte aligned, or NULL (no split) */
  size_t workspace_bytes;
} rkv_prefill_args;

/* ---- kernel-level entry points (explicit device pointers) -----------------
 * pages: one layer's pool (num_pages * rkv_page_bytes).  block_tables:
 * device int32 [n_seqs][bt_stride]; seq_lens: device int32 [n_seqs]. */

/* Quantize-and-append.  Replaces q8_0_quantize (attention.rs:25-42) /
 * r4kv::quant::encode (quant.rs:138-170) followed by the host copy into the
 * shader's K/V buffers (har-serve-vulkan-attn-smoke.rs:62-69, 95-127). */
rkv_status rkv_append_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         int32_t n_seqs, const rkv_append_args *args, void *stream);

/* Paged flash-decode (+ causal verify when q_len > 1).  Replaces
 * flash_decode_reference / flash_decode_online (attention.rs:148-215) and
 * the flash_decode_q8.comp dispatch (har-serve-vulkan-attn-smoke.rs:149-161).
 * With more than one partition per sequence the partials go to `workspace`
 * and a second kernel merges them (rkv_splitk_combine's algebra). */
rkv_status rkv_decode_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_lens, int32_t n_seqs,
                         const rkv_decode_args *args, void *stream);
/* rkv_decode_q8 that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  args->workspace and workspace_bytes are
 * ignored: the split-K partials go to a static device array of
 * RKV_DECODE_SCRATCH_BYTES that the library holds on each device it runs on
 * until the process ends.  A launch whose partials need more (see
 * rkv_decode_workspace_bytes) is refused with RKV_ERR_INVALID_ARG.  Every
 * call on one device shares that array, and a call leaves its contents
 * behind (no call needs them cleared): calls that overlap on one device --
 * queued on different streams, or from several threads -- race and give
 * wrong results; calls queued on one stream are ordered. */
#define RKV_DECODE_SCRATCH_BYTES ((size_t)64 << 20)
rkv_status rkv_decode_q8_noalloc(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                                 const int32_t *block_tables, int32_t bt_stride,
                                 const int32_t *seq_lens, int32_t n_seqs,
                                 const rkv_decode_args *args, void *stream);
/* Workspace bytes rkv_decode_q8 needs for these arguments (0 if none); it
 * depends on batch, q_len, q_heads, max_seq_len and partition_tokens, and
 * needs no initialisation. */
size_t rkv_decode_workspace_bytes(const rkv_kv_geometry *g, const rkv_decode_args *args);
/* The explicit partition length of these arguments, or 0 when the device
 * chooses it per launch. */
int32_t rkv_decode_partition_tokens(const rkv_kv_geometry *g, const rkv_decode_args *args);

/* Split-K stage alone (for parity tests): writes per-partition partials
 * (m, l) into ml [B][q_len*q_heads][n_parts][2] and o into
 * o [B][q_len*q_heads][n_parts][head_dim].  m is the running max of
 * scale*log2(e)*q.k (base-2 domain); l and o are unnormalised sums of
 * 2^(s - m) and 2^(s - m) * v.  n_parts = ceil(max_seq_len/partition_tokens);
 * partition_tokens must be explicit (> 0). */
rkv_status rkv_decode_q8_partials(rkv_ctx *ctx, const rkv_kv_geometry *g,
                                  const void *pages, const int32_t *block_tables,
                                  int32_t bt_stride, const int32_t *seq_lens,
                                  int32_t n_seqs, const rkv_decode_args *args,
                                  float *ml, float *o, void *stream);
/* Log-sum-exp combine of the partials above (attention.rs:205-212 algebra):
 * M = max m_p, L = sum l_p 2^(m_p-M), out = sum o_p 2^(m_p-M) / L; L == 0
 * gives zeros (flash_decode_q8.comp:144-148).  Only the first
 * ceil(seq_lens[seq_ids[b]]/partition_tokens) partitions of entry b are read. */
rkv_status rkv_splitk_combine(rkv_ctx *ctx, const float *ml, const float *o,
                              int32_t batch, int32_t rows, int32_t n_parts,
                              int32_t head_dim, const int32_t *seq_ids,
                              const int32_t *seq_lens, int32_t n_seqs,
                              int32_t partition_tokens, void *out, int32_t out_dtype,
                              void *stream);

/* Chunked prefill attention over the pages (see rkv_prefill_args); rows of
 * entries whose range exceeds the block-table row (or 4096 pages) are
 * refused with RKV_ERR_UNSUPPORTED.  An explicit segment_tokens whose
 * partials do not fit workspace_bytes is refused with RKV_ERR_INVALID_ARG. */
rkv_status rkv_prefill_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                          const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                          const rkv_prefill_args *args, void *stream);
/* Workspace bytes the split of these arguments uses: with segment_tokens > 0
 * that split, with 0 the split chosen when the workspace is large enough
 * (0 when none is); with a bf16 query (q_dtype) also room for every tile of
 * the entries' causal ranges widened once (head_dim * 132 bytes, padded to
 * whole KiB, per 32 tokens and kv head), which the prefill then copies
 * instead of widening it in each of the row blocks that read it.  A smaller
 * workspace still works: the tiles are widened per row block.  The device
 * pointers in args are not read. */
size_t rkv_prefill_workspace_bytes(const rkv_kv_geometry *g, const rkv_prefill_args *args);

/* Export seq's K or V cache in the reference contiguous layout
 * [kv_heads][len][head_dim/32*34] bytes (what flash_decode_reference reads,
 * attention.rs:144-147; row_to_words is a reinterpretation, :115-120). */
rkv_status rkv_gather_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                         const int32_t *block_table, int32_t len, int32_t kind,
                         uint8_t *out, void *stream);
/* Inverse of rkv_gather_q8: write reference rows into the pages. */
rkv_status rkv_import_q8(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                         const int32_t *block_table, int32_t len, int32_t kind,
                         const uint8_t *rows, void *stream);

/* Copy-on-write page copies: page dst := page src for each (src, dst) pair
 * of `pairs` (device, n_pairs pairs), in each of `layers` page arrays
 * starting layer_stride_bytes apart at `pages`.  No reference counterpart:
 * the reference never copies a KV page (har-kv/src/graph.rs:447-533 shares
 * them only logically).  Pairs naming pages outside [0, num_pages) are
 * skipped. */
rkv_status rkv_copy_pages(rkv_ctx *ctx, const rkv_kv_geometry *g, void *pages,
                          int64_t layer_stride_bytes, int32_t layers,
                          const int32_t *pairs, int32_t n_pairs, void *stream);

/* Batch f32 -> binary16 bits with the device encoder of one rule
 * (RKV_Q8_CANONICAL = r4kv/src/f16.rs:27-86, RKV_Q8_HARSERVE =
 * attention.rs:45-76); used to pin the scale encoder over many inputs. */
rkv_status rkv_f32_to_f16(rkv_ctx *ctx, const float *in, uint16_t *out, int64_t n,
                          int32_t rule, void *stream);

/* Drop-in for the flash_decode_q8.comp ABI (:36-52): contiguous K/V words
 * [kv_heads][seq_len][head_dim/32*34/4], query f32 [q_heads][head_dim],
 * out f32 [q_heads][head_dim], no softmax scale, l == 0 -> zeros.
 * `scratch` must hold rkv_flash_decode_scratch_bytes(); the rows are
 * imported into a scratch pool and decoded there. */
typedef struct rkv_flash_decode_params {
  int32_t q_heads;
  int32_t kv_heads;
  int32_t seq_len;
  int32_t chunk;    /* accepted for API parity (attention.rs:128-130) */
  int32_t head_dim;
} rkv_flash_decode_params;
size_t rkv_flash_decode_scratch_bytes(const rkv_flash_decode_params *p);
rkv_status rkv_flash_decode_q8(rkv_ctx *ctx, const rkv_flash_decode_params *p,
                               const uint32_t *k_words, const uint32_t *v_words,
                               const float *query, float *out, void *scratch,
                               void *stream);

/* ---- pool: device pages for `layers` layers + allocator + device tables ----
 * The operator-level API a serving adapter (BatchStepModel, adapter.rs:28-72)
 * would hold per model.  Block-table edits made through the allocator are
 * uploaded by rkv_pool_sync_tables() before the next launch.
 * A pool's calls that queue device work (sync, append, decode, prefill,
 * gather, spill, restore) run in call order, whatever streams they are
 * queued on: a call on another stream than the pool's previous call first
 * makes its stream wait, on the device, for the work queued so far on that
 * previous stream (which must still exist then, unless it was released with
 * rkv_pool_release_stream).  Calls on one stream add
 * nothing. */
/* Where a pool's pages live.  RKV_PAGES_HOST puts them in pinned host
 * memory mapped for the device (the reference's host-KV tier,
 * research/host-kv/README.md:1-24): every kernel reads and writes them
 * over the host link instead of HBM, and each K/V tile a kernel stages in
 * LDS still serves every query row of its kv head (the GQA group times
 * q_len, or a prefill block's 128 rows), so the rows served per fetched
 * byte multiply the link's bandwidth. */
#define RKV_PAGES_DEVICE 0
#define RKV_PAGES_HOST 1
typedef struct rkv_pool_desc {
  int32_t layers;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;
  int32_t num_pages;
  int32_t max_seqs;
  int32_t max_pages_per_seq;
  uint64_t free_list_seed;
  int32_t page_memory;  /* RKV_PAGES_DEVICE (0) | RKV_PAGES_HOST */
} rkv_pool_desc;
typedef struct rkv_pool rkv_pool;
rkv_status rkv_pool_create(rkv_ctx *ctx, const rkv_pool_desc *desc, rkv_pool **out);
rkv_status rkv_pool_destroy(rkv_pool *pool);
/* The pool forgets `stream` if its previous call was queued there: the work
 * queued on it so far is marked (an event recorded now), and the next call,
 * on any stream, waits for that mark instead of touching `stream`.  Call it
 * before destroying a stream the pool's last call used; other calls need
 * nothing.  No reference counterpart (Vulkan queues outlive their
 * submissions, har-vulkan/src/lib.rs:1673-1777). */
rkv_status rkv_pool_release_stream(rkv_pool *pool, void *stream);
rkv_alloc *rkv_pool_allocator(rkv_pool *pool);
/* Upload the allocator's changed block-table rows and all lengths and run
 * its queued copy-on-write page copies (all layers), ordered on `stream`:
 * launches enqueued on `stream` afterwards see the new tables and copied
 * pages, earlier ones the old.  One or two small kernels that read the
 * changes from a pinned staging buffer in place (no copy and no event in
 * the stream); the host waits only if the staging buffer of the call before
 * last has not been read yet.  Refused (RKV_ERR_INVALID_ARG) on a stream
 * that is capturing a graph: the upload carries the allocator's state at
 * the call, which a replay would repeat. */
rkv_status rkv_pool_sync_tables(rkv_pool *pool, void *stream);
/* Device pointers owned by the pool (for a host-memory pool, the device
 * mapping of its pinned pages). */
void *rkv_pool_layer_pages(rkv_pool *pool, int32_t layer);
const int32_t *rkv_pool_block_tables(rkv_pool *pool); /* [max_seqs][max_pages_per_seq] */
const int32_t *rkv_pool_seq_lens(rkv_pool *pool);     /* [max_seqs] */
rkv_status rkv_pool_append(rkv_pool *pool, int32_t layer, const rkv_append_args *args,
                           void *stream);
rkv_status rkv_pool_decode(rkv_pool *pool, int32_t layer, const rkv_decode_args *args,
                           void *stream);
/* rkv_prefill_q8 on a layer; also checks ctx_lens[e] + q_rows[e] against the
 * allocator's length of each sequence. */
rkv_status rkv_pool_prefill(rkv_pool *pool, int32_t layer, const rkv_prefill_args *args,
                            void *stream);
/* rkv_prefill_workspace_bytes for rkv_pool_prefill on this pool: a pool in
 * host memory widens each tile in the row blocks that read it (its pages
 * cross the host link once per row block either way), so it needs only the
 * split partials, planned for its dispatch order. */
size_t rkv_pool_prefill_workspace_bytes(const rkv_pool *pool, const rkv_prefill_args *args);
rkv_status rkv_pool_gather(rkv_pool *pool, int32_t layer, int32_t seq, int32_t kind,
                           uint8_t *out, void *stream);

/* ---- R4KV pages: off-HBM tier spill / restore ------------------------------
 * The container of har/crates/r4kv/src/page.rs: a 96-byte little-endian
 * header with a trailing CRC32C of its first 92 bytes (PageHeader::to_bytes,
 * :100-126), then the payload body and a CRC32C of the body (pack_page,
 * :213-224).  CRC32C is crc32c.rs:1-31 (reflected 0x82f63b78, init and
 * final xor 0xffffffff).  Restores fail closed (check_restore, :151-210). */
#define RKV_R4KV_HEADER_BYTES 96
#define RKV_R4KV_MAGIC 0x52344B56u /* "R4KV", page.rs:11 */
#define RKV_R4KV_VERSION 1
enum { RKV_FMT_F16 = 0, RKV_FMT_Q8 = 1, RKV_FMT_Q6 = 2, RKV_FMT_Q4 = 3, RKV_FMT_Q3 = 4 }; /* lib.rs:23-31 */
typedef struct rkv_r4kv_header {  /* PageHeader, page.rs:15-30 */
  uint64_t prefix_digest;
  uint32_t token_start;
  uint32_t token_count;
  uint32_t pos_start;
  uint16_t layer_lo;
  uint16_t layer_hi;   /* inclusive */
  uint8_t k_fmt;
  uint8_t v_fmt;
  uint32_t epoch;
  uint32_t generation;
  uint64_t payload_len; /* body bytes, without the trailing CRC */
  uint32_t sketch_offset;
  uint16_t flags;       /* bit0 has_sketch, bit1 rotated_k */
} rkv_r4kv_header;
/* RestoreError variants (page.rs:63-76) */
enum {
  RKV_R4KV_ACCEPTED = 0,
  RKV_R4KV_BAD_MAGIC = 1,
  RKV_R4KV_BAD_VERSION = 2,
  RKV_R4KV_HEADER_CHECKSUM = 3,
  RKV_R4KV_PAYLOAD_CHECKSUM = 4,
  RKV_R4KV_LENGTH = 5,
  RKV_R4KV_PREFIX = 6,
  RKV_R4KV_TOKEN_RANGE = 7,
  RKV_R4KV_POS = 8,
  RKV_R4KV_LAYER_RANGE = 9,
  RKV_R4KV_FORMAT = 10,
  RKV_R4KV_GENERATION = 11
};
/* RestoreExpectation (page.rs:32-45); k_fmt / v_fmt < 0 = any; the
 * generation predicate is generation_min <= generation <= generation_max
 * when check_generation is non-zero. */
typedef struct rkv_r4kv_expect {
  uint64_t prefix_digest;
  uint32_t token_start;
  uint32_t pos_start;
  uint16_t layer_lo;
  uint16_t layer_hi;
  int32_t k_fmt;
  int32_t v_fmt;
  int32_t check_generation;
  uint32_t generation_min;
  uint32_t generation_max;
} rkv_r4kv_expect;

/* Host CRC32C (crc32c.rs:23-31). */
uint32_t rkv_crc32c_host(const uint8_t *data, size_t n);
/* CRC32C of n device bytes (16-byte aligned) into *out (device word),
 * stream-ordered.  No reference counterpart on the device: crc32c.rs is
 * CPU-only. */
rkv_status rkv_crc32c(rkv_ctx *ctx, const void *data, uint64_t n, uint32_t *out, void *stream);
/* PageHeader::to_bytes / from_bytes (page.rs:100-149).  decode sets
 * *refusal (BAD_MAGIC, BAD_VERSION, HEADER_CHECKSUM, FORMAT) and returns
 * RKV_ERR_REFUSED when the bytes are refused. */
rkv_status rkv_r4kv_header_encode(const rkv_r4kv_header *h, uint8_t out[RKV_R4KV_HEADER_BYTES]);
rkv_status rkv_r4kv_header_decode(const uint8_t in[RKV_R4KV_HEADER_BYTES], rkv_r4kv_header *h,
                                  int32_t *refusal);
/* PageHeader::check_restore (page.rs:151-210), same order of checks. */
rkv_status rkv_r4kv_check_restore(const rkv_r4kv_header *h, const rkv_r4kv_expect *e,
                                  uint64_t payload_body_len, int32_t *refusal);
/* unpack_page (page.rs:227-260) on host bytes: header, body length and the
 * payload CRC.  On success *body points into `page`. */
rkv_status rkv_r4kv_unpack_host(const uint8_t *page, size_t len, rkv_r4kv_header *h,
                                const uint8_t **body, int32_t *refusal);

/* Page size of a spill: 96 + layers*2*kv_heads*token_count*(head_dim/32*34) + 4. */
size_t rkv_r4kv_page_bytes(const rkv_pool *pool, int32_t token_count, int32_t layer_lo,
                           int32_t layer_hi);
/* Spill (the T1 mirror of r4kv/src/tier.rs): rows of tokens [token_start,
 * token_start+token_count) of `seq`, layers [layer_lo, layer_hi], become one
 * R4KV page: header from `identity` (prefix_digest, pos_start, epoch,
 * generation, flags bit1; the rest is set here: k_fmt = v_fmt = Q8,
 * payload_len, no sketch), body = per layer, K then V, per kv head, the
 * reference rows (attention.rs:144-147 layout), then the body's CRC32C
 * computed on the device.  The page is assembled in `staging` (device,
 * >= rkv_r4kv_page_bytes) and then copied to `dst` (host or device, may be
 * `staging` itself), all ordered on `stream`. */
rkv_status rkv_pool_spill(rkv_pool *pool, int32_t seq, int32_t token_start, int32_t token_count,
                          int32_t layer_lo, int32_t layer_hi, const rkv_r4kv_header *identity,
                          void *staging, size_t staging_bytes, void *dst, size_t dst_bytes,
                          void *stream);
/* Restore (promotion): `page` (host bytes) is unpacked and gated on the
 * host -- header, length, identity against `expect` -- before any device
 * work; its body is copied to `staging` (device, >= the page size) and its
 * CRC32C checked on the device (the call waits for that one word); only
 * then are the rows written into the pages of `seq`, at the header's token
 * range (which must lie within the sequence's reserved length), for the
 * header's layers.  A refused page returns RKV_ERR_REFUSED with *refusal
 * set and writes nothing. */
rkv_status rkv_pool_restore(rkv_pool *pool, int32_t seq, const uint8_t *page, size_t page_bytes,
                            const rkv_r4kv_expect *expect, void *staging, size_t staging_bytes,
                            int32_t *refusal, void *stream);

/* ---- serving adapter ------------------------------------------------------
 * The KV side of a BatchStepModel backend (har-serve/src/adapter.rs:28-72)
 * as ServeScheduler::step drives it (har-serve/src/scheduler.rs:603-960):
 * the scheduler names sequences by SequenceId (scheduler.rs:122) and each
 * step runs prefill chunks (prefill_batch) and one-token decode rows
 * (batch_step) as separate model calls.  The adapter owns one pool (all
 * layers), maps live ids to pool sequences, grows them by the tokens a step
 * consumes, and runs each layer's attention for the step's rows.  The model
 * code around attention (projections, sampling) stays the caller's.
 *
 * Per step, on one stream:
 *   rkv_serve_begin_step(prefill entries, decode entries)
 *   for each layer: rkv_serve_prefill(...) and/or rkv_serve_decode(...)
 *   (then rkv_serve_truncate / rkv_serve_finish as the step's outcome says;
 *   they take effect at the next rkv_serve_begin_step).
 * Steps may change streams: the pool orders its calls whatever streams they
 * use (rkv_pool_create), and the step's row layout is uploaded behind that
 * ordering. */
typedef struct rkv_serve_desc {
  int32_t layers;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;        /* the scheduler's page_size (scheduler.rs:1045-1052;
                                 ServeConfig::default() has 8, :103-120): a power
                                 of two, 1..256.  The pool's pages hold whole
                                 scheduler pages: page_tokens tokens when that
                                 is 16 or more, else 32 (rkv_serve_geometry) */
  int32_t num_pages;          /* scheduler pages the pool holds */
  int32_t max_seqs;           /* live sequences at once */
  int32_t max_pages_per_seq;  /* scheduler pages of one sequence */
  int32_t q_heads;            /* multiple of kv_heads */
  int32_t max_decode;         /* decode rows per step, 1..max_seqs */
  int32_t max_prefill_rows;   /* prefill query rows per step, >= 0 */
  int32_t rule;               /* RKV_Q8_CANONICAL | RKV_Q8_HARSERVE */
  uint64_t free_list_seed;
  int32_t page_memory;        /* RKV_PAGES_DEVICE (0) | RKV_PAGES_HOST */
} rkv_serve_desc;

/* One sequence in one step. */
typedef struct rkv_serve_entry {
  uint64_t id;       /* SequenceId */
  int32_t tokens;    /* tokens consumed this step: 1 for a decode row, the
                        chunk length (>= 1) for a prefill entry */
  int32_t fork_len;  /* read at an id's first step only: > 0 starts it from the
                        first fork_len tokens of live sequence `parent`, whose
                        pages it shares (prefix reuse, copy-on-write) */
  uint64_t parent;
} rkv_serve_entry;

/* Where one KV page record lives: the ExactHotQ8 representation's
 * PhysicalPageLocation (har-kv/src/page.rs:100-115) for scheduler page
 * `ordinal` of a sequence, i.e. tokens [ordinal*page_tokens,
 * (ordinal+1)*page_tokens), all layers and kv heads (the KVPageId of
 * scheduler.rs:1056-1066).  The record is slots [first_slot, first_slot +
 * slots) of pool page `page`, whose bytes (all its slots) are at offset +
 * l*layer_stride for layer l in the pool's page memory
 * (rkv_pool_layer_pages(pool, 0)); a page's slots are not contiguous bytes
 * (K rows, V columns and scales are separate runs), so a record smaller
 * than its pool page names the page and its slots. */
typedef struct rkv_page_location {
  int32_t page;           /* pool page id */
  uint64_t offset;        /* bytes from the start of a layer's page array */
  uint64_t length;        /* page bytes of one layer (rkv_page_bytes) */
  uint64_t layer_stride;  /* bytes between layers' page arrays */
  uint64_t generation;    /* rkv_page_generation of the page */
  int32_t first_slot;     /* the record's first token slot in the page */
  int32_t slots;          /* the record's tokens (page_tokens of the desc) */
} rkv_page_location;

typedef struct rkv_serve rkv_serve;
rkv_status rkv_serve_create(rkv_ctx *ctx, const rkv_serve_desc *desc, rkv_serve **out);
rkv_status rkv_serve_destroy(rkv_serve *s);
rkv_pool *rkv_serve_pool(rkv_serve *s);
/* The pool's geometry: kv heads, head_dim, tokens of a pool page (see
 * rkv_serve_desc.page_tokens) and pool pages per layer. */
rkv_status rkv_serve_geometry(const rkv_serve *s, rkv_kv_geometry *out);
/* Admit ids seen for the first time (forking those with fork_len > 0), grow
 * every entry's sequence by its tokens and upload the tables and the step's
 * row layout, ordered on `stream`.  An id appears at most once per step;
 * decode entries have tokens == 1; prefill rows total <= max_prefill_rows.
 * All-or-nothing: on RKV_ERR_OUT_OF_PAGES (or any refusal) no sequence is
 * changed or admitted. */
rkv_status rkv_serve_begin_step(rkv_serve *s, const rkv_serve_entry *prefill, int32_t n_prefill,
                                const rkv_serve_entry *decode, int32_t n_decode, void *stream);
/* One layer's attention for the step's decode rows (batch_step): q
 * [n_decode][q_heads][head_dim], k and v [n_decode][kv_heads][head_dim] (the
 * rows' own K/V, appended inside the decode launch), out
 * [n_decode][q_heads][head_dim]; row b is decode entry b. */
rkv_status rkv_serve_decode(rkv_serve *s, int32_t layer, const void *q, const void *k,
                            const void *v, int32_t dtype, void *out, int32_t out_dtype,
                            float scale, void *stream);
/* One layer's attention for the step's prefill chunks (prefill_batch): rows
 * in entry order, entry e's chunk contiguous; q [rows][q_heads][head_dim],
 * k and v [rows][kv_heads][head_dim], out [rows][q_heads][head_dim].  Row i
 * of a chunk that follows ctx cached tokens attends positions [0, ctx+i]. */
rkv_status rkv_serve_prefill(rkv_serve *s, int32_t layer, const void *q, const void *k,
                             const void *v, int32_t dtype, void *out, int32_t out_dtype,
                             float scale, void *stream);
/* Speculative rollback of a live id to len tokens (rkv_seq_truncate). */
rkv_status rkv_serve_truncate(rkv_serve *s, uint64_t id, int32_t len);
/* The id finished: its pages (those no other sequence shares) return to the
 * free list and its pool sequence is reused. */
rkv_status rkv_serve_finish(rkv_serve *s, uint64_t id);
rkv_status rkv_serve_seq_len(const rkv_serve *s, uint64_t id, int32_t *len);
/* The pool sequence of a live id, for pool-level calls on it: rkv_pool_spill
 * / rkv_pool_restore (off-HBM tier), rkv_pool_gather, rkv_pool_append. */
rkv_status rkv_serve_seq_slot(const rkv_serve *s, uint64_t id, int32_t *slot);
rkv_status rkv_serve_page_location(const rkv_serve *s, uint64_t id, int32_t ordinal,
                                   rkv_page_location *out);

/* ---- measurement --------------------------------------------------------
 * HBM streaming-read ceiling.  No counterpart in the reference: it gives the
 * practical read rate that the decode's bandwidth is set against, measured
 * in the same run.  Reads the `bytes` device bytes at `data` once (16-byte
 * aligned, bytes a multiple of 16) with `blocks` workgroups:
 *   mode 0: 1024-thread workgroups, each wave reading 16 KiB contiguous per
 *           round with 16-byte vector loads, the grid's waves taking the
 *           rounds in turn; *out (device word) receives the xor of every
 *           32-bit word read;
 *   mode 1: one-wave workgroups, workgroup b streaming the b-th of `blocks`
 *           equal contiguous chunks with 1 KiB LDS-DMA copies (the decode's
 *           order and stage copy), 16 KiB in flight per wave; bytes must be
 *           a multiple of blocks * RKV_STREAM_DMA_UNIT; `out` is not written.
 * Both modes read with the nontemporal cache policy, as the decode does.
 * blocks in [1, 2^20].  Stream-ordered. */
#define RKV_STREAM_DMA_UNIT 16384
rkv_status rkv_stream_read(rkv_ctx *ctx, const void *data, uint64_t bytes, int32_t mode,
                           int32_t blocks, uint32_t *out, void *stream);
/* The decode's tile order over a pool's pages.  No counterpart in the
 * reference: it gives the practical read rate of the decode's own access
 * pattern, with the pages wherever the block tables put them, in the same
 * run.  For n_seqs block-table rows ([n_seqs][bt_stride]) of seq_tokens
 * tokens each and every kv head, partitions of partition_tokens tokens are
 * read by one one-wave workgroup each, 32-token tile after tile: its K
 * codes, V codes and both scale runs, with the decode's nontemporal 1 KiB
 * LDS-DMA copies and one tile in flight.  Nothing is written.  head_dim 128
 * or 256, page_tokens >= 32; seq_tokens a multiple of 32; partition_tokens a
 * multiple of 32 (partitions start on 32-token tiles, inside a page when it
 * is not a whole number of pages, as the decode's do) whose every partition
 * spans at most 64 pages; the rows must hold
 * ceil(seq_tokens / page_tokens) pages (a page id outside the pool reads
 * page 0).  Reads n_seqs * kv_heads * seq_tokens * head_dim * 17/8 bytes.
 * Stream-ordered. */
rkv_status rkv_stream_read_tiles(rkv_ctx *ctx, const rkv_kv_geometry *g, const void *pages,
                                 const int32_t *block_tables, int32_t bt_stride, int32_t n_seqs,
                                 int32_t seq_tokens, int32_t partition_tokens, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* RKV_H */
