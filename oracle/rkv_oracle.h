/*
 * rkv_oracle.h -- CPU restatement of the reference's paged-Q8 KV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * HIP kernels in remora-lab_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only as the checker or
 * as the timed CPU baseline -- never as the product path.
 *
 * Every function restates one reference function (path:line under the
 * reference tree leoinfer/remora-lab) in plain C99, compiled with
 * -O2 -ffp-contract=off and no fast-math so that f32 arithmetic happens in
 * the same order and with the same rounding as the Rust code (Rust never
 * contracts a*b+c into an FMA).  Functions the reference does not have
 * (paged layout, block tables, split-K partials, causal verify) are built
 * on top of the restated functions and say which invariant pins them.
 */
#ifndef RKV_ORACLE_H
#define RKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- generators --------------------------------------------------------- */
/* tools/repro-harness/src/main.rs:81-88 */
uint64_t rko_splitmix64(uint64_t x);
/* tools/repro-harness/src/main.rs:90-95 */
float rko_seeded_float(uint64_t index);
/* har/crates/har-serve/src/q4k.rs:109-120 */
void rko_lcg_values(float *out, size_t count, uint64_t seed);
/* Not in the reference: N(0,1) f32 from splitmix64 counters + Box-Muller in
 * f64 (the synthetic-input generator of the benchmark configs). */
void rko_normal_f32(float *out, size_t count, uint64_t seed);
/* f32 -> bf16 round-to-nearest-even (NaN kept quiet); bf16 -> f32 exact. */
uint16_t rko_f32_to_bf16(float v);
float rko_bf16_to_f32(uint16_t b);

/* ---- binary16 ------------------------------------------------------------ */
/* har/crates/r4kv/src/f16.rs:4-25 */
float rko_f16_to_f32(uint16_t bits);
/* har/crates/har-serve/src/q4k.rs:22-50 (byte-pair form used by attention.rs) */
float rko_f16_to_f32_harserve(uint8_t b0, uint8_t b1);
/* har/crates/r4kv/src/f16.rs:27-86 (RTNE, carries, subnormals) */
uint16_t rko_f32_to_f16(float v);
/* har/crates/har-serve/src/attention.rs:45-76 (f64 path, mantissa carry dropped) */
uint16_t rko_f32_to_f16_harserve(float v);

/* ---- Q8_0 codecs ---------------------------------------------------------- */
#define RKO_Q8_GROUP 32
#define RKO_Q8_GROUP_BYTES 34
/* har/crates/r4kv/src/quant.rs:45-90 + 138-170 (Fmt::Q8): canonical rule.
 * n must be a multiple of 32; dst gets n/32*34 bytes.  Returns worst group
 * max-abs error (quant.rs:61-69). */
float rko_q8_encode(const float *src, size_t n, uint8_t *dst);
/* har/crates/har-serve/src/attention.rs:25-42: the har-serve rule
 * (true division v/d, attention.rs f16 encoder). */
void rko_q8_quantize_harserve(const float *src, size_t n, uint8_t *dst);
/* har/crates/r4kv/src/quant.rs:173-225 (Fmt::Q8) */
void rko_q8_decode(const uint8_t *src, size_t n, float *dst);
/* har/crates/har-serve/src/attention.rs:79-90 generalised to n values */
void rko_q8_dequant_row(const uint8_t *row, size_t n, float *dst);
/* har/crates/r4kv/src/quant.rs:138-170 + 173-225 (Fmt::F16) */
void rko_f16_encode(const float *src, size_t n, uint16_t *dst);
void rko_f16_decode(const uint16_t *src, size_t n, float *dst);

/* har/crates/r4kv/src/quant.rs:19-33, 228-245: fmt 0 = F16, 1 = Q8 */
typedef struct rko_group_stats {
  float max_abs_err;
  double sum_sq_err;
  double sum_sq_ref;
} rko_group_stats;
void rko_roundtrip_stats(const float *src, size_t n, int fmt, float *decoded,
                         rko_group_stats *st);
float rko_rel_rms(const rko_group_stats *st);
/* tools/repro-harness/src/main.rs:192-204 */
double rko_normalized_kl(const float *ref, const float *cand, size_t n);

/* ---- reference (contiguous) flash decode, head_dim generalised ------------ */
/* har/crates/har-serve/src/attention.rs:123-141 */
typedef struct rko_fd_params {
  int32_t q_heads;
  int32_t kv_heads;
  int32_t seq_len;
  int32_t chunk;
  int32_t head_dim; /* the reference fixes 256 (attention.rs:17) */
} rko_fd_params;
/* attention.rs:98-112 */
float rko_q8_kv_value(const uint32_t *words, size_t row_word, size_t index);
/* attention.rs:115-120 */
void rko_row_to_words(const uint8_t *row, size_t nbytes, uint32_t *words);
/* attention.rs:169-215 */
void rko_flash_decode_online(const rko_fd_params *p, const uint32_t *k_words,
                             const uint32_t *v_words, const float *q, int32_t kvh,
                             float *m, float *l, float *o);
/* attention.rs:148-165 */
void rko_flash_decode_reference(const rko_fd_params *p, const uint32_t *k_words,
                                const uint32_t *v_words, const float *query,
                                float *out);
/* rko_flash_decode_reference over n sequences on `threads` OpenMP threads
 * (by sequence and q head); for timing the CPU path on all host cores */
void rko_flash_decode_reference_many(const rko_fd_params *p, int32_t n,
                                     const uint32_t *const *k_words,
                                     const uint32_t *const *v_words, const float *queries,
                                     float *out, int32_t threads);
/* attention.rs:219-250 */
void rko_flash_decode_bruteforce(const rko_fd_params *p, const uint32_t *k_words,
                                 const uint32_t *v_words, const float *q,
                                 int32_t kvh, float *out);
/* Per-chunk partials of attention.rs:182-204 before the combine at :205-212:
 * chunk c of `chunk` positions yields (cm[c], lc[c], oc[c][head_dim]).
 * Returns the number of chunks. */
int32_t rko_flash_decode_partials(const rko_fd_params *p, const uint32_t *k_words,
                                  const uint32_t *v_words, const float *q,
                                  int32_t kvh, float *cm, float *lc, float *oc);
/* The combine of attention.rs:205-212 applied over n partials in order,
 * starting from (m,l,o) = (-inf, 0, 0); writes normalized o/l. */
void rko_lse_combine(int32_t n, int32_t head_dim, const float *cm, const float *lc,
                     const float *oc, float *out, float *m_out, float *l_out);
/* f64 canonical softmax attention over dequantized rows (not in the
 * reference; the truth used to bound both oracle and kernel error). */
void rko_attention_f64(int32_t seq_len, int32_t head_dim, const uint32_t *k_words,
                       const uint32_t *v_words, const float *q, double *out);

/* ---- paged layout (this build's HBM layout, restated for the checker) ----- */
typedef struct rko_layout {
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;
  int32_t num_pages;
} rko_layout;
size_t rko_region_bytes(const rko_layout *L);
size_t rko_page_bytes(const rko_layout *L);
/* byte offset of code (slot, dim) inside a K (kind 0) or V (kind 1) region */
size_t rko_code_offset(const rko_layout *L, int kind, int32_t slot, int32_t dim);
/* byte offset of the f16 scale of (slot, block) inside a region */
size_t rko_scale_offset(const rko_layout *L, int32_t slot, int32_t block);
/* Quantize rows [n_rows][kv_heads][head_dim] of K and V (f32 values) and
 * scatter them through block tables into `pages` (one layer).
 * rule 0 = canonical (r4kv), 1 = har-serve.  Returns 0, or -3 for a bad
 * block-table entry / position. */
int32_t rko_paged_append(const rko_layout *L, uint8_t *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_ids, const int32_t *positions,
                         int32_t n_rows, const float *k_src, const float *v_src,
                         int rule);
/* Export seq's K (kind 0) or V (kind 1) rows in the reference contiguous
 * layout [kv_head][len][head_dim/32*34] (what attention.rs:144-147 reads). */
int32_t rko_paged_gather(const rko_layout *L, const uint8_t *pages,
                         const int32_t *block_table, int32_t len, int kind,
                         uint8_t *out);
/* Paged decode through the reference loop: for batch entry b, rows
 * j < q_len, q head h: gather rows, prescale q by `scale` in f32, run
 * attention.rs:169-215 over the first len_b - q_len + j + 1 positions
 * (causal; q_len == 1 is plain decode) with chunk = `chunk`, out = o/l.
 * q: [B][q_len][q_heads][head_dim] f32; out same shape. */
int32_t rko_paged_decode(const rko_layout *L, const uint8_t *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_lens, const int32_t *seq_ids, int32_t batch,
                         int32_t q_len, int32_t q_heads, const float *q, float scale,
                         int32_t chunk, float *out);

/* ---- R4KV page container ---------------------------------------------------- */
/* har/crates/r4kv/src/crc32c.rs:4-31: reflected 0x82f63b78, init/final xor ~0 */
uint32_t rko_crc32c(const uint8_t *data, size_t n);
/* har/crates/r4kv/src/page.rs:15-30 */
typedef struct rko_r4kv_header {
  uint64_t prefix_digest;
  uint32_t token_start, token_count, pos_start;
  uint16_t layer_lo, layer_hi;
  uint8_t k_fmt, v_fmt;
  uint32_t epoch, generation;
  uint64_t payload_len;
  uint32_t sketch_offset;
  uint16_t flags;
} rko_r4kv_header;
/* PageHeader::to_bytes, page.rs:100-126 */
void rko_r4kv_header_bytes(const rko_r4kv_header *h, uint8_t out[96]);
/* pack_page, page.rs:213-224: header, body, LE CRC32C of the body;
 * `out` holds 96 + n + 4 bytes */
void rko_r4kv_pack_page(const rko_r4kv_header *h, const uint8_t *body, size_t n, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
