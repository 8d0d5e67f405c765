// rkv_launch.h -- internal launcher interface between the C-ABI runtime
// (rkv_runtime.cpp) and the gfx950 kernels (rkv_append.hip, rkv_decode.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rkv_device.h"

namespace rkv {

struct AppendLaunch {
  Geo g;
  uint8_t *pages;
  const int32_t *bt;
  int32_t bt_stride;
  int32_t n_seqs;
  int32_t n_rows;
  const int32_t *seq_ids;
  const int32_t *positions;
  const void *k_src;
  const void *v_src;
  int32_t src_bf16;
  int32_t rule;
  int32_t *fault;
};
hipError_t launch_append(const AppendLaunch &a, hipStream_t s);

// gather: pages -> reference rows; import: reference rows -> pages
hipError_t launch_gather(const Geo &g, const uint8_t *pages, const int32_t *bt, int32_t len,
                         int32_t kind, uint8_t *rows, int32_t *fault, hipStream_t s);
hipError_t launch_import(const Geo &g, uint8_t *pages, const int32_t *bt, int32_t len,
                         int32_t kind, const uint8_t *rows, int32_t *fault, hipStream_t s);
hipError_t launch_f32_to_f16(const float *in, uint16_t *out, int64_t n, int32_t rule,
                             hipStream_t s);
// block-table update: records [seq][W ids] x n_rows, then n_seqs lengths,
// read from `packed` (pinned host memory, device-mapped); n_rows + 1 blocks,
// each counted once in *count, and the block that takes the count `last`
// stores `seq` to *done (host-visible) after every block has read `packed`
hipError_t launch_table_scatter(const int32_t *packed, int32_t n_rows, int32_t W, int32_t n_seqs,
                                int32_t *tables, int32_t *lens, unsigned long long *count,
                                unsigned long long last, unsigned long long *done,
                                unsigned long long seq, hipStream_t s);
// copy-on-write: page dst := page src for each (src, dst) pair in `pairs`
// (device), in `layers` page arrays `layer_stride` bytes apart
hipError_t launch_copy_pages(uint8_t *pages, int64_t layer_stride, int32_t layers,
                             int32_t num_pages, const int32_t *pairs, int32_t n_pairs,
                             int64_t page_bytes, hipStream_t s);

struct DecodeLaunch {
  Geo g;
  const uint8_t *pages;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  int32_t n_seqs;
  const int32_t *seq_ids;
  int32_t batch;
  const void *q;
  int32_t q_bf16;
  int32_t q_len;
  int32_t q_heads;
  float scale_log2;  // softmax scale * log2(e)
  // Partition plan.  part_tokens > 0 fixes the partition length; 0 lets every
  // workgroup derive the same length from the device lengths: the smallest
  // k*pt_unit (pt_unit = one 32-token tile), k in [pt_kmin, pt_kmax], whose
  // partition count over the batch is <= target_parts (else the longest);
  // a length whose partitions could start inside a page and span more than
  // 64 pages rounds up to 64 pages.  Workgroup x of the grid (n_wg,
  // kv_heads) takes the x-th partition of the batch in entry order.
  int32_t part_tokens;
  int32_t pt_unit, pt_kmin, pt_kmax, target_parts;
  int32_t max_len;  // >= every length of the batch
  int32_t n_wg;     // upper bound of the batch's partition count
  int32_t n_parts;  // per-entry layout only: ceil(max_len / part_tokens)
  // direct output (ws_o == nullptr) ...
  void *out;
  int32_t out_bf16;
  // ... or split-K partials (m, l) and o, either flat [kv_head][n_wg][R][2 | D]
  // with ws_hdr = {partition length, then per entry: first partition, count},
  // or per entry [batch][q_len*q_heads][n_parts][2 | D] (ws_hdr == nullptr)
  float *ws_ml;
  float *ws_o;
  int32_t *ws_hdr;
  int32_t *fault;
  int32_t stages;  // LDS ring depth: 2 or 3 (tiles in flight = stages - 1)
  // Optional append (app_k == nullptr: none): row b*q_len + j of app_k/app_v
  // ([rows][kv_heads][head_dim]) goes to position app_pos[row] of sequence
  // seq_ids[b] before the decode reads it; the workgroup whose partition
  // holds that position writes it.
  uint8_t *pages_w;  // == pages, writable
  const int32_t *app_seq_ids;
  const int32_t *app_pos;
  const void *app_k;
  const void *app_v;
  int32_t app_bf16;
  int32_t app_rule;
};
// rows per kv head = q_len * q_heads / kv_heads must be <= 32
hipError_t launch_decode(const DecodeLaunch &d, hipStream_t s);

// Chunked prefill attention: entry e holds rows[e] query rows of sequence
// seq[e] at positions ctx[e] .. ctx[e]+rows[e]-1 (already appended), stored
// at rows qoff[e].. of q/out ([rows][q_heads][head_dim]); row i attends
// positions [0, ctx[e]+i].  A row block is tq query tokens x
// q_heads/kv_heads heads = kPrefillRows rows; its causal range is split into
// nseg[e] segments of seg[e] tokens.  Entry e owns units [first[e]*H,
// first[e+1]*H) of the launch (H = kv_heads), one per (segment, kv head,
// row block).  Workgroups go to the 8 XCDs round robin; XCD x takes list
// chunks x, x + 8, ... of xcd_chunk consecutive units.  An entry with one segment writes its rows normalized; a
// split one writes per-segment partials (m, l) and o at partial row
// wsoff[e] + (row * q_heads + head) * nseg[e] + segment, which
// launch_prefill's combine merges into the rows.
constexpr int kPrefillWaves = 8;
constexpr int kPrefillRows = 16 * kPrefillWaves;
constexpr int kPrefillMaxEntries = 64;
constexpr int kPrefillMaxPages = 4096;  // page-list capacity of one unit (LDS)
constexpr int kPrefillMaxSegs = 64;
constexpr int kPrefillWgsPerCu = 2;  // the prefill kernel's launch bounds
// xcd_chunk of a launch over HBM pages (a causal range's 32 row blocks per kv
// head on 4 XCDs: 2% faster than 1 on config 7, 1% on the serving step; 16
// unbalances the serving step's mixed lengths) and over host-memory pages
// (one XCD per range: the link, not the CUs, is the bound)
constexpr int kPrefillXcdChunkHbm = 8;
constexpr int kPrefillXcdChunkHost = 32;
struct PrefillLaunch {
  DecodeLaunch d;  // geometry, pages, tables, q, out, dtypes, scale, fault, stages
  int32_t tq;
  int32_t n_entries;
  int32_t seq[kPrefillMaxEntries];
  int32_t ctx[kPrefillMaxEntries];
  int32_t rows[kPrefillMaxEntries];
  int32_t qoff[kPrefillMaxEntries];
  int32_t nseg[kPrefillMaxEntries];
  int32_t seg[kPrefillMaxEntries];     // tokens, a multiple of max(32, page_tokens)
  int64_t wsoff[kPrefillMaxEntries];   // first partial row of a split entry
  int32_t first[kPrefillMaxEntries + 1];
  int32_t xcd_chunk;  // 1: plain round robin; more: row blocks of one range share an L2
  float *ws_ml;  // split partials: (m, l) [partial row][2] ...
  float *ws_o;   // ... and o [partial row][head_dim]
  // Tiles widened once (bf16 query): the widening pass writes every 32-token
  // tile of every entry's causal range, per kv head, as the image the
  // compute reads from LDS (prefill_tile_bytes each, K and V as f16 and
  // both scale runs); the prefill copies those images instead of widening
  // per workgroup.  Entry k's tiles start at tile index preoff[k] (kv head h:
  // + h * tiles of the entry); preoff[n_entries] is the total.  nullptr: the
  // workgroups widen their tiles themselves.
  uint8_t *pre;
  int64_t preoff[kPrefillMaxEntries + 1];
};
hipError_t launch_prefill(const PrefillLaunch &pf, hipStream_t s);
// bytes of one widened tile image: K and V f16 (64*D each), the K and V
// scale runs (2*D each), padded to whole 1 KiB copies
constexpr int64_t prefill_tile_bytes(int head_dim) { return (132LL * head_dim + 1023) / 1024 * 1024; }

// CRC32C of n bytes at `data` (16-byte aligned, device-readable) into *out
// (device word), stream-ordered; the word is cleared by the launch itself.
hipError_t launch_crc32c(const uint8_t *data, int64_t n, uint32_t *out, hipStream_t s);

// R4KV page body <-> pool: rows of tokens [t0, t0+count) of one sequence
// (block-table row `bt`), layers [layer_lo, layer_lo+n_layers) of page
// arrays layer_stride bytes apart.  Pack writes header, body and payload
// CRC (through crc_word) to page_out; unpack writes a verified body back.
struct R4kvLaunch {
  Geo g;
  int64_t layer_stride;
  int32_t layer_lo, n_layers;
  int32_t t0, count;
  uint8_t header[96];
};
hipError_t launch_r4kv_pack(const R4kvLaunch &r, const uint8_t *pages, const int32_t *bt,
                            uint8_t *page_out, uint32_t *crc_word, int32_t *fault, hipStream_t s);
hipError_t launch_r4kv_unpack(const R4kvLaunch &r, uint8_t *pages, const int32_t *bt,
                              const uint8_t *body, int32_t *fault, hipStream_t s);
// HBM streaming-read ceiling (rkv_stream.hip): mode 0 vector loads with the
// xor of the words read into *out, mode 1 LDS-DMA copies of
// stream_read_dma_unit() bytes per wave round
hipError_t launch_stream_read(const uint8_t *data, int64_t bytes, int32_t mode, int32_t blocks,
                              uint32_t *out, hipStream_t s);
int64_t stream_read_dma_unit();
// The decode's tile order over a pool's pages, for its read rate
// (rkv_stream_read_tiles): n_seqs block-table rows of seq_tokens tokens,
// partitions of part_tokens tokens (parts per sequence), each kv head.
struct TileStreamLaunch {
  Geo g;
  const uint8_t *pages;
  const int32_t *bt;
  int32_t bt_stride;
  int32_t n_seqs;
  int32_t seq_tokens;
  int32_t part_tokens;
  int32_t parts;
};
hipError_t launch_stream_tiles(const TileStreamLaunch &t, hipStream_t s);
// the 17..32-row instantiations (own translation unit)
hipError_t launch_decode_rows32(const DecodeLaunch &d, hipStream_t s);

// Decode workgroups (one wave each) resident per CU, the lesser of
//  - LDS: `stages` tile stages of 68*head_dim bytes, padded to 1 KiB, out of
//    the CU's 160 KiB;
//  - registers: head_dim 256, or more than 16 rows per kv head, takes more
//    than half of a SIMD's 512 VGPR+AGPR per lane (one wave per SIMD);
//    smaller shapes fit two waves per SIMD.
// The 2-stage, <= 16-row kernel on pages of >= 32 tokens keeps K codes in
// registers and stages only 36*head_dim bytes; registers bind before LDS for
// both stage sizes, so the count is the same.
constexpr int decode_wgs_per_cu(int head_dim, int rows, int stages) {
  const int stage = (68 * head_dim / 16 + 63) / 64 * 1024;
  const int by_lds = 160 * 1024 / (stages * stage);
  const int by_regs = (head_dim == 256 || rows > 16) ? 4 : 8;
  return by_lds < by_regs ? by_lds : by_regs;
}
constexpr int kComputeUnits = 256;  // MI355X (gfx950): 8 XCDs of 32 CUs

// Static device scratch of rkv_decode_q8_noalloc (rkv_scratch.hip): its
// size, and its device address on `device`, which must be the current
// device (resolved once per device, then cached).
constexpr size_t kDecodeScratchBytes = 64u << 20;
hipError_t scratch_address(int device, void **ptr);

struct CombineLaunch {
  const float *ml;
  const float *o;
  int32_t batch;
  int32_t rows;
  int32_t n_parts;
  int32_t head_dim;
  const int32_t *seq_ids;
  const int32_t *seq_lens;
  int32_t n_seqs;
  int32_t part_tokens;
  void *out;
  int32_t out_bf16;
};
hipError_t launch_combine(const CombineLaunch &c, hipStream_t s);

// Combine of the flat partials layout written by a decode launch: `slices`
// 256-thread blocks per (row, entry), each merging all of the entry's
// partitions (from the header the decode wrote) for head_dim/slices dims.
struct FlatCombineLaunch {
  const float *ml;
  const float *o;
  const int32_t *hdr;
  int32_t batch;
  int32_t q_len;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t n_wg;
  int32_t slices;    // blocks per (row, entry), each merging head_dim/slices dims; a power of two
  void *out;
  int32_t out_bf16;
};
hipError_t launch_combine_flat(const FlatCombineLaunch &c, hipStream_t s);

}  // namespace rkv
