// rkv_append.hip -- quantize-and-append of K/V rows into Q8_0 pages, the
// bit-exact gather/import between pages and reference rows, and a batch
// f16 encoder (gfx950).
//
// Quantization rules (bit-exact with the CPU reference): q8_quantize_lane
// in rkv_device.h -- canonical (har/crates/r4kv/src/quant.rs:45-90) or
// har-serve (har/crates/har-serve/src/attention.rs:25-42).
#include <algorithm>

#include "rkv_launch.h"

namespace rkv {

namespace {

// One group of 8 lanes quantizes one 32-value block; lane `sub` owns values
// 4*sub..4*sub+3.  The block index enumerates (row, kv_head, kind, block).
__global__ __launch_bounds__(256) void append_kernel(AppendLaunch a) {
  const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  const int32_t D = a.g.head_dim;
  const int32_t NB = D >> 5;
  const uint32_t nblocks = (uint32_t)a.n_rows * (uint32_t)a.g.kv_heads * 2u * (uint32_t)NB;
  const uint32_t blk = tid >> 3;
  const int32_t sub = (int32_t)(tid & 7u);
  // Every lane takes part in the shuffles; out-of-range lanes use zeros.
  const bool live = blk < nblocks;
  const uint32_t blkc = live ? blk : 0u;
  const int32_t b = (int32_t)(blkc % (uint32_t)NB);
  uint32_t t = blkc / (uint32_t)NB;
  const int32_t kind = (int32_t)(t & 1u);
  t >>= 1;
  const int32_t kvh = (int32_t)(t % (uint32_t)a.g.kv_heads);
  const int32_t row = (int32_t)(t / (uint32_t)a.g.kv_heads);

  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    const uint64_t off =
        ((uint64_t)row * (uint64_t)a.g.kv_heads + (uint64_t)kvh) * (uint64_t)D + (uint64_t)(b * 32 + sub * 4);
    load_src4(kind == 0 ? a.k_src : a.v_src, off, a.src_bf16 != 0, v);
  }
  uint16_t scale;
  const uint32_t codes = q8_quantize_lane(v, a.rule, scale);
  if (!live) return;

  const int32_t seq = a.seq_ids[row];
  const int32_t pos = a.positions[row];
  if (seq < 0 || seq >= a.n_seqs) {
    if (sub == 0) atomicOr(a.fault, FAULT_BAD_SEQ);
    return;
  }
  if (pos < 0 || pos / a.g.page_tokens >= a.bt_stride) {
    if (sub == 0) atomicOr(a.fault, FAULT_BAD_POSITION);
    return;
  }
  const int32_t page = a.bt[(int64_t)seq * a.bt_stride + pos / a.g.page_tokens];
  if (page < 0 || page >= a.g.num_pages) {
    if (sub == 0) atomicOr(a.fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot = pos % a.g.page_tokens;
  store_q8_lane(a.g, a.pages + region_base(a.g, page, kvh, kind), kind, slot, b, sub, codes, scale);
}

// One thread per (kv_head, position, block): 34 reference-row bytes.
__global__ __launch_bounds__(256) void gather_kernel(Geo g, const uint8_t *pages, const int32_t *bt,
                                                     int32_t len, int32_t kind, uint8_t *rows,
                                                     int32_t *fault) {
  const int32_t NB = g.head_dim >> 5;
  const int64_t n = (int64_t)g.kv_heads * len * NB;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tid >= n) return;
  const int32_t b = (int32_t)(tid % NB);
  const int64_t t = tid / NB;
  const int32_t pos = (int32_t)(t % len);
  const int32_t kvh = (int32_t)(t / len);
  const int32_t page = bt[pos / g.page_tokens];
  if (page < 0 || page >= g.num_pages) {
    atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot = pos % g.page_tokens;
  const uint8_t *region = pages + region_base(g, page, kvh, kind);
  uint8_t *dst = rows + ((int64_t)kvh * len + pos) * (NB * 34) + b * 34;
  const uint16_t sc = *reinterpret_cast<const uint16_t *>(region + scale_offset(g, slot, b));
  dst[0] = (uint8_t)(sc & 0xffu);
  dst[1] = (uint8_t)(sc >> 8);
  const uint8_t bias = code_bias(kind);
  for (int i = 0; i < 32; ++i) dst[2 + i] = region[code_offset(g, kind, slot, b * 32 + i)] ^ bias;
}

__global__ __launch_bounds__(256) void import_kernel(Geo g, uint8_t *pages, const int32_t *bt,
                                                     int32_t len, int32_t kind, const uint8_t *rows,
                                                     int32_t *fault) {
  const int32_t NB = g.head_dim >> 5;
  const int64_t n = (int64_t)g.kv_heads * len * NB;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tid >= n) return;
  const int32_t b = (int32_t)(tid % NB);
  const int64_t t = tid / NB;
  const int32_t pos = (int32_t)(t % len);
  const int32_t kvh = (int32_t)(t / len);
  const int32_t page = bt[pos / g.page_tokens];
  if (page < 0 || page >= g.num_pages) {
    atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot = pos % g.page_tokens;
  uint8_t *region = pages + region_base(g, page, kvh, kind);
  const uint8_t *src = rows + ((int64_t)kvh * len + pos) * (NB * 34) + b * 34;
  *reinterpret_cast<uint16_t *>(region + scale_offset(g, slot, b)) =
      (uint16_t)(src[0] | ((uint16_t)src[1] << 8));
  const uint8_t bias = code_bias(kind);
  for (int i = 0; i < 32; ++i) region[code_offset(g, kind, slot, b * 32 + i)] = src[2 + i] ^ bias;
}

__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float *in, uint16_t *out, int64_t n,
                                                         int32_t rule) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] = rule == 0 ? f16_rtne(in[i]) : f16_harserve(in[i]);
}

inline unsigned grid_for(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace

hipError_t launch_append(const AppendLaunch &a, hipStream_t s) {
  const int64_t threads = (int64_t)a.n_rows * a.g.kv_heads * 2 * (a.g.head_dim / 32) * 8;
  if (threads == 0) return hipSuccess;
  hipLaunchKernelGGL(append_kernel, dim3(grid_for(threads)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gather(const Geo &g, const uint8_t *pages, const int32_t *bt, int32_t len,
                         int32_t kind, uint8_t *rows, int32_t *fault, hipStream_t s) {
  const int64_t n = (int64_t)g.kv_heads * len * (g.head_dim / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(grid_for(n)), dim3(256), 0, s, g, pages, bt, len, kind,
                     rows, fault);
  return hipGetLastError();
}

hipError_t launch_import(const Geo &g, uint8_t *pages, const int32_t *bt, int32_t len,
                         int32_t kind, const uint8_t *rows, int32_t *fault, hipStream_t s) {
  const int64_t n = (int64_t)g.kv_heads * len * (g.head_dim / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(import_kernel, dim3(grid_for(n)), dim3(256), 0, s, g, pages, bt, len, kind,
                     rows, fault);
  return hipGetLastError();
}

namespace {
// Unpack a block-table update: `n_rows` records of [seq][W page ids] then
// the lengths of all `n_seqs` sequences.  Block i < n_rows copies record i;
// block n_rows copies the lengths.
__global__ __launch_bounds__(256) void table_scatter_kernel(const int32_t *packed, int32_t n_rows,
                                                           int32_t W, int32_t n_seqs,
                                                           int32_t *tables, int32_t *lens) {
  const int32_t r = blockIdx.x;
  if (r < n_rows) {
    const int32_t *rec = packed + (int64_t)r * (W + 1);
    const int32_t seq = rec[0];
    if (seq < 0 || seq >= n_seqs) return;  // packed by the host from its own table
    for (int32_t i = threadIdx.x; i < W; i += 256) tables[(int64_t)seq * W + i] = rec[1 + i];
  } else {
    const int32_t *src = packed + (int64_t)n_rows * (W + 1);
    for (int32_t i = threadIdx.x; i < n_seqs; i += 256) lens[i] = src[i];
  }
}

// Copy-on-write page copies: for each (src, dst) pair and each of `layers`
// layer arrays, page dst := page src.  A unit is one 16 KiB piece of one
// (pair, layer) page; each block walks units with a grid stride and each
// thread moves four 16-byte vectors per unit, all loads issued before the
// stores.  Pairs naming pages outside [0, num_pages) are skipped.
constexpr int32_t kCopyVecs = 4;
constexpr int32_t kCopyUnitBytes = 256 * 16 * kCopyVecs;

__global__ __launch_bounds__(256) void copy_pages_kernel(uint8_t *pages, int64_t layer_stride,
                                                         int32_t layers, int32_t num_pages,
                                                         const int32_t *pairs, int64_t page_bytes,
                                                         int32_t units_per_page, int64_t n_units) {
  for (int64_t u = blockIdx.x; u < n_units; u += gridDim.x) {
    const int64_t pl = u / units_per_page;
    const int32_t part = (int32_t)(u - pl * units_per_page);
    const int32_t layer = (int32_t)(pl % layers);
    const int64_t pair = pl / layers;
    const int32_t src = pairs[2 * pair], dst = pairs[2 * pair + 1];
    if (src < 0 || src >= num_pages || dst < 0 || dst >= num_pages) continue;
    const uint8_t *from = pages + layer * layer_stride + (int64_t)src * page_bytes;
    uint8_t *to = pages + layer * layer_stride + (int64_t)dst * page_bytes;
    const int64_t base = (int64_t)part * kCopyUnitBytes + (int64_t)threadIdx.x * 16;
    uint4 v[kCopyVecs];
#pragma unroll
    for (int32_t k = 0; k < kCopyVecs; ++k) {
      const int64_t off = base + (int64_t)k * 256 * 16;
      if (off < page_bytes) v[k] = *reinterpret_cast<const uint4 *>(from + off);
    }
#pragma unroll
    for (int32_t k = 0; k < kCopyVecs; ++k) {
      const int64_t off = base + (int64_t)k * 256 * 16;
      if (off < page_bytes) *reinterpret_cast<uint4 *>(to + off) = v[k];
    }
  }
}
}  // namespace

hipError_t launch_copy_pages(uint8_t *pages, int64_t layer_stride, int32_t layers,
                             int32_t num_pages, const int32_t *pairs, int32_t n_pairs,
                             int64_t page_bytes, hipStream_t s) {
  if (n_pairs <= 0 || layers <= 0) return hipSuccess;
  const int32_t units_per_page = (int32_t)((page_bytes + kCopyUnitBytes - 1) / kCopyUnitBytes);
  const int64_t n_units = (int64_t)n_pairs * layers * units_per_page;
  const unsigned grid = (unsigned)std::min<int64_t>(n_units, 8192);
  hipLaunchKernelGGL(copy_pages_kernel, dim3(grid), dim3(256), 0, s, pages, layer_stride, layers,
                     num_pages, pairs, page_bytes, units_per_page, n_units);
  return hipGetLastError();
}

hipError_t launch_table_scatter(const int32_t *packed, int32_t n_rows, int32_t W, int32_t n_seqs,
                                int32_t *tables, int32_t *lens, hipStream_t s) {
  hipLaunchKernelGGL(table_scatter_kernel, dim3((unsigned)n_rows + 1), dim3(256), 0, s, packed,
                     n_rows, W, n_seqs, tables, lens);
  return hipGetLastError();
}

hipError_t launch_f32_to_f16(const float *in, uint16_t *out, int64_t n, int32_t rule,
                             hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n, rule);
  return hipGetLastError();
}

}  // namespace rkv
