// rkv_append.hip -- quantize-and-append of K/V rows into Q8_0 pages, the
// bit-exact gather/import between pages and reference rows, and a batch
// f16 encoder (gfx950).
//
// Quantization rules (bit-exact with the CPU reference): q8_quantize_values
// in rkv_device.h -- canonical (har/crates/r4kv/src/quant.rs:45-90) or
// har-serve (har/crates/har-serve/src/attention.rs:25-42).
#include <algorithm>

#include "rkv_launch.h"

namespace rkv {

namespace {

// Eight consecutive source values (f32 or bf16) starting at element `off`.
template <bool kBf16>
__device__ inline void load_src8(const void *src, uint64_t off, float v[8]) {
  if constexpr (kBf16) {
    const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(src) + off);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_bits_to_f32((uint16_t)(ws[i] & 0xffffu));
      v[2 * i + 1] = bf16_bits_to_f32((uint16_t)(ws[i] >> 16));
    }
  } else {
    const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + off);
    const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + off + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

// One workgroup of 256 threads appends input rows [ROWS*blockIdx.x, +ROWS)
// of kv head blockIdx.y, K and V (ROWS = 32 for large launches, 8 for small
// ones, so that a few thousand rows still spread over several workgroups per
// CU: the quantizer's VALU work, not HBM, bounds a workgroup):
//  1. each row's destination (region offset and slot; invalid rows are
//     reported and skipped, nothing is written for them);
//  2. quantize, 4 lanes per 32-value block with 8 values each (lanes of a
//     row read its values in contiguous 16-byte loads), into LDS: K and V
//     codes row-major (row stride D + 8 bytes: conflict-free for both the
//     8-byte writes here and the transposing byte reads below) and scales;
//  3. write the page bytes so that a wave's stores are contiguous whenever
//     the rows are consecutive tokens: K rows as 16-byte stores; V codes
//     (page layout [slot/TT][dim][slot%TT]) as one 4-byte store per 4 rows
//     that are 4 aligned consecutive slots of one page, lanes ordered by
//     slot group then dim (256 contiguous bytes per wave for a whole tile),
//     else byte stores; scales with lanes ordered by slot.
template <int D, int kAppRows, bool kBf16, int kRule>
__global__ __launch_bounds__(256) void append_kernel(AppendLaunch a) {
  static_assert(kAppRows % 4 == 0 && kAppRows <= 64, "rows come in quads, resolved by wave 0");
  constexpr int NB = D / 32;
  constexpr int RS = D + 8;  // LDS row stride
  __shared__ __attribute__((aligned(16))) uint8_t codes[2][kAppRows][RS];
  __shared__ uint16_t scl[2][kAppRows][NB];
  __shared__ int64_t rbase[kAppRows];  // region offset of (page, kv head, K); -1: skip the row
  __shared__ int32_t rslot[kAppRows];
  __shared__ int32_t quad[kAppRows / 4];  // rows 4i..4i+3 are slots s..s+3 (s % 4 == 0) of one page
  const Geo g = a.g;
  const int tid = (int)threadIdx.x;
  const int kvh = (int)blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * kAppRows;
  const int nr = (int)min<int64_t>(kAppRows, (int64_t)a.n_rows - row0);

  // ---- loads: lanes 0..nr-1 of wave 0 read their row's sequence and
  // position, then every thread issues its quantize tasks' source loads
  // (tasks (row, kind, block, lane), lane fastest; dtype and rule fixed at
  // compile time, rows past the last read as the last row and never
  // written), all before the first wait; the page lookup that needs the
  // position follows, so wave 0's critical path is two dependent loads
  const bool resolver = tid < 64;
  int32_t seq = -1, pos = -1;
  if (resolver && tid < nr) {
    seq = a.seq_ids[row0 + tid];
    pos = a.positions[row0 + tid];
  }
  // kWhole (32-row workgroups): one lane per (row, kind, block) task, its 32
  // values in registers (q8_quantize_block: no shuffles, one scale per
  // lane); 8-row workgroups keep 4 lanes per block so that every thread has
  // a task.  Tasks run block fastest, so consecutive lanes read consecutive
  // source bytes.
  constexpr bool kWhole = kAppRows == 32;
  constexpr int kVPL = kWhole ? 32 : 8;  // values per lane and task
  constexpr int kTasks = kAppRows * 2 * NB * (32 / kVPL);
  constexpr int kPer = kTasks / 256;
  static_assert(kTasks % 256 == 0, "every thread takes part in every task round");
  float v[kPer][kVPL];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int t = 256 * i + tid;
    const int sub = kWhole ? 0 : t & 3;
    const int tb = kWhole ? t : t >> 2;
    const int blk = tb % NB;
    const int kind = (tb / NB) & 1;
    const int r = min(tb / NB / 2, nr - 1);
    const uint64_t off = ((uint64_t)(row0 + r) * (uint64_t)g.kv_heads + (uint64_t)kvh) * D +
                         (uint64_t)(blk * 32 + sub * 8);
#pragma unroll
    for (int e = 0; e < kVPL / 8; ++e)
      load_src8<kBf16>(kind == 0 ? a.k_src : a.v_src, off + 8 * e, &v[i][8 * e]);
  }

  // ---- rows' destinations (wave 0) --------------------------------------
  if (resolver) {
    int64_t base = -1;
    int32_t slot = 0;
    if (tid < nr) {
      if (seq < 0 || seq >= a.n_seqs) {
        if (kvh == 0) atomicOr(a.fault, FAULT_BAD_SEQ);
      } else if (pos < 0 || pos / g.page_tokens >= a.bt_stride) {
        if (kvh == 0) atomicOr(a.fault, FAULT_BAD_POSITION);
      } else {
        const int32_t page = a.bt[(int64_t)seq * a.bt_stride + pos / g.page_tokens];
        if (page < 0 || page >= g.num_pages) {
          if (kvh == 0) atomicOr(a.fault, FAULT_BAD_PAGE);
        } else {
          base = (int64_t)region_base(g, page, kvh, 0);
          slot = pos % g.page_tokens;
        }
      }
    }
    // rows 4i..4i+3 form a quad when they are 4 aligned consecutive slots of one page
    bool run = base >= 0 && slot % 4 == 0;
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      const int64_t b2 = __shfl_down(base, i);
      const int32_t s2 = __shfl_down(slot, i);
      run = run && b2 == base && s2 == slot + i;
    }
    if (tid < kAppRows) {
      rbase[tid] = base;
      rslot[tid] = slot;
      if ((tid & 3) == 0) quad[tid >> 2] = run;
    }
  }

  // ---- quantize into LDS ---------------------------------------------------
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int t = 256 * i + tid;
    const int sub = kWhole ? 0 : t & 3;
    const int tb = kWhole ? t : t >> 2;
    const int blk = tb % NB;
    const int kind = (tb / NB) & 1;
    const int r = tb / NB / 2;
    uint16_t scale;
    if constexpr (kWhole) {
      uint32_t c[8];
      q8_quantize_block(v[i], kRule, scale, c);
      const uint32_t bias = kind == 1 ? 0x80808080u : 0u;  // V codes are stored biased (code_bias)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<uint2 *>(&codes[kind][r][blk * 32 + 8 * j]) =
            uint2{c[2 * j] ^ bias, c[2 * j + 1] ^ bias};
    } else {
      uint64_t c = q8_quantize_values<8>(v[i], kRule, scale);
      if (kind == 1) c ^= 0x8080808080808080ull;  // V codes are stored biased (code_bias)
      *reinterpret_cast<uint64_t *>(&codes[kind][r][blk * 32 + sub * 8]) = c;
    }
    if (sub == 0) scl[kind][r][blk] = scale;
  }
  __syncthreads();

  uint8_t *pages = a.pages;
  const uint64_t RB = region_bytes(g);
  // K codes: row r's D bytes at slot * D of the K region
  for (int t = tid; t < kAppRows * (D / 16); t += 256) {
    const int r = t / (D / 16), c = t % (D / 16);
    const int64_t b = rbase[r];
    if (b < 0) continue;
    // (LDS rows are 8-byte aligned: two 8-byte reads)
    const uint2 lo = *reinterpret_cast<const uint2 *>(&codes[0][r][16 * c]);
    const uint2 hi = *reinterpret_cast<const uint2 *>(&codes[0][r][16 * c + 8]);
    *reinterpret_cast<uint4 *>(pages + b + (uint64_t)rslot[r] * D + 16 * c) = uint4{lo.x, lo.y, hi.x, hi.y};
  }
  // V codes: tasks (4-row group, dim), group fastest
  for (int t = tid; t < (kAppRows / 4) * D; t += 256) {
    const int q = t % (kAppRows / 4), d = t / (kAppRows / 4);
    const int r = 4 * q;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) w |= (uint32_t)codes[1][r + i][d] << (8 * i);
    if (quad[q]) {
      *reinterpret_cast<uint32_t *>(pages + rbase[r] + RB + code_offset(g, 1, rslot[r], d)) = w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rbase[r + i] >= 0)
          pages[rbase[r + i] + RB + code_offset(g, 1, rslot[r + i], d)] = (uint8_t)(w >> (8 * i));
    }
  }
  // scales: tasks (row, block, kind), row fastest
  for (int t = tid; t < 2 * NB * kAppRows; t += 256) {
    const int r = t % kAppRows, blk = (t / kAppRows) % NB, kind = t / (kAppRows * NB);
    const int64_t b = rbase[r];
    if (b < 0) continue;
    *reinterpret_cast<uint16_t *>(pages + b + kind * RB + scale_offset(g, rslot[r], blk)) =
        scl[kind][r][blk];
  }
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

namespace {
template <int D, int ROWS>
void launch_append_r(const AppendLaunch &a, hipStream_t s) {
  const dim3 grid((unsigned)((a.n_rows + ROWS - 1) / ROWS), (unsigned)a.g.kv_heads);
  if (a.src_bf16) {
    if (a.rule == 0) hipLaunchKernelGGL((append_kernel<D, ROWS, true, 0>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((append_kernel<D, ROWS, true, 1>), grid, dim3(256), 0, s, a);
  } else {
    if (a.rule == 0) hipLaunchKernelGGL((append_kernel<D, ROWS, false, 0>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((append_kernel<D, ROWS, false, 1>), grid, dim3(256), 0, s, a);
  }
}
template <int D>
void launch_append_d(const AppendLaunch &a, hipStream_t s) {
  // 32-row workgroups once there are at least 8 per CU, else 8-row ones
  if ((int64_t)a.n_rows * a.g.kv_heads >= (int64_t)32 * 8 * kComputeUnits)
    launch_append_r<D, 32>(a, s);
  else
    launch_append_r<D, 8>(a, s);
}
}  // namespace

hipError_t launch_append(const AppendLaunch &a, hipStream_t s) {
  if (a.n_rows <= 0) return hipSuccess;
  if (a.g.head_dim == 256) launch_append_d<256>(a, s);
  else launch_append_d<128>(a, s);
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
// `packed` is the host's pinned staging buffer, read over the host link
// (no separate copy).  When every block has read it, the last one to finish
// stores `seq` to the host-visible word `done`, which tells the host that
// the buffer may be rewritten: each block counts itself in the device
// counter `count` (never reset; the launch's blocks are the counts from
// `last` - gridDim.x + 1 to `last`).
__global__ __launch_bounds__(256) void table_scatter_kernel(const int32_t *packed, int32_t n_rows,
                                                           int32_t W, int32_t n_seqs,
                                                           int32_t *tables, int32_t *lens,
                                                           unsigned long long *count,
                                                           unsigned long long last,
                                                           unsigned long long *done,
                                                           unsigned long long seq) {
  const int32_t r = blockIdx.x;
  if (r < n_rows) {
    const int32_t *rec = packed + (int64_t)r * (W + 1);
    const int32_t sq = rec[0];
    if (sq >= 0 && sq < n_seqs)  // packed by the host from its own table
      for (int32_t i = threadIdx.x; i < W; i += 256) tables[(int64_t)sq * W + i] = rec[1 + i];
  } else {
    const int32_t *src = packed + (int64_t)n_rows * (W + 1);
    for (int32_t i = threadIdx.x; i < n_seqs; i += 256) lens[i] = src[i];
  }
  // every value read above was stored, so the block's reads are done
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(count, 1ull) == last) {
      __threadfence_system();
      __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
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
                                int32_t *tables, int32_t *lens, unsigned long long *count,
                                unsigned long long last, unsigned long long *done,
                                unsigned long long seq, hipStream_t s) {
  hipLaunchKernelGGL(table_scatter_kernel, dim3((unsigned)n_rows + 1), dim3(256), 0, s, packed,
                     n_rows, W, n_seqs, tables, lens, count, last, done, seq);
  return hipGetLastError();
}

hipError_t launch_f32_to_f16(const float *in, uint16_t *out, int64_t n, int32_t rule,
                             hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n, rule);
  return hipGetLastError();
}

}  // namespace rkv
