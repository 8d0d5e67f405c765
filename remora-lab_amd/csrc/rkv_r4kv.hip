// rkv_r4kv.hip -- R4KV page spill/restore kernels for gfx950: a device
// CRC32C (har/crates/r4kv/src/crc32c.rs) and the pack/unpack of a token
// range of Q8_0 rows between the page pool and a page payload.
//
// CRC32C.  Each wave covers a 128 KiB segment; the segments are laid out
// back from the end of the 16-byte-aligned prefix, so the first may start
// before byte 0 (those leading bytes read as zero, which leaves the raw CRC
// unchanged) and every 16-byte piece is aligned.  Lane l folds the pieces
// l, l+64, ... of its segment (Horner: shift the running value 1024 bytes,
// xor the piece's raw CRC from the slicing tables), and the lanes combine
// in a 6-level tree of shifts by 16*2^j bytes.  The four waves of a block
// hold consecutive segments: each is shifted to the block's end and xor-ed
// in LDS, and the block's value is shifted once to the end of the message
// and xor-ed into the output word.  Block 0 also adds the raw CRC of the
// unaligned tail and the init/final-xor term.  Reads stay inside [0, n).
#include "rkv_crc32c.h"
#include "rkv_launch.h"

namespace rkv {
namespace {

constexpr int kCrcIter = 128;                      // pieces per lane
constexpr int64_t kCrcSeg = 16LL * 64 * kCrcIter;  // bytes per wave (128 KiB = 2^17)
constexpr int kCrcSegLog2 = 17;

__constant__ crc::Slice16 c_slice16 = crc::kSlice16;
__constant__ crc::Shift1024 c_shift1024 = crc::kShift1024;
__constant__ crc::Shifts c_shifts = crc::kShift;
__constant__ crc::ByteTable c_byte = crc::kByte;

__device__ __forceinline__ uint32_t mat_apply_dev(const crc::Mat &m, uint32_t c) {
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) r ^= m.col[i] & (0u - ((c >> i) & 1u));
  return r;
}

__global__ void zero_word_kernel(uint32_t *w) { *w = 0; }

__global__ __launch_bounds__(256) void crc32c_kernel(const uint8_t *data, int64_t n,
                                                     int64_t n_waves, uint32_t finish,
                                                     uint32_t *out) {
  __shared__ uint32_t ts[16][256];
  __shared__ uint32_t tm[4][256];
  for (int i = threadIdx.x; i < 16 * 256; i += 256) ts[i >> 8][i & 255] = c_slice16.t[i >> 8][i & 255];
  for (int i = threadIdx.x; i < 4 * 256; i += 256) tm[i >> 8][i & 255] = c_shift1024.t[i >> 8][i & 255];
  __syncthreads();
  __shared__ uint32_t wave_acc[4];
  const int wib = threadIdx.x >> 6;
  const int64_t wave = (int64_t)blockIdx.x * 4 + wib;
  const int lane = threadIdx.x & 63;
  // blocks are laid out back from the end like the waves: the last block is
  // full, the first may hold waves before the first segment (all zero)
  const int64_t n_blocks = (n_waves + 3) / 4;
  const int64_t vwave = wave - (n_blocks * 4 - n_waves);  // < 0: before byte 0
  const int64_t n16 = n & ~(int64_t)15;
  const int64_t seg = n16 - (n_waves - vwave) * kCrcSeg;
  uint32_t acc = 0;
  for (int k = 0; k < kCrcIter; ++k) {
    const int64_t p = seg + 1024 * k + 16 * lane;
    uint4 w = {0u, 0u, 0u, 0u};
    if (p >= 0) w = *reinterpret_cast<const uint4 *>(data + p);
    acc = tm[0][acc & 0xffu] ^ tm[1][(acc >> 8) & 0xffu] ^ tm[2][(acc >> 16) & 0xffu] ^ tm[3][acc >> 24];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 16; ++q) acc ^= ts[15 - q][(ws[q >> 2] >> (8 * (q & 3))) & 0xffu];
  }
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const uint32_t other = __shfl_xor(acc, 1 << j);
    const uint32_t sh = mat_apply_dev(c_shifts.m[4 + j], acc) ^ other;
    if ((lane & (1 << j)) == 0) acc = sh;
  }
  // lane 0 holds the wave's raw CRC aligned at its segment end; the block's
  // four segments are consecutive, so wave w's value moves (3-w) segments
  if (lane == 0) {
    const int k = 3 - wib;
    if (k & 1) acc = mat_apply_dev(c_shifts.m[kCrcSegLog2], acc);
    if (k & 2) acc = mat_apply_dev(c_shifts.m[kCrcSegLog2 + 1], acc);
    wave_acc[wib] = acc;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  acc = wave_acc[0] ^ wave_acc[1] ^ wave_acc[2] ^ wave_acc[3];
  const int64_t block_end = seg + (int64_t)(4 - wib) * kCrcSeg;  // wib == 0 here
  uint64_t d = (uint64_t)(n - block_end);
  for (int j = 0; j < crc::kShiftBits && d; ++j, d >>= 1)
    if (d & 1u) acc = mat_apply_dev(c_shifts.m[j], acc);
  if (blockIdx.x == 0) {
    uint32_t t = 0;
    for (int64_t i = n16; i < n; ++i) t = c_byte.t[(t ^ data[i]) & 0xffu] ^ (t >> 8);
    acc ^= t ^ finish;
  }
  atomicXor(out, acc);
}

// Payload body of a page: for each layer of [layer_lo, layer_lo+n_layers),
// kind (K, V) and kv head, the rows of tokens [t0, t0+count) in the
// reference layout ((D/32) blocks of LE f16 scale + 32 int8).
//
// A unit is one page tile (TT = min(32, page_tokens) slots) of one (layer,
// kind, kv head) that the range touches.  In the page, the tile's codes
// (TT*D bytes) and scales (TT*D/32 f16) are two contiguous, 16-byte aligned
// runs; in the body, its rows are one contiguous, 8-byte aligned run.  So
// both kernels move each side with wide coalesced accesses and do the byte
// permutation in LDS: pack reads the tile and writes the rows, unpack reads
// the rows and the tile (slots outside the range keep their bytes) and
// writes the tile back.
struct BodyMap {
  Geo g;
  int64_t layer_stride;
  int32_t layer_lo, n_layers;
  int32_t t0, count;
  int32_t NB;
  int32_t tile0, n_tiles;  // page tiles touched: [tile0, tile0 + n_tiles) in units of TT
  __host__ __device__ int64_t units() const {
    return (int64_t)n_layers * 2 * g.kv_heads * n_tiles;
  }
};

constexpr int kMaxTileBytes = 32 * 256;       // TT * D
constexpr int kMaxRowRun = 32 * 8 * 34;       // TT rows * NB blocks * 34 bytes

struct Unit {
  int32_t layer, kind, kvh;
  int32_t p0, s_lo, s_hi;  // tile start position, slots [s_lo, s_hi) in range
  int32_t TT;
  int64_t body_off;        // body byte offset of the unit's first row
};

__device__ __forceinline__ Unit unit_of(const BodyMap &m, int64_t u) {
  Unit r;
  r.TT = tile_tokens(m.g.page_tokens);
  const int32_t j = (int32_t)(u % m.n_tiles);
  int64_t q = u / m.n_tiles;
  r.kvh = (int32_t)(q % m.g.kv_heads);
  q /= m.g.kv_heads;
  r.kind = (int32_t)(q & 1);
  r.layer = m.layer_lo + (int32_t)(q >> 1);
  r.p0 = (m.tile0 + j) * r.TT;
  const int32_t a = max(m.t0, r.p0), b = min(m.t0 + m.count, r.p0 + r.TT);
  r.s_lo = a - r.p0;
  r.s_hi = b - r.p0;
  const int64_t RB = (int64_t)m.NB * 34;
  r.body_off = ((((int64_t)(r.layer - m.layer_lo) * 2 + r.kind) * m.g.kv_heads + r.kvh) * m.count +
                (a - m.t0)) * RB;
  return r;
}

// LDS tile offsets: code (s, d) and the f16 scale (s, b) of a tile
__device__ __forceinline__ int32_t tile_code(int32_t kind, int32_t TT, int32_t D, int32_t s, int32_t d) {
  return kind == 0 ? s * D + d : d * TT + s;
}
__device__ __forceinline__ int32_t tile_scale(int32_t TT, int32_t s, int32_t b) {
  return 2 * (b * TT + (TT == 32 ? (int32_t)scale_pos32((uint32_t)s) : s));
}

__global__ __launch_bounds__(256) void pack_kernel(BodyMap m, const uint8_t *pages,
                                                   const int32_t *bt, uint8_t *body,
                                                   int32_t *fault) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kMaxTileBytes + 512];
  __shared__ __attribute__((aligned(16))) uint8_t rows[kMaxRowRun];
  const Unit u = unit_of(m, blockIdx.x);
  const int32_t D = m.g.head_dim, NB = m.NB, TT = u.TT;
  const int32_t page = bt[u.p0 / m.g.page_tokens];
  if (page < 0 || page >= m.g.num_pages) {
    if (threadIdx.x == 0) atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot0 = u.p0 % m.g.page_tokens;
  const uint8_t *region = pages + u.layer * m.layer_stride + region_base(m.g, page, u.kvh, u.kind);
  const uint4 *codes = reinterpret_cast<const uint4 *>(region + code_offset(m.g, u.kind, slot0, 0));
  const uint4 *scales = reinterpret_cast<const uint4 *>(region + scale_offset(m.g, slot0, 0));
  const int32_t nc = TT * D / 16, ns = TT * NB * 2 / 16;
  for (int32_t i = threadIdx.x; i < nc + ns; i += 256)
    reinterpret_cast<uint4 *>(tile)[i] = i < nc ? codes[i] : scales[i - nc];
  __syncthreads();
  const uint8_t *tsc = tile + TT * D;
  const uint8_t bias = code_bias(u.kind);
  const int32_t nrows = u.s_hi - u.s_lo;
  for (int32_t i = threadIdx.x; i < nrows * NB; i += 256) {
    const int32_t s = u.s_lo + i / NB, b = i % NB;
    uint8_t *dst = rows + (i / NB) * NB * 34 + b * 34;
    const int32_t so = tile_scale(TT, s, b);
    dst[0] = tsc[so];
    dst[1] = tsc[so + 1];
    for (int32_t k = 0; k < 32; ++k) dst[2 + k] = tile[tile_code(u.kind, TT, D, s, 32 * b + k)] ^ bias;
  }
  __syncthreads();
  uint2 *out = reinterpret_cast<uint2 *>(body + u.body_off);
  for (int32_t i = threadIdx.x; i < nrows * NB * 34 / 8; i += 256)
    out[i] = reinterpret_cast<const uint2 *>(rows)[i];
}

__global__ __launch_bounds__(256) void unpack_kernel(BodyMap m, uint8_t *pages, const int32_t *bt,
                                                     const uint8_t *body, int32_t *fault) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kMaxTileBytes + 512];
  __shared__ __attribute__((aligned(16))) uint8_t rows[kMaxRowRun];
  const Unit u = unit_of(m, blockIdx.x);
  const int32_t D = m.g.head_dim, NB = m.NB, TT = u.TT;
  const int32_t page = bt[u.p0 / m.g.page_tokens];
  if (page < 0 || page >= m.g.num_pages) {
    if (threadIdx.x == 0) atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot0 = u.p0 % m.g.page_tokens;
  uint8_t *region = pages + u.layer * m.layer_stride + region_base(m.g, page, u.kvh, u.kind);
  uint4 *codes = reinterpret_cast<uint4 *>(region + code_offset(m.g, u.kind, slot0, 0));
  uint4 *scales = reinterpret_cast<uint4 *>(region + scale_offset(m.g, slot0, 0));
  const int32_t nc = TT * D / 16, ns = TT * NB * 2 / 16;
  const int32_t nrows = u.s_hi - u.s_lo;
  const bool whole = nrows == TT;
  if (!whole)  // slots outside the range keep their bytes
    for (int32_t i = threadIdx.x; i < nc + ns; i += 256)
      reinterpret_cast<uint4 *>(tile)[i] = i < nc ? codes[i] : scales[i - nc];
  const uint2 *in = reinterpret_cast<const uint2 *>(body + u.body_off);
  for (int32_t i = threadIdx.x; i < nrows * NB * 34 / 8; i += 256)
    reinterpret_cast<uint2 *>(rows)[i] = in[i];
  __syncthreads();
  uint8_t *tsc = tile + TT * D;
  const uint8_t bias = code_bias(u.kind);
  for (int32_t i = threadIdx.x; i < nrows * NB; i += 256) {
    const int32_t s = u.s_lo + i / NB, b = i % NB;
    const uint8_t *src = rows + (i / NB) * NB * 34 + b * 34;
    const int32_t so = tile_scale(TT, s, b);
    tsc[so] = src[0];
    tsc[so + 1] = src[1];
    for (int32_t k = 0; k < 32; ++k) tile[tile_code(u.kind, TT, D, s, 32 * b + k)] = src[2 + k] ^ bias;
  }
  __syncthreads();
  for (int32_t i = threadIdx.x; i < nc + ns; i += 256) {
    const uint4 v = reinterpret_cast<const uint4 *>(tile)[i];
    if (i < nc) codes[i] = v;
    else scales[i - nc] = v;
  }
}

// The 96 header bytes (already serialized on the host) at the page start,
// and the payload CRC word as 4 LE bytes after the body.
struct Header96 {
  uint32_t w[24];
};
__global__ void write_header_kernel(Header96 h, uint8_t *page) {
  if (threadIdx.x < 24) reinterpret_cast<uint32_t *>(page)[threadIdx.x] = h.w[threadIdx.x];
}
__global__ void store_word_kernel(const uint32_t *w, uint8_t *dst) {
  const uint32_t v = *w;
  dst[0] = (uint8_t)v;
  dst[1] = (uint8_t)(v >> 8);
  dst[2] = (uint8_t)(v >> 16);
  dst[3] = (uint8_t)(v >> 24);
}

int64_t body_blocks(const BodyMap &m) {
  return (int64_t)m.n_layers * 2 * m.g.kv_heads * m.count * m.NB;
}

BodyMap body_map(const R4kvLaunch &r) {
  BodyMap m{r.g, r.layer_stride, r.layer_lo, r.n_layers, r.t0, r.count, r.g.head_dim / 32, 0, 0};
  const int32_t TT = tile_tokens(r.g.page_tokens);
  if (r.count > 0) {
    m.tile0 = r.t0 / TT;
    m.n_tiles = (r.t0 + r.count - 1) / TT - m.tile0 + 1;
  }
  return m;
}

}  // namespace

hipError_t launch_crc32c(const uint8_t *data, int64_t n, uint32_t *out, hipStream_t s) {
  hipLaunchKernelGGL(zero_word_kernel, dim3(1), dim3(1), 0, s, out);
  if (n <= 0) return hipGetLastError();
  const int64_t n16 = n & ~(int64_t)15;
  int64_t waves = (n16 + kCrcSeg - 1) / kCrcSeg;
  if (waves == 0) waves = 1;
  const int64_t blocks = (waves + 3) / 4;  // the kernel derives the same count
  hipLaunchKernelGGL(crc32c_kernel, dim3((unsigned)blocks), dim3(256), 0, s, data, n, waves,
                     crc::finish_term((uint64_t)n), out);
  return hipGetLastError();
}

hipError_t launch_r4kv_pack(const R4kvLaunch &r, const uint8_t *pages, const int32_t *bt,
                            uint8_t *page_out, uint32_t *crc_word, int32_t *fault, hipStream_t s) {
  const BodyMap m = body_map(r);
  Header96 h;
  for (int i = 0; i < 24; ++i)
    h.w[i] = (uint32_t)r.header[4 * i] | ((uint32_t)r.header[4 * i + 1] << 8) |
             ((uint32_t)r.header[4 * i + 2] << 16) | ((uint32_t)r.header[4 * i + 3] << 24);
  hipLaunchKernelGGL(write_header_kernel, dim3(1), dim3(64), 0, s, h, page_out);
  const int64_t nb = body_blocks(m);
  uint8_t *body = page_out + 96;
  if (m.units() > 0)
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)m.units()), dim3(256), 0, s, m, pages, bt, body,
                       fault);
  hipError_t e = launch_crc32c(body, nb * 34, crc_word, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(store_word_kernel, dim3(1), dim3(1), 0, s, crc_word, body + nb * 34);
  return hipGetLastError();
}

hipError_t launch_r4kv_unpack(const R4kvLaunch &r, uint8_t *pages, const int32_t *bt,
                              const uint8_t *body, int32_t *fault, hipStream_t s) {
  const BodyMap m = body_map(r);
  if (m.units() > 0)
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)m.units()), dim3(256), 0, s, m, pages, bt,
                       body, fault);
  return hipGetLastError();
}

}  // namespace rkv
