// rkv_r4kv.hip -- R4KV page spill/restore kernels for gfx950: a device
// CRC32C (har/crates/r4kv/src/crc32c.rs) and the pack/unpack of a token
// range of Q8_0 rows between the page pool and a page payload.
//
// CRC32C.  Each wave covers a 64 KiB segment; the segments are laid out
// back from the end of the 16-byte-aligned prefix, so the first may start
// before byte 0 (those leading bytes read as zero, which leaves the raw CRC
// unchanged) and every 16-byte piece is aligned.  Lane l folds the pieces
// l, l+64, ... of its segment (Horner: shift the running value 1024 bytes,
// xor the piece's raw CRC from the slicing tables), the lanes combine in a
// 6-level tree of shifts by 16*2^j bytes, and the wave's value is shifted
// to the end of the message and xor-ed into the output word.  Wave 0 also
// adds the raw CRC of the unaligned tail and the init/final-xor term.
// Reads stay inside [0, n).
#include "rkv_crc32c.h"
#include "rkv_launch.h"

namespace rkv {
namespace {

constexpr int kCrcIter = 64;                       // pieces per lane
constexpr int64_t kCrcSeg = 16LL * 64 * kCrcIter;  // bytes per wave

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
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= n_waves) return;
  const int64_t n16 = n & ~(int64_t)15;
  const int64_t seg = n16 - (n_waves - wave) * kCrcSeg;
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
  if (lane != 0) return;
  uint64_t d = (uint64_t)(n - (seg + kCrcSeg));
  for (int j = 0; j < crc::kShiftBits && d; ++j, d >>= 1)
    if (d & 1u) acc = mat_apply_dev(c_shifts.m[j], acc);
  if (wave == 0) {
    uint32_t t = 0;
    for (int64_t i = n16; i < n; ++i) t = c_byte.t[(t ^ data[i]) & 0xffu] ^ (t >> 8);
    acc ^= t ^ finish;
  }
  atomicXor(out, acc);
}

// Payload body of a page: for each layer of [layer_lo, layer_lo+n_layers),
// kind (K, V) and kv head, the rows of tokens [t0, t0+count) in the
// reference layout ((D/32) blocks of LE f16 scale + 32 int8).  One thread
// per 34-byte block.
struct BodyMap {
  Geo g;
  int64_t layer_stride;
  int32_t layer_lo, n_layers;
  int32_t t0, count;
  int32_t NB;
  __device__ __forceinline__ int64_t blocks() const {
    return (int64_t)n_layers * 2 * g.kv_heads * count * NB;
  }
};

__global__ __launch_bounds__(256) void pack_kernel(BodyMap m, const uint8_t *pages,
                                                   const int32_t *bt, uint8_t *body,
                                                   int32_t *fault) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tid >= m.blocks()) return;
  const int32_t b = (int32_t)(tid % m.NB);
  int64_t r = tid / m.NB;
  const int32_t t = (int32_t)(r % m.count);
  r /= m.count;
  const int32_t kvh = (int32_t)(r % m.g.kv_heads);
  r /= m.g.kv_heads;
  const int32_t kind = (int32_t)(r & 1);
  const int32_t layer = m.layer_lo + (int32_t)(r >> 1);
  const int32_t pos = m.t0 + t;
  const int32_t page = bt[pos / m.g.page_tokens];
  uint8_t *dst = body + tid * 34;
  if (page < 0 || page >= m.g.num_pages) {
    atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot = pos % m.g.page_tokens;
  const uint8_t *region = pages + layer * m.layer_stride + region_base(m.g, page, kvh, kind);
  const uint16_t sc = *reinterpret_cast<const uint16_t *>(region + scale_offset(m.g, slot, b));
  dst[0] = (uint8_t)(sc & 0xffu);
  dst[1] = (uint8_t)(sc >> 8);
  const uint8_t bias = code_bias(kind);
  for (int i = 0; i < 32; ++i) dst[2 + i] = region[code_offset(m.g, kind, slot, b * 32 + i)] ^ bias;
}

__global__ __launch_bounds__(256) void unpack_kernel(BodyMap m, uint8_t *pages, const int32_t *bt,
                                                     const uint8_t *body, int32_t *fault) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tid >= m.blocks()) return;
  const int32_t b = (int32_t)(tid % m.NB);
  int64_t r = tid / m.NB;
  const int32_t t = (int32_t)(r % m.count);
  r /= m.count;
  const int32_t kvh = (int32_t)(r % m.g.kv_heads);
  r /= m.g.kv_heads;
  const int32_t kind = (int32_t)(r & 1);
  const int32_t layer = m.layer_lo + (int32_t)(r >> 1);
  const int32_t pos = m.t0 + t;
  const int32_t page = bt[pos / m.g.page_tokens];
  if (page < 0 || page >= m.g.num_pages) {
    atomicOr(fault, FAULT_BAD_PAGE);
    return;
  }
  const int32_t slot = pos % m.g.page_tokens;
  uint8_t *region = pages + layer * m.layer_stride + region_base(m.g, page, kvh, kind);
  const uint8_t *src = body + tid * 34;
  *reinterpret_cast<uint16_t *>(region + scale_offset(m.g, slot, b)) =
      (uint16_t)(src[0] | ((uint16_t)src[1] << 8));
  const uint8_t bias = code_bias(kind);
  for (int i = 0; i < 32; ++i) region[code_offset(m.g, kind, slot, b * 32 + i)] = src[2 + i] ^ bias;
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

}  // namespace

hipError_t launch_crc32c(const uint8_t *data, int64_t n, uint32_t *out, hipStream_t s) {
  hipLaunchKernelGGL(zero_word_kernel, dim3(1), dim3(1), 0, s, out);
  if (n <= 0) return hipGetLastError();
  const int64_t n16 = n & ~(int64_t)15;
  int64_t waves = (n16 + kCrcSeg - 1) / kCrcSeg;
  if (waves == 0) waves = 1;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL(crc32c_kernel, dim3((unsigned)blocks), dim3(256), 0, s, data, n, waves,
                     crc::finish_term((uint64_t)n), out);
  return hipGetLastError();
}

hipError_t launch_r4kv_pack(const R4kvLaunch &r, const uint8_t *pages, const int32_t *bt,
                            uint8_t *page_out, uint32_t *crc_word, int32_t *fault, hipStream_t s) {
  BodyMap m{r.g, r.layer_stride, r.layer_lo, r.n_layers, r.t0, r.count, r.g.head_dim / 32};
  Header96 h;
  for (int i = 0; i < 24; ++i)
    h.w[i] = (uint32_t)r.header[4 * i] | ((uint32_t)r.header[4 * i + 1] << 8) |
             ((uint32_t)r.header[4 * i + 2] << 16) | ((uint32_t)r.header[4 * i + 3] << 24);
  hipLaunchKernelGGL(write_header_kernel, dim3(1), dim3(64), 0, s, h, page_out);
  const int64_t nb = body_blocks(m);
  uint8_t *body = page_out + 96;
  if (nb > 0)
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, m, pages,
                       bt, body, fault);
  hipError_t e = launch_crc32c(body, nb * 34, crc_word, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(store_word_kernel, dim3(1), dim3(1), 0, s, crc_word, body + nb * 34);
  return hipGetLastError();
}

hipError_t launch_r4kv_unpack(const R4kvLaunch &r, uint8_t *pages, const int32_t *bt,
                              const uint8_t *body, int32_t *fault, hipStream_t s) {
  BodyMap m{r.g, r.layer_stride, r.layer_lo, r.n_layers, r.t0, r.count, r.g.head_dim / 32};
  const int64_t nb = body_blocks(m);
  if (nb > 0)
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, m, pages,
                       bt, body, fault);
  return hipGetLastError();
}

}  // namespace rkv
