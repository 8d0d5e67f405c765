// rkv_stream.hip -- HBM streaming-read ceiling for gfx950: the practical
// read rate the decode kernel is measured against, taken in the same run.
//
// Both modes read with the nontemporal cache policy, which streams about
// 15% faster than the default one, and both give each wave contiguous runs:
//  - vector mode: 1024-thread workgroups, each wave reading kVecLoads KiB
//    contiguous per round (one 16-byte load per lane per KiB, all in
//    flight), the waves of the grid taking the rounds in turn; the words read
//    are folded by xor into one word per workgroup and then into *out, so no
//    load can be dropped and the result is checkable;
//  - LDS-DMA mode, the decode's order and copy: one-wave workgroups each
//    streaming its own contiguous chunk with kDmaLoads 1 KiB global_load_lds
//    copies into a wave-private LDS ring, then waiting for them, round after
//    round.
#include "rkv_launch.h"

namespace rkv {
namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

constexpr int kVecLoads = 16;
constexpr int kDmaLoads = 16;  // 16 KiB in flight per wave, about one decode tile
constexpr int kNT = 2;         // cache policy bits: nontemporal

constexpr int kVecWaves = 16;  // waves per vector-mode workgroup

__global__ __launch_bounds__(64 * kVecWaves) void stream_read_vec_kernel(const v4i *p, int64_t n16,
                                                                         uint32_t *out) {
  __shared__ int32_t wave_acc[kVecWaves];
  const int64_t waves = (int64_t)gridDim.x * kVecWaves;
  const int wib = threadIdx.x >> 6;
  const int64_t w = (int64_t)blockIdx.x * kVecWaves + wib;
  const int lane = threadIdx.x & 63;
  constexpr int64_t kRound = 64 * kVecLoads;  // 16-byte items per wave round
  int32_t acc = 0;
  int64_t c = w * kRound;
  for (; c + kRound <= n16; c += waves * kRound) {
    v4i v[kVecLoads];
#pragma unroll
    for (int u = 0; u < kVecLoads; ++u) v[u] = __builtin_nontemporal_load(p + c + 64 * u + lane);
#pragma unroll
    for (int u = 0; u < kVecLoads; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  // the last, partial round (one wave takes it)
  if (c < n16) {
    for (int64_t i = c + lane; i < n16; i += 64) {
      const v4i v = __builtin_nontemporal_load(p + i);
      acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
  // one atomic per workgroup: same-address atomics serialize in L2
  if (lane == 0) wave_acc[wib] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t t = 0;
    for (int i = 0; i < kVecWaves; ++i) t ^= wave_acc[i];
    atomicXor(out, (uint32_t)t);
  }
}

// One wave per workgroup; chunk16 is a multiple of 64 * kDmaLoads, so every
// copy instruction is whole and inside the chunk.
__global__ __launch_bounds__(64) void stream_read_dma_kernel(const uint8_t *p, int64_t chunk) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kDmaLoads][1024];
  const uint8_t *base = p + (int64_t)blockIdx.x * chunk + 16 * threadIdx.x;
  for (int64_t off = 0; off < chunk; off += 1024 * kDmaLoads) {
#pragma unroll
    for (int u = 0; u < kDmaLoads; ++u)
      __builtin_amdgcn_global_load_lds(base + off + 1024 * u,
                                       (__attribute__((address_space(3))) void *)ring[u], 16, 0, kNT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// The decode's tile order over a pool's pages (see launch_stream_tiles):
// workgroup (entry b's partition, kv head) reads each 32-token tile of its
// partition as the decode stages it -- K codes, V codes (D/32 KiB each) and
// both scale runs (2*D bytes each, one copy) -- with nontemporal 1 KiB
// LDS-DMA copies, waits for them, and moves to the next tile.
template <int D>
__global__ __launch_bounds__(64) void stream_tiles_kernel(TileStreamLaunch t) {
  constexpr int kCodeCopies = D / 32;  // 1 KiB copies per code run of a tile
  constexpr int kCopies = 2 * kCodeCopies + 1;
  __shared__ __attribute__((aligned(1024))) uint8_t st[2][kCopies * 1024];
  const Geo g = t.g;
  const int lane = threadIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.x / t.parts, part = blockIdx.x % t.parts;
  // a partition starts on a 32-token tile, possibly inside a page; the host
  // checked that every partition spans at most 64 pages
  const int32_t tok0 = part * t.part_tokens;
  const int32_t tok_end = min(t.seq_tokens, tok0 + t.part_tokens);
  const int n_tiles = (tok_end - tok0) / 32;
  const int pg0 = tok0 / g.page_tokens;
  const int npg = (tok_end - 1) / g.page_tokens - pg0 + 1;
  int32_t pid = lane < npg ? t.bt[(int64_t)b * t.bt_stride + pg0 + lane] : 0;
  if (pid < 0 || pid >= g.num_pages) pid = 0;  // every copy stays inside the pool
  const uint64_t RB = region_bytes(g), PB = page_bytes(g);
  const uint32_t PTD = (uint32_t)g.page_tokens * D;
  // the scale copy: lanes [0, D/8) K scales, [D/8, D/4) V scales, the rest
  // re-read the K scales' first chunk
  const uint32_t sc_off = lane < D / 8 ? PTD + 16u * lane
                                       : (lane < D / 4 ? (uint32_t)RB + PTD + 16u * (lane - D / 8) : PTD);
  for (int i = 0; i < n_tiles; ++i) {
    const int32_t tk = tok0 + i * 32;
    const int32_t s0 = tk % g.page_tokens;
    const int32_t p = __builtin_amdgcn_readlane(pid, tk / g.page_tokens - pg0);
    const uint8_t *kb = t.pages + (uint64_t)p * PB + (uint64_t)(2 * kvh) * RB;
    uint8_t *dst = st[i & 1];
#pragma unroll
    for (int c = 0; c < kCodeCopies; ++c) {
      __builtin_amdgcn_global_load_lds(kb + (uint64_t)s0 * D + 1024 * c + 16 * lane,
                                       (__attribute__((address_space(3))) void *)(dst + 1024 * c), 16, 0, kNT);
      __builtin_amdgcn_global_load_lds(kb + RB + (uint64_t)s0 * D + 1024 * c + 16 * lane,
                                       (__attribute__((address_space(3))) void *)(dst + 1024 * (kCodeCopies + c)),
                                       16, 0, kNT);
    }
    __builtin_amdgcn_global_load_lds(kb + sc_off + (uint64_t)s0 * (D / 16),
                                     (__attribute__((address_space(3))) void *)(dst + 1024 * (2 * kCodeCopies)),
                                     16, 0, kNT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

__global__ void clear_word_kernel(uint32_t *w) { *w = 0u; }

}  // namespace

int64_t stream_read_dma_unit() { return 1024LL * kDmaLoads; }

hipError_t launch_stream_tiles(const TileStreamLaunch &t, hipStream_t s) {
  const dim3 grid((unsigned)(t.n_seqs * t.parts), (unsigned)t.g.kv_heads);
  if (t.g.head_dim == 256)
    hipLaunchKernelGGL(stream_tiles_kernel<256>, grid, dim3(64), 0, s, t);
  else
    hipLaunchKernelGGL(stream_tiles_kernel<128>, grid, dim3(64), 0, s, t);
  return hipGetLastError();
}

hipError_t launch_stream_read(const uint8_t *data, int64_t bytes, int32_t mode, int32_t blocks,
                              uint32_t *out, hipStream_t s) {
  if (mode == 0) {
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, out);
    hipLaunchKernelGGL(stream_read_vec_kernel, dim3((unsigned)blocks), dim3(64 * kVecWaves), 0, s,
                       reinterpret_cast<const v4i *>(data), bytes / 16, out);
  } else {
    hipLaunchKernelGGL(stream_read_dma_kernel, dim3((unsigned)blocks), dim3(64), 0, s, data,
                       bytes / blocks);
  }
  return hipGetLastError();
}

}  // namespace rkv
