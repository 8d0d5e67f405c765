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

__global__ void clear_word_kernel(uint32_t *w) { *w = 0u; }

}  // namespace

int64_t stream_read_dma_unit() { return 1024LL * kDmaLoads; }

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
