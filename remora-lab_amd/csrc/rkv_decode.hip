// rkv_decode.hip -- launches of the paged Q8_0 flash-decode kernel
// (rkv_decode_kernel.h) for up to 16 query rows per kv head, and the split-K
// log-sum-exp combine kernel, for gfx950 (CDNA4).
//
// Built with -mllvm -amdgpu-mfma-vgpr-form: MFMA results and accumulators
// live in VGPRs, so the VALU work on them (K-scale FMAs, lazy rescale) needs
// no v_accvgpr_read/write copies.
#include "rkv_decode_kernel.h"

namespace rkv {

namespace {

// One 256-thread block per (batch entry, row); thread = dimension.  Partials
// are read once: (m, l) of every partition first (at most 64 in registers),
// then the o vectors with all loads of a group in flight together.
__global__ __launch_bounds__(256) void combine_kernel(CombineLaunch c) {
  const int row = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int32_t seq = c.seq_ids[b];
  const int32_t len = (seq >= 0 && seq < c.n_seqs) ? c.seq_lens[seq] : 0;
  const int32_t np = len > 0 ? min(c.n_parts, (len + c.part_tokens - 1) / c.part_tokens) : 0;
  const int64_t prow = ((int64_t)b * c.rows + row) * c.n_parts;
  const float2 *ml = reinterpret_cast<const float2 *>(c.ml) + prow;
  float M = -INFINITY;
  for (int i = 0; i < np; ++i) M = fmaxf(M, ml[i].x);
  float L = 0.0f, O = 0.0f;
  if (M != -INFINITY && d < c.head_dim) {
    const float *o = c.o + prow * c.head_dim + d;
    int i = 0;
    for (; i + 8 <= np; i += 8) {
      float w[8], ov[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ov[k] = o[(int64_t)(i + k) * c.head_dim];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float2 v = ml[i + k];
        w[k] = __builtin_amdgcn_exp2f(v.x - M);
        L += v.y * w[k];
        O += ov[k] * w[k];
      }
    }
    for (; i < np; ++i) {
      const float2 v = ml[i];
      const float w = __builtin_amdgcn_exp2f(v.x - M);
      L += v.y * w;
      O += o[(int64_t)i * c.head_dim] * w;
    }
  }
  if (d >= c.head_dim) return;
  const float r = L > 0.0f ? O / L : 0.0f;
  const int64_t oi = ((int64_t)b * c.rows + row) * c.head_dim + d;
  if (c.out_bf16) static_cast<uint16_t *>(c.out)[oi] = f32_to_bf16_rtne(r);
  else static_cast<float *>(c.out)[oi] = r;
}

// Flat-layout combine.  Block (row, entry, split) merges partitions
// [chunk*split, chunk*(split+1)) of the entry (from the header the decode
// wrote).  Up to 16 partitions: one thread per dimension,
// all loads in one round, no LDS.  More: groups of head_dim/4 threads (4 dims
// each, float4 loads), group g taking partitions g, g + groups, ... 16 at a
// time, merged online (running max, rescaled sums), then the groups merge
// through LDS.  With one split per row the block writes the output; with
// more it stores its (m, l, o) and combine_splits_kernel merges the splits in
// a second launch.  All merges are the chunk combine of attention.rs:205-212
// in base 2.
struct Merge {
  float m, l;
  float4 o;
  __device__ void add(float mi, float li, float4 oi) {
    if (mi == -INFINITY) return;
    const float mn = fmaxf(m, mi);
    const float a = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
    const float w = __builtin_amdgcn_exp2f(mi - mn);
    l = l * a + li * w;
    o.x = o.x * a + oi.x * w;
    o.y = o.y * a + oi.y * w;
    o.z = o.z * a + oi.z * w;
    o.w = o.w * a + oi.w * w;
    m = mn;
  }
};

__device__ __forceinline__ void store_res(const FlatCombineLaunch &c, int64_t oi, float4 res) {
  if (c.out_bf16) {
    uint16_t *dst = static_cast<uint16_t *>(c.out) + oi;
    const uint32_t w0 = (uint32_t)f32_to_bf16_rtne(res.x) | ((uint32_t)f32_to_bf16_rtne(res.y) << 16);
    const uint32_t w1 = (uint32_t)f32_to_bf16_rtne(res.z) | ((uint32_t)f32_to_bf16_rtne(res.w) << 16);
    *reinterpret_cast<uint2 *>(dst) = uint2{w0, w1};
  } else {
    *reinterpret_cast<float4 *>(static_cast<float *>(c.out) + oi) = res;
  }
}

__device__ __forceinline__ void store_row(const FlatCombineLaunch &c, int64_t orow, int dt,
                                          const Merge &t) {
  const float inv = t.l > 0.0f ? 1.0f / t.l : 0.0f;
  const float4 res = t.l > 0.0f ? float4{t.o.x * inv, t.o.y * inv, t.o.z * inv, t.o.w * inv}
                                : float4{0.f, 0.f, 0.f, 0.f};
  store_res(c, orow * c.head_dim + 4 * dt, res);
}

constexpr int kCombineThreads = 256;

__global__ __launch_bounds__(kCombineThreads) void combine_flat_kernel(FlatCombineLaunch c) {
  const int row = blockIdx.x;  // j * q_heads + h
  const int b = blockIdx.y;
  const int split = blockIdx.z;
  const int t = threadIdx.x;
  const int j = row / c.q_heads, h = row % c.q_heads;
  const int q_per_kv = c.q_heads / c.kv_heads;
  const int kvh = h / q_per_kv;
  const int R = c.q_len * q_per_kv;
  const int r = j * q_per_kv + h % q_per_kv;
  const int32_t start = c.hdr[1 + 2 * b];
  int32_t n = c.hdr[2 + 2 * b];
  if (start < 0 || n < 1 || start > c.n_wg - n) n = 0;
  const int32_t n_splits = n > 0 ? (n + c.chunk - 1) / c.chunk : 1;
  if (split >= n_splits) return;
  const int32_t i_beg = split * c.chunk;
  const int32_t i_end = min(n, i_beg + c.chunk);
  const int64_t p0 = ((int64_t)kvh * c.n_wg + start) * R + r;  // partition i at p0 + i*R
  const int64_t orow = (int64_t)b * c.q_len * c.q_heads + row;

  if (c.splits == 1 && n <= 16) {
    // one thread per dimension
    if (t >= c.head_dim) return;
    float2 ml[16];
    float ov[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool in = k < n;
      const int64_t pr = p0 + (int64_t)k * R;
      ml[k] = in ? *reinterpret_cast<const float2 *>(c.ml + 2 * pr) : float2{-INFINITY, 0.0f};
      ov[k] = in ? c.o[pr * c.head_dim + t] : 0.0f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; ++k) M = fmaxf(M, ml[k].x);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float w = ml[k].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[k].x - M);
        L += ml[k].y * w;
        O += ov[k] * w;
      }
    }
    const float res = L > 0.0f ? O / L : 0.0f;
    const int64_t oi = orow * c.head_dim + t;
    if (c.out_bf16) static_cast<uint16_t *>(c.out)[oi] = f32_to_bf16_rtne(res);
    else static_cast<float *>(c.out)[oi] = res;
    return;
  }

  const int GS = c.head_dim / 4;          // threads per group
  const int NG = kCombineThreads / GS;    // groups
  const int grp = t / GS, dt = t % GS;
  Merge mg{-INFINITY, 0.0f, {0.f, 0.f, 0.f, 0.f}};
  for (int32_t i0 = i_beg + grp; i0 < i_end; i0 += 16 * NG) {
    float2 ml[16];
    float4 ov[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int32_t i = i0 + k * NG;
      const int64_t pr = p0 + (int64_t)i * R;
      const bool in = i < i_end;
      ml[k] = in ? *reinterpret_cast<const float2 *>(c.ml + 2 * pr) : float2{-INFINITY, 0.0f};
      ov[k] = in ? *reinterpret_cast<const float4 *>(c.o + pr * c.head_dim + 4 * dt)
                 : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) mg.add(ml[k].x, ml[k].y, ov[k]);
  }

  __shared__ float s_m[8], s_l[8];
  __shared__ float4 s_o[8][64];
  if (dt == 0) {
    s_m[grp] = mg.m;
    s_l[grp] = mg.l;
  }
  s_o[grp][dt] = mg.o;
  __syncthreads();
  if (grp != 0) return;
  Merge tot{-INFINITY, 0.0f, {0.f, 0.f, 0.f, 0.f}};
  for (int g = 0; g < NG; ++g) tot.add(s_m[g], s_l[g], s_o[g][dt]);
  if (c.splits == 1) {
    store_row(c, orow, dt, tot);
    return;
  }
  if (dt == 0)
    *reinterpret_cast<float2 *>(c.split_ml + 2 * (orow * c.splits + split)) = float2{tot.m, tot.l};
  *reinterpret_cast<float4 *>(c.split_o + (orow * c.splits + split) * c.head_dim + 4 * dt) = tot.o;
}

// Second level: merge the splits of every (row, entry), head_dim/4 threads.
__global__ __launch_bounds__(64) void combine_splits_kernel(FlatCombineLaunch c) {
  const int row = blockIdx.x;
  const int b = blockIdx.y;
  const int dt = threadIdx.x;
  if (dt >= c.head_dim / 4) return;
  int32_t n = c.hdr[2 + 2 * b];
  const int32_t start = c.hdr[1 + 2 * b];
  if (start < 0 || n < 1 || start > c.n_wg - n) n = 0;
  const int32_t n_splits = n > 0 ? min(c.splits, (n + c.chunk - 1) / c.chunk) : 0;
  const int64_t orow = (int64_t)b * c.q_len * c.q_heads + row;
  Merge tot{-INFINITY, 0.0f, {0.f, 0.f, 0.f, 0.f}};
  for (int32_t q0 = 0; q0 < n_splits; q0 += 8) {
    float2 ml[8];
    float4 ov[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool in = q0 + k < n_splits;
      const int64_t sp = orow * c.splits + q0 + k;
      ml[k] = in ? *reinterpret_cast<const float2 *>(c.split_ml + 2 * sp) : float2{-INFINITY, 0.0f};
      ov[k] = in ? *reinterpret_cast<const float4 *>(c.split_o + sp * c.head_dim + 4 * dt)
                 : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) tot.add(ml[k].x, ml[k].y, ov[k]);
  }
  store_row(c, orow, dt, tot);
}

template <int D, int NS>
hipError_t launch_decode_d(const DecodeLaunch &d, int NT, hipStream_t s) {
  if (NT == 1) return launch_decode_t<D, 1, NS>(d, s);
  return launch_decode_t<D, 2, NS>(d, s);
}

}  // namespace

hipError_t launch_decode(const DecodeLaunch &d, hipStream_t s) {
  if (d.batch == 0 || d.n_wg == 0) return hipSuccess;
  const int R = d.q_len * (d.q_heads / d.g.kv_heads);
  const int NT = R <= 8 ? 1 : (R <= 16 ? 2 : 4);
  if (NT == 4) return launch_decode_rows32(d, s);
  const bool three = d.stages != 2;
  if (d.g.head_dim == 256)
    return three ? launch_decode_d<256, 3>(d, NT, s) : launch_decode_d<256, 2>(d, NT, s);
  return three ? launch_decode_d<128, 3>(d, NT, s) : launch_decode_d<128, 2>(d, NT, s);
}

hipError_t launch_combine_flat(const FlatCombineLaunch &c, hipStream_t s) {
  if (c.batch == 0) return hipSuccess;
  const dim3 grid((unsigned)(c.q_len * c.q_heads), (unsigned)c.batch);
  hipLaunchKernelGGL(combine_flat_kernel, dim3(grid.x, grid.y, (unsigned)c.splits),
                     dim3(kCombineThreads), 0, s, c);
  if (c.splits > 1) hipLaunchKernelGGL(combine_splits_kernel, grid, dim3(64), 0, s, c);
  return hipGetLastError();
}

hipError_t launch_combine(const CombineLaunch &c, hipStream_t s) {
  if (c.batch == 0 || c.rows == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)c.rows, (unsigned)c.batch), dim3(256), 0, s, c);
  return hipGetLastError();
}

}  // namespace rkv
