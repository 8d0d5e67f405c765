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

// Flat-layout combine.  Block (row, entry, slice) merges all of the entry's
// partitions (from the header the decode wrote) for one slice of the row's
// dimensions.  With one slice and up to 16 partitions: one thread per
// dimension, all loads in one round, no LDS.  Otherwise the slice's
// head_dim/slices dims are read as float4s by LP lanes per partition and the
// block's 256/LP lane groups take partitions g, g + groups, ...  Every block
// first merges the row's (m, l) pairs into (M, L) and then sums
// o_i * 2^(m_i - M) over its partitions; the o loads of the first 8
// partitions per group are issued before the (m, l) loads, so both land in
// one round.  Slicing by dimension gives rows with long partition lists
// (config 3: 16 rows, 512 partitions) enough blocks in one launch, with no
// second launch to merge splits.  All merges are the chunk combine of
// attention.rs:205-212 in base 2.
__device__ __forceinline__ void merge_ml(float &m, float &l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
  const float b = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - mn);
  l = l * a + l2 * b;
  m = mn;
}

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

__global__ __launch_bounds__(256) void combine_flat_kernel(FlatCombineLaunch c) {
  const int row = blockIdx.x;  // j * q_heads + h
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  const int j = row / c.q_heads, h = row % c.q_heads;
  const int q_per_kv = c.q_heads / c.kv_heads;
  const int kvh = h / q_per_kv;
  const int R = c.q_len * q_per_kv;
  const int r = j * q_per_kv + h % q_per_kv;
  const int32_t start = c.hdr[1 + 2 * b];
  int32_t n = c.hdr[2 + 2 * b];
  if (start < 0 || n < 1 || start > c.n_wg - n) n = 0;
  const int64_t p0 = ((int64_t)kvh * c.n_wg + start) * R + r;  // partition i at p0 + i*R
  const int64_t orow = (int64_t)b * c.q_len * c.q_heads + row;

  if (gridDim.z == 1 && n <= 16) {
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

  const int CH = c.head_dim / (int)gridDim.z;  // dims of this slice (>= 16)
  const int LP = CH / 4;                       // lanes per partition
  const int NG = 256 / LP;                     // partition groups
  const int grp = t / LP, dt = t % LP;
  const int dim = blockIdx.z * CH + 4 * dt;
  const int lane = t & 63, wave = t >> 6;

  constexpr int kB = 8;  // partitions per group and load round
  // first batch of this group's partitions: o and m
  float mi[kB];
  float4 ov[kB];
#pragma unroll
  for (int k = 0; k < kB; ++k) {
    const int32_t i = grp + k * NG;
    const int64_t pr = p0 + (int64_t)i * R;
    const bool in = i < n;
    ov[k] = in ? *reinterpret_cast<const float4 *>(c.o + pr * c.head_dim + dim)
               : float4{0.f, 0.f, 0.f, 0.f};
    mi[k] = in ? c.ml[2 * pr] : -INFINITY;
  }

  // (M, L) of the row over all n partitions
  float m = -INFINITY, l = 0.0f;
  for (int32_t i = t; i < n; i += 256) {
    const float2 v = *reinterpret_cast<const float2 *>(c.ml + 2 * (p0 + (int64_t)i * R));
    merge_ml(m, l, v.x, v.y);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
    merge_ml(m, l, m2, l2);
  }
  __shared__ float s_m[4], s_l[4];
  __shared__ float4 s_o[4][64];
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
  __syncthreads();
  float M = s_m[0], L = s_l[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) merge_ml(M, L, s_m[w], s_l[w]);

  float4 acc{0.f, 0.f, 0.f, 0.f};
  for (int32_t i0 = grp;;) {
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const float w = mi[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mi[k] - M);
      acc.x += ov[k].x * w;
      acc.y += ov[k].y * w;
      acc.z += ov[k].z * w;
      acc.w += ov[k].w * w;
    }
    i0 += kB * NG;
    if (i0 >= n) break;
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int32_t i = i0 + k * NG;
      const int64_t pr = p0 + (int64_t)i * R;
      const bool in = i < n;
      ov[k] = in ? *reinterpret_cast<const float4 *>(c.o + pr * c.head_dim + dim)
                 : float4{0.f, 0.f, 0.f, 0.f};
      mi[k] = in ? c.ml[2 * pr] : -INFINITY;
    }
  }
  // sum over the groups: lanes LP apart in a wave, then the 4 waves
  for (int off = LP; off < 64; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off);
    acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off);
    acc.w += __shfl_xor(acc.w, off);
  }
  if (lane < LP) s_o[wave][lane] = acc;
  __syncthreads();
  if (t >= LP) return;
  float4 o = s_o[0][t];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    o.x += s_o[w][t].x;
    o.y += s_o[w][t].y;
    o.z += s_o[w][t].z;
    o.w += s_o[w][t].w;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  store_res(c, orow * c.head_dim + dim, float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv});
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
  if (c.slices < 1 || (c.slices & (c.slices - 1)) || c.head_dim % c.slices || c.head_dim / c.slices < 16 ||
      c.head_dim / c.slices > 256)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(c.q_len * c.q_heads), (unsigned)c.batch, (unsigned)c.slices);
  hipLaunchKernelGGL(combine_flat_kernel, grid, dim3(256), 0, s, c);
  return hipGetLastError();
}

hipError_t launch_combine(const CombineLaunch &c, hipStream_t s) {
  if (c.batch == 0 || c.rows == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)c.rows, (unsigned)c.batch), dim3(256), 0, s, c);
  return hipGetLastError();
}

}  // namespace rkv
