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

template <int D, int NS>
hipError_t launch_decode_d(const DecodeLaunch &d, int NT, hipStream_t s) {
  if (NT == 1) return launch_decode_t<D, 1, NS>(d, s);
  return launch_decode_t<D, 2, NS>(d, s);
}

}  // namespace

hipError_t launch_decode(const DecodeLaunch &d, hipStream_t s) {
  if (d.batch == 0 || d.n_parts == 0) return hipSuccess;
  const int R = d.q_len * (d.q_heads / d.g.kv_heads);
  const int NT = R <= 8 ? 1 : (R <= 16 ? 2 : 4);
  if (NT == 4) return launch_decode_rows32(d, s);
  const bool three = d.stages != 2;
  if (d.g.head_dim == 256)
    return three ? launch_decode_d<256, 3>(d, NT, s) : launch_decode_d<256, 2>(d, NT, s);
  return three ? launch_decode_d<128, 3>(d, NT, s) : launch_decode_d<128, 2>(d, NT, s);
}

hipError_t launch_combine(const CombineLaunch &c, hipStream_t s) {
  if (c.batch == 0 || c.rows == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)c.rows, (unsigned)c.batch), dim3(256), 0, s, c);
  return hipGetLastError();
}

}  // namespace rkv
