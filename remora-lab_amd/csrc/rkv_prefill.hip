// rkv_prefill.hip -- chunked prefill attention over paged Q8_0 K/V for gfx950.
//
// The reference's chunked prefill (har-serve/src/adapter.rs:31-60,
// BatchStepModel::prefill_batch) folds the one-token step over the chunk:
// query row i of a chunk that starts after ctx cached tokens sees exactly
// the decode of length ctx+i+1 (attention.rs:148-165 over positions
// [0, ctx+i]).  Here one workgroup of 8 waves takes a block of 128 query
// rows of one (entry, kv head) -- tq = 128 / (q_heads/kv_heads) chunk tokens
// times the q heads that share the kv head -- so each K/V tile staged in
// LDS is read from memory once per 128 rows.  Wave w owns rows 16w..16w+15;
// the per-tile work (int8 QK MFMA with exact K dequant, base-2 online
// softmax, f16 PV MFMA) is the decode kernel's, with the causal limit of
// every row at ctx + its token + 1; the V codes of each tile are widened to
// f16 once per workgroup (each wave its share) instead of once per wave.
// The block walks its whole causal range [0, ctx + last token of the
// block], with the range's page ids staged in an LDS list.  Output rows are
// written normalized; no workspace.
#include "rkv_decode_kernel.h"

namespace rkv {
namespace {

template <int D, bool kSmall, int NS>
__global__ __launch_bounds__(64 * kPrefillWaves, 2) void prefill_kernel(PrefillLaunch pf) {
#if defined(__HIP_DEVICE_COMPILE__)
  using Dec = Decoder<D, 2, kSmall, NS, kPrefillWaves, true, true>;
  using S = StageShape<D>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS][S::kAlloc];
  __shared__ int32_t page_list[kPrefillMaxPages];
  __shared__ __attribute__((aligned(16))) uint8_t v_f16[D * 64];  // the tile's V as f16
  const DecodeLaunch &p = pf.d;
  const Geo g = p.g;

  // entry of this row block (the table is in the kernel arguments); an
  // entry's row blocks are taken last block first (longest causal range
  // first, as the entries themselves are ordered)
  const int32_t x = (int32_t)blockIdx.x;
  int e = 0;
  while (e + 1 < pf.n_entries && x >= pf.first[e + 1]) ++e;
  const int32_t rb = pf.first[e + 1] - 1 - x;
  const int32_t seq = pf.seq[e], ctx = pf.ctx[e], n = pf.rows[e];
  const int32_t j0 = pf.tq * rb;
  const int32_t jn = min(pf.tq, n - j0);
  const int32_t len = ctx + j0 + jn;  // causal extent of the block's last token
  if (seq < 0 || seq >= p.n_seqs || jn <= 0) {
    if (threadIdx.x == 0) atomicOr(p.fault, FAULT_BAD_SEQ);
    return;
  }
  const int32_t npg = (len + g.page_tokens - 1) / g.page_tokens;
  if (len > p.bt_stride * g.page_tokens || npg > kPrefillMaxPages) {
    if (threadIdx.x == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  // the block's page ids; bad entries are reported and replaced by page 0 so
  // every copy stays inside the pool
  for (int32_t i = threadIdx.x; i < npg; i += 64 * kPrefillWaves) {
    int32_t pid = p.bt[(int64_t)seq * p.bt_stride + i];
    if (pid < 0 || pid >= g.num_pages) {
      atomicOr(p.fault, FAULT_BAD_PAGE);
      pid = 0;
    }
    page_list[i] = pid;
  }
  __syncthreads();

  Dec dc(p);
  dc.lane = threadIdx.x & 63;
  dc.wave = (int)(threadIdx.x >> 6);
  dc.li = dc.lane & 15;
  dc.lg = dc.lane >> 4;
  const int lane = dc.lane, li = dc.li, lg = dc.lg;
  const int kvh = blockIdx.y;
  const int r0 = 16 * dc.wave;
  dc.kvh = kvh;
  dc.b = e;
  dc.seq = seq;
  dc.len = len;
  dc.tok0 = 0;
  dc.tok_end = len;
  dc.n_tiles = (len + kTile - 1) / kTile;
  dc.app_mode = 0;
  dc.pg_first = 0;
  dc.pidv = 0;
  dc.pg_lds = (const __attribute__((address_space(3))) int32_t *)page_list;
  dc.vf16 = (lds_u8 *)v_f16;

  const int32_t G = p.q_heads / g.kv_heads;  // rows of one chunk token
  // row r of the block: chunk token j0 + r / G, q head kvh*G + r % G
  float qmul[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = r0 + 8 * nt + (li & 7);
    const int jl = r / G;
    int64_t qbase = -1;
    if (jl < jn)
      qbase = ((int64_t)(pf.qoff[e] + j0 + jl) * p.q_heads + kvh * G + r % G) * D;
    load_q_planes<D>(p.q, p.q_bf16 != 0, qbase, li, lg, p.scale_log2, dc.qhi[nt], dc.qlo[nt],
                     qmul[nt]);
  }
  {
    const int r = r0 + li;  // softmax row of this lane (PV n-tile 0, column li)
    const int jl = r / G;
    dc.rmul[0] = li < 8 ? qmul[0] : qmul[1];
    dc.rlim[0] = jl < jn ? ctx + j0 + jl + 1 : 0;
    dc.mref[0] = -INFINITY;
    dc.lrun[0] = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) dc.oacc[0][m] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  make_plan<D, kSmall>(dc.plan, g, lane);
  dc.PB = page_bytes(g);
  dc.kv_base = p.pages + (uint64_t)kvh * 2u * region_bytes(g);

  dc.run((lds_u8 *)lds[0], (lds_u8 *)lds[1], (lds_u8 *)lds[NS - 1]);

  float l = dc.lrun[0];
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  const int r = r0 + li;
  const int jl = r / G;
  if (jl < jn) {
    const int64_t orow = (int64_t)(pf.qoff[e] + j0 + jl) * p.q_heads + kvh * G + r % G;
    store_out_row<D>(p.out, p.out_bf16 != 0, orow, dc.oacc[0], l, lg);
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <int D, int NS>
hipError_t launch_prefill_t(const PrefillLaunch &pf, hipStream_t s) {
  dim3 grid((unsigned)pf.first[pf.n_entries], (unsigned)pf.d.g.kv_heads);
  if (pf.d.g.page_tokens < kTile)
    hipLaunchKernelGGL((prefill_kernel<D, true, NS>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  else
    hipLaunchKernelGGL((prefill_kernel<D, false, NS>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill(const PrefillLaunch &pf, hipStream_t s) {
  if (pf.n_entries <= 0 || pf.first[pf.n_entries] <= 0) return hipSuccess;
  if (pf.d.g.head_dim == 256) return launch_prefill_t<256, 2>(pf, s);
  return launch_prefill_t<128, 2>(pf, s);
}

}  // namespace rkv
