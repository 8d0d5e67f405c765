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
// A block walks its causal range [0, ctx + last token of the block] in one
// workgroup, or, when the launch has too few blocks to fill the chip, in
// nseg workgroups that take a segment each and write unnormalized partials
// (m, l, o) to a workspace; a combine kernel then merges the segments of
// each row (the decode's split-K and LSE merge, here across a block's rows).
// The unit's page ids are staged in an LDS list.
#include "rkv_decode_kernel.h"

namespace rkv {
namespace {

// kQF16: a bf16 query, whose QK runs on f16 MFMA against K codes the
// workgroup widens once per tile (Decoder kF16K); an f32 query keeps the
// int8 QK with three query planes.
// kPre (with kQF16): the tiles come widened from the widening pass
// (PrefillLaunch::pre) and are copied into three f16 buffers; no stage ring
// and no page list.
template <int D, bool kSmall, int NS, bool kQF16, bool kPre = false>
__global__ __launch_bounds__(64 * kPrefillWaves, kPrefillWgsPerCu) void prefill_kernel(PrefillLaunch pf) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(!kPre || kQF16, "widened tiles feed the f16 QK");
  using Dec = Decoder<D, 2, kSmall, NS, kPrefillWaves, true, true, false, kQF16>;
  using S = StageShape<D>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kPre ? 1 : NS][kPre ? 1024 : S::kAlloc];
  __shared__ int32_t page_list[kPre ? 1 : kPrefillMaxPages];
  // kQF16: two f16 buffers, each a tile's K and V widened and its K scales
  // (Decoder::run_pipe widens tile t+1 into one while tile t is computed from
  // the other); kPre: three buffers of copied tile images; otherwise the
  // tile's V as f16
  __shared__ __attribute__((aligned(1024))) uint8_t
      f16buf[kPre ? 3 * Dec::kPBytes : (kQF16 ? 2 * Dec::kFBytes : D * 64)];
  __shared__ __attribute__((aligned(16))) uint8_t v_scl[kPrefillWaves * 2 * D];  // each wave's scaled V scales
  const DecodeLaunch &p = pf.d;
  const Geo g = p.g;

  // Unit of this workgroup.  Units are listed entry by entry (the entries
  // ordered by causal extent), an entry's segment by segment, a segment's kv
  // head by kv head, and a (segment, kv head)'s row blocks last first, so
  // they come about longest first (every segment but a block's last is seg
  // tokens long).  Workgroups go to the 8 XCDs round robin, and each XCD
  // takes chunks of xcd_chunk consecutive units (chunks xcd, xcd + 8, ...):
  // with chunks of 32, the row blocks that read one causal range share that
  // XCD's L2, which pays when the pages sit behind the host link.
  const uint32_t C = (uint32_t)max(pf.xcd_chunk, 1);
  const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
  const int64_t j = ((int64_t)xcd + 8 * (int64_t)(slot / C)) * C + slot % C;
  const int32_t H = g.kv_heads;
  if (j >= (int64_t)pf.first[pf.n_entries] * H) return;  // padding of the last chunks
  int e = 0;
  while (e + 1 < pf.n_entries && j >= (int64_t)pf.first[e + 1] * H) ++e;
  const int32_t ns = pf.nseg[e];
  const int32_t nb = (pf.first[e + 1] - pf.first[e]) / ns;  // row blocks of the entry
  const int32_t v = (int32_t)(j - (int64_t)pf.first[e] * H);
  const int32_t sg = v / (H * nb);
  const int kvh = (v / nb) % H;
  const int32_t rb = nb - 1 - v % nb;
  const int32_t seq = pf.seq[e], ctx = pf.ctx[e], n = pf.rows[e];
  const int32_t j0 = pf.tq * rb;
  const int32_t jn = min(pf.tq, n - j0);
  const int32_t len = ctx + j0 + jn;  // causal extent of the block's last token
  if (seq < 0 || seq >= p.n_seqs || jn <= 0) {
    if (threadIdx.x == 0) atomicOr(p.fault, FAULT_BAD_SEQ);
    return;
  }
  if (len > p.bt_stride * g.page_tokens) {
    if (threadIdx.x == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  // this unit's part of the causal range, tokens [tok0, tok_end): the whole
  // range, or segment sg (empty past the block's extent; seg is a multiple
  // of the tile and of the page, so every tile but the range's last is whole
  // and lies in the unit's pages)
  const int32_t tok0 = min(sg * pf.seg[e], len);
  const int32_t tok_end = ns == 1 ? len : min(len, tok0 + pf.seg[e]);
  const int32_t pg0 = tok0 / g.page_tokens;
  const int32_t npg = tok_end > tok0 ? (tok_end - 1) / g.page_tokens - pg0 + 1 : 0;
  if (npg > kPrefillMaxPages) {
    if (threadIdx.x == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  // the unit's page ids; bad entries are reported and replaced by page 0 so
  // every copy stays inside the pool (kPre: the widening pass did that)
  if constexpr (!kPre) {
    for (int32_t i = threadIdx.x; i < npg; i += 64 * kPrefillWaves) {
      int32_t pid = p.bt[(int64_t)seq * p.bt_stride + pg0 + i];
      if (pid < 0 || pid >= g.num_pages) {
        atomicOr(p.fault, FAULT_BAD_PAGE);
        pid = 0;
      }
      page_list[i] = pid;
    }
    __syncthreads();
  }

  Dec dc(p);
  dc.lane = threadIdx.x & 63;
  // uniform within a wave: a scalar, so that the per-wave choices (which
  // tile copies it issues, which chunks it widens) are scalar branches
  dc.wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  dc.swave = dc.wave;
  dc.li = dc.lane & 15;
  dc.lg = dc.lane >> 4;
  const int lane = dc.lane, li = dc.li, lg = dc.lg;
  const int r0 = 16 * dc.wave;
  dc.kvh = kvh;
  dc.b = e;
  dc.seq = seq;
  dc.len = len;
  dc.tok0 = tok0;
  dc.tok_end = tok_end;
  dc.n_tiles = (tok_end - tok0 + kTile - 1) / kTile;
  dc.app_mode = 0;
  dc.pg_first = pg0;
  dc.pidv = 0;
  dc.pg_lds = (const __attribute__((address_space(3))) int32_t *)page_list;
  dc.vf16 = (lds_u8 *)f16buf;
  dc.kf16 = (lds_u8 *)f16buf;
  dc.vsc = (lds_u8 *)v_scl + dc.wave * 2 * D;

  const int32_t G = p.q_heads / g.kv_heads;  // rows of one chunk token
  // row r of the block: chunk token j0 + r / G, q head kvh*G + r % G; the
  // wave's 16 rows take the 16x16x32 QK (Dec::kWide), lane (li, lg) row r0 + li
  static_assert(Dec::kWide, "prefill waves hold 16 rows");
  {
    const int r = r0 + li;  // query and softmax row of this lane (PV n-tile 0, column li)
    const int jl = r / G;
    const int64_t qbase =
        jl < jn ? ((int64_t)(pf.qoff[e] + j0 + jl) * p.q_heads + kvh * G + r % G) * D : -1;
    if constexpr (kQF16)
      load_q_f16<D>(static_cast<const uint16_t *>(p.q), qbase, lg, p.scale_log2, dc.qf, dc.rmul[0]);
    else
      load_q_wide<D>(p.q, p.q_bf16 != 0, qbase, lg, p.scale_log2, dc.qhi[0], dc.qmd[0], dc.qlo[0],
                     dc.rmul[0]);
    dc.rlim[0] = jl < jn ? ctx + j0 + jl + 1 : 0;
    dc.mref[0] = -INFINITY;
    dc.lrun[0] = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) dc.oacc[0][m] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  // chunk token j0 (row 0 of the block) attends the fewest positions
  dc.rlim_min = jn > 0 ? ctx + j0 + 1 : 0;
  make_plan<D, kSmall, false, kPrefillWaves>(dc.plan, g, lane, dc.swave);
  dc.PB = page_bytes(g);
  dc.kv_base = p.pages + (uint64_t)kvh * 2u * region_bytes(g);

  if constexpr (kPre) {
    // entry e's images: kv head after kv head, each its causal range's tiles
    const int64_t tiles_e = ((int64_t)ctx + n + kTile - 1) / kTile;
    dc.pre_src = pf.pre + (uint64_t)(pf.preoff[e] + kvh * tiles_e + tok0 / kTile) * Dec::kPBytes;
    dc.run_pre((lds_u8 *)f16buf, (lds_u8 *)f16buf + Dec::kPBytes, (lds_u8 *)f16buf + 2 * Dec::kPBytes);
  } else if constexpr (kQF16) {
    static_assert(NS == 2, "the pipelined prefill runs a two-stage ring");
    dc.run_pipe((lds_u8 *)lds[0], (lds_u8 *)lds[1], (lds_u8 *)f16buf, (lds_u8 *)f16buf + Dec::kFBytes);
  } else {
    dc.run((lds_u8 *)lds[0], (lds_u8 *)lds[1], (lds_u8 *)lds[NS - 1]);
  }
  dc.finish();

  float l = dc.lrun[0];
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  const int r = r0 + li;
  const int jl = r / G;
  if (jl < jn) {
    const int64_t erow = (int64_t)(j0 + jl) * p.q_heads + kvh * G + r % G;  // row within the entry
    if (ns == 1) {
      store_out_row<D>(p.out, p.out_bf16 != 0, (int64_t)pf.qoff[e] * p.q_heads + erow,
                       dc.oacc[0], l, lg);
    } else {
      const int64_t prow = pf.wsoff[e] + erow * ns + sg;
#pragma unroll
      for (int m = 0; m < D / 16; ++m)
        *reinterpret_cast<v4f *>(pf.ws_o + prow * D + 16 * m + 4 * lg) = dc.oacc[0][m];
      if (lg == 0) *reinterpret_cast<float2 *>(pf.ws_ml + 2 * prow) = float2{dc.mref[0], l};
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// The widening pass (PrefillLaunch::pre): one 256-thread workgroup per
// (entry, kv head, 32-token tile of the entry's causal range [0, ctx+rows)),
// in the order of the images: entry by entry (launch order), kv head by kv
// head, tile by tile.  It writes the tile as the f16 compute reads it from
// LDS (Decoder kFK/kFV/kFS, what widen_k, widen_v and widen_into produce
// from a staged tile), plus the V scales at kPVS:
//  - K: token row r as exact f16, 16-byte chunk c of the row at
//    c ^ (r mod D/8);
//  - V: chunk (dim d, k-group g) = the 8 tokens 4g..4g+3, 16+4g..16+4g+3 of
//    dim d as exact f16 (the codes are stored biased), at slot g ^ (d & 3);
//  - scales: each run [block][32 positions] in the staged order (position q
//    of a block holds token tok32(q)), V scales past the entry's end zeroed.
// Every tile is read from its pages once, instead of once per row block.
__device__ __forceinline__ int tok32(int q) {
  const int lg = q >> 3, i = (q >> 1) & 3;
  return (i < 2 ? 0 : 16) + 4 * lg + 2 * (i & 1) + (q & 1);
}

template <int D>
__global__ __launch_bounds__(256) void widen_tiles_kernel(PrefillLaunch pf) {
#if defined(__HIP_DEVICE_COMPILE__)
  using Dec = Decoder<D, 2, false, 2, kPrefillWaves, true, true, false, true>;
  const DecodeLaunch &p = pf.d;
  const Geo g = p.g;
  const int64_t x = blockIdx.x;
  if (x >= pf.preoff[pf.n_entries]) return;
  int e = 0;
  while (e + 1 < pf.n_entries && x >= pf.preoff[e + 1]) ++e;
  const int32_t len = pf.ctx[e] + pf.rows[e];
  const int64_t tiles = ((int64_t)len + kTile - 1) / kTile;
  const int64_t v = x - pf.preoff[e];
  const int kvh = (int)(v / tiles);
  const int32_t j = (int32_t)(v % tiles);
  const int32_t seq = pf.seq[e];
  uint8_t *dst = pf.pre + (uint64_t)x * Dec::kPBytes;
  const int tid = threadIdx.x;
  if (seq < 0 || seq >= p.n_seqs) return;  // the prefill kernel reports it
  // The tile's two 16-token halves each lie inside one page (page_tokens is a
  // multiple of 16).  Their page ids are looked up once; bad ids are reported
  // and read as page 0.  A half that starts past the entry's end (possible
  // only for the second: the tile's first token is inside the range) reads
  // the first half's page instead, since with 16-token pages it may have none.
  int32_t hpid[2], hslot[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int32_t pos = j * kTile + 16 * h < len ? j * kTile + 16 * h : j * kTile;
    hslot[h] = pos % g.page_tokens;
    int32_t pid = p.bt[(int64_t)seq * p.bt_stride + pos / g.page_tokens];
    if (pid < 0 || pid >= g.num_pages) {
      if (tid == 0) atomicOr(p.fault, FAULT_BAD_PAGE);
      pid = 0;
    }
    hpid[h] = pid;
  }
  // page and slot of tile token r (r < 32).  Tokens past the entry's end read
  // the tile's first token (written data: its K scale is finite); their V
  // scales are zeroed below and the causal mask drops their scores.
  auto page_of = [&](int r, int32_t &slot) -> int32_t {
    if (j * kTile + r < len) {
      slot = hslot[r >> 4] + (r & 15);
      return hpid[r >> 4];
    }
    slot = hslot[0];
    return hpid[0];
  };
  // K: 32 rows x D/16 chunks of 16 codes
  for (int c = tid; c < 32 * (D / 16); c += 256) {
    const int r = c / (D / 16), lc = c % (D / 16);
    int32_t slot;
    const int32_t pid = page_of(r, slot);
    const v4i w = *reinterpret_cast<const v4i *>(p.pages + region_base(g, pid, kvh, 0) +
                                                 code_offset(g, 0, slot, 16 * lc));
    v2h h[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) v8x4_to_f16((uint32_t)w[q] ^ 0x80808080u, h[2 * q], h[2 * q + 1]);
    const v8h f0 = {h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
    const v8h f1 = {h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
    uint8_t *row = dst + Dec::kFK + r * (2 * D);
    *reinterpret_cast<v8h *>(row + 16 * ((2 * lc) ^ (r & (D / 8 - 1)))) = f0;
    *reinterpret_cast<v8h *>(row + 16 * ((2 * lc + 1) ^ (r & (D / 8 - 1)))) = f1;
  }
  // V: one dim per thread, each half's 16 codes of the dim in one 16-byte
  // load (the V codes of a dim are contiguous within a 16-token half, at a
  // 16-byte aligned offset); chunk (d, g) takes tokens 4g..4g+3 of each half.
  // Codes past the entry's end are finite junk under zeroed V scales.
  for (int d = tid; d < D; d += 256) {
    v4i w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      w[h] = *reinterpret_cast<const v4i *>(p.pages + region_base(g, hpid[h], kvh, 1) +
                                            code_offset(g, 1, hslot[h], d));
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      v2h a0, a1, a2, a3;
      v8x4_to_f16((uint32_t)w[0][gq], a0, a1);
      v8x4_to_f16((uint32_t)w[1][gq], a2, a3);
      const v8h va = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
      *reinterpret_cast<v8h *>(dst + Dec::kFV + 16 * (4 * d + (gq ^ (d & 3)))) = va;
    }
  }
  // scales: kind, block, position
  for (int c = tid; c < 2 * D; c += 256) {
    const int kind = c / D, b = (c % D) / 32, q = c % 32;
    const int t = tok32(q);
    int32_t slot;
    const int32_t pid = page_of(t, slot);
    uint16_t sc = *reinterpret_cast<const uint16_t *>(p.pages + region_base(g, pid, kvh, kind) +
                                                      scale_offset(g, slot, b));
    if (kind == 1 && j * kTile + t >= len) sc = 0;  // past the entry's end: junk
    *reinterpret_cast<uint16_t *>(dst + (kind == 0 ? Dec::kFS : Dec::kPVS) + 2 * (32 * b + q)) = sc;
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// Rows of the split entries, one workgroup of 64 threads each, four
// dimensions a thread: merge the row's nseg partials in base 2 (M = max m,
// L = sum l 2^(m-M), O = sum o 2^(m-M)) and write O / L (0 when L is 0).
// Workgroup x takes row x - cfirst[k] of split entry k, cfirst[k] <= x <
// cfirst[k+1].
struct PrefillCombine {
  int32_t n_entries;
  int32_t q_heads;
  int32_t out_bf16;
  void *out;
  const float *ml, *o;
  int32_t cfirst[kPrefillMaxEntries + 1];  // rows * q_heads of the split entries, cumulative
  int32_t qoff[kPrefillMaxEntries];
  int32_t nseg[kPrefillMaxEntries];
  int64_t wsoff[kPrefillMaxEntries];
};

template <int D>
__global__ __launch_bounds__(64) void prefill_combine_kernel(PrefillCombine c) {
  const int32_t x = (int32_t)blockIdx.x;
  int e = 0;
  while (e + 1 < c.n_entries && x >= c.cfirst[e + 1]) ++e;
  const int32_t erow = x - c.cfirst[e];  // token * q_heads + head within the entry
  const int dt = threadIdx.x;
  if (dt >= D / 4) return;
  const int32_t ns = c.nseg[e];
  const int64_t p0 = c.wsoff[e] + (int64_t)erow * ns;
  float M = -INFINITY;
  for (int32_t s = 0; s < ns; ++s) M = fmaxf(M, c.ml[2 * (p0 + s)]);
  float L = 0.0f;
  float o4[4] = {0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
    for (int32_t s = 0; s < ns; ++s) {
      const float2 ml = *reinterpret_cast<const float2 *>(c.ml + 2 * (p0 + s));
      if (ml.x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml.x - M);
      const v4f o = *reinterpret_cast<const v4f *>(c.o + (p0 + s) * D + 4 * dt);
      L += ml.y * w;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] += o[i] * w;
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int64_t oi = ((int64_t)c.qoff[e] * c.q_heads + erow) * D + 4 * dt;
  if (c.out_bf16) {
    const uint32_t w0 = (uint32_t)f32_to_bf16_rtne(o4[0] * inv) |
                        ((uint32_t)f32_to_bf16_rtne(o4[1] * inv) << 16);
    const uint32_t w1 = (uint32_t)f32_to_bf16_rtne(o4[2] * inv) |
                        ((uint32_t)f32_to_bf16_rtne(o4[3] * inv) << 16);
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(c.out) + oi) = uint2{w0, w1};
  } else {
    *reinterpret_cast<v4f *>(static_cast<float *>(c.out) + oi) =
        v4f{o4[0] * inv, o4[1] * inv, o4[2] * inv, o4[3] * inv};
  }
}

template <int D, int NS>
hipError_t launch_prefill_t(const PrefillLaunch &pf, hipStream_t s) {
  const int64_t units = (int64_t)pf.first[pf.n_entries] * pf.d.g.kv_heads;
  const int64_t round = 8 * (int64_t)std::max(pf.xcd_chunk, 1);
  dim3 grid((unsigned)((units + round - 1) / round * round));
  const bool small = pf.d.g.page_tokens < kTile, qf16 = pf.d.q_bf16 != 0;
  if (pf.pre != nullptr && qf16) {
    // widen every tile once, then copy the images
    hipLaunchKernelGGL(widen_tiles_kernel<D>, dim3((unsigned)pf.preoff[pf.n_entries]), dim3(256), 0, s, pf);
    hipLaunchKernelGGL((prefill_kernel<D, false, NS, true, true>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  } else if (small && qf16)
    hipLaunchKernelGGL((prefill_kernel<D, true, NS, true>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  else if (small)
    hipLaunchKernelGGL((prefill_kernel<D, true, NS, false>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  else if (qf16)
    hipLaunchKernelGGL((prefill_kernel<D, false, NS, true>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  else
    hipLaunchKernelGGL((prefill_kernel<D, false, NS, false>), grid, dim3(64 * kPrefillWaves), 0, s, pf);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // merge the split entries' partials into their rows
  PrefillCombine c{};
  c.q_heads = pf.d.q_heads;
  c.out_bf16 = pf.d.out_bf16;
  c.out = pf.d.out;
  c.ml = pf.ws_ml;
  c.o = pf.ws_o;
  int32_t rows = 0;
  for (int32_t i = 0; i < pf.n_entries; ++i) {
    if (pf.nseg[i] < 2) continue;
    c.cfirst[c.n_entries] = rows;
    c.qoff[c.n_entries] = pf.qoff[i];
    c.nseg[c.n_entries] = pf.nseg[i];
    c.wsoff[c.n_entries] = pf.wsoff[i];
    rows += pf.rows[i] * pf.d.q_heads;
    ++c.n_entries;
  }
  c.cfirst[c.n_entries] = rows;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_combine_kernel<D>, dim3((unsigned)rows), dim3(64), 0, s, c);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill(const PrefillLaunch &pf, hipStream_t s) {
  if (pf.n_entries <= 0 || pf.first[pf.n_entries] <= 0) return hipSuccess;
  if (pf.d.g.head_dim == 256) return launch_prefill_t<256, 2>(pf, s);
  return launch_prefill_t<128, 2>(pf, s);
}

}  // namespace rkv
