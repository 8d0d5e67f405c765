// rkv_decode.hip -- paged Q8_0 flash-decode (GQA, causal multi-query verify,
// split-K partitions) and the log-sum-exp combine, for gfx950 (CDNA4).
//
// Algorithm: the online-softmax flash decode of
// har/crates/har-serve/src/attention.rs:169-215 (chunked scores, running
// max, rescale-and-accumulate), with the chunk combine (:205-212) reused as
// the split-K combine across workgroups.  Softmax runs in base 2 with the
// scale folded in: s2 = scale*log2(e)*q.k, p = 2^(s2 - m2); the result is
// identical in exact arithmetic to e^(scale*q.k - m).
//
// Work unit (one 64-lane workgroup = one wavefront):
//   (partition of part_tokens tokens, batch entry b, kv head).
// All R = q_len * q_heads/kv_heads query rows that share the kv head are
// processed together, so each K/V byte is read from HBM once.
//
// Per 32-token tile:
//   stage   : the tile's K codes, K scales, V codes and V scales (68*D bytes)
//             are copied HBM -> LDS with global_load_lds_dwordx4 (16 B per
//             lane, 1 KiB per instruction, fully coalesced), NSTAGE deep.
//   QK      : S^T[token][row] on v_mfma_i32_16x16x64_i8.  A = K codes (int8,
//             exactly the stored bytes, no dequant), B = the query split
//             into two int8 planes q ~ sq*(128*hi + lo).  The B operand's 16
//             columns are 8 rows x 2 block parities: columns 0-7 carry the
//             even 32-dim block of the 64-dim step, columns 8-15 the odd
//             one, so every int32 result is one (token, row, Q8 block) dot
//             product and gets its own f16 K scale on the VALU (exact
//             dequant order: d_k * sum(q_int * k_int)).
//   softmax : scores live one row per lane column; max across the 4 lane
//             groups with two shuffles, exp2 on the VALU.
//   PV      : O^T[dim][row] on v_mfma_f32_16x16x32_f16.  A = V codes
//             widened int8 -> f16 exactly (bias trick: 0x6400|(x^0x80) is
//             1024+x+128, minus 1152), B = p * d_v (the f16 V scale of that
//             token and block) rounded once to f16; f32 accumulation.
#include "rkv_launch.h"

namespace rkv {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kTile = 32;    // tokens per tile
constexpr int kStages = 2;   // LDS ring depth
// s_waitcnt immediate with expcnt/lgkmcnt at their maxima (no wait) and
// vmcnt = 0; OR in vmcnt bits [3:0] and [5:4] (at 15:14) to wait for less.
constexpr int kWaitBase = 0x0f70;

// LDS stage: [K codes 32*D][K scales 2*D][V codes 32*D][V scales 2*D],
// padded to whole 1 KiB global_load_lds instructions.
template <int D>
struct StageShape {
  static constexpr int kKC = 0;
  static constexpr int kKS = 32 * D;
  static constexpr int kVC = 34 * D;
  static constexpr int kVS = 66 * D;
  static constexpr int kBytes = 68 * D;
  static constexpr int kChunks = kBytes / 16;
  static constexpr int kInstr = (kChunks + 63) / 64;
  static constexpr int kAlloc = kInstr * 1024;
  static constexpr int kCPR = D / 16;  // 16-byte chunks per K row
};

__device__ __forceinline__ float dpp_ror8(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}

// 4 int8 codes (one dword) -> 4 exact f16 values.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, v2h &lo, v2h &hi) {
  const uint32_t u = w ^ 0x80808080u;  // x + 128 as unsigned bytes
  const uint32_t l = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const v2h bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(v2h, l) - bias;
  hi = __builtin_bit_cast(v2h, h) - bias;
}

__device__ __forceinline__ v4f f16x4_to_f32(uint2 w) {
  v4f r;
  r[0] = f16_bits_to_f32((uint16_t)(w.x & 0xffffu));
  r[1] = f16_bits_to_f32((uint16_t)(w.x >> 16));
  r[2] = f16_bits_to_f32((uint16_t)(w.y & 0xffffu));
  r[3] = f16_bits_to_f32((uint16_t)(w.y >> 16));
  return r;
}

// Global source offsets of the 16-byte LDS chunks one lane copies per tile.
// `half` says which 16-token half of the tile a chunk belongs to (the page
// of that half is looked up per tile); `mul` scales the tile's starting
// slot into the region (D for code runs, D/16 for scale runs).
template <int D, bool kSmallPage>
struct ChunkPlan {
  using S = StageShape<D>;
  uint32_t off[S::kInstr];
  uint32_t mul[S::kInstr];  // D for code runs, D/16 for scale runs
  uint32_t halves;          // bit k: chunk k lies in the tile's second 16-token half
};

template <int D, bool kSmallPage>
__device__ __forceinline__ void make_plan(ChunkPlan<D, kSmallPage> &pl, const Geo &g, int lane) {
  using S = StageShape<D>;
  const uint32_t RB = (uint32_t)region_bytes(g);
  const uint32_t PTD = (uint32_t)g.page_tokens * D;
  const uint32_t TT = (uint32_t)tile_tokens(g.page_tokens);
  pl.halves = 0;
#pragma unroll
  for (int k = 0; k < S::kInstr; ++k) {
    const int c = 64 * k + lane;
    uint32_t off = 0;
    uint32_t half = 0, is_scale = 0;
    if (c < 2 * D) {  // K codes: row r, physical chunk pc holds logical chunk pc ^ (r mod CPR)
      const int r = c / S::kCPR;
      const int pc = c % S::kCPR;
      const int lc = pc ^ (r & (S::kCPR - 1));
      half = r >= 16;
      off = (uint32_t)((kSmallPage ? (r & 15) : r) * D + 16 * lc);
    } else if (c < 2 * D + D / 8) {  // K scales: block b, tokens 8*piece..+7
      const int i = c - 2 * D;
      const int b = i >> 2, piece = i & 3;
      half = piece >= 2;
      is_scale = 1;
      off = PTD + 2u * ((uint32_t)b * TT + (uint32_t)(kSmallPage ? 8 * (piece & 1) : 8 * piece));
    } else if (c < 4 * D + D / 8) {  // V codes: dim row d, 16-token piece (halves swapped when (d>>2)&1)
      const int i = c - (2 * D + D / 8);
      const int d = i >> 1;
      const int lh = (i & 1) ^ ((d >> 2) & 1);
      half = lh;
      off = RB + (uint32_t)d * TT + (uint32_t)(kSmallPage ? 0 : 16 * lh);
    } else if (c < 4 * D + D / 4) {  // V scales
      const int i = c - (4 * D + D / 8);
      const int b = i >> 2, piece = i & 3;
      half = piece >= 2;
      is_scale = 1;
      off = RB + PTD + 2u * ((uint32_t)b * TT + (uint32_t)(kSmallPage ? 8 * (piece & 1) : 8 * piece));
    } else {  // padding lanes of the last instruction: re-read chunk 0 of the tile
      off = 0;
    }
    pl.off[k] = off;
    pl.mul[k] = is_scale ? (uint32_t)(D / 16) : (uint32_t)D;
    pl.halves |= half << k;
  }
}

#if defined(__HIP_DEVICE_COMPILE__)
// LDS-typed pointers exist only in the device pass.
typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <typename T>
__device__ __forceinline__ T lds_load(const lds_u8 *p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T *>(p);
}

// One workgroup's decode of one (partition, batch entry, kv head).
template <int D, int NT, bool kSmall>
struct Decoder {
  using S = StageShape<D>;
  static constexpr int NP = (NT + 1) / 2;  // PV n-tiles of 16 rows
  static constexpr int NC = D / 64;        // 64-dim QK steps
  static constexpr int NB = D / 32;        // Q8 blocks per row

  const DecodeLaunch &p;
  int lane, li, lg, kvh;
  int32_t len, tok0, n_tiles;
  int32_t pg_first;        // first page index (within the sequence) of the partition
  int32_t pidv;            // lane i: page id of the partition's i-th page
  const uint8_t *kv_base;  // pages + kv head offset
  uint64_t PB;
  ChunkPlan<D, kSmall> plan;
  v4i qhi[NT][NC], qlo[NT][NC];
  float rmul[NP];
  int32_t rlim[NP];
  v4f oacc[NP][D / 16];
  float mrun[NP], lrun[NP];

  __device__ __forceinline__ Decoder(const DecodeLaunch &p_) : p(p_) {}

  // Copy tile `tile` (32 tokens) of this work unit HBM -> LDS stage `dst`.
  // Page ids come from `pidv` (lane i holds the partition's i-th page id).
  __device__ __forceinline__ void issue(int tile, lds_u8 *__restrict__ dst) {
    const Geo &g = p.g;
    const int32_t t0 = tok0 + tile * kTile;
    const int32_t pi = t0 / g.page_tokens - pg_first;
    if constexpr (!kSmall) {
      const int32_t pid = __builtin_amdgcn_readlane(pidv, pi);
      const uint8_t *base = kv_base + (uint64_t)pid * PB;
      const uint32_t s0 = (uint32_t)(t0 % g.page_tokens);
#pragma unroll
      for (int k = 0; k < S::kInstr; ++k) {
        const uint32_t voff = plan.off[k] + s0 * plan.mul[k];
        __builtin_amdgcn_global_load_lds(base + voff, dst + 1024 * k, 16, 0, 0);
      }
    } else {
      // 16-token pages: the two halves of the tile live in two pages
      const int32_t pid0 = __builtin_amdgcn_readlane(pidv, pi);
      const int32_t pid1 = (t0 + 16 < len) ? __builtin_amdgcn_readlane(pidv, pi + 1) : pid0;
      const uint8_t *base0 = kv_base + (uint64_t)pid0 * PB;
      const uint8_t *base1 = kv_base + (uint64_t)pid1 * PB;
#pragma unroll
      for (int k = 0; k < S::kInstr; ++k) {
        const bool h = (plan.halves >> k) & 1u;
        __builtin_amdgcn_global_load_lds((h ? base1 : base0) + plan.off[k], dst + 1024 * k, 16, 0, 0);
      }
    }
  }

  // Scores, online softmax and PV for the tile held in LDS stage `st`.
  __device__ __forceinline__ void compute(int tile, const lds_u8 *__restrict__ st) {
    const int32_t t0 = tok0 + tile * kTile;
    // ---- QK^T ----
    float sacc[NT][2][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[nt][mt][r] = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int krow = 16 * mt + li;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int pc = (4 * c + lg) ^ (krow & (S::kCPR - 1));
        const v4i a = lds_load<v4i>(st + S::kKC + krow * D + 16 * pc);
        const int blk = 2 * c + (li >> 3);
        const v4f dk = f16x4_to_f32(lds_load<uint2>(st + S::kKS + 2 * (blk * 32 + 16 * mt + 4 * lg)));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const v4i z = {0, 0, 0, 0};
          const v4i ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qhi[nt][c], z, 0, 0, 0);
          const v4i cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qlo[nt][c], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) sacc[nt][mt][r] += (float)((ch[r] << 7) + cl[r]) * dk[r];
        }
      }
    }

    // ---- online softmax (base 2) ----
    float pr[NP][8];
#pragma unroll
    for (int np = 0; np < NP; ++np) {
      float s[8];
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // the even- and odd-block halves of a row sit 8 columns apart
          float lo_t = 0.f, hi_t = 0.f;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            if (nt != 2 * np && nt != 2 * np + 1) continue;
            const float tot = sacc[nt][mt][r] + dpp_ror8(sacc[nt][mt][r]);
            if (nt == 2 * np) lo_t = tot;
            else hi_t = tot;
          }
          const float v = (li < 8 ? lo_t : hi_t) * rmul[np];
          const int tok = t0 + 16 * mt + 4 * lg + r;
          const float sv = tok < rlim[np] ? v : -INFINITY;
          s[4 * mt + r] = sv;
          tmax = fmaxf(tmax, sv);
        }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float mnew = fmaxf(mrun[np], tmax);
      const float muse = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(mrun[np] - muse);
      float lsum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pr[np][e] = __builtin_amdgcn_exp2f(s[e] - muse);
        lsum += pr[np][e];
      }
      lrun[np] = lrun[np] * alpha + lsum;
      mrun[np] = mnew;
      // alpha == 1 exactly unless this row's max moved; rescale only then
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int m = 0; m < D / 16; ++m) oacc[np][m] *= alpha;
      }
    }

    // ---- PV ----
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      const v4f dv0 = f16x4_to_f32(lds_load<uint2>(st + S::kVS + 2 * (blk * 32 + 4 * lg)));
      const v4f dv1 = f16x4_to_f32(lds_load<uint2>(st + S::kVS + 2 * (blk * 32 + 16 + 4 * lg)));
      v8h pb[NP];
#pragma unroll
      for (int np = 0; np < NP; ++np) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // masked tokens have p == 0 and may carry junk scales: keep them 0
          pb[np][e] = (_Float16)(pr[np][e] > 0.0f ? pr[np][e] * dv0[e] : 0.0f);
          pb[np][4 + e] = (_Float16)(pr[np][4 + e] > 0.0f ? pr[np][4 + e] * dv1[e] : 0.0f);
        }
      }
#pragma unroll
      for (int hm = 0; hm < 2; ++hm) {
        const int d = 32 * blk + 16 * hm + li;
        const int sw = (d >> 2) & 1;
        const uint32_t w0 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * sw + 4 * lg);
        const uint32_t w1 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * (sw ^ 1) + 4 * lg);
        v2h a0, a1, a2, a3;
        i8x4_to_f16(w0, a0, a1);
        i8x4_to_f16(w1, a2, a3);
        const v8h va = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
#pragma unroll
        for (int np = 0; np < NP; ++np)
          oacc[np][2 * blk + hm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[np], oacc[np][2 * blk + hm], 0, 0, 0);
      }
    }
  }

  // Prefetch the next tile into `next`, wait for `cur`, compute `cur`.  The
  // two stages are distinct restrict pointers so the compiler can see that
  // the reads of `cur` do not depend on the copies into `next` and keeps the
  // explicit vmcnt wait below instead of draining every copy.
  __device__ __forceinline__ void step(int tile, const lds_u8 *__restrict__ cur,
                                       lds_u8 *__restrict__ next) {
    if (tile + 1 < n_tiles) {
      issue(tile + 1, next);
      // vmcnt <= kInstr: every copy into `cur` has landed
      __builtin_amdgcn_s_waitcnt(kWaitBase | (S::kInstr & 0xf) | ((S::kInstr >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitBase);
    }
    compute(tile, cur);
  }
};

#endif  // __HIP_DEVICE_COMPILE__

template <int D, int NT, bool kSmall>
__global__ __launch_bounds__(64) void decode_kernel(DecodeLaunch p) {
#if defined(__HIP_DEVICE_COMPILE__)
  using Dec = Decoder<D, NT, kSmall>;
  using S = StageShape<D>;
  constexpr int NP = Dec::NP;
  constexpr int NC = Dec::NC;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages][S::kAlloc];

  Dec dc(p);
  dc.lane = threadIdx.x;
  dc.li = dc.lane & 15;  // MFMA row/column within a 16-lane group
  dc.lg = dc.lane >> 4;  // MFMA k-group
  const int lane = dc.lane, li = dc.li, lg = dc.lg;
  const int part = blockIdx.x;
  const int b = blockIdx.y;
  const int kvh = blockIdx.z;
  dc.kvh = kvh;
  const Geo g = p.g;

  const int32_t seq = p.seq_ids[b];
  if (seq < 0 || seq >= p.n_seqs) {
    if (lane == 0) atomicOr(p.fault, FAULT_BAD_SEQ);
    return;
  }
  const int32_t len = p.seq_lens[seq];
  if (len < 0 || len > p.bt_stride * g.page_tokens) {
    if (lane == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  if (len > p.n_parts * p.part_tokens) {  // longer than max_seq_len promised
    if (lane == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  const int32_t tok0 = part * p.part_tokens;
  if (tok0 >= len && part > 0) return;  // past the end: the combine never reads it
  const int32_t tok_end = min(len, tok0 + p.part_tokens);
  dc.len = len;
  dc.tok0 = tok0;
  dc.n_tiles = tok_end > tok0 ? (tok_end - tok0 + kTile - 1) / kTile : 0;

  const int32_t q_per_kv = p.q_heads / g.kv_heads;
  const int32_t R = p.q_len * q_per_kv;

  // ---- query: int8 hi/lo planes as MFMA B operands -------------------------
  // Lane (n = li, group lg) of QK n-tile nt serves row 8*nt + (n & 7), dims
  // 64*c + 16*lg .. +15; it is live for the even block (lg < 2) when n < 8
  // and for the odd block (lg >= 2) when n >= 8.
  float qmul[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = 8 * nt + (li & 7);
    float qv[NC][16];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) qv[c][e] = 0.0f;
    if (row < R) {
      const int j = row / q_per_kv;
      const int h = kvh * q_per_kv + row % q_per_kv;
      const int64_t base = (((int64_t)b * p.q_len + j) * p.q_heads + h) * D + 16 * lg;
      if (p.q_bf16) {
        const uint16_t *q = static_cast<const uint16_t *>(p.q) + base;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const uint4 w0 = *reinterpret_cast<const uint4 *>(q + 64 * c);
          const uint4 w1 = *reinterpret_cast<const uint4 *>(q + 64 * c + 8);
          const uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            qv[c][2 * e] = bf16_bits_to_f32((uint16_t)(ws[e] & 0xffffu));
            qv[c][2 * e + 1] = bf16_bits_to_f32((uint16_t)(ws[e] >> 16));
          }
        }
      } else {
        const float *q = static_cast<const float *>(p.q) + base;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const float4 w = *reinterpret_cast<const float4 *>(q + 64 * c + 4 * e4);
            qv[c][4 * e4] = w.x;
            qv[c][4 * e4 + 1] = w.y;
            qv[c][4 * e4 + 2] = w.z;
            qv[c][4 * e4 + 3] = w.w;
          }
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(qv[c][e]));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    // q ~ sq * Q with |Q| <= 16256 = 127*128; Q = 128*hi + lo with hi in
    // [-127, 127] and lo in [-64, 63].
    const float inv = amax > 0.0f ? 16256.0f / amax : 0.0f;
    qmul[nt] = amax > 0.0f ? (amax / 16256.0f) * p.scale_log2 : 0.0f;
    const bool live = (li < 8) == (lg < 2);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint32_t hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        int32_t Q = (int32_t)rintf(qv[c][e] * inv);
        Q = live ? max(-16256, min(16256, Q)) : 0;
        const int32_t hi = (Q + 64) >> 7;
        const int32_t lo = Q - 128 * hi;
        hw[e >> 2] |= ((uint32_t)(uint8_t)(int8_t)hi) << (8 * (e & 3));
        lw[e >> 2] |= ((uint32_t)(uint8_t)(int8_t)lo) << (8 * (e & 3));
      }
      dc.qhi[nt][c] = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
      dc.qlo[nt][c] = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
    }
  }

  // ---- per-lane softmax rows: PV n-tile np, column li -> row 16*np + li ---
#pragma unroll
  for (int np = 0; np < NP; ++np) {
    const int row = 16 * np + li;
    const int nt = 2 * np + (li >> 3);
    // every lane of column li computed the scale of row 8*nt + (li & 7)
    float mul = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t == nt) mul = qmul[t];
    dc.rmul[np] = mul;
    dc.rlim[np] = (row < R && nt < NT) ? len - p.q_len + row / q_per_kv + 1 : 0;
    dc.mrun[np] = -INFINITY;
    dc.lrun[np] = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) dc.oacc[np][m] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  make_plan<D, kSmall>(dc.plan, g, lane);
  dc.PB = page_bytes(g);
  dc.kv_base = p.pages + (uint64_t)kvh * 2u * region_bytes(g);
  // The partition's page ids, one per lane (the host keeps part_tokens <=
  // 64 * page_tokens); bad entries are reported and replaced by page 0 so
  // every copy stays inside the pool.
  dc.pg_first = tok0 / g.page_tokens;
  {
    const int32_t npg = tok_end > tok0 ? (tok_end - 1) / g.page_tokens - dc.pg_first + 1 : 0;
    int32_t pid = lane < npg ? p.bt[(int64_t)seq * p.bt_stride + dc.pg_first + lane] : 0;
    if (pid < 0 || pid >= g.num_pages) {
      atomicOr(p.fault, FAULT_BAD_PAGE);
      pid = 0;
    }
    dc.pidv = pid;
  }

  lds_u8 *s0 = (lds_u8 *)lds[0];
  lds_u8 *s1 = (lds_u8 *)lds[1];
  const int nt_total = dc.n_tiles;
  if (nt_total > 0) dc.issue(0, s0);
  int tile = 0;
  for (; tile + 1 < nt_total; tile += 2) {
    dc.step(tile, s0, s1);
    dc.step(tile + 1, s1, s0);
  }
  if (tile < nt_total) dc.step(tile, s0, s1);

  // ---- epilogue ---------------------------------------------------------------
#pragma unroll
  for (int np = 0; np < NP; ++np) {
    float l = dc.lrun[np];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int row = 16 * np + li;
    if (row >= R) continue;
    const int j = row / q_per_kv;
    const int h = kvh * q_per_kv + row % q_per_kv;
    const int64_t orow = ((int64_t)b * p.q_len + j) * p.q_heads + h;
    if (p.ws_o == nullptr) {
      const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
      for (int m = 0; m < D / 16; ++m) {
        const int d0 = 16 * m + 4 * lg;
        const v4f o = l > 0.0f ? dc.oacc[np][m] * inv_l : v4f{0.f, 0.f, 0.f, 0.f};
        if (p.out_bf16) {
          uint16_t *dst = static_cast<uint16_t *>(p.out) + orow * D + d0;
          const uint32_t w0 = (uint32_t)f32_to_bf16_rtne(o[0]) | ((uint32_t)f32_to_bf16_rtne(o[1]) << 16);
          const uint32_t w1 = (uint32_t)f32_to_bf16_rtne(o[2]) | ((uint32_t)f32_to_bf16_rtne(o[3]) << 16);
          *reinterpret_cast<uint2 *>(dst) = uint2{w0, w1};
        } else {
          *reinterpret_cast<v4f *>(static_cast<float *>(p.out) + orow * D + d0) = o;
        }
      }
    } else {
      const int64_t prow = orow * p.n_parts + part;
#pragma unroll
      for (int m = 0; m < D / 16; ++m)
        *reinterpret_cast<v4f *>(p.ws_o + prow * D + 16 * m + 4 * lg) = dc.oacc[np][m];
      if (lg == 0) *reinterpret_cast<float2 *>(p.ws_ml + 2 * prow) = float2{dc.mrun[np], l};
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// One 256-thread block per (batch entry, row); thread = dimension.
__global__ __launch_bounds__(256) void combine_kernel(CombineLaunch c) {
  const int row = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int32_t seq = c.seq_ids[b];
  const int32_t len = (seq >= 0 && seq < c.n_seqs) ? c.seq_lens[seq] : 0;
  const int32_t np = len > 0 ? min(c.n_parts, (len + c.part_tokens - 1) / c.part_tokens) : 0;
  const int64_t prow = ((int64_t)b * c.rows + row) * c.n_parts;
  float M = -INFINITY;
  for (int i = 0; i < np; ++i) M = fmaxf(M, c.ml[2 * (prow + i)]);
  float L = 0.0f, O = 0.0f;
  if (M != -INFINITY) {
    for (int i = 0; i < np; ++i) {
      const float w = __builtin_amdgcn_exp2f(c.ml[2 * (prow + i)] - M);
      L += c.ml[2 * (prow + i) + 1] * w;
      if (d < c.head_dim) O += c.o[(prow + i) * c.head_dim + d] * w;
    }
  }
  if (d >= c.head_dim) return;
  const float r = L > 0.0f ? O / L : 0.0f;
  const int64_t oi = ((int64_t)b * c.rows + row) * c.head_dim + d;
  if (c.out_bf16) static_cast<uint16_t *>(c.out)[oi] = f32_to_bf16_rtne(r);
  else static_cast<float *>(c.out)[oi] = r;
}

template <int D, int NT>
hipError_t launch_decode_t(const DecodeLaunch &d, hipStream_t s) {
  dim3 grid((unsigned)d.n_parts, (unsigned)d.batch, (unsigned)d.g.kv_heads);
  if (d.g.page_tokens < kTile)
    hipLaunchKernelGGL((decode_kernel<D, NT, true>), grid, dim3(64), 0, s, d);
  else
    hipLaunchKernelGGL((decode_kernel<D, NT, false>), grid, dim3(64), 0, s, d);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const DecodeLaunch &d, hipStream_t s) {
  if (d.batch == 0 || d.n_parts == 0) return hipSuccess;
  const int R = d.q_len * (d.q_heads / d.g.kv_heads);
  const int NT = R <= 8 ? 1 : (R <= 16 ? 2 : 4);
  if (d.g.head_dim == 256) {
    if (NT == 1) return launch_decode_t<256, 1>(d, s);
    if (NT == 2) return launch_decode_t<256, 2>(d, s);
    return launch_decode_t<256, 4>(d, s);
  }
  if (NT == 1) return launch_decode_t<128, 1>(d, s);
  if (NT == 2) return launch_decode_t<128, 2>(d, s);
  return launch_decode_t<128, 4>(d, s);
}

hipError_t launch_combine(const CombineLaunch &c, hipStream_t s) {
  if (c.batch == 0 || c.rows == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)c.rows, (unsigned)c.batch), dim3(256), 0, s, c);
  return hipGetLastError();
}

}  // namespace rkv
