// rkv_decode_kernel.h -- the paged Q8_0 flash-decode kernel template (GQA,
// causal multi-query verify, split-K partitions) for gfx950 (CDNA4), shared
// by rkv_decode.hip (up to 16 rows per kv head, one wave per workgroup) and
// rkv_decode_rows32.hip (17..32 rows, two waves per workgroup).
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
//             into three int8 planes q ~ sq*(128*hi + md + lo/128) (22
//             significant bits per row).  The B operand's 16 columns are 8
//             rows x 2 block parities: columns 0-7 carry the even 32-dim
//             block of the 64-dim step, columns 8-15 the odd one, so every
//             int32 result is one (token, row, Q8 block) dot product and
//             gets its own f16 K scale on the VALU (exact dequant order:
//             d_k * sum(q_int * k_int)).  The lo plane's dot, shifted right
//             by 7, is the accumulator input of the md plane's MFMA, so the
//             third plane costs one MFMA and one shift per result.
//   softmax : scores live one row per lane column; max across the 4 lane
//             groups with two shuffles, exp2 on the VALU.
//   PV      : O^T[dim][row] on v_mfma_f32_16x16x32_f16.  A = V codes
//             widened to f16 exactly (they are stored as x+128: 0x6400|byte
//             is 1024+x+128, minus 1152), B = the weight p * d_v (the f16 V
//             scale of that token and block) as two f16 terms; f32
//             accumulation.
#pragma once

#include <type_traits>

#include "rkv_launch.h"

namespace rkv {

namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kTile = 32;    // tokens per tile
// s_waitcnt immediate with expcnt/lgkmcnt at their maxima (no wait) and
// vmcnt = 0; OR in vmcnt bits [3:0] and [5:4] (at 15:14) to wait for less.
constexpr int kWaitBase = 0x0f70;

// LDS stage: [K codes 32*D][K scales 2*D][V codes 32*D][V scales 2*D],
// padded to whole 1 KiB global_load_lds instructions.  kKReg: the K codes
// go to registers instead, and the stage is [V codes][K scales][V scales].
template <int D, bool kKReg = false>
struct StageShape {
  static constexpr int kKC = 0;
  static constexpr int kKS = 32 * D;
  static constexpr int kVC = kKReg ? 0 : 34 * D;
  static constexpr int kVS = kKReg ? 34 * D : 66 * D;
  static constexpr int kBytes = kKReg ? 36 * D : 68 * D;
  static constexpr int kChunks = kBytes / 16;
  static constexpr int kInstr = (kChunks + 63) / 64;
  static constexpr int kAlloc = kInstr * 1024;
  static constexpr int kCPR = D / 16;  // 16-byte chunks per K row
};

__device__ __forceinline__ float dpp_ror8(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}

// The second f16 term of a pair of PV weights p0, p1 whose first terms are
// h = f16(p): f16(p - h), where p - h is exact in f32.  Computed as
// fma(h, m1, p) with the f16 halves of h as v_fma_mix operands (one
// instruction per value, where a conversion back to f32 and a subtraction
// take two); m1 = -1 comes from a register so that the compiler keeps the
// fma instead of rewriting it into that subtraction.
__device__ __forceinline__ v2h p_residual(v2h h, float p0, float p1) {
  float m1;
  asm("v_mov_b32 %0, -1.0" : "=v"(m1));
  return v2h{(_Float16)__builtin_fmaf((float)h[0], m1, p0), (_Float16)__builtin_fmaf((float)h[1], m1, p1)};
}

// The maximum of x over lanes li, li+16, li+32 and li+48 (the four 16-lane
// rows), on every lane.  gfx950's row swaps hand each lane its partner's
// value in a register: v_permlane16_swap pairs rows 0-1 and 2-3,
// v_permlane32_swap the two halves.  Each swap leaves the lane's own and its
// partner's value in the two outputs, in either order; the maximum does not
// depend on which.  No LDS round trip (a shuffle by ds_bpermute waits on the
// LDS queue, which the tile's scale reads also occupy).
__device__ __forceinline__ float row_group_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
  const uint32_t w = __builtin_bit_cast(uint32_t, x);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}

// 4 stored V codes (one dword of x + 128 bytes) -> 4 exact f16 values x.
__device__ __forceinline__ void v8x4_to_f16(uint32_t u, v2h &lo, v2h &hi) {
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

// Per-lane copy plan of one tile: source offsets (relative to the kv head's
// base in the page of the chunk's 16-token half) of the LDS chunks this lane
// copies.  Pages of >= 32 tokens hold the whole tile in one page laid out
// exactly like the LDS stage, so the copy is S::kInstr 16-byte instructions
// over the stage in order (the last one padded by re-reading chunk 0).
// 16-token pages hold half a tile each: the code runs are still 16-byte
// copies, but the lane-ordered scale runs interleave the two pages every 4
// bytes, so they use 4-byte copies.
template <int D, bool kSmallPage, bool kKReg = false, int NW = 1>
struct ChunkPlan {
  using S = StageShape<D, kKReg>;
  static constexpr int kNKC = D / 32;                       // 1 KiB K-code (or V-code) copies
  static constexpr int kN16 = kSmallPage ? 2 * kNKC : S::kInstr;
  static constexpr int kN4 = kSmallPage ? 2 * (D / 128) : 0;  // 256-byte scale copies
  static constexpr int kInstr = kN16 + kN4;                  // vmcnt units per tile
  // Pages of >= 32 tokens with NW waves: wave w issues copies k = i*NW + w
  // and holds only their offsets (entry i), so its copies go out as
  // straight-line code; 16-token pages keep every copy's entry.
  static constexpr int kWaves = kSmallPage ? 1 : NW;
  static constexpr int kPer = (kN16 + kWaves - 1) / kWaves;  // 16-byte copy entries per wave
  uint32_t off[kPer + kN4];
  uint32_t mul[kPer + kN4];  // D for code runs, D/16 for scale runs (pages >= 32 tokens)
  uint32_t halves;           // bit k: chunk k lies in the tile's second 16-token half
  __host__ __device__ static constexpr int dst16(int k) {  // LDS byte offset of 16-B copy k
    return kSmallPage ? (k < kNKC ? S::kKC + 1024 * k : S::kVC + 1024 * (k - kNKC)) : 1024 * k;
  }
  __host__ __device__ static constexpr int dst4(int k) {  // LDS byte offset of 4-B copy k
    return k < kN4 / 2 ? S::kKS + 256 * k : S::kVS + 256 * (k - kN4 / 2);
  }
};

template <int D, bool kSmallPage, bool kKReg = false, int NW = 1>
__device__ __forceinline__ void make_plan(ChunkPlan<D, kSmallPage, kKReg, NW> &pl, const Geo &g,
                                          int lane, int wave = 0) {
  using S = StageShape<D, kKReg>;
  using PL = ChunkPlan<D, kSmallPage, kKReg, NW>;
  const uint32_t RB = (uint32_t)region_bytes(g);
  const uint32_t PTD = (uint32_t)g.page_tokens * D;
  pl.halves = 0;
  if constexpr (kKReg) {
    static_assert(!kSmallPage, "K codes in registers need 32-token tiles in one page");
#pragma unroll
    for (int k = 0; k < S::kInstr; ++k) {
      const int c = 64 * k + lane;
      uint32_t off = 0, is_scale = 0;
      if (c < 2 * D) {  // V codes: dim row d, 16-token piece (halves swapped when (d>>2)&1)
        const int d = c >> 1;
        const int lh = (c & 1) ^ ((d >> 2) & 1);
        off = RB + (uint32_t)(d * 32 + 16 * lh);
      } else if (c < 2 * D + D / 8) {  // K scales
        const int i = c - 2 * D;
        off = PTD + 2u * (uint32_t)(32 * (i >> 2) + 8 * (i & 3));
        is_scale = 1;
      } else if (c < 2 * D + D / 4) {  // V scales
        const int i = c - (2 * D + D / 8);
        off = RB + PTD + 2u * (uint32_t)(32 * (i >> 2) + 8 * (i & 3));
        is_scale = 1;
      }  // else: padding lane of the last copy, re-reads chunk 0 of the tile
      pl.off[k] = off;
      pl.mul[k] = is_scale ? (uint32_t)(D / 16) : (uint32_t)D;
    }
  } else if constexpr (!kSmallPage) {
#pragma unroll
    for (int i = 0; i < PL::kPer; ++i) {
      const int k = i * PL::kWaves + wave;  // copy k (past the last: unused)
      const int c = 64 * k + lane;
      uint32_t off = 0, is_scale = 0;
      if (c < 2 * D) {  // K codes: row r, physical chunk pc holds logical chunk pc ^ (r mod CPR)
        const int r = c / S::kCPR;
        const int lc = (c % S::kCPR) ^ (r & (S::kCPR - 1));
        off = (uint32_t)(r * D + 16 * lc);
      } else if (c < 2 * D + D / 8) {  // K scales: block b, lane-ordered positions 8*j..8*j+7
        const int i = c - 2 * D;
        off = PTD + 2u * (uint32_t)(32 * (i >> 2) + 8 * (i & 3));
        is_scale = 1;
      } else if (c < 4 * D + D / 8) {  // V codes: dim row d, 16-token piece (halves swapped when (d>>2)&1)
        const int i = c - (2 * D + D / 8);
        const int d = i >> 1;
        const int lh = (i & 1) ^ ((d >> 2) & 1);
        off = RB + (uint32_t)(d * 32 + 16 * lh);
      } else if (c < 4 * D + D / 4) {  // V scales
        const int i = c - (4 * D + D / 8);
        off = RB + PTD + 2u * (uint32_t)(32 * (i >> 2) + 8 * (i & 3));
        is_scale = 1;
      }  // else: padding lane of the last copy, re-reads chunk 0 of the tile
      pl.off[i] = off;
      pl.mul[i] = is_scale ? (uint32_t)(D / 16) : (uint32_t)D;
    }
  } else {
#pragma unroll
    for (int k = 0; k < PL::kN16; ++k) {
      const int c = 64 * (k % PL::kNKC) + lane;
      uint32_t off, half;
      if (k < PL::kNKC) {  // K codes
        const int r = c / S::kCPR;
        const int lc = (c % S::kCPR) ^ (r & (S::kCPR - 1));
        half = r >= 16;
        off = (uint32_t)((r & 15) * D + 16 * lc);
      } else {  // V codes [d][16] per page
        const int d = c >> 1;
        half = (c & 1) ^ ((d >> 2) & 1);
        off = RB + (uint32_t)d * 16u;
      }
      pl.off[k] = off;
      pl.mul[k] = 0;
      pl.halves |= half << k;
    }
#pragma unroll
    for (int k = 0; k < PL::kN4; ++k) {
      // dword w of a kind's scale run: block b, lane-ordered positions p, p+1
      const int kind = k < PL::kN4 / 2 ? 0 : 1;
      const int w = 64 * (k % (PL::kN4 / 2)) + lane;
      const int b = w >> 4, p = 2 * (w & 15);
      const uint32_t half = (p >> 2) & 1;
      const uint32_t tk = (uint32_t)(4 * (p >> 3) + (p & 3));
      pl.off[PL::kN16 + k] = (kind ? RB : 0u) + PTD + 2u * ((uint32_t)b * 16u + tk);
      pl.mul[PL::kN16 + k] = 0;
      pl.halves |= half << (PL::kN16 + k);
    }
  }
}

#if defined(__HIP_DEVICE_COMPILE__)
// LDS-typed pointers exist only in the device pass.
typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <typename T>
__device__ __forceinline__ T lds_load(const lds_u8 *p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T *>(p);
}

// Rescale threshold (base-2 log units): the running reference max of a row
// only moves when a tile's max exceeds it by more than kTau, so p = 2^(s-m)
// stays <= 2^kTau and the accumulators are rescaled only a few times.
constexpr float kTau = 4.0f;

// Workgroup barrier without memory fences: a fenced barrier would also wait
// for every tile copy in flight.  The explicit vmcnt waits order the copies;
// the "memory" clobber keeps the compiler from moving LDS accesses across.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }
// Barrier after LDS writes that other waves read next: s_barrier does not
// wait for the wave's outstanding LDS operations, so lgkmcnt(0) first.
__device__ __forceinline__ void wg_barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One wave's share of the decode of one (partition, batch entry, kv head).
// With NW > 1 waves per workgroup, wave w owns query rows 16w .. 16w+15 and
// issues copy k of each tile when k % NW == w; the waves share the LDS
// stages and meet at two barriers per tile (stage free, tile landed).
// kPageList: page ids come from a workgroup list in LDS (any length) instead
// of one register lane per page (at most 64 pages).
// kF16V: after a tile lands the waves widen its V codes to f16 once, each
// its share, into an LDS tile laid out as the PV MFMA's A operand (one
// 16-byte read per operand); without it every wave widens the whole tile.
// kKReg (one wave, pages of >= 32 tokens): each tile's K codes are loaded
// straight into the QK MFMA's A-operand registers (8 x 16 bytes per lane,
// 16 rows x 64 contiguous bytes per load) instead of through the LDS stage;
// the next tile's are loaded as soon as this tile's QK has read them.  The
// stage then holds only V codes and the scales, 9 KiB at D=256.
template <int D, int NT, bool kSmall, int NS, int NW = 1, bool kPageList = false,
          bool kF16V = false, bool kKReg = false, bool kF16K = false>
struct Decoder {
  using S = StageShape<D, kKReg>;
  static constexpr bool kSplitP = true;    // two-term f16 PV weights (see compute)
  // Cache policy of the tile reads.  A decode or verify launch reads every
  // K/V byte once, so its reads are nontemporal (NT): they do not displace
  // cached lines, and a streaming read runs about 15% faster.  The prefill
  // (kPageList) re-reads a sequence's tiles from every row block and keeps
  // the default policy so those re-reads hit the caches.
  static constexpr int kCpol = kPageList ? 0 : 2;
  // With one QK n-tile (at most 8 rows) the PV MFMA's columns 8-15 are free:
  // they carry the second weight term of rows 0-7 instead of a second MFMA,
  // and the epilogue adds column c + 8 to column c.
  static constexpr bool kColSplit = kSplitP && NT == 1;
  static constexpr int NP = (NT + 1) / 2;  // PV n-tiles of 16 rows
  static constexpr int NC = D / 64;        // 64-dim QK steps
  static constexpr int NB = D / 32;        // Q8 blocks per row
  // 16 rows per wave (NT == 2): the QK runs on v_mfma_i32_16x16x32_i8, one
  // Q8 block per MFMA with the wave's 16 rows in its 16 columns, so each
  // lane's int32 result is a whole (token, row, block) dot and the query
  // operands hold no zero half (8 bytes per block and plane).  With at most
  // 8 rows the 16x16x64 form packs 8 rows x 2 block parities instead.
  static constexpr bool kWide = NT == 2;
  using QOp = typename std::conditional<kWide, int64_t, v4i>::type;
  static constexpr int kQR = kWide ? 1 : NT;   // query operand sets
  static constexpr int kQC = kWide ? NB : NC;  // operands per set and plane
  // kF16K (16 rows per wave, bf16 query): the QK runs on
  // v_mfma_f32_16x16x32_f16 against the query as one f16 operand per block
  // (a bf16 value times a power of two is exact in f16) and the K codes
  // widened to exact f16: once per tile by the workgroup into kf16 when it
  // widens V too (the prefill's 8 waves), else by each wave in registers
  // (8 codes per operand: two xors, four perms, four packed subtractions).
  // Each (token, row, block) result then costs one K-scale fma instead of
  // the int8 form's shift, add, convert and fma.
  static_assert(!kF16K || kWide, "f16 K: 16-row waves");
  static constexpr int kQF = kF16K ? NB : 1;
  // kDSplit (the two-wave verify with a bf16 query, 2-stage ring): wave w
  // owns half of the head dimension, blocks w*NB/2 .. +NB/2-1, for all 32
  // rows, and the softmax of its own 16 rows.  Each wave widens and reads
  // only its half of every K and V tile; the halves' partial scores and
  // the rows' p values cross through LDS (see compute_split).  qf then holds
  // [n-tile][own block] and oacc[0] holds [n-tile][own 16-dim tile].  Not on
  // 16-token pages: their copy plan leaves the split too few registers.
  static constexpr bool kDSplit = NW == 2 && kF16K && !kF16V && NS == 2 && !kSmall;
  // kPipe (the prefill with a bf16 query: kF16V and kF16K): the workgroup
  // widens tile t+1 into a second f16 buffer while it computes tile t (see
  // run_pipe), so the tile's compute reads only f16 buffers and the stage
  // is refilled as soon as it is widened: one barrier per tile.
  static constexpr bool kPipe = kF16V && kF16K;
  static constexpr int kHB = NB / 2;  // kDSplit: blocks of a wave's half
  static constexpr int kHM = D / 32;  // kDSplit: 16-dim PV tiles of a wave's half

  const DecodeLaunch &p;
  int lane, li, lg, kvh, b, wave;
  int swave;               // wave, read into a scalar: indexes this wave's tile copies
  int32_t seq, len, tok0, tok_end, n_tiles;
  int32_t app_mode;        // 0: no rows to append here; 1: before the first copy; 2: after the prologue copies
  int32_t app_first;       // first tile of this partition that holds an appended row
  bool issued0 = false;    // kKReg: tile 0's copies and K codes went out in the prologue
  int32_t pg_first;        // first page index (within the sequence) of the partition
  int32_t pidv;            // lane i: page id of the partition's i-th page
  uint64_t pid_bad;        // lanes whose page id was out of range (replaced by page 0)
  int32_t apos[4];         // positions of this entry's appended rows (-1: another sequence)
  const __attribute__((address_space(3))) int32_t *pg_lds;  // kPageList: page id of page index i
  lds_u8 *vf16;            // kF16V: [dim][4 k-groups] x 8 f16, k-group slot lg ^ (dim & 3)
  const uint8_t *kv_base;  // pages + kv head offset
  uint64_t PB;
  ChunkPlan<D, kSmall, kKReg, NW> plan;
  QOp kreg[2][kQC];        // kKReg: K codes of the tile being computed (A operands)
  QOp qhi[kQR][kQC], qmd[kQR][kQC], qlo[kQR][kQC];  // query planes (see split_q_planes)
  v8h qf[kQF];             // kF16K: query f16 operand per Q8 block (see load_q_f16)
  lds_u8 *kf16;            // kF16K: [token][D] f16, 16-byte chunk c of row r at c ^ (r & (D/8 - 1))
  const lds_u8 *ks;        // kPipe: the computed tile's K scales (copied out of its stage)
  lds_u8 *xs;              // kDSplit: partial scores [wave][lane][8] f32, then alphas [wave][lane] f32
  float rmul[NP];
  int32_t rlim[NP];
  int32_t rlim_min;        // the smallest rlim of the live rows (wave-uniform)
  v4f oacc[NP][D / 16];
  float mref[NP], lrun[NP];
  // The PV weights multiply the V scales times 2^vexp (see scale_v), so
  // oacc carries that factor; finish() divides it out.
  static constexpr int32_t kVexpMax = 30;
  int32_t vexp = kVexpMax;
  lds_u8 *vsc;             // NW > 1: this wave's 2*D-byte copy of the tile's scaled V scales

  __device__ __forceinline__ Decoder(const DecodeLaunch &p_) : p(p_) {}

  // The V scales of the tile in stage `st` times 2^vexp, for the PV: in
  // place with one wave (its LDS accesses are performed in order), else in
  // this wave's copy vsc (the waves of a workgroup share the stage).
  // The PV weights are f16 products p * d_v (two terms, see compute).  With
  // the scales as stored, a V of small magnitude (d_v below about 2^-12,
  // |v| below about 0.03) puts them in the f16 subnormal range, whose
  // absolute spacing 2^-24 is far coarser than the two terms carry.  vexp
  // is the largest exponent with 2^vexp * max d_v <= 2^11 over the
  // partition's tiles so far (0 <= d_v; the maximum's f16 exponent field e
  // gives d_v < 2^(e-14), so vexp = 25 - max(e, 1), at most kVexpMax): a
  // power-of-two step that is exact, keeps every weight below 2^15 (p <=
  // 2^kTau) and every weight of a p >= 2^-25 on the tile's largest scale
  // normal.  vexp only decreases; when it does, the accumulators take the
  // same exact step.  probe_v reads the scales and tests them against the
  // current vexp (each lane its own: a few instructions per tile); only a
  // tile that needs a smaller vexp (a partition's first, then rarely) takes
  // apply_v's wave-wide maximum and the accumulators' step.  Split so that
  // a tile's QK can hide the probe's latency.
  static constexpr int kVW = D / 128;  // 32-bit words of the tile's 2*D bytes of V scales per lane
  struct VProbe {
    uint32_t w[kVW];  // the lane's scales, as stored
    int32_t mx;       // their largest |d_v| bit pattern
  };
  __device__ __forceinline__ bool probe_v(const lds_u8 *st, VProbe &v) const {
    const lds_u8 *src = st + S::kVS + 4 * kVW * lane;
    uint32_t mx = 0;
#pragma unroll
    for (int i = 0; i < kVW; ++i) {
      v.w[i] = lds_load<uint32_t>(src + 4 * i);
      const uint32_t a = v.w[i] & 0x7fff7fffu;  // |d_v| as u16 pairs: ordered as the values
      mx = max(mx, max(a & 0xffffu, a >> 16));
    }
    v.mx = (int32_t)mx;
    // exponent field e > 25 - vexp: this vexp would take a weight past 2^15
    return v.mx >= (26 - vexp) * 1024;
  }
  __device__ __forceinline__ const lds_u8 *apply_v(const lds_u8 *st, bool over, const VProbe &v) {
    if (__any(over)) {
      int32_t m = v.mx;
      m = max(m, __builtin_amdgcn_update_dpp(0, m, 0x111, 0xf, 0xf, false));  // row_shr:1
      m = max(m, __builtin_amdgcn_update_dpp(0, m, 0x112, 0xf, 0xf, false));  // row_shr:2
      m = max(m, __builtin_amdgcn_update_dpp(0, m, 0x114, 0xf, 0xf, false));  // row_shr:4
      m = max(m, __builtin_amdgcn_update_dpp(0, m, 0x118, 0xf, 0xf, false));  // row_shr:8
      const int32_t mw = max(max(__builtin_amdgcn_readlane(m, 15), __builtin_amdgcn_readlane(m, 31)),
                             max(__builtin_amdgcn_readlane(m, 47), __builtin_amdgcn_readlane(m, 63)));
      const int32_t et = 25 - max(mw >> 10, 1);  // < vexp: some lane was over
      const float f = __builtin_amdgcn_ldexpf(1.0f, et - vexp);
#pragma unroll
      for (int np = 0; np < NP; ++np)
#pragma unroll
        for (int m2 = 0; m2 < D / 16; ++m2) oacc[np][m2] *= f;
      vexp = et;
    }
    // 2^vexp as at most two normal f16 factors (-6 <= vexp <= 30), as bits
    const uint32_t b1 = (uint32_t)(min(vexp, 15) + 15) << 10;
    const uint32_t b2 = (uint32_t)(max(vexp - 15, 0) + 15) << 10;
    const v2h f1 = __builtin_bit_cast(v2h, b1 | (b1 << 16));
    const v2h f2 = __builtin_bit_cast(v2h, b2 | (b2 << 16));
    lds_u8 *dst = NW == 1 ? const_cast<lds_u8 *>(st) + S::kVS : vsc;
#pragma unroll
    for (int i = 0; i < kVW; ++i) {
      v2h h = __builtin_bit_cast(v2h, v.w[i]) * f1;
      if (vexp > 15) h *= f2;
      *reinterpret_cast<__attribute__((address_space(3))) uint32_t *>(dst + 4 * kVW * lane + 4 * i) =
          __builtin_bit_cast(uint32_t, h);
    }
    return dst;
  }
  __device__ __forceinline__ const lds_u8 *scale_v(const lds_u8 *st) {
    VProbe v;
    const bool over = probe_v(st, v);
    return apply_v(st, over, v);
  }

  // Divides the accumulators by 2^vexp (after the last tile).
  __device__ __forceinline__ void finish() {
    const float f = __builtin_amdgcn_ldexpf(1.0f, -vexp);
#pragma unroll
    for (int np = 0; np < NP; ++np)
#pragma unroll
      for (int m = 0; m < D / 16; ++m) oacc[np][m] *= f;
  }

  // kKReg: V-code copies 0..K-1 of a tile (see issue); the immediate offset
  // must be a constant expression, hence the recursion.
  template <int K>
  __device__ __forceinline__ static void copy_v_codes(const uint8_t *vsrc, lds_u8 *dst) {
    if constexpr (K > 0) {
      copy_v_codes<K - 1>(vsrc, dst);
      constexpr int k = K - 1;
      __builtin_amdgcn_global_load_lds(vsrc + 4096 * (k / 4), dst + 4096 * (k / 4), 16, 1024 * (k % 4), kCpol);
    }
  }

  // Copy tile `tile` (32 tokens) of this work unit HBM -> LDS stage `dst`.
  // Page ids come from `pidv` (lane i holds the partition's i-th page id).
  __device__ __forceinline__ void issue(int tile, lds_u8 *dst) {
    const Geo &g = p.g;
    const int32_t t0 = tok0 + tile * kTile;
    // page_tokens is a power of two (checked on the host): shifts, not the
    // generic signed division
    const int32_t psh = __builtin_ctz((uint32_t)g.page_tokens);
    const int32_t pi = (t0 >> psh) - pg_first;
    using PL = ChunkPlan<D, kSmall, kKReg, NW>;
    if constexpr (!kSmall) {
      const int32_t pid = kPageList ? __builtin_amdgcn_readfirstlane(pg_lds[pi])
                                    : __builtin_amdgcn_readlane(pidv, pi);
      const uint8_t *base = kv_base + (uint64_t)pid * PB;
      const uint32_t s0 = (uint32_t)(t0 & (g.page_tokens - 1));
      if constexpr (kKReg) {
        // The V codes of a tile are 32*D contiguous bytes (D rows of 32
        // slots), copied to the stage's first 32*D bytes: 2D/64 copies from
        // one lane address at offsets of 1 KiB.  The copy's immediate offset
        // moves the global and the LDS address alike, so the copies of each
        // 4 KiB group share one address register and one M0.  The last copy
        // carries the K and V scale runs (plan entry 2D/64).
        constexpr int kNV = 2 * D / 64;
        static_assert(S::kInstr == kNV + 1, "V codes, then one copy of both scale runs");
        copy_v_codes<kNV>(base + plan.off[0] + s0 * (uint32_t)D, dst);
        __builtin_amdgcn_global_load_lds(base + plan.off[kNV] + s0 * (uint32_t)(D / 16),
                                         dst + PL::dst16(kNV), 16, 0, kCpol);
        return;
      }
      // this wave's copies k = i*NW + wave, entry i of its plan
#pragma unroll
      for (int i = 0; i < PL::kPer; ++i) {
        const int k = i * PL::kWaves + swave;
        if (PL::kWaves > 1 && PL::kN16 % PL::kWaves != 0 && k >= PL::kN16) break;
        // kKReg: copies 0..2D/64-1 are V codes, the rest scales (their
        // padding lanes read inside the region either way)
        const uint32_t mul = kKReg ? (64 * k < 2 * D ? (uint32_t)D : (uint32_t)(D / 16)) : plan.mul[i];
        const uint32_t voff = plan.off[i] + s0 * mul;
        __builtin_amdgcn_global_load_lds(base + voff, dst + PL::dst16(k), 16, 0, kCpol);
      }
    } else {
      // 16-token pages: the two halves of the tile live in two pages
      const int32_t pid0 = kPageList ? __builtin_amdgcn_readfirstlane(pg_lds[pi])
                                     : __builtin_amdgcn_readlane(pidv, pi);
      const int32_t pid1 = (t0 + 16 < len) ? (kPageList ? __builtin_amdgcn_readfirstlane(pg_lds[pi + 1])
                                                        : __builtin_amdgcn_readlane(pidv, pi + 1))
                                           : pid0;
      const uint8_t *base0 = kv_base + (uint64_t)pid0 * PB;
      const uint8_t *base1 = kv_base + (uint64_t)pid1 * PB;
#pragma unroll
      for (int k = 0; k < PL::kN16; ++k) {
        if (NW > 1 && k % NW != wave) continue;
        const bool h = (plan.halves >> k) & 1u;
        __builtin_amdgcn_global_load_lds((h ? base1 : base0) + plan.off[k], dst + PL::dst16(k), 16, 0, kCpol);
      }
#pragma unroll
      for (int k = 0; k < PL::kN4; ++k) {
        if (NW > 1 && (PL::kN16 + k) % NW != wave) continue;
        const bool h = (plan.halves >> (PL::kN16 + k)) & 1u;
        __builtin_amdgcn_global_load_lds((h ? base1 : base0) + plan.off[PL::kN16 + k], dst + PL::dst4(k), 4, 0, kCpol);
      }
    }
  }

  // Quantize and store this partition's appended rows for kv head `kvh`
  // (canonical or har-serve rule, bit-exact with rkv_append_q8), then wait
  // until the stores are done so the tile copies that follow read them.
  __device__ __forceinline__ void append_rows() {
    const Geo &g = p.g;
    for (int j = 0; j < p.q_len; ++j) {
      const int32_t row = b * p.q_len + j;
      const int32_t pos = p.app_pos[row];
      if (p.app_seq_ids[row] != seq || pos < tok0 || pos >= tok_end) continue;
      const int32_t page = p.bt[(int64_t)seq * p.bt_stride + pos / g.page_tokens];
      if (page < 0 || page >= g.num_pages) continue;  // reported by the page-id prefetch
      const int32_t slot = pos % g.page_tokens;
      // 2 kinds x D/32 blocks x 8 lanes = D/2 lane-tasks
#pragma unroll
      for (int pass = 0; pass < D / 128; ++pass) {
        const int u = 64 * pass + lane;
        const int kind = u / (D / 4);
        const int blk = (u % (D / 4)) >> 3;
        const int sub = u & 7;
        float v[4];
        load_src4(kind == 0 ? p.app_k : p.app_v,
                  ((uint64_t)row * g.kv_heads + kvh) * D + (uint64_t)(32 * blk + 4 * sub),
                  p.app_bf16 != 0, v);
        uint16_t scale;
        const uint32_t codes = q8_quantize_lane(v, p.app_rule, scale);
        store_q8_lane(g, p.pages_w + region_base(g, page, kvh, kind), kind, slot, blk, sub, codes, scale);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  // kKReg (one wave): the appended rows are handled in two halves around
  // tile 0's copies.  app_load loads the source values of this partition's
  // rows (row j is live when its position lies in [tok0, tok_end) on a valid
  // page); app_store quantizes and stores them, with the page id taken from
  // pidv.  Neither reloads positions or page ids, so the loads ride with the
  // prologue's and no dependent round trip follows tile 0's copies.
  __device__ __forceinline__ void app_load(uint4 (&w)[4][D / 128], bool (&live)[4]) {
    const Geo &g = p.g;
    const bool bf16 = p.app_bf16 != 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t pos = apos[j];
      live[j] = pos >= tok0 && pos < tok_end &&
                !((pid_bad >> (pos / g.page_tokens - pg_first)) & 1u);
      if (!live[j]) continue;
      const int32_t row = b * p.q_len + j;
#pragma unroll
      for (int pass = 0; pass < D / 128; ++pass) {
        const int u = 64 * pass + lane;
        const int kind = u / (D / 4);
        const int blk = (u % (D / 4)) >> 3;
        const int sub = u & 7;
        const uint64_t off = ((uint64_t)row * g.kv_heads + kvh) * D + (uint64_t)(32 * blk + 4 * sub);
        const void *src = kind == 0 ? p.app_k : p.app_v;
        // raw words only: the values are converted in app_store, so no wait
        // follows a load here
        if (bf16) {
          const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(src) + off);
          w[j][pass] = uint4{v.x, v.y, 0u, 0u};
        } else {
          w[j][pass] = *reinterpret_cast<const uint4 *>(static_cast<const float *>(src) + off);
        }
      }
    }
  }
  __device__ __forceinline__ void app_store(const uint4 (&w)[4][D / 128], const bool (&live)[4]) {
    const Geo &g = p.g;
    const bool bf16 = p.app_bf16 != 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!live[j]) continue;
      const int32_t pos = apos[j];
      const int32_t page = __builtin_amdgcn_readlane(pidv, pos / g.page_tokens - pg_first);
      const int32_t slot = pos % g.page_tokens;
#pragma unroll
      for (int pass = 0; pass < D / 128; ++pass) {
        const int u = 64 * pass + lane;
        const int kind = u / (D / 4);
        const int blk = (u % (D / 4)) >> 3;
        const int sub = u & 7;
        float v[4];
        if (bf16) {
          v[0] = bf16_bits_to_f32((uint16_t)(w[j][pass].x & 0xffffu));
          v[1] = bf16_bits_to_f32((uint16_t)(w[j][pass].x >> 16));
          v[2] = bf16_bits_to_f32((uint16_t)(w[j][pass].y & 0xffffu));
          v[3] = bf16_bits_to_f32((uint16_t)(w[j][pass].y >> 16));
        } else {
          v[0] = __uint_as_float(w[j][pass].x);
          v[1] = __uint_as_float(w[j][pass].y);
          v[2] = __uint_as_float(w[j][pass].z);
          v[3] = __uint_as_float(w[j][pass].w);
        }
        uint16_t scale;
        const uint32_t codes = q8_quantize_lane(v, p.app_rule, scale);
        store_q8_lane(g, p.pages_w + region_base(g, page, kvh, kind), kind, slot, blk, sub, codes, scale);
      }
    }
  }

  // kKReg: K codes of tile `tile` into kreg.  Lane (li, lg) of M-tile mt
  // holds token row 16*mt + li: dims 64*c + 16*lg .. +15 of 64-dim step c,
  // or (kWide) dims 32*blk + 8*lg .. +7 of block blk.
  __device__ __forceinline__ void load_k(int tile) {
    const Geo &g = p.g;
    const int32_t t0 = tok0 + tile * kTile;
    const int32_t psh = __builtin_ctz((uint32_t)g.page_tokens);
    const int32_t pid = __builtin_amdgcn_readlane(pidv, (t0 >> psh) - pg_first);
    const uint8_t *base = kv_base + (uint64_t)pid * PB +
                          (uint64_t)((t0 & (g.page_tokens - 1)) + li) * D + (kWide ? 8 : 16) * lg;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int c = 0; c < kQC; ++c)
        kreg[mt][c] = __builtin_nontemporal_load(
            reinterpret_cast<const QOp *>(base + (uint64_t)(16 * mt) * D + (kWide ? 32 : 64) * c));
  }

  // Scores, online softmax and PV for the tile held in LDS stage `st`
  // (kKReg: the next tile is copied into `next_stage` meanwhile).
  // drain: wait for this wave's stores before the next tile's copies (the
  // appended rows of that tile were stored during this one)
  __device__ __forceinline__ void compute(int tile, const lds_u8 *st, lds_u8 *next_stage = nullptr,
                                         bool drain = false) {
    const int32_t t0 = tok0 + tile * kTile;
    // ---- QK^T: int32 block dots, scaled by the f16 K scale of (token, block) ----
    // Each plane set computes t = 128*dot(hi) + dot(md) + floor(dot(lo)/128):
    // the lo plane's dot, shifted, is the accumulator input of the md
    // plane's MFMA.  |t| < 2^27, so every step is exact in int32 and the f32
    // conversion rounds once.
    float sacc[kQR][2][4];
    // tiles wholly below every live row's limit skip the per-token mask
    const bool full = t0 + kTile <= rlim_min;
    // the V scales' exponent (scale_v), probed before the QK so that it
    // hides the probe's latency: one wave.  The verify's two waves hold too
    // many registers across the QK for that and scale after the softmax;
    // the prefill's (kF16V) waves scale in step(), before its barrier.
    constexpr bool kEarlyProbe = NW == 1;
    VProbe vp;
    bool vover = false;
    if constexpr (kEarlyProbe) {
      if (t0 + kTile > len) mask_tail_scales(st, t0);
      vover = probe_v(st, vp);
    }
#pragma unroll
    for (int nt = 0; nt < kQR; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[nt][mt][r] = 0.0f;
    if constexpr (kF16K && kF16V) {
      // K f16 operands and scales from LDS: block blk+1's are read before
      // block blk's MFMAs, so each block's LDS latency hides behind the
      // previous block's work.  Lane-ordered scales: 8 f16 = tokens 4*lg+r
      // of M-tile 0, then of M-tile 1; the operand of M-tile mt is dims
      // 32*blk + 8*lg .. +7 of token row 16*mt + li, f16 chunk 4*blk + lg.
      const lds_u8 *ksrc = kPipe ? ks : st + S::kKS;
      v8h ka[2], kn[2], dka, dkn;
      auto load_blk = [&](int blk, v8h(&a)[2], v8h &dk) {
        dk = lds_load<v8h>(ksrc + 2 * (blk * 32 + 8 * lg));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int krow = 16 * mt + li;
          const int pc = (4 * blk + lg) ^ (krow & (D / 8 - 1));
          a[mt] = lds_load<v8h>(kf16 + krow * (2 * D) + 16 * pc);
        }
      };
      load_blk(0, ka, dka);
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) {
        if (blk + 1 < NB) load_blk(blk + 1, kn, dkn);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[mt], qf[blk], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sacc[0][mt][r] = __builtin_fmaf(c[r], (float)dka[4 * mt + r], sacc[0][mt][r]);
        }
        if (blk + 1 < NB) {
          ka[0] = kn[0];
          ka[1] = kn[1];
          dka = dkn;
        }
      }
    } else if constexpr (kF16K) {
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) {
        // lane-ordered scales: 8 f16 = tokens 4*lg+r of M-tile 0, then of M-tile 1
        const v8h dk8 = lds_load<v8h>(st + S::kKS + 2 * (blk * 32 + 8 * lg));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int krow = 16 * mt + li;
          // the int8 operand (see the kWide QK below), widened
          const int pc = (2 * blk + (lg >> 1)) ^ (krow & (S::kCPR - 1));
          const int64_t k8 = kKReg ? kreg[mt][blk]
                                   : lds_load<int64_t>(st + S::kKC + krow * D + 16 * pc + 8 * (lg & 1));
          v2h h0, h1, h2, h3;
          v8x4_to_f16((uint32_t)k8 ^ 0x80808080u, h0, h1);
          v8x4_to_f16((uint32_t)((uint64_t)k8 >> 32) ^ 0x80808080u, h2, h3);
          const v8h a = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[blk], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sacc[0][mt][r] = __builtin_fmaf(c[r], (float)dk8[4 * mt + r], sacc[0][mt][r]);
        }
      }
    } else if constexpr (kWide) {
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) {
        // lane-ordered scales: 8 f16 = tokens 4*lg+r of M-tile 0, then of M-tile 1
        const v8h dk8 = lds_load<v8h>(st + S::kKS + 2 * (blk * 32 + 8 * lg));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int krow = 16 * mt + li;
          // dims 32*blk + 8*lg .. +7: half (lg & 1) of logical 16-byte chunk 2*blk + (lg >> 1)
          const int pc = (2 * blk + (lg >> 1)) ^ (krow & (S::kCPR - 1));
          const int64_t a = kKReg ? kreg[mt][blk]
                                  : lds_load<int64_t>(st + S::kKC + krow * D + 16 * pc + 8 * (lg & 1));
          const v4i z = {0, 0, 0, 0};
          const v4i cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, qlo[0][blk], z, 0, 0, 0);
          const v4i cls = {cl[0] >> 7, cl[1] >> 7, cl[2] >> 7, cl[3] >> 7};
          const v4i cm = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, qmd[0][blk], cls, 0, 0, 0);
          const v4i ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, qhi[0][blk], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sacc[0][mt][r] = __builtin_fmaf((float)((ch[r] << 7) + cm[r]), (float)dk8[4 * mt + r],
                                            sacc[0][mt][r]);
        }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int krow = 16 * mt + li;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int pc = (4 * c + lg) ^ (krow & (S::kCPR - 1));
          const v4i a = kKReg ? kreg[mt][c] : lds_load<v4i>(st + S::kKC + krow * D + 16 * pc);
          const int blk = 2 * c + (li >> 3);
          // lane-ordered scales: 8 f16 = tokens 4*lg+r of M-tile 0, then of M-tile 1
          const v8h dk8 = lds_load<v8h>(st + S::kKS + 2 * (blk * 32 + 8 * lg));
          const float dk[4] = {(float)dk8[4 * mt], (float)dk8[4 * mt + 1], (float)dk8[4 * mt + 2],
                               (float)dk8[4 * mt + 3]};
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const v4i z = {0, 0, 0, 0};
            const v4i cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qlo[nt][c], z, 0, 0, 0);
            const v4i cls = {cl[0] >> 7, cl[1] >> 7, cl[2] >> 7, cl[3] >> 7};
            const v4i cm = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qmd[nt][c], cls, 0, 0, 0);
            const v4i ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qhi[nt][c], z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              sacc[nt][mt][r] = __builtin_fmaf((float)((ch[r] << 7) + cm[r]), dk[r], sacc[nt][mt][r]);
          }
        }
      }
    }

    // kKReg: the QK above has read this tile's K codes and K scales; the
    // next tile's K codes and stage copy start now and land during this
    // tile's softmax and PV.  (They cannot start earlier: before a register
    // use of loaded data the compiler waits for every outstanding load,
    // stage copies included, so copies issued before a QK complete before
    // it.)
    if constexpr (kKReg) {
      if (tile + 1 < n_tiles) {
        if (drain) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        issue(tile + 1, next_stage);
        load_k(tile + 1);
      }
    }

    const lds_u8 *vs = vsc;
    if constexpr (kEarlyProbe) vs = apply_v(st, vover, vp);

    // ---- online softmax (base 2, lazily rescaled reference max) ----
    uint32_t pp[NP][4];  // p of the lane's 8 tokens as packed f16 pairs
    uint32_t pl[NP][4];  // kSplitP: p - f16(p), rounded to f16
    uint32_t pz[NP][4];  // kColSplit: f16(p) on lanes li >= 8, 0 on lanes li < 8
#pragma unroll
    for (int np = 0; np < NP; ++np) {
      float s[8];
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v;  // unscaled: the softmax multiplies by rmul (> 0) in the fma below
          if constexpr (kWide) {
            v = sacc[0][mt][r];
          } else {
            // the even- and odd-block halves of a row sit 8 columns apart
            float lo_t = 0.f, hi_t = 0.f;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              if (nt != 2 * np && nt != 2 * np + 1) continue;
              const float tot = sacc[nt][mt][r] + dpp_ror8(sacc[nt][mt][r]);
              if (nt == 2 * np) lo_t = tot;
              else hi_t = tot;
            }
            // kColSplit: lanes li >= 8 hold row li - 8 (the ror-8 sum is symmetric)
            v = kColSplit || li < 8 ? lo_t : hi_t;
          }
          s[4 * mt + r] = v;
          tmax = fmaxf(tmax, v);
        }
      if (!full) {
        // token t0 + 16*mt + 4*lg + r is visible below rlim: compare the
        // tile offset 16*mt + r with the lane's limit (immediates, one
        // subtraction per tile)
        const int32_t lim = (rlim[np] - 4 * lg) - t0;
        tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sv = 16 * mt + r < lim ? s[4 * mt + r] : -INFINITY;
            s[4 * mt + r] = sv;
            tmax = fmaxf(tmax, sv);
          }
      }
      tmax = row_group_max(tmax) * rmul[np];  // max(s) * rmul = max(s * rmul), rmul > 0
      const bool need = tmax > mref[np] + kTau;  // also true for the first visible tile
      if (__any(need)) {
        const float mnew = need ? tmax : mref[np];
        const float alpha = !need ? 1.0f : (mref[np] == -INFINITY ? 0.0f
                                                                  : __builtin_amdgcn_exp2f(mref[np] - mnew));
        lrun[np] *= alpha;
#pragma unroll
        for (int m = 0; m < D / 16; ++m) oacc[np][m] *= alpha;
        mref[np] = mnew;
      }
      const float muse = mref[np] == -INFINITY ? 0.0f : mref[np];
      float pr[8];
      float lsum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], rmul[np], -muse));
        lsum += pr[e];
      }
      lrun[np] += lsum;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v2h h2 = {(_Float16)pr[2 * i], (_Float16)pr[2 * i + 1]};
        pp[np][i] = __builtin_bit_cast(uint32_t, h2);
        if constexpr (kSplitP) {
          const v2h l2 = p_residual(h2, pr[2 * i], pr[2 * i + 1]);
          pl[np][i] = __builtin_bit_cast(uint32_t, l2);
          if constexpr (kColSplit) {
            // columns 0-7 take p and no second term: zero their p_lo and
            // (below) their product subtrahend
            pz[np][i] = li >= 8 ? pp[np][i] : 0u;
            if (li < 8) pl[np][i] = 0u;
          }
        }
      }
    }

    // ---- PV: B = p * d_v as packed f16.  Without kSplitP that is one f16
    // value per (token, row): p rounded to f16, times the stored f16 scale,
    // rounded again (up to 2^-11 relative per weight).  With kSplitP a second
    // operand carries what those roundings drop -- the product's rounding
    // error, exact from an f16 fma, plus (p - f16(p)) * d_v -- and a second
    // MFMA on the same V operand adds it, so the weights are exact to about
    // 2^-22. ----
    if constexpr (!kEarlyProbe && !kF16V) {
      if (t0 + kTile > len) mask_tail_scales(st, t0);
      vs = scale_v(st);
    }
    pv(st, vs, pp, pl, pz);
  }

  // kDSplit: tile `tile` (stage `st`) on this wave's half of the dims.
  //  1. QK of all 32 rows over the half's blocks (f16 MFMA, K widened in
  //     registers): partial scores of n-tiles 0 and 1.
  //  2. The other wave's rows' partials go to LDS (slot w of xs); after a
  //     barrier this wave adds the other half's partials of its own rows.
  //  3. Online softmax of the own rows (as compute's, one n-tile).
  //  4. p (two f16 terms) and the rescale factor of the own rows go to LDS
  //     (p in the stage's K-code area, which the QK no longer needs); after a
  //     barrier this wave reads the other rows' and rescales their
  //     accumulators if the other wave moved its maxima.
  //  5. PV of all 32 rows over the half's dims (V widened in registers).
  // The wave number is a template argument so that every register array
  // index below is a constant.
  __device__ __forceinline__ void compute_split(int tile, const lds_u8 *st) {
    if (wave == 0) compute_split_w<0>(tile, st);
    else compute_split_w<1>(tile, st);
  }
  template <int W>
  __device__ __forceinline__ void compute_split_w(int tile, const lds_u8 *st) {
    const int32_t t0 = tok0 + tile * kTile;
    const bool full = t0 + kTile <= rlim_min;
    constexpr int w = W, o = 1 - W;
    // the PV's V scales (scale_v): probed before the QK, which hides the
    // probe's latency, and scaled into vsc after it
    if (t0 + kTile > len) mask_tail_scales(st, t0);
    VProbe vp;
    const bool vover = probe_v(st, vp);
    float sacc[2][2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[nt][mt][r] = 0.0f;
#pragma unroll
    for (int bl = 0; bl < kHB; ++bl) {
      const int blk = w * kHB + bl;
      const v8h dk8 = lds_load<v8h>(st + S::kKS + 2 * (blk * 32 + 8 * lg));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int krow = 16 * mt + li;
        const int pc = (2 * blk + (lg >> 1)) ^ (krow & (S::kCPR - 1));
        const int64_t k8 = lds_load<int64_t>(st + S::kKC + krow * D + 16 * pc + 8 * (lg & 1));
        v2h h0, h1, h2, h3;
        v8x4_to_f16((uint32_t)k8 ^ 0x80808080u, h0, h1);
        v8x4_to_f16((uint32_t)((uint64_t)k8 >> 32) ^ 0x80808080u, h2, h3);
        const v8h a = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[nt * kHB + bl], z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sacc[nt][mt][r] = __builtin_fmaf(c[r], (float)dk8[4 * mt + r], sacc[nt][mt][r]);
        }
      }
    }

    const lds_u8 *vs = apply_v(st, vover, vp);

    // ---- 2. partial-score exchange ----
    __attribute__((address_space(3))) v4f *ps = reinterpret_cast<__attribute__((address_space(3))) v4f *>(xs);
    ps[(w * 64 + lane) * 2] = v4f{sacc[o][0][0], sacc[o][0][1], sacc[o][0][2], sacc[o][0][3]};
    ps[(w * 64 + lane) * 2 + 1] = v4f{sacc[o][1][0], sacc[o][1][1], sacc[o][1][2], sacc[o][1][3]};
    wg_barrier_lds();
    const v4f q0 = ps[(o * 64 + lane) * 2], q1 = ps[(o * 64 + lane) * 2 + 1];
    float sown[2][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sown[0][r] = sacc[w][0][r] + q0[r];
      sown[1][r] = sacc[w][1][r] + q1[r];
    }

    // ---- 3. online softmax of the own rows ----
    float s[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = sown[mt][r];  // unscaled, as in compute
        s[4 * mt + r] = v;
        tmax = fmaxf(tmax, v);
      }
    if (!full) {
      // compared by position (see mask_tail_scales)
      tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = t0 + 16 * mt + 4 * lg + r;
          const float sv = tok < rlim[0] ? s[4 * mt + r] : -INFINITY;
          s[4 * mt + r] = sv;
          tmax = fmaxf(tmax, sv);
        }
    }
    tmax = row_group_max(tmax) * rmul[0];
    const bool need = tmax > mref[0] + kTau;  // also true for the first visible tile
    float alpha = 1.0f;
    if (__any(need)) {
      const float mnew = need ? tmax : mref[0];
      alpha = !need ? 1.0f : (mref[0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[0] - mnew));
      lrun[0] *= alpha;
#pragma unroll
      for (int m = 0; m < kHM; ++m) oacc[0][w * kHM + m] *= alpha;
      mref[0] = mnew;
    }
    const float muse = mref[0] == -INFINITY ? 0.0f : mref[0];
    float pr[8];
    float lsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], rmul[0], -muse));
      lsum += pr[e];
    }
    lrun[0] += lsum;
    uint32_t pq[2][8];  // [n-tile][p hi x4, p lo x4]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v2h h2 = {(_Float16)pr[2 * i], (_Float16)pr[2 * i + 1]};
      const v2h l2 = p_residual(h2, pr[2 * i], pr[2 * i + 1]);
      pq[w][i] = __builtin_bit_cast(uint32_t, h2);
      pq[w][4 + i] = __builtin_bit_cast(uint32_t, l2);
    }

    // ---- 4. p and rescale exchange (p in this stage's K-code area) ----
    __attribute__((address_space(3))) v4i *px =
        reinterpret_cast<__attribute__((address_space(3))) v4i *>(const_cast<lds_u8 *>(st) + S::kKC);
    __attribute__((address_space(3))) float *ax =
        reinterpret_cast<__attribute__((address_space(3))) float *>(xs + 2 * 64 * 32);
    px[(w * 64 + lane) * 2] = v4i{(int)pq[w][0], (int)pq[w][1], (int)pq[w][2], (int)pq[w][3]};
    px[(w * 64 + lane) * 2 + 1] = v4i{(int)pq[w][4], (int)pq[w][5], (int)pq[w][6], (int)pq[w][7]};
    ax[w * 64 + lane] = alpha;
    wg_barrier_lds();
    {
      const v4i a0 = px[(o * 64 + lane) * 2], a1 = px[(o * 64 + lane) * 2 + 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pq[o][i] = (uint32_t)a0[i];
        pq[o][4 + i] = (uint32_t)a1[i];
      }
      const float alpha_o = ax[o * 64 + lane];
      if (__any(alpha_o != 1.0f)) {
#pragma unroll
        for (int m = 0; m < kHM; ++m) oacc[0][o * kHM + m] *= alpha_o;
      }
    }

    // ---- 5. PV of all 32 rows over the half's dims ----
#pragma unroll
    for (int bl = 0; bl < kHB; ++bl) {
      const int blk = w * kHB + bl;
      const v4i sv = lds_load<v4i>(vs + 2 * (blk * 32 + 8 * lg));
      // weights step by step across the eight pairs (see pv_weights), then
      // both dim tiles' V operands, then the MFMAs: no MFMA reads a register
      // the instruction just before it wrote
      v8h pb[2], pbl[2];
      v2h prod[2][4], err[2][4];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          prod[nt][i] = __builtin_bit_cast(v2h, pq[nt][i]) * __builtin_bit_cast(v2h, (uint32_t)sv[i]);
          pb[nt][2 * i] = prod[nt][i][0];
          pb[nt][2 * i + 1] = prod[nt][i][1];
        }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          err[nt][i] = __builtin_elementwise_fma(__builtin_bit_cast(v2h, pq[nt][i]),
                                                 __builtin_bit_cast(v2h, (uint32_t)sv[i]), -prod[nt][i]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v2h lo = __builtin_elementwise_fma(__builtin_bit_cast(v2h, pq[nt][4 + i]),
                                                   __builtin_bit_cast(v2h, (uint32_t)sv[i]), err[nt][i]);
          pbl[nt][2 * i] = lo[0];
          pbl[nt][2 * i + 1] = lo[1];
        }
      v8h va[2];
#pragma unroll
      for (int hm = 0; hm < 2; ++hm) {
        const int d = 32 * blk + 16 * hm + li;
        const int sw = (d >> 2) & 1;
        const uint32_t w0 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * sw + 4 * lg);
        const uint32_t w1 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * (sw ^ 1) + 4 * lg);
        v2h a0, a1, a2, a3;
        v8x4_to_f16(w0, a0, a1);
        v8x4_to_f16(w1, a2, a3);
        va[hm] = v8h{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
      }
#pragma unroll
      for (int hm = 0; hm < 2; ++hm)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          v4f &acc = oacc[0][nt * kHM + 2 * bl + hm];
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[hm], pb[nt], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[hm], pbl[nt], acc, 0, 0, 0);
        }
    }
  }

  // Tokens past the sequence end may carry junk V scales (an f16 NaN or
  // Inf): the tail tile zeroes them in its landed stage before the PV reads
  // them, so 0 * junk cannot turn into NaN and no other tile pays for a
  // mask.  Lane li == 0 of each k-group rewrites the group's 8 scales of
  // every block; LDS accesses of a wave are performed in order, and the
  // waves of a workgroup that share the stage write the same values.
  __device__ __forceinline__ void mask_tail_scales(const lds_u8 *st, int32_t t0) {
    // token t0 + 4*lg + k is kept when the tile offset k is below the
    // lane's limit (kDSplit: compared by position; the limit would hold one
    // more register across the loop, and that kernel has none to spare)
    uint32_t m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = (i < 2 ? 0 : 16) + 2 * (i & 1);
      if constexpr (kDSplit) {
        const int tk = t0 + 4 * lg + k;
        m[i] = (tk < len ? 0xffffu : 0u) | (tk + 1 < len ? 0xffff0000u : 0u);
      } else {
        const int32_t lim = (len - 4 * lg) - t0;
        m[i] = (k < lim ? 0xffffu : 0u) | (k + 1 < lim ? 0xffff0000u : 0u);
      }
    }
    if (li != 0) return;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      lds_u8 *a = const_cast<lds_u8 *>(st) + S::kVS + 2 * (blk * 32 + 8 * lg);
      v4i sv = lds_load<v4i>(a);
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = (int)((uint32_t)sv[i] & m[i]);
      *reinterpret_cast<__attribute__((address_space(3))) v4i *>(a) = sv;
    }
  }

  // The PV weights of one Q8 block from its lane-ordered V scales `sv`:
  // pb = p * d_v and (kSplitP) pbl = its second term (see compute).
  __device__ __forceinline__ void pv_weights(const v4i sv, const uint32_t (&pp)[NP][4],
                                             const uint32_t (&pl)[NP][4], const uint32_t (&pz)[NP][4],
                                             v8h (&pb)[NP], v8h (&pbl)[NP]) const {
    // Step by step across the four pairs: each step depends on the one
    // before, and back-to-back dependent packed-f16 operations take wait
    // states (s_nop) that four independent pairs in between hide.
#pragma unroll
    for (int np = 0; np < NP; ++np) {
      v2h ph[4], dv[4], q[4], e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ph[i] = __builtin_bit_cast(v2h, pp[np][i]);
        dv[i] = __builtin_bit_cast(v2h, (uint32_t)sv[i]);
      }
      if constexpr (kColSplit) {
        // lanes li < 8: q = 0, so e = f16(p)*d_v rounded once and the
        // second fma adds 0 * d_v; lanes li >= 8: e is the product's
        // exact rounding error and the result the second weight term
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = __builtin_bit_cast(v2h, pz[np][i]) * dv[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = __builtin_elementwise_fma(ph[i], dv[i], -q[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v2h hi = __builtin_elementwise_fma(__builtin_bit_cast(v2h, pl[np][i]), dv[i], e[i]);
          pb[np][2 * i] = hi[0];
          pb[np][2 * i + 1] = hi[1];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          q[i] = ph[i] * dv[i];
          pb[np][2 * i] = q[i][0];
          pb[np][2 * i + 1] = q[i][1];
        }
        if constexpr (kSplitP) {
#pragma unroll
          for (int i = 0; i < 4; ++i) e[i] = __builtin_elementwise_fma(ph[i], dv[i], -q[i]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const v2h lo = __builtin_elementwise_fma(__builtin_bit_cast(v2h, pl[np][i]), dv[i], e[i]);
            pbl[np][2 * i] = lo[0];
            pbl[np][2 * i + 1] = lo[1];
          }
        }
      }
    }
  }
  // The PV MFMAs of 16-dim tile m of every n-tile on V operand va.
  __device__ __forceinline__ void pv_mfma(int m, const v8h va, const v8h (&pb)[NP], const v8h (&pbl)[NP]) {
#pragma unroll
    for (int np = 0; np < NP; ++np) {
      oacc[np][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[np], oacc[np][m], 0, 0, 0);
      if constexpr (kSplitP && !kColSplit)
        oacc[np][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pbl[np], oacc[np][m], 0, 0, 0);
    }
  }

  // PV of one tile (see compute), with the V scales `vs` (scale_v).
  __device__ __forceinline__ void pv(const lds_u8 *st, const lds_u8 *vs, const uint32_t (&pp)[NP][4],
                                     const uint32_t (&pl)[NP][4], const uint32_t (&pz)[NP][4]) {
    if constexpr (kF16V) {
      // V f16 operands and scales from LDS: block blk+1's are read before
      // block blk's weights and MFMAs, so each block's LDS latency hides
      // behind the previous block's work.  The operand of dim tile hm is
      // the 8 tokens lane (d = 32*blk + 16*hm + li, lg) takes.
      v4i svc, svn;
      v8h vac[2], van[2];
      auto load_blk = [&](int blk, v4i &sv, v8h(&va)[2]) {
        sv = lds_load<v4i>(vs + 2 * (blk * 32 + 8 * lg));
#pragma unroll
        for (int hm = 0; hm < 2; ++hm) {
          const int d = 32 * blk + 16 * hm + li;
          va[hm] = lds_load<v8h>(vf16 + 16 * (4 * d + (lg ^ (d & 3))));
        }
      };
      load_blk(0, svc, vac);
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) {
        if (blk + 1 < NB) load_blk(blk + 1, svn, van);
        v8h pb[NP], pbl[NP];
        pv_weights(svc, pp, pl, pz, pb, pbl);
#pragma unroll
        for (int hm = 0; hm < 2; ++hm) pv_mfma(2 * blk + hm, vac[hm], pb, pbl);
        if (blk + 1 < NB) {
          svc = svn;
          vac[0] = van[0];
          vac[1] = van[1];
        }
      }
      return;
    }
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      // (ext-vector loads only: an LDS load of the uint4 struct type makes the
      // compiler drain every in-flight copy before it)
      const v4i sv = lds_load<v4i>(vs + 2 * (blk * 32 + 8 * lg));
      v8h pb[NP], pbl[NP];
      pv_weights(sv, pp, pl, pz, pb, pbl);
#pragma unroll
      for (int hm = 0; hm < 2; ++hm) {
        const int d = 32 * blk + 16 * hm + li;
        const int sw = (d >> 2) & 1;
        const uint32_t w0 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * sw + 4 * lg);
        const uint32_t w1 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * (sw ^ 1) + 4 * lg);
        v2h a0, a1, a2, a3;
        v8x4_to_f16(w0, a0, a1);
        v8x4_to_f16(w1, a2, a3);
        const v8h va = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
        pv_mfma(2 * blk + hm, va, pb, pbl);
      }
    }
  }


  // vmcnt wait for the tile about to be computed when `ahead` later tiles'
  // copies are still in flight.  A tile is kInstr copies, split over the NW
  // waves; counting floor(kInstr / NW) per tile is exact for the waves with
  // that many and waits one copy longer for the others.
  __device__ __forceinline__ static void wait_tiles_ahead(int ahead) {
    constexpr int kI = ChunkPlan<D, kSmall, kKReg, NW>::kInstr / NW;
    static_assert(kI >= 1, "every wave issues at least one copy per tile");
    if (ahead >= 2) {
      constexpr int n = 2 * kI;
      __builtin_amdgcn_s_waitcnt(kWaitBase | (n & 0xf) | ((n >> 4) << 14));
    } else if (ahead == 1) {
      constexpr int n = kI;
      __builtin_amdgcn_s_waitcnt(kWaitBase | (n & 0xf) | ((n >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitBase);
    }
  }

  // Tile t: prefetch tile t+NS-1 into `fill`, wait for `cur`, compute it.
  // kF16V: widen this wave's share of the landed tile's V codes into vf16.
  // Chunk (dim d, k-group g) is the 8 tokens lane (d, g) of the PV MFMA
  // holds: 4g..4g+3 then 16+4g..16+4g+3 (the halves are swapped in the
  // stage when (d >> 2) & 1, as the tile copy put them).
  __device__ __forceinline__ void widen_v(const lds_u8 *st, lds_u8 *dst) {
    constexpr int kChunks = 4 * D;
    // a fixed trip count (chunks c = wave*64 + lane + i*64*NW) keeps the
    // widening straight-line code that the compiler can interleave with the
    // compute that follows it
    constexpr int kIt = (kChunks + 64 * NW - 1) / (64 * NW);
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
      const int c = (i * NW + wave) * 64 + lane;
      if (kChunks % (64 * NW) != 0 && c >= kChunks) continue;
      const int d = c >> 2, g = c & 3;
      const int sw = (d >> 2) & 1;
      const uint32_t w0 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * sw + 4 * g);
      const uint32_t w1 = lds_load<uint32_t>(st + S::kVC + d * 32 + 16 * (sw ^ 1) + 4 * g);
      v2h a0, a1, a2, a3;
      v8x4_to_f16(w0, a0, a1);
      v8x4_to_f16(w1, a2, a3);
      const v8h va = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
      *reinterpret_cast<__attribute__((address_space(3))) v8h *>(dst + 16 * (4 * d + (g ^ (d & 3)))) = va;
    }
  }


  // kF16K: widen this wave's share of the landed tile's K codes into kf16.
  // Physical 16-byte chunk pc of K row r holds logical chunk pc ^ (r mod
  // D/16), the codes of dims 16*lc .. +15 (signed; xor 0x80 makes them the
  // biased form v8x4_to_f16 takes).  They become f16 chunks 2*lc and 2*lc+1.
  __device__ __forceinline__ void widen_k(const lds_u8 *st, lds_u8 *dst) {
    constexpr int kCPR = D / 16;
    constexpr int kChunks = 32 * kCPR;
    constexpr int kIt = (kChunks + 64 * NW - 1) / (64 * NW);  // fixed trip count, as widen_v
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
      const int c = (i * NW + wave) * 64 + lane;
      if (kChunks % (64 * NW) != 0 && c >= kChunks) continue;
      const int r = c / kCPR, pc = c % kCPR;
      const int lc = pc ^ (r & (kCPR - 1));
      const v4i w = lds_load<v4i>(st + S::kKC + r * D + 16 * pc);
      v2h h[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) v8x4_to_f16((uint32_t)w[j] ^ 0x80808080u, h[2 * j], h[2 * j + 1]);
      const v8h f0 = {h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
      const v8h f1 = {h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
      lds_u8 *row = dst + r * (2 * D);
      *reinterpret_cast<__attribute__((address_space(3))) v8h *>(row + 16 * ((2 * lc) ^ (r & (D / 8 - 1)))) = f0;
      *reinterpret_cast<__attribute__((address_space(3))) v8h *>(row + 16 * ((2 * lc + 1) ^ (r & (D / 8 - 1)))) = f1;
    }
  }


  // kPipe: an f16 buffer holds one tile as the compute reads it: K widened
  // [token][D] (kf16's layout, 64*D bytes), V widened (vf16's layout, 64*D
  // bytes), then the tile's K scales as staged (2*D bytes).
  static constexpr int kFK = 0, kFV = 64 * D, kFS = 128 * D;
  static constexpr int kFBytes = 130 * D;

  // kPipe: tile t's stage `src` into f16 buffer `f`, this wave's share.
  __device__ __forceinline__ void widen_into(const lds_u8 *src, lds_u8 *f) {
    widen_v(src, f + kFV);
    widen_k(src, f + kFK);
    for (int c = wave * 64 + lane; c < D / 8; c += 64 * NW)
      *reinterpret_cast<__attribute__((address_space(3))) v4i *>(f + kFS + 16 * c) =
          lds_load<v4i>(src + S::kKS + 16 * c);
  }
  // kPipe: tile t's V scales from its stage `src` into this wave's vsc (the
  // tail tile's junk scales zeroed first), with the accumulators' 2^vexp
  // step (scale_v); after tile t-1's PV, which used the previous vsc.
  __device__ __forceinline__ void prep_v(int t, const lds_u8 *src) {
    const int32_t t0 = tok0 + t * kTile;
    if (t0 + kTile > len) mask_tail_scales(src, t0);
    scale_v(src);
  }
  // kPipe, step t.  Entering it, f16 buffer fc holds tile t (written by every
  // wave in step t-1), this wave's vsc holds tile t's V scales, and tile
  // t+1's copies into stage rn were issued in step t-1.  One barrier: after
  // it tile t+1 has landed, fc is complete, and every wave is done with the
  // stage rc (widened in step t-1) and with fn (computed in step t-1).  Then
  // tile t+2's copies go into rc, tile t+1 is widened into fn while tile t
  // is computed from fc, and tile t+1's V scales are taken after tile t's PV.
  __device__ __forceinline__ void pipe_step(int t, lds_u8 *__restrict__ rc, lds_u8 *__restrict__ rn,
                                            lds_u8 *__restrict__ fc, lds_u8 *__restrict__ fn) {
    const bool more = t + 1 < n_tiles;
    if (more) __builtin_amdgcn_s_waitcnt(kWaitBase);  // this wave's copies of tile t+1
    wg_barrier_lds();
    if (t + 2 < n_tiles) issue(t + 2, rc);
    if (more) widen_into(rn, fn);
    kf16 = fc + kFK;
    vf16 = fc + kFV;
    ks = fc + kFS;
    compute(t, rc);  // reads fc and vsc only: rc is being refilled
    if (more) prep_v(t + 1, rn);
  }
  // kPipe: the tile loop over stages r0, r1 and f16 buffers f0, f1 (tile k
  // in r[k % 2] and f[k % 2]).
  __device__ __forceinline__ void run_pipe(lds_u8 *__restrict__ r0, lds_u8 *__restrict__ r1,
                                           lds_u8 *__restrict__ f0, lds_u8 *__restrict__ f1) {
    if (n_tiles == 0) return;
    issue(0, r0);
    if (n_tiles > 1) issue(1, r1);
    wait_tiles_ahead(n_tiles > 1 ? 1 : 0);
    wg_barrier();  // every wave's copies of tile 0 have landed
    widen_into(r0, f0);
    prep_v(0, r0);
    int t = 0;
    for (; t + 1 < n_tiles; t += 2) {
      pipe_step(t, r0, r1, f0, f1);
      pipe_step(t + 1, r1, r0, f1, f0);
    }
    if (t < n_tiles) pipe_step(t, r0, r1, f0, f1);
  }

  // Tiles widened once (PrefillLaunch::pre): tile t's image (kPBytes: K and
  // V f16, K scales, V scales, as the compute reads them) is copied from the
  // unit's run of images in the workspace straight into f16 buffer t % 3,
  // two tiles ahead of the compute; nothing is widened here.
  static constexpr int kPBytes = (int)prefill_tile_bytes(D);
  static constexpr int kPCopies = kPBytes / 1024;  // 1 KiB copies per tile
  static constexpr int kPVS = 130 * D;             // V scales in the image
  const uint8_t *pre_src;                          // the unit's first tile image
  __device__ __forceinline__ void issue_pre(int tile, lds_u8 *dst) {
    static_assert(kPipe, "widened tiles feed the f16 compute");
    const uint8_t *src = pre_src + (uint64_t)tile * kPBytes + 16 * lane;
    // this wave's copies k = i*NW + wave; re-read by every row block of the
    // range, so the default cache policy
#pragma unroll
    for (int i = 0; i < (kPCopies + NW - 1) / NW; ++i) {
      const int k = i * NW + swave;
      if (kPCopies % NW != 0 && k >= kPCopies) break;
      __builtin_amdgcn_global_load_lds(src + 1024 * k, dst + 1024 * k, 16, 0, 0);
    }
  }
  // Step t with widened tiles: tile t in fc (copied two steps ago), fn the
  // buffer of tile t-1, which tile t+2 refills.  One barrier: after it every
  // wave's copies of tile t have landed and every wave is done with fn.
  __device__ __forceinline__ void pre_step(int t, lds_u8 *__restrict__ fc, lds_u8 *__restrict__ fn) {
    // this wave's copies of tile t; tile t+1's (the floor of kPCopies / NW
    // of them, one more on some waves) may stay in flight
    if (t + 1 < n_tiles) {
      constexpr int n = kPCopies / NW;
      __builtin_amdgcn_s_waitcnt(kWaitBase | (n & 0xf) | ((n >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitBase);
    }
    wg_barrier_lds();
    if (t + 2 < n_tiles) issue_pre(t + 2, fn);
    // tile t's V scales into this wave's vsc, with the accumulators' 2^vexp
    // step (scale_v reads them at S::kVS of the pointer it is given); the
    // widening pass zeroed the scales past the entry's end
    scale_v(fc + kPVS - S::kVS);
    kf16 = fc + kFK;
    vf16 = fc + kFV;
    ks = fc + kFS;
    compute(t, fc);  // reads fc and vsc only
  }
  __device__ __forceinline__ void run_pre(lds_u8 *__restrict__ f0, lds_u8 *__restrict__ f1,
                                          lds_u8 *__restrict__ f2) {
    if (n_tiles == 0) return;
    issue_pre(0, f0);
    if (n_tiles > 1) issue_pre(1, f1);
    int t = 0;
    for (; t + 2 < n_tiles; t += 3) {
      pre_step(t, f0, f2);
      pre_step(t + 1, f1, f0);
      pre_step(t + 2, f2, f1);
    }
    if (t < n_tiles) pre_step(t, f0, f2);
    if (t + 1 < n_tiles) pre_step(t + 1, f1, f0);
  }

  __device__ __forceinline__ void step(int t, const lds_u8 *cur, lds_u8 *fill) {
    if constexpr (kKReg) {
      // tile t's K codes and stage copy were the last loads issued
      __builtin_amdgcn_s_waitcnt(kWaitBase);
      compute(t, cur, fill);
      return;
    }
    if (NW > 1) wg_barrier();  // every wave is done with `fill` (tile t-1) and vf16
    if (t + NS - 1 < n_tiles) issue(t + NS - 1, fill);
    const int ahead = min(n_tiles - 1 - t, NS - 1);
    wait_tiles_ahead(ahead);
    if (NW > 1) wg_barrier();  // every wave's copies of tile t have landed
    if constexpr (kF16V) {
      // the V scales are probed first, so that the widening overlaps the
      // probe's read; the scaled copy goes to this wave's vsc
      const int32_t t0 = tok0 + t * kTile;
      if (t0 + kTile > len) mask_tail_scales(cur, t0);
      VProbe vp;
      const bool over = probe_v(cur, vp);
      widen_v(cur, vf16);
      if constexpr (kF16K) widen_k(cur, kf16);
      apply_v(cur, over, vp);
      wg_barrier_lds();  // vf16 (and kF16K: kf16) hold tile t
    }
    if constexpr (kDSplit) compute_split(t, cur);
    else compute(t, cur);
  }

  // The whole tile loop.  The stages are distinct restrict pointers of this
  // one function, so the compiler can prove that reading one stage does not
  // depend on the copies still landing in the others and keeps the explicit
  // vmcnt waits above instead of draining every copy.
  __device__ __forceinline__ void run(lds_u8 *__restrict__ s0, lds_u8 *__restrict__ s1,
                                      lds_u8 *__restrict__ s2) {
    if constexpr (kKReg) {
      // Tile 0's copies and K codes normally went out in the prologue
      // (issued0).  The appended rows' source values are loaded next, with
      // the prologue's loads still landing.  Position in tile 0 (app_mode
      // 1): they are quantized and stored, and the stores complete, before
      // tile 0's copies are issued here.  Later tiles (app_mode 2): tile 0 is peeled
      // off the loop and they are stored after its wait, before its compute;
      // the vmcnt(0) of step 1 drains them before tile 2's copies, and a
      // drain in compute(0) precedes tile 1's when a row lies there.
      uint4 av[4][D / 128];
      bool alive[4] = {false, false, false, false};
      if (app_mode != 0) app_load(av, alive);
      if (app_mode == 1) {
        app_store(av, alive);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      if (n_tiles == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prologue's copies
        return;
      }
      if (!issued0) {
        issue(0, s0);
        load_k(0);
      }
      __builtin_amdgcn_s_waitcnt(kWaitBase);
      if (app_mode == 2) app_store(av, alive);
      compute(0, s0, s1, app_mode == 2 && app_first == 1);
      int t = 1;
      for (; t + 1 < n_tiles; t += 2) {
        step(t, s1, s0);
        step(t + 1, s0, s1);
      }
      if (t < n_tiles) step(t, s1, s0);
      return;
    }
    // appended rows are written by wave 0; the other waves copy their tiles
    // only after a barrier that follows the stores
    if (app_mode == 1) {
      if (wave == 0) append_rows();
      if (NW > 1) wg_barrier();
    }
    if (n_tiles > 0) issue(0, s0);
    if constexpr (NS == 3 && !kKReg) {
      if (n_tiles > 1) issue(1, s1);
    }
    if (app_mode == 2 && wave == 0) append_rows();
    if constexpr (NS == 2) {
      int t = 0;
      for (; t + 1 < n_tiles; t += 2) {
        step(t, s0, s1);
        step(t + 1, s1, s0);
      }
      if (t < n_tiles) step(t, s0, s1);
    } else {
      int t = 0;
      for (; t + 2 < n_tiles; t += 3) {
        step(t, s0, s2);
        step(t + 1, s1, s0);
        step(t + 2, s2, s1);
      }
      if (t < n_tiles) step(t, s0, s2);
      if (t + 1 < n_tiles) step(t + 1, s1, s0);
    }
  }
};

// One QK n-tile's query operands: lane (n = li, group lg) serves the row
// whose D values start at element `qbase` of q (qbase < 0: a dead row, all
// zeros), dims 64*c + 16*lg .. +15.  It is live for the even block (lg < 2)
// when li < 8 and for the odd block (lg >= 2) when li >= 8.  The row is
// split into three int8 planes, q ~ sq * (128*hi + md + lo/128) with
// sq = amax/16256: u = q/sq is rounded to the integer Q = 128*hi + md
// (|hi| <= 127, md in [-64, 63]) and its remainder u - Q (exact in f32) to
// lo/128 (|lo| <= 64).  Each element is then within sq/256 = amax*2^-22 of
// q: a bf16 q is exact when its exponent is within 13 of the row maximum's,
// and outlier channels (amax >> typical |q|) leave the other elements
// 2^7 times finer than a two-plane split would.  `qmul` returns
// sq * scale_log2 (the same on every lane of the row).
// Bytes of the three planes of one query element, u = q / sq (|u| <= 16256).
__device__ __forceinline__ void q_split(float u, uint32_t &hi8, uint32_t &md8, uint32_t &lo8) {
  const float r = fminf(fmaxf(rintf(u), -16256.0f), 16256.0f);
  const int32_t Q = (int32_t)r;
  const int32_t hi = (Q + 64) >> 7;
  const int32_t md = Q - 128 * hi;
  const int32_t lo = max(-127, min(127, (int32_t)rintf((u - r) * 128.0f)));
  hi8 = (uint32_t)(uint8_t)(int8_t)hi;
  md8 = (uint32_t)(uint8_t)(int8_t)md;
  lo8 = (uint32_t)(uint8_t)(int8_t)lo;
}

// The three-plane split of the 8-row query in two steps: load_q_raw loads
// the words, split_q_planes splits them, so that a caller can issue other
// loads in between (nothing reads the words before the split).  Lanes li
// and li ^ 8 serve the same row and dims and exactly one of them is live, so
// each loads and splits half of the 16 elements -- elements 8h .. 8h+7, h =
// li >> 3 -- and the live lane takes the other half's plane words from its
// partner over a DPP row rotation; the dead lane's words are zeros.
// Raw words: bf16 pairs in 0..3, or f32 bits in 0..7, per 64-dim step.
template <int D>
__device__ __forceinline__ void load_q_raw(const void *qp, bool bf16, int64_t qbase, int li, int lg,
                                           uint32_t (&qw)[D / 64][8]) {
  constexpr int NC = D / 64;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) qw[c][e] = 0u;
  if (qbase >= 0) {
    const int64_t base = qbase + 16 * lg + 8 * (li >> 3);
    if (bf16) {
      const uint16_t *q = static_cast<const uint16_t *>(qp) + base;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 w = *reinterpret_cast<const uint4 *>(q + 64 * c);
        qw[c][0] = w.x, qw[c][1] = w.y, qw[c][2] = w.z, qw[c][3] = w.w;
      }
    } else {
      const uint32_t *q = static_cast<const uint32_t *>(qp) + base;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e4 = 0; e4 < 2; ++e4) {
          const uint4 w = *reinterpret_cast<const uint4 *>(q + 64 * c + 4 * e4);
          qw[c][4 * e4] = w.x, qw[c][4 * e4 + 1] = w.y, qw[c][4 * e4 + 2] = w.z, qw[c][4 * e4 + 3] = w.w;
        }
    }
  }
}
// The softmax multiplier of a query row stored as q * sign(scale) / sq:
// |scale_log2| * sq, and at least FLT_MIN, so that it is positive (a zero
// row or a zero scale gives scores of about 2^-80, i.e. a uniform softmax):
// the softmax then takes the maximum of the unscaled scores and scales it
// once, and every exponent is one fma of the unscaled score.
__device__ __forceinline__ float softmax_mul(float amax, float sq, float scale_log2) {
  return fmaxf(amax > 0.0f ? sq * fabsf(scale_log2) : 0.0f, 1.17549435e-38f);
}

template <int D>
__device__ __forceinline__ void split_q_planes(const uint32_t (&qw)[D / 64][8], bool bf16, int li,
                                               int lg, float scale_log2, v4i *qhi, v4i *qmd,
                                               v4i *qlo, float &qmul) {
  constexpr int NC = D / 64;
  float qv[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (bf16) {
        qv[c][2 * e] = bf16_bits_to_f32((uint16_t)(qw[c][e] & 0xffffu));
        qv[c][2 * e + 1] = bf16_bits_to_f32((uint16_t)(qw[c][e] >> 16));
      } else {
        qv[c][2 * e] = __uint_as_float(qw[c][2 * e]);
        qv[c][2 * e + 1] = __uint_as_float(qw[c][2 * e + 1]);
      }
    }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[c][e]));
  amax = fmaxf(amax, dpp_ror8(amax));  // the partner's half of the chunks
  amax = row_group_max(amax);
  // a negative scale negates the planes (exact), so that qmul >= 0
  const float inv = amax > 0.0f ? copysignf(16256.0f / amax, scale_log2) : 0.0f;
  qmul = softmax_mul(amax, amax / 16256.0f, scale_log2);
  const bool live = (li < 8) == (lg < 2);
  const bool upper = li >= 8;  // this lane split elements 8..15
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    uint32_t w[3][2] = {{0, 0}, {0, 0}, {0, 0}};  // plane, word: own elements
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t b[3];
      q_split(qv[c][e] * inv, b[0], b[1], b[2]);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) w[pl][e >> 2] |= b[pl] << (8 * (e & 3));
    }
    v4i out[3];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t part = __builtin_bit_cast(
            uint32_t, __builtin_amdgcn_update_dpp(0, (int)w[pl][k], 0x128, 0xf, 0xf, false));  // row_ror:8
        o[k] = live ? (upper ? part : w[pl][k]) : 0u;
        o[2 + k] = live ? (upper ? w[pl][k] : part) : 0u;
      }
      out[pl] = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    }
    qhi[c] = out[0];
    qmd[c] = out[1];
    qlo[c] = out[2];
  }
}

// The query operand of the f16 QK (kF16K), one v8h per Q8 block: lane
// (li, lg) serves row li (qbase < 0: a dead row, zeros) with dims
// 32*b + 8*lg .. +7 of a bf16 query.  The row is scaled by 2^s, s chosen so
// that amax * 2^s lies in [2^14, 2^15): a bf16 value (8 significant bits)
// times a power of two is then exact in f16 down to 2^-14, i.e. for every
// element above amax * 2^-28, and the rest are within amax * 2^-39 of their
// value.  The row is negated for a negative scale, and qmul =
// |scale_log2| * 2^-s (softmax_mul) undoes the scaling in the softmax.
// kParts > 1: only blocks kPart*NB/kParts .. +NB/kParts-1 go to qf (the
// scale still follows the whole row).
template <int D, int kParts = 1, int kPart = 0>
__device__ __forceinline__ void load_q_f16(const uint16_t *qp, int64_t qbase, int lg,
                                           float scale_log2, v8h *qf, float &qmul) {
  constexpr int NB = D / 32;
  float qv[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[b][e] = 0.0f;
  if (qbase >= 0) {
    const uint16_t *q = qp + qbase + 8 * lg;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint4 w = *reinterpret_cast<const uint4 *>(q + 32 * b);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[b][2 * e] = bf16_bits_to_f32((uint16_t)(ws[e] & 0xffffu));
        qv[b][2 * e + 1] = bf16_bits_to_f32((uint16_t)(ws[e] >> 16));
      }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[b][e]));
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  int ex = 0;
  (void)frexpf(amax, &ex);  // amax = m * 2^ex, m in [0.5, 1)
  ex = max(ex, -111);       // keeps 2^(15 - ex) finite
  const float sc = amax > 0.0f ? copysignf(ldexpf(1.0f, 15 - ex), scale_log2) : 0.0f;
  qmul = softmax_mul(amax, ldexpf(1.0f, ex - 15), scale_log2);
  constexpr int kNB = NB / kParts;
#pragma unroll
  for (int b = 0; b < kNB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[b][e] = (_Float16)(qv[kPart * kNB + b][e] * sc);
}

// The query operands of the 16-row QK (Decoder::kWide): lane (li, lg) holds
// row li's dims 32*blk + 8*lg .. +7 of every block blk, as the B operand of
// v_mfma_i32_16x16x32_i8 (k = 8*lg .. 8*lg+7, column li); qbase < 0 is a
// dead row (zeros).  Same planes and `qmul` as split_q_planes.
template <int D>
__device__ __forceinline__ void load_q_wide(const void *qp, bool bf16, int64_t qbase, int lg,
                                            float scale_log2, int64_t *qhi, int64_t *qmd,
                                            int64_t *qlo, float &qmul) {
  constexpr int NB = D / 32;
  float qv[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[b][e] = 0.0f;
  if (qbase >= 0) {
    const int64_t base = qbase + 8 * lg;
    if (bf16) {
      const uint16_t *q = static_cast<const uint16_t *>(qp) + base;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint4 w = *reinterpret_cast<const uint4 *>(q + 32 * b);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qv[b][2 * e] = bf16_bits_to_f32((uint16_t)(ws[e] & 0xffffu));
          qv[b][2 * e + 1] = bf16_bits_to_f32((uint16_t)(ws[e] >> 16));
        }
      }
    } else {
      const float *q = static_cast<const float *>(qp) + base;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e4 = 0; e4 < 2; ++e4) {
          const float4 w = *reinterpret_cast<const float4 *>(q + 32 * b + 4 * e4);
          qv[b][4 * e4] = w.x;
          qv[b][4 * e4 + 1] = w.y;
          qv[b][4 * e4 + 2] = w.z;
          qv[b][4 * e4 + 3] = w.w;
        }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[b][e]));
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  const float inv = amax > 0.0f ? copysignf(16256.0f / amax, scale_log2) : 0.0f;
  qmul = softmax_mul(amax, amax / 16256.0f, scale_log2);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    uint64_t h = 0, m = 0, l = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t h8, m8, l8;
      q_split(qv[b][e] * inv, h8, m8, l8);
      h |= (uint64_t)h8 << (8 * e);
      m |= (uint64_t)m8 << (8 * e);
      l |= (uint64_t)l8 << (8 * e);
    }
    qhi[b] = (int64_t)h;
    qmd[b] = (int64_t)m;
    qlo[b] = (int64_t)l;
  }
}

// Normalized output row `orow` ([rows][D], f32 or bf16) from one PV n-tile's
// accumulators: lane (li, lg) holds dims 16*m + 4*lg .. +3 for every m.
template <int D>
__device__ __forceinline__ void store_out_row(void *out, bool bf16, int64_t orow, const v4f *oacc,
                                              float l, int lg) {
  const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int m = 0; m < D / 16; ++m) {
    const int d0 = 16 * m + 4 * lg;
    const v4f o = l > 0.0f ? oacc[m] * inv_l : v4f{0.f, 0.f, 0.f, 0.f};
    if (bf16) {
      uint16_t *dst = static_cast<uint16_t *>(out) + orow * D + d0;
      const uint32_t w0 = (uint32_t)f32_to_bf16_rtne(o[0]) | ((uint32_t)f32_to_bf16_rtne(o[1]) << 16);
      const uint32_t w1 = (uint32_t)f32_to_bf16_rtne(o[2]) | ((uint32_t)f32_to_bf16_rtne(o[3]) << 16);
      *reinterpret_cast<uint2 *>(dst) = uint2{w0, w1};
    } else {
      *reinterpret_cast<v4f *>(static_cast<float *>(out) + orow * D + d0) = o;
    }
  }
}
#endif  // __HIP_DEVICE_COMPILE__

// Length of batch entry e, 0 when its sequence id or length is out of range
// (the entry then has one partition, whose workgroup reports the fault).
__device__ __forceinline__ int32_t entry_len(const DecodeLaunch &p, int32_t sq) {
  if (sq < 0 || sq >= p.n_seqs) return 0;
  const int32_t L = p.seq_lens[sq];
  return (L < 0 || L > p.max_len) ? 0 : L;
}

// Inclusive prefix sum over the wave: DPP row shifts inside each 16-lane row,
// then the row totals by readlane (no LDS round trips).
__device__ __forceinline__ int32_t wave_iscan(int32_t v, int lane) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  const int32_t r0 = __builtin_amdgcn_readlane(v, 15);
  const int32_t r1 = __builtin_amdgcn_readlane(v, 31);
  const int32_t r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}
__device__ __forceinline__ int32_t wave_isum(int32_t v, int lane) {
  return __builtin_amdgcn_readlane(wave_iscan(v, lane), 63);
}

// The partition length of the launch and this workgroup's entry b (its
// sequence id and length), partition `part` of nb.  Every workgroup computes
// the same length and the same order (entries in batch order, partitions in
// token order), so workgroup x takes the x-th partition.  Returns false past
// the last one.
__device__ __forceinline__ bool locate(const DecodeLaunch &p, int lane, int32_t x, int32_t &pt,
                                       int32_t &b, int32_t &seq, int32_t &len, int32_t &part,
                                       int32_t &nb) {
  constexpr int kCached = 4;  // entries < 256 stay in registers
  int32_t lc[kCached], sc[kCached];
#pragma unroll
  for (int c = 0; c < kCached; ++c) {
    const int32_t e = 64 * c + lane;
    sc[c] = e < p.batch ? p.seq_ids[e] : -1;
    lc[c] = e < p.batch ? entry_len(p, sc[c]) : -1;  // -1: no entry
  }
  auto len_at = [&](int c, int32_t &sq) -> int32_t {
    if (c < kCached) {
      int32_t v = lc[0];
      sq = sc[0];
#pragma unroll
      for (int k = 1; k < kCached; ++k)
        if (c == k) {
          v = lc[k];
          sq = sc[k];
        }
      return v;
    }
    const int32_t e = 64 * c + lane;
    sq = e < p.batch ? p.seq_ids[e] : -1;
    return e < p.batch ? entry_len(p, sq) : -1;
  };
  const int n_chunks = (p.batch + 63) / 64;
  // Partitions of a length-L entry at partition length t: ceil(L / t), the
  // last one taking the rest.
  auto parts = [&](int32_t L, int32_t t) -> int32_t {
    if (L <= 0) return L < 0 ? 0 : 1;
    return (L + t - 1) / t;
  };
  pt = p.part_tokens;
  if (pt == 0) {
    int32_t sq;
    auto count = [&](int32_t t) -> int32_t {
      int32_t tot = 0;
      for (int c = 0; c < n_chunks; ++c) tot += wave_isum(parts(len_at(c, sq), t), lane);
      return tot;
    };
    // Candidate lengths are whole tiles (pt_unit = 32 tokens), so a
    // partition may start inside a page and then spans one page more than
    // its length: a length that is not a multiple of the page must keep
    // that span within the 64 page ids of a workgroup, else it rounds up to
    // 64 whole pages.  The rounding keeps the length monotone in k, so the
    // binary search below stays valid.
    const int32_t PT = p.g.page_tokens;
    auto len_of = [&](int32_t k) -> int32_t {
      const int32_t t = k * p.pt_unit;
      return (t % PT != 0 && t + PT - kTile > 64 * PT) ? 64 * PT : t;
    };
    // count(k*unit) >= (sum of ceil(L/unit)) / k, so no k below
    // ceil(that sum / target) can do: start the search there (exact in one
    // evaluation when the lengths are equal)
    int32_t units = 0;
    for (int c = 0; c < n_chunks; ++c) {
      const int32_t L = len_at(c, sq);
      units += wave_isum(L > 0 ? (L + p.pt_unit - 1) / p.pt_unit : 0, lane);
    }
    const int32_t k0 = (units + p.target_parts - 1) / p.target_parts;
    int32_t lo = max(p.pt_kmin, min(k0, p.pt_kmax)), hi = p.pt_kmax;
    if (count(len_of(lo)) > p.target_parts) {
      if (count(len_of(hi)) > p.target_parts) {
        lo = hi;
      } else {
        ++lo;
        while (lo < hi) {
          const int32_t mid = (lo + hi) >> 1;
          if (count(len_of(mid)) <= p.target_parts) hi = mid;
          else lo = mid + 1;
        }
      }
    }
    pt = len_of(lo);
  }
  int32_t base = 0;
  for (int c = 0; c < n_chunks; ++c) {
    int32_t sq;
    const int32_t L = len_at(c, sq);
    const int32_t n = parts(L, pt);
    const int32_t cum = wave_iscan(n, lane);
    const uint64_t hit = __ballot(L >= 0 && base + cum > x);
    if (hit != 0) {
      const int l = __builtin_ctzll(hit);
      b = 64 * c + l;
      nb = __builtin_amdgcn_readlane(n, l);
      seq = __builtin_amdgcn_readlane(sq, l);
      len = __builtin_amdgcn_readlane(L, l);
      part = x - (base + __builtin_amdgcn_readlane(cum, l) - nb);
      return true;
    }
    base += __builtin_amdgcn_readlane(cum, 63);
  }
  return false;
}

// NW = 1: one wave per workgroup, NT n-tiles of 8 rows (up to 16 rows).
// NW = 2: two waves, 16 rows each (NT = 2 per wave, up to 32 rows), two
// waves per SIMD.
// kQF16: a bf16 query with 16 rows per wave, whose QK runs on f16 MFMA
// (Decoder kF16K); otherwise the int8 QK with three query planes.
template <int D, int NT, bool kSmall, int NS, int NW = 1, bool kQF16 = false>
__global__ __launch_bounds__(64 * NW, NW) void decode_kernel(DecodeLaunch p) {
#if defined(__HIP_DEVICE_COMPILE__)
  // single-wave workgroups over pages of >= 32 tokens with the two-stage
  // ring take the K codes straight to registers (compute copies tile t+1
  // into the stage tile t-1 used)
  constexpr bool kKReg = NW == 1 && !kSmall && NS == 2;
  static_assert(!kQF16 || NT == 2, "the f16 QK serves 16-row waves");
  using Dec = Decoder<D, NT, kSmall, NS, NW, false, false, kKReg, kQF16>;
  using S = typename Dec::S;
  constexpr int NP = Dec::NP;
  constexpr int NC = Dec::NC;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS][S::kAlloc];
  // kDSplit: partial scores [2][64][8] f32, then rescale factors [2][64] f32
  __shared__ __attribute__((aligned(16))) uint8_t xsbuf[Dec::kDSplit ? 2 * 64 * 32 + 2 * 64 * 4 : 16];
  // NW > 1: each wave's scaled V scales of the tile (Decoder::scale_v)
  __shared__ __attribute__((aligned(16))) uint8_t vscbuf[NW > 1 ? NW * 2 * D : 16];

  Dec dc(p);
  dc.xs = (lds_u8 *)xsbuf;
  dc.lane = threadIdx.x & 63;
  dc.wave = NW > 1 ? (int)(threadIdx.x >> 6) : 0;
  // the same value read into a scalar, so that the wave's share of each
  // tile's copies (ChunkPlan) is addressed with scalar arithmetic (the
  // split verify's per-wave code paths keep the vector form: with a scalar
  // they hold more registers than the wave has)
  dc.swave = NW > 1 ? (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  const int r0 = 16 * dc.wave;  // first query row of this wave
  dc.li = dc.lane & 15;  // MFMA row/column within a 16-lane group
  dc.lg = dc.lane >> 4;  // MFMA k-group
  const int lane = dc.lane, li = dc.li, lg = dc.lg;
  const int kvh = blockIdx.y;
  dc.kvh = kvh;
  const Geo g = p.g;

  int32_t pt, b, seq, lenc, part, nb;
  if (!locate(p, lane, (int32_t)blockIdx.x, pt, b, seq, lenc, part, nb)) return;
  // the combine finds entry b's partials through the header, written before
  // any check can end this workgroup
  if (p.ws_hdr != nullptr && kvh == 0 && threadIdx.x == 0) {
    if (blockIdx.x == 0) p.ws_hdr[0] = pt;
    if (part == 0) {
      p.ws_hdr[1 + 2 * b] = (int32_t)blockIdx.x;
      p.ws_hdr[2 + 2 * b] = nb;
    }
  }

  if (seq < 0 || seq >= p.n_seqs) {
    if (lane == 0) atomicOr(p.fault, FAULT_BAD_SEQ);
    return;
  }
  // locate() maps an out-of-range length to 0; reread it to tell the two apart
  const int32_t len = lenc > 0 ? lenc : p.seq_lens[seq];
  if (len < 0 || len > p.bt_stride * g.page_tokens || len > p.max_len) {
    if (lane == 0) atomicOr(p.fault, FAULT_BAD_POSITION);
    return;
  }
  const int32_t tok0 = part * pt;
  const int32_t tok_end = part == nb - 1 ? len : min(len, tok0 + pt);  // the last takes the rest
  dc.b = b;
  dc.seq = seq;
  dc.len = len;
  dc.tok0 = tok0;
  dc.tok_end = tok_end;
  dc.n_tiles = tok_end > tok0 ? (tok_end - tok0 + kTile - 1) / kTile : 0;

  // ---- prologue loads, issued together so their latencies overlap: the
  // partition's page ids, this entry's appended-row positions and the query
  // rows (each of them needs only the entry and partition located above)
  make_plan<D, kSmall, kKReg, NW>(dc.plan, g, lane, dc.swave);
  dc.PB = page_bytes(g);
  dc.kv_base = p.pages + (uint64_t)kvh * 2u * region_bytes(g);
  // The partition's page ids, one per lane (partitions start on a page
  // boundary and span at most 64 pages); bad entries are reported and
  // replaced by page 0 so every copy stays inside the pool.
  dc.pg_first = tok0 / g.page_tokens;
  const int32_t npg = tok_end > tok0 ? (tok_end - 1) / g.page_tokens - dc.pg_first + 1 : 0;
  int32_t pid = lane < npg ? p.bt[(int64_t)seq * p.bt_stride + dc.pg_first + lane] : 0;
  // rows appended by this launch (q_len <= 4 per entry)
  const bool appending = p.app_k != nullptr;
  int32_t app_pos[4], app_seq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = appending && j < p.q_len;
    app_pos[j] = in ? p.app_pos[b * p.q_len + j] : -1;
    app_seq[j] = in ? p.app_seq_ids[b * p.q_len + j] : -1;
  }

  const int32_t q_per_kv = p.q_heads / g.kv_heads;
  const int32_t R = p.q_len * q_per_kv;

  // ---- query: int8 hi/md/lo planes as MFMA B operands ----------------------
  // Lane (li, lg) of QK n-tile nt serves row 8*nt + (li & 7) of this wave;
  // with Dec::kWide it serves row li.  qrow(row) is the row's first element
  // in q, or -1 past the last row.
  auto qrow = [&](int row) -> int64_t {
    if (row >= R) return -1;
    const int j = row / q_per_kv;
    const int h = kvh * q_per_kv + row % q_per_kv;
    return (((int64_t)b * p.q_len + j) * p.q_heads + h) * D;
  };
  float qmul[NT];
  if constexpr (Dec::kDSplit) {
    // all 32 rows (n-tiles 0 and 1) on this wave's half of the blocks; the
    // softmax scale is the own n-tile's
    const uint16_t *q16 = static_cast<const uint16_t *>(p.q);
    constexpr int HB = Dec::kHB;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      float qm;
      if (dc.wave == 0) load_q_f16<D, 2, 0>(q16, qrow(16 * nt + li), lg, p.scale_log2, &dc.qf[nt * HB], qm);
      else load_q_f16<D, 2, 1>(q16, qrow(16 * nt + li), lg, p.scale_log2, &dc.qf[nt * HB], qm);
      if (nt == dc.wave) qmul[0] = qm;
    }
  } else if constexpr (kQF16) {
    load_q_f16<D>(static_cast<const uint16_t *>(p.q), qrow(r0 + li), lg, p.scale_log2, dc.qf,
                  qmul[0]);
  } else if constexpr (Dec::kWide) {
    load_q_wide<D>(p.q, p.q_bf16 != 0, qrow(r0 + li), lg, p.scale_log2, dc.qhi[0], dc.qmd[0],
                   dc.qlo[0], qmul[0]);
  }
  // The 8-row three-plane query: its words are loaded here and split below,
  // after tile 0's copies went out (kKReg), so the split overlaps their
  // latency.
  constexpr bool kPlanes = !(Dec::kDSplit || kQF16 || Dec::kWide);
  uint32_t qw[D / 64][8];
  if constexpr (kPlanes) {
    static_assert(NT == 1, "the three-plane split with one n-tile");
    load_q_raw<D>(p.q, p.q_bf16 != 0, qrow(r0 + (li & 7)), li, lg, qw);
  }

  const bool pid_bad = pid < 0 || pid >= g.num_pages;
  if (pid_bad) {
    atomicOr(p.fault, FAULT_BAD_PAGE);
    pid = 0;
  }
  dc.pidv = pid;
  dc.pid_bad = __ballot(pid_bad);

  // ---- rows appended by this launch: checked once per batch entry; written
  // by the partition that holds their position, before its copies read them
  dc.app_mode = 0;
  if (appending) {
    if (part == 0 && kvh == 0 && lane == 0) {
      for (int j = 0; j < p.q_len; ++j) {
        if (app_seq[j] != seq) atomicOr(p.fault, FAULT_BAD_SEQ);
        else if (app_pos[j] < 0 || app_pos[j] >= len) atomicOr(p.fault, FAULT_BAD_POSITION);
      }
    }
    int32_t first = dc.n_tiles;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (app_seq[j] == seq && app_pos[j] >= tok0 && app_pos[j] < tok_end)
        first = min(first, (app_pos[j] - tok0) / kTile);
    if (first < dc.n_tiles) dc.app_mode = first < NS - 1 ? 1 : 2;
    dc.app_first = first;
#pragma unroll
    for (int j = 0; j < 4; ++j) dc.apos[j] = app_seq[j] == seq ? app_pos[j] : -1;
  }

  // kKReg: tile 0's copies and K codes go out now, ahead of the query split,
  // unless an appended row must be stored into tile 0 first (app_mode 1,
  // done in run()).  Branch-free, so that the wait for the query words
  // after it does not also drain every copy on one side of a branch: with
  // app_mode 1 the copies are a throwaway prefetch into stage 1 (run()
  // drains them, copies tile 0 after the stores, and tile 1 overwrites
  // stage 1); an empty partition reads page 0, and run() drains that too.
  if constexpr (kKReg) {
    const bool mode1 = __builtin_amdgcn_readfirstlane(dc.app_mode) == 1;
    dc.issue(0, (lds_u8 *)lds[mode1 ? 1 : 0]);
    dc.load_k(0);
    dc.issued0 = !mode1;
  }
  if constexpr (kPlanes)
    split_q_planes<D>(qw, p.q_bf16 != 0, li, lg, p.scale_log2, dc.qhi[0], dc.qmd[0], dc.qlo[0],
                      qmul[0]);

  // ---- per-lane softmax rows: PV n-tile np, column li -> row 16*np + li ---
#pragma unroll
  for (int np = 0; np < NP; ++np) {
    // kColSplit: lanes li and li + 8 both follow row li & 7
    const int row = r0 + 16 * np + (Dec::kColSplit ? (li & 7) : li);
    const int nt = Dec::kColSplit ? 0 : 2 * np + (li >> 3);
    // every lane of column li computed the scale of row 8*nt + (li & 7)
    // (kWide: of row li itself)
    float mul = 1.17549435e-38f;  // dead n-tiles: positive, as softmax_mul's
    if constexpr (Dec::kWide) {
      mul = qmul[0];
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t == nt) mul = qmul[t];
    }
    dc.rmul[np] = mul;
    dc.rlim[np] = (row < R && nt < NT) ? len - p.q_len + row / q_per_kv + 1 : 0;
    dc.mref[np] = -INFINITY;
    dc.lrun[np] = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 16; ++m) dc.oacc[np][m] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  // rows of draft j attend len - q_len + j + 1 positions; row 0 is live
  dc.rlim_min = len - p.q_len + 1;

  dc.vsc = (lds_u8 *)vscbuf + (NW > 1 ? dc.wave * 2 * D : 0);
  dc.run((lds_u8 *)lds[0], (lds_u8 *)lds[1], (lds_u8 *)lds[NS - 1]);
  dc.finish();

  if constexpr (Dec::kDSplit) {
    // o of all 32 rows over this wave's half of the dims; (m, l) of its own
    // 16 rows.  A direct output needs the other rows' l too: through the
    // partial-score slots of xs, which the last tile read before its second
    // barrier.
    float l = dc.lrun[0];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    float l_other = 0.0f;
    if (p.ws_o == nullptr) {
      __attribute__((address_space(3))) float *lx = reinterpret_cast<__attribute__((address_space(3))) float *>(dc.xs);
      lx[dc.wave * 64 + lane] = l;
      wg_barrier_lds();
      l_other = lx[(1 - dc.wave) * 64 + lane];
    }
    constexpr int HM = Dec::kHM;
    const int d_half = dc.wave * (D / 2);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int row = 16 * nt + li;
      if (row >= R) continue;
      const bool own = nt == dc.wave;
      const float lr = own ? l : l_other;
      const int j = row / q_per_kv;
      const int h = kvh * q_per_kv + row % q_per_kv;
      const int64_t orow = ((int64_t)b * p.q_len + j) * p.q_heads + h;
      if (p.ws_o == nullptr) {
        const float inv_l = lr > 0.0f ? 1.0f / lr : 0.0f;
#pragma unroll
        for (int m = 0; m < HM; ++m) {
          const int d0 = d_half + 16 * m + 4 * lg;
          const v4f o = lr > 0.0f ? dc.oacc[0][nt * HM + m] * inv_l : v4f{0.f, 0.f, 0.f, 0.f};
          if (p.out_bf16 != 0) {
            uint16_t *dst = static_cast<uint16_t *>(p.out) + orow * D + d0;
            const uint32_t w0 = (uint32_t)f32_to_bf16_rtne(o[0]) | ((uint32_t)f32_to_bf16_rtne(o[1]) << 16);
            const uint32_t w1 = (uint32_t)f32_to_bf16_rtne(o[2]) | ((uint32_t)f32_to_bf16_rtne(o[3]) << 16);
            *reinterpret_cast<uint2 *>(dst) = uint2{w0, w1};
          } else {
            *reinterpret_cast<v4f *>(static_cast<float *>(p.out) + orow * D + d0) = o;
          }
        }
      } else {
        const int64_t prow = p.ws_hdr != nullptr
                                 ? ((int64_t)kvh * p.n_wg + (int64_t)blockIdx.x) * R + row
                                 : orow * p.n_parts + part;
#pragma unroll
        for (int m = 0; m < HM; ++m)
          *reinterpret_cast<v4f *>(p.ws_o + prow * D + d_half + 16 * m + 4 * lg) = dc.oacc[0][nt * HM + m];
        if (own && lg == 0) *reinterpret_cast<float2 *>(p.ws_ml + 2 * prow) = float2{dc.mref[0], l};
      }
    }
    return;
  }

  // ---- epilogue ---------------------------------------------------------------
  if constexpr (Dec::kColSplit) {
    // column li + 8 holds the second weight term of row li
#pragma unroll
    for (int m = 0; m < D / 16; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) dc.oacc[0][m][r] += dpp_ror8(dc.oacc[0][m][r]);
  }
#pragma unroll
  for (int np = 0; np < NP; ++np) {
    float l = dc.lrun[np];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int row = r0 + 16 * np + li;
    if (row >= R || (Dec::kColSplit && li >= 8)) continue;
    const int j = row / q_per_kv;
    const int h = kvh * q_per_kv + row % q_per_kv;
    const int64_t orow = ((int64_t)b * p.q_len + j) * p.q_heads + h;
    if (p.ws_o == nullptr) {
      store_out_row<D>(p.out, p.out_bf16 != 0, orow, dc.oacc[np], l, lg);
    } else {
      const int64_t prow = p.ws_hdr != nullptr
                               ? ((int64_t)kvh * p.n_wg + (int64_t)blockIdx.x) * R + row
                               : orow * p.n_parts + part;
#pragma unroll
      for (int m = 0; m < D / 16; ++m)
        *reinterpret_cast<v4f *>(p.ws_o + prow * D + 16 * m + 4 * lg) = dc.oacc[np][m];
      if (lg == 0) *reinterpret_cast<float2 *>(p.ws_ml + 2 * prow) = float2{dc.mref[np], l};
    }
  }

#endif  // __HIP_DEVICE_COMPILE__
}

template <int D, int NT, int NS, int NW = 1>
hipError_t launch_decode_t(const DecodeLaunch &d, hipStream_t s) {
  dim3 grid((unsigned)d.n_wg, (unsigned)d.g.kv_heads);
  const bool small = d.g.page_tokens < kTile;
  if constexpr (NT == 2) {
    if (d.q_bf16 != 0) {
      if (small)
        hipLaunchKernelGGL((decode_kernel<D, NT, true, NS, NW, true>), grid, dim3(64 * NW), 0, s, d);
      else
        hipLaunchKernelGGL((decode_kernel<D, NT, false, NS, NW, true>), grid, dim3(64 * NW), 0, s, d);
      return hipGetLastError();
    }
  }
  if (small)
    hipLaunchKernelGGL((decode_kernel<D, NT, true, NS, NW>), grid, dim3(64 * NW), 0, s, d);
  else
    hipLaunchKernelGGL((decode_kernel<D, NT, false, NS, NW>), grid, dim3(64 * NW), 0, s, d);
  return hipGetLastError();
}

}  // namespace
}  // namespace rkv
