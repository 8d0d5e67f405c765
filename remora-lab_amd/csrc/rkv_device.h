// rkv_device.h -- device-side building blocks shared by the gfx950 kernels:
// the page layout in HBM, the binary16 scale encoders and the Q8_0 group
// quantizer.  Everything here is bit-exact integer/IEEE code; nothing uses
// fast-math.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rkv {

// ---------------------------------------------------------------------------
// Page layout (one layer of the pool).
//
// A page holds page_tokens token slots for every kv head, K then V:
//   page   = [kv_head][kind K|V][region]
//   region = codes (page_tokens*D bytes) then scales (page_tokens*D/32 f16)
//   K codes : [slot][dim]                     -- the reference row order
//   V codes : [slot/TT][dim][slot%TT]         -- dim-major inside 32-slot tiles,
//                                                stored as x ^ 0x80 (code_bias)
//   scales  : [slot/TT][block][sigma(slot%TT)] -- K and V alike
// with TT = min(32, page_tokens).  Inside a 32-slot tile the scales are kept
// in the order the decode kernel's lanes consume them: slot t = 16*m + 4*g + r
// (m < 2, g < 4, r < 4) sits at position sigma(t) = 8*g + 4*m + r, so one
// 16-byte read gives a lane the 8 scales of its tokens; 16-slot tiles keep
// slot order.  The bytes of one reference row
// (har/crates/har-serve/src/attention.rs:17-21: per 32-value block an LE f16
// scale then 32 int8 codes) are a fixed permutation of these; rkv_gather_q8
// applies the inverse.  Why: a 32-token tile of K codes, of V codes and of
// each scale array is a contiguous, 16-byte aligned run, so the decode
// kernel streams it with full 128-byte lines, the QK product reads K rows
// and the PV product reads V columns without byte shuffles.
// ---------------------------------------------------------------------------
struct Geo {
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;
  int32_t num_pages;
};

__host__ __device__ inline int32_t tile_tokens(int32_t page_tokens) {
  return page_tokens < 32 ? page_tokens : 32;
}
__host__ __device__ inline uint64_t region_bytes(const Geo &g) {
  return (uint64_t)g.page_tokens * (uint64_t)g.head_dim * 17u / 16u;
}
__host__ __device__ inline uint64_t page_bytes(const Geo &g) {
  return (uint64_t)g.kv_heads * 2u * region_bytes(g);
}
__host__ __device__ inline uint64_t region_base(const Geo &g, int32_t page, int32_t kvh,
                                                int32_t kind) {
  return (uint64_t)page * page_bytes(g) + (uint64_t)(kvh * 2 + kind) * region_bytes(g);
}
// V codes are stored biased, as x ^ 0x80 (x + 128 as an unsigned byte): the
// decode widens them to f16 with two byte permutes and no sign flip.  K codes
// are stored as they are (the int8 MFMA reads them).
__host__ __device__ constexpr uint8_t code_bias(int32_t kind) { return kind == 1 ? 0x80 : 0x00; }
// byte offset of code (slot, dim) inside a region of `kind`
__host__ __device__ inline uint32_t code_offset(const Geo &g, int32_t kind, int32_t slot,
                                                int32_t dim) {
  const uint32_t D = (uint32_t)g.head_dim;
  if (kind == 0) return (uint32_t)slot * D + (uint32_t)dim;
  const uint32_t TT = (uint32_t)tile_tokens(g.page_tokens);
  return ((uint32_t)slot / TT) * D * TT + (uint32_t)dim * TT + (uint32_t)slot % TT;
}
// position of tile slot t inside a 32-slot scale run
__host__ __device__ inline uint32_t scale_pos32(uint32_t t) {
  return 8u * ((t >> 2) & 3u) + 4u * (t >> 4) + (t & 3u);
}
// byte offset of the f16 scale of (slot, block) inside a region
__host__ __device__ inline uint32_t scale_offset(const Geo &g, int32_t slot, int32_t block) {
  const uint32_t D = (uint32_t)g.head_dim;
  const uint32_t TT = (uint32_t)tile_tokens(g.page_tokens);
  const uint32_t t = (uint32_t)slot % TT;
  return (uint32_t)g.page_tokens * D +
         2u * (((uint32_t)slot / TT) * (D / 32u) * TT + (uint32_t)block * TT +
               (TT == 32u ? scale_pos32(t) : t));
}

// Device-side fault word bits (read back by rkv_ctx_sync).
enum : int32_t { FAULT_BAD_PAGE = 1, FAULT_BAD_POSITION = 2, FAULT_BAD_SEQ = 4 };

// ---------------------------------------------------------------------------
// binary16 encoders.
// ---------------------------------------------------------------------------

// IEEE binary16, round to nearest even, subnormals and carries handled:
// the encoder of har/crates/r4kv/src/f16.rs:27-86.
__host__ __device__ inline uint16_t f16_rtne(float v) {
  uint32_t x = __builtin_bit_cast(uint32_t, v);
  uint32_t sign = (x >> 16) & 0x8000u;
  int32_t bexp = (int32_t)((x >> 23) & 0xffu);
  uint32_t frac = x & 0x7fffffu;
  if (bexp == 0xff) return (uint16_t)(sign | 0x7c00u | (frac ? 0x200u : 0u));
  int32_t e = bexp - 127;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  uint32_t m = frac | 0x800000u;
  if (e >= -14) {
    // keep 11 significant bits; round on the 13 dropped bits
    uint32_t r = (m >> 13) + (((m & 0x1fffu) > 0x1000u) ||
                              ((m & 0x1fffu) == 0x1000u && ((m >> 13) & 1u)));
    uint32_t h = ((uint32_t)(e + 15) << 10) + (r - 0x400u);  // carry flows into exponent
    if (h >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | h);
  }
  if (bexp == 0 && frac == 0) return (uint16_t)sign;
  uint32_t sh = (uint32_t)(-1 - e);  // >= 14
  if (sh >= 31) return (uint16_t)sign;
  uint32_t whole = m >> sh;
  uint32_t rem = m & ((1u << sh) - 1u);
  uint32_t half = 1u << (sh - 1);
  whole += (rem > half) || (rem == half && (whole & 1u));
  return (uint16_t)(sign | whole);  // whole == 0x400 is the smallest normal
}

// The f16 encoder of har/crates/har-serve/src/attention.rs:45-76, in integer
// form.  That code takes exp = floor(log2|v|) and rounds the 10-bit
// mantissa half away from zero, but keeps only `mantissa & 0x3ff`, so a
// round-up to 1024 drops the carry (value encodes as 2^exp).  For negative
// normal inputs its (v/2^exp - 1)*1024 is negative and `as u16` saturates
// to 0; negative subnormals saturate to -0.
__host__ __device__ inline uint16_t f16_harserve(float v) {
  uint32_t x = __builtin_bit_cast(uint32_t, v);
  uint32_t sign = (x >> 16) & 0x8000u;
  int32_t bexp = (int32_t)((x >> 23) & 0xffu);
  uint32_t frac = x & 0x7fffffu;
  if ((x & 0x7fffffffu) == 0) return (uint16_t)sign;
  if (bexp == 0xff) return frac ? (uint16_t)0x7e00u : (uint16_t)(sign | 0x7c00u);
  if (bexp == 0) return (uint16_t)sign;  // f32 subnormal: rounds to (+/-)0 units
  int32_t e = bexp - 127;
  if (e < -14) {
    if (sign) return 0x8000u;
    uint32_t sh = (uint32_t)(-1 - e);  // v * 2^24 = m * 2^-sh, sh >= 14
    if (sh >= 26) return 0;
    uint32_t m = frac | 0x800000u;
    return (uint16_t)((m + (1u << (sh - 1))) >> sh);
  }
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  uint32_t mant = sign ? 0u : ((frac + 0x1000u) >> 13);
  return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | (mant & 0x3ffu));
}

// binary16 bits -> f32 (exact), as r4kv/src/f16.rs:4-25 and q4k.rs:22-50.
__device__ inline float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ inline float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ inline uint16_t f32_to_bf16_rtne(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Rust `x.round() as i32` then clamp to [-127, 127] (NaN -> 0), for the
// product or quotient x of the quantizer.  round() is half away from zero:
// trunc(x + copysign(0.5 - 2^-25, x)) in f32 (round-to-nearest-even add)
// equals it for every f32 x -- checked exhaustively for |x| < 2^23, above
// which x is an integer that the add leaves unchanged -- and the clamp to
// integer bounds commutes with the truncation, so the truncating convert
// finishes it.  ±inf clamp to ±127; NaN gives 0.
// The add must not fuse with the multiply that produced x (the reference
// rounds the product first): contraction is off here and in the callers.
__device__ inline int32_t q8_round_code(float x) {
#pragma clang fp contract(off)
  const float y = x + __builtin_copysignf(0x1.fffffep-2f, x);
  if (y != y) return 0;
  return (int32_t)fminf(fmaxf(y, -127.0f), 127.0f);
}

// ---------------------------------------------------------------------------
// Q8_0 quantization of one 32-value block by 8 consecutive lanes; lane `sub`
// of the group owns values 4*sub..4*sub+3 (q8_quantize_lane), or by 4 lanes
// of 8 values (q8_quantize_values<8>).  Every lane of the wave must make the
// call (the group max is two or three xor-shuffles).
//   canonical (har/crates/r4kv/src/quant.rs:45-90): d = amax/127, inv = 1/d,
//     q = clamp(round_half_away(v*inv)), scale = f16_rtne(d);
//   har-serve (har/crates/har-serve/src/attention.rs:25-42): same d,
//     q = clamp(round_half_away(v/d)), scale = f16_harserve(d).
// amax ignores NaN (quant.rs:49-55 compares `a > amax`; attention.rs:29
// uses f32::max).  f32 division is IEEE (the build keeps it correctly
// rounded) and nothing here contracts into an FMA.
// ---------------------------------------------------------------------------
// The same rule with VPL values per lane (32/VPL consecutive lanes per
// block, VPL in {4, 8}); code i of this lane is byte i of the result.
template <int VPL>
__device__ inline uint64_t q8_quantize_values(const float *v, int32_t rule, uint16_t &scale) {
#pragma clang fp contract(off)
  static_assert(VPL == 4 || VPL == 8, "4 or 8 values per lane");
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const float x = fabsf(v[i]);
    amax = x > amax ? x : amax;
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  if (VPL == 4) amax = fmaxf(amax, __shfl_xor(amax, 4));
  const float d = amax == 0.0f ? 0.0f : amax / 127.0f;
  uint64_t codes = 0;
  if (rule == 0) {
    const float inv = d == 0.0f ? 0.0f : 1.0f / d;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      codes |= ((uint64_t)(uint8_t)(int8_t)q8_round_code(v[i] * inv)) << (8 * i);
    scale = f16_rtne(d);
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int32_t q = d == 0.0f ? 0 : q8_round_code(v[i] / d);
      codes |= ((uint64_t)(uint8_t)(int8_t)q) << (8 * i);
    }
    scale = f16_harserve(d);
  }
  return codes;
}

// The same rule for a whole 32-value block held by one lane: no shuffles,
// and the scale's divisions and f16 encoding run once per block.  codes[j]
// holds codes 4j..4j+3, code i in byte i % 4.
__device__ inline void q8_quantize_block(const float (&v)[32], int32_t rule, uint16_t &scale,
                                         uint32_t (&codes)[8]) {
#pragma clang fp contract(off)
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float x = fabsf(v[i]);
    amax = x > amax ? x : amax;
  }
  const float d = amax == 0.0f ? 0.0f : amax / 127.0f;
  int32_t q[32];
  if (rule == 0) {
    const float inv = d == 0.0f ? 0.0f : 1.0f / d;
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = q8_round_code(v[i] * inv);
    scale = f16_rtne(d);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = d == 0.0f ? 0 : q8_round_code(v[i] / d);
    scale = f16_harserve(d);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    codes[j] = ((uint32_t)(uint8_t)q[4 * j]) | ((uint32_t)(uint8_t)q[4 * j + 1] << 8) |
               ((uint32_t)(uint8_t)q[4 * j + 2] << 16) | ((uint32_t)(uint8_t)q[4 * j + 3] << 24);
}

__device__ inline uint32_t q8_quantize_lane(const float v[4], int32_t rule, uint16_t &scale) {
  return (uint32_t)q8_quantize_values<4>(v, rule, scale);
}

// Four consecutive source values (f32 or bf16) starting at element `off`.
__device__ inline void load_src4(const void *src, uint64_t off, bool bf16, float v[4]) {
  if (bf16) {
    const uint2 w = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(src) + off);
    v[0] = bf16_bits_to_f32((uint16_t)(w.x & 0xffffu));
    v[1] = bf16_bits_to_f32((uint16_t)(w.x >> 16));
    v[2] = bf16_bits_to_f32((uint16_t)(w.y & 0xffffu));
    v[3] = bf16_bits_to_f32((uint16_t)(w.y >> 16));
  } else {
    const float4 w = *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + off);
    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
  }
}

// Store lane `sub`'s 4 codes of block `blk` of token `slot` into a K or V
// region, and (lane 0 of the group) the block's scale.
__device__ inline void store_q8_lane(const Geo &g, uint8_t *region, int32_t kind, int32_t slot,
                                     int32_t blk, int32_t sub, uint32_t codes, uint16_t scale) {
  const int32_t dim0 = blk * 32 + sub * 4;
  if (kind == 0) {
    *reinterpret_cast<uint32_t *>(region + code_offset(g, 0, slot, dim0)) = codes;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      region[code_offset(g, 1, slot, dim0 + i)] = (uint8_t)(codes >> (8 * i)) ^ code_bias(1);
  }
  if (sub == 0) *reinterpret_cast<uint16_t *>(region + scale_offset(g, slot, blk)) = scale;
}

}  // namespace rkv
