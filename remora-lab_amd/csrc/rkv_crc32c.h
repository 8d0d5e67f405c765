// rkv_crc32c.h -- CRC32C (Castagnoli, reflected polynomial 0x82f63b78, init
// and final xor 0xffffffff), the checksum of R4KV pages
// (har/crates/r4kv/src/crc32c.rs:1-31).  Tables are computed at compile
// time and shared by host code and the device kernel.
//
// The device kernel works on the "raw" CRC: the register after the table
// loop started from 0, without the final xor.  raw is linear over GF(2) in
// the message bits, leading zero bytes do not change it, and
//   raw(A || B) = shift(raw(A), |B|) ^ raw(B),
// where shift(c, k) runs the register c through k zero bytes, a linear map
// kept as a 32x32 bit matrix per power of two.  The standard CRC of a
// message of n bytes is raw(message) ^ shift(0xffffffff, n) ^ 0xffffffff.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace rkv {
namespace crc {

constexpr uint32_t kPoly = 0x82f63b78u;

struct ByteTable {
  uint32_t t[256];
};
constexpr ByteTable make_byte_table() {
  ByteTable r{};
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c & 1u) ? (kPoly ^ (c >> 1)) : (c >> 1);
    r.t[i] = c;
  }
  return r;
}
constexpr ByteTable kByte = make_byte_table();

// A linear map on the 32-bit register: col[i] is the image of bit i.
struct Mat {
  uint32_t col[32];
};
constexpr uint32_t mat_apply(const Mat &m, uint32_t c) {
  uint32_t r = 0;
  for (int i = 0; i < 32; ++i)
    if ((c >> i) & 1u) r ^= m.col[i];
  return r;
}
constexpr Mat mat_square(const Mat &a) {
  Mat r{};
  for (int i = 0; i < 32; ++i) r.col[i] = mat_apply(a, a.col[i]);
  return r;
}

// kShift.m[j]: the register through 2^j zero bytes (j < 40, so n < 2^40).
constexpr int kShiftBits = 40;
struct Shifts {
  Mat m[kShiftBits];
};
constexpr Shifts make_shifts() {
  Shifts s{};
  for (int i = 0; i < 32; ++i) {
    const uint32_t c = 1u << i;
    s.m[0].col[i] = kByte.t[c & 0xffu] ^ (c >> 8);
  }
  for (int j = 1; j < kShiftBits; ++j) s.m[j] = mat_square(s.m[j - 1]);
  return s;
}
constexpr Shifts kShift = make_shifts();

// Slicing tables for 16-byte pieces: t[j][b] = raw(b followed by j zero
// bytes), so raw(p0..p15) = xor over k of t[15-k][p_k].
struct Slice16 {
  uint32_t t[16][256];
};
constexpr Slice16 make_slice16() {
  Slice16 s{};
  for (int b = 0; b < 256; ++b) s.t[0][b] = kByte.t[b];
  for (int j = 1; j < 16; ++j)
    for (int b = 0; b < 256; ++b) {
      const uint32_t c = s.t[j - 1][b];
      s.t[j][b] = kByte.t[c & 0xffu] ^ (c >> 8);
    }
  return s;
}
constexpr Slice16 kSlice16 = make_slice16();

// The 1024-byte shift as four byte tables: shift(c, 1024) = xor over i of
// t[i][(c >> 8i) & 0xff].
struct Shift1024 {
  uint32_t t[4][256];
};
constexpr Shift1024 make_shift1024() {
  Shift1024 s{};
  for (int i = 0; i < 4; ++i)
    for (uint32_t b = 0; b < 256; ++b) s.t[i][b] = mat_apply(kShift.m[10], b << (8 * i));
  return s;
}
constexpr Shift1024 kShift1024 = make_shift1024();

// Host helpers.
inline uint32_t shift(uint32_t c, uint64_t n) {
  for (int j = 0; j < kShiftBits && n; ++j, n >>= 1)
    if (n & 1u) c = mat_apply(kShift.m[j], c);
  return c;
}
inline uint32_t update(uint32_t c, const uint8_t *p, size_t n) {
  for (size_t i = 0; i < n; ++i) c = kByte.t[(c ^ p[i]) & 0xffu] ^ (c >> 8);
  return c;
}
inline uint32_t crc32c(const uint8_t *p, size_t n) { return update(0xffffffffu, p, n) ^ 0xffffffffu; }
// What the device adds to the raw CRC of n bytes to give the CRC.
inline uint32_t finish_term(uint64_t n) { return shift(0xffffffffu, n) ^ 0xffffffffu; }

}  // namespace crc
}  // namespace rkv
