// HiFloat8 (Ascend byte layout) format arithmetic, usable on host and device.
//
// Byte = sign bit 7 + 7-bit magnitude code.  Magnitude codes (codec.py:27-82):
//   0x00            zero (there is no signed zero; 0x80 is NaN)
//   0x01..0x07      2^(code-23)                      (2^-22 .. 2^-16)
//   0x08..0x3F      |e|<=3, 3 mantissa bits, base per exponent:
//                   e: 0->0x08 1->0x10 -1->0x18 2->0x20 3->0x28 -2->0x30 -3->0x38
//   0x40..0x4F      e = 4..7,   2 mantissa bits      (0x40 + (e-4)*4 + m)
//   0x50..0x5F      e = -4..-7, 2 mantissa bits      (0x50 + (-e-4)*4 + m)
//   0x60..0x6E      e = 8..15,  1 mantissa bit       (0x60 + (e-8)*2 + m)
//   0x6F            +Inf (the would-be 1.5*2^15)
//   0x70..0x7F      e = -8..-15, 1 mantissa bit      (0x70 + (-e-8)*2 + m)
// Encode rounds to nearest with ties away from zero, |x| < 2^-23 -> 0x00,
// |x| >= 1.25*2^15 -> Inf, NaN -> 0x80 (codec.py:148-180).  The static
// (saturating) encode clamps finite values to +-2^15 first, so finite overflow
// gives 0x6E|sign (calibration.py:139-158).
//
// Everything here is derived from those rules; the tables are built by
// constexpr evaluation at compile time, so there is no generated header.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define HIF8_HD __host__ __device__
#else
#define HIF8_HD
#endif

namespace hif8 {

constexpr uint8_t kZero = 0x00;
constexpr uint8_t kNan = 0x80;
constexpr uint8_t kPosInf = 0x6F;
constexpr uint8_t kMaxFinite = 0x6E;
constexpr uint16_t kBf16Nan = 0x7FC0;
constexpr uint16_t kF16Nan = 0x7E00;

// Base code of the three-mantissa-bit exponents -3..3, byte e+3 of this word
// (0x38, 0x30, 0x18, 0x08, 0x10, 0x20, 0x28): a shift instead of a table, so
// device code never indexes memory for it.
constexpr uint64_t kSmallExponentBase = 0x0028201008183038ull;

HIF8_HD constexpr int mantissa_bits(int e) {
  return (e <= 3 && e >= -3) ? 3 : ((e <= 7 && e >= -7) ? 2 : 1);
}

// 7-bit code of (1 + m / 2^mb) * 2^e for a HiF8 normal exponent -15 <= e <= 15.
HIF8_HD constexpr uint32_t normal_code(int e, uint32_t m) {
  if (e >= -3 && e <= 3) return uint32_t((kSmallExponentBase >> (8 * (e + 3))) & 0xFFu) + m;
  if (e >= 4 && e <= 7) return 0x40u + uint32_t(e - 4) * 4u + m;
  if (e <= -4 && e >= -7) return 0x50u + uint32_t(-e - 4) * 4u + m;
  if (e >= 8) return 0x60u + uint32_t(e - 8) * 2u + m;
  return 0x70u + uint32_t(-e - 8) * 2u + m;
}

// Magnitude code of a finite non-negative FP32 value given its biased exponent
// field E (0..254) and its top four mantissa bits m4.  Four bits decide every
// rounding exactly: the finest HiF8 grid has three mantissa bits, so a value
// is at or above the midpoint iff the fourth bit (or a higher one) says so.
// Returns 0x6F (Inf) for finite overflow; the static encoder saturates it.
HIF8_HD constexpr uint32_t encode_magnitude(int E, uint32_t m4) {
  const int e = E - 127;
  if (e < -23) return 0u;
  if (e == -23) return 1u;                           // [2^-23, 2^-22) rounds up to 2^-22
  if (e <= -17) return uint32_t(e + 23) + (m4 >> 3);  // grid {2^e, 2^(e+1)}
  if (e == -16) return (m4 >> 3) ? normal_code(-15, 0) : 7u;
  if (e >= 16) return kPosInf;
  const int mb = mantissa_bits(e);
  uint32_t mant = m4 >> (4 - mb);
  mant += (m4 >> (3 - mb)) & 1u;                     // ties away from zero
  int ee = e;
  if (mant >> mb) { mant = 0; ++ee; }
  if (ee > 15) return kPosInf;
  return normal_code(ee, mant);                      // e=15, m=1 is 0x6F = Inf
}

// FP32 bits of the decoded magnitude code (0x6F -> +Inf).
HIF8_HD constexpr uint32_t decode_magnitude_bits(uint32_t mag) {
  if (mag == 0) return 0u;
  if (mag == kPosInf) return 0x7F800000u;
  if (mag < 8) return uint32_t(127 - 23 + int(mag)) << 23;
  int e = 0;
  uint32_t m = 0;
  int mb = 3;
  if (mag < 0x40) {
    // Exponent of code groups 1..7 (mag >> 3): 0, 1, -1, 2, 3, -2, -3, as 4-bit
    // two's-complement fields of one word.
    const uint32_t field = (0xDE32F100u >> (4 * (mag >> 3))) & 0xFu;
    e = int(field) - (field & 8u ? 16 : 0);
    m = mag & 7u;
  } else if (mag < 0x60) {
    const int em = 4 + int((mag >> 2) & 3u);
    e = (mag & 0x10u) ? -em : em;
    m = mag & 3u;
    mb = 2;
  } else {
    const int em = 8 + int((mag >> 1) & 7u);
    e = (mag & 0x10u) ? -em : em;
    m = mag & 1u;
    mb = 1;
  }
  return (uint32_t(e + 127) << 23) | (m << (23 - mb));
}

// FP32 bits of any decoded byte; NaN is the canonical quiet 0x7FC00000.
HIF8_HD constexpr uint32_t decode_bits(uint32_t byte) {
  if (byte == kNan) return 0x7FC00000u;
  return decode_magnitude_bits(byte & 0x7Fu) | ((byte & 0x80u) << 24);
}

// Static (saturating) encode of FP32 bits: finite overflow -> 0x6E|sign,
// Inf kept, NaN (any nonzero mantissa) -> 0x80, zero magnitude drops the sign.
HIF8_HD constexpr uint32_t static_encode_bits(uint32_t u) {
  const uint32_t E = (u >> 23) & 0xFFu;
  const uint32_t sign = (u >> 24) & 0x80u;
  if (E == 0xFFu) return (u & 0x7FFFFFu) ? kNan : (kPosInf | sign);
  uint32_t mag = encode_magnitude(int(E), (u >> 19) & 0xFu);
  if (mag == kPosInf) mag = kMaxFinite;
  return mag ? (mag | sign) : 0u;
}

// FP16 bits of a decoded byte.  Every HiF8 value is exact in fp16: magnitudes
// are multiples of 2^-23 (fp16 subnormal step 2^-24) with at most four
// significant bits, and the largest finite value 1.25*2^15 is below 65504.
HIF8_HD constexpr uint16_t decode_f16_bits(uint32_t byte) {
  if (byte == kNan) return kF16Nan;
  const uint32_t f = decode_magnitude_bits(byte & 0x7Fu);
  const uint16_t sign = uint16_t((byte & 0x80u) << 8);
  if (f == 0) return 0;
  if (f == 0x7F800000u) return uint16_t(sign | 0x7C00u);
  const int e = int(f >> 23) - 127;
  const uint32_t m = f & 0x7FFFFFu;                 // at most the top 3 bits set
  if (e >= -14) return uint16_t(sign | (uint32_t(e + 15) << 10) | (m >> 13));
  // fp16 subnormal: the value (2^23 + m) * 2^(e-23) counted in units of 2^-24.
  return uint16_t(sign | ((0x800000u | m) >> (-e - 1)));
}

struct alignas(16) Tables {
  // (sign, exp8, top-4 mantissa) 13-bit index -> static-encoded byte.  For
  // exponent 0xFF the entry follows the top four mantissa bits only; callers
  // that may see a NaN with those bits clear treat NaN separately.
  uint8_t static_encode[8192];
  uint16_t decode_bf16[256];  // byte -> bf16 payload (NaN 0x7FC0)
  uint32_t decode_f32[256];   // byte -> fp32 bits (NaN 0x7FC00000)
  uint16_t decode_f16[256];   // byte -> fp16 payload (NaN 0x7E00)
};

constexpr Tables make_tables() {
  Tables t{};
  for (uint32_t i = 0; i < 8192; ++i) {
    t.static_encode[i] = uint8_t(static_encode_bits(i << 19));
  }
  for (uint32_t b = 0; b < 256; ++b) {
    const uint32_t f = decode_bits(b);
    t.decode_f32[b] = f;
    t.decode_bf16[b] = uint16_t(f >> 16);  // every finite HiF8 value is exact in bf16
    t.decode_f16[b] = decode_f16_bits(b);
  }
  return t;
}

}  // namespace hif8
