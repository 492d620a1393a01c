// Decoders of 8-code runs to exact bf16 pairs, shared by the one-row and few-row decode
// kernels: the bias-less 4-bit modes nvfp4 (e2m1 codes, 16-value groups, e4m3 scales) and
// mxfp4 (e2m1 codes, 32-value groups, e8m0 scales), where a code times its group scale is
// exact in bf16 (at most 2 x 4 significant bits); mxfp8 (e4m3 codes, 32-value groups, e8m0
// scales, exact as well); and affine 2/3/5/6-bit codes as 128 + q.
#pragma once
#include "mi_common.h"

namespace mi {
namespace code_runs {

// e4m3 (nvfp4 scales) with the reference's reading of every code as finite, as fp32.
MI_DEV float fp_e4m3(uint32_t b) {
  const uint32_t m = b & 0x7Fu, e = m >> 3, f = m & 7u;
  const float mag = e ? __uint_as_float(((e + 120u) << 23) | (f << 20)) : (float)f * 0.001953125f;
  return (b & 0x80u) ? -mag : mag;
}

// 8 e2m1 codes (one per nibble, low nibble first) times one power-of-two scale -> 4 bf16
// pairs. v_cvt_scalef32_pk_bf16_fp4 reads only the exponent field of its fp32 scale, as an
// e8m0 byte (0 -> 2^-127), which is exactly mxfp4's scale: pass the byte as the exponent.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
MI_DEV u32x4_t fp4_run(uint32_t codes, float sc) {
  return u32x4_t{
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, sc, 0)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, sc, 1)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, sc, 2)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, sc, 3))};
}
// nvfp4: e4m3 scales are not powers of two. The code converts to fp32 with the scale's
// power of two, is multiplied by the scale's signed mantissa factor (exact: at most 2 x 4
// significant bits) and rounds to bf16 without loss.
MI_DEV u32x4_t fp4_run_e4m3(uint32_t codes, float sc) {
  const uint32_t sb = __float_as_uint(sc);
  const float p = __uint_as_float(sb & 0x7F800000u);
  const float m = sc == 0.f ? 0.f : __uint_as_float((sb & 0x807FFFFFu) | 0x3F800000u);
  auto pair = [&](f32x2v v) {
    const f32x2v w = {v.x * m, v.y * m};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(w, bf16x2v));
  };
  return u32x4_t{pair(__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, p, 0)),
                 pair(__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, p, 1)),
                 pair(__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, p, 2)),
                 pair(__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, p, 3))};
}

// 8 e4m3 codes (two words, low byte first) times an e8m0 scale -> 4 bf16 pairs.
// v_cvt_scalef32_pk_bf16_fp8 reads 0x7F / 0xFF as NaN; the reference reads them as +-480
// (2^8 x 1.875). A run holding one (never in weights the format's quantizer writes, but
// any byte is a valid code) keeps the conversion's other values and patches those codes
// with +-bf16(480 x scale), exact: the scale is a power of two (2^-127 for scale byte 0).
MI_DEV u32x4_t fp8_run(uint32_t w0, uint32_t w1, float sc) {
  const uint32_t m7 = 0x7F7F7F7Fu, c1 = 0x01010101u, top = 0x80808080u;
  // bit 7 of each byte: the code's low 7 bits are all ones
  const uint32_t e0 = ((w0 & m7) + c1) & top, e1 = ((w1 & m7) + c1) & top;
  u32x4_t r{
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, false)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, true)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, false)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, true))};
  if (__builtin_expect((e0 | e1) != 0u, 0)) {
    const float s = sc == 0.f ? __uint_as_float(0x00400000u) : sc;  // e8m0 byte 0: 2^-127
    const uint32_t mag = __float_as_uint(480.f * s) >> 16;           // exact in bf16
    const uint32_t mp = mag | (mag << 16);
    // dword d of word w holds codes 2d, 2d+1: v_perm's sign-extending selectors spread their
    // flags (e bits 7, 15 / 23, 31, reached as bits 15 / 31 of e << 8 and of e) over the two
    // bf16 halves, and byte selectors move the codes' sign bits to bits 15 and 31
    auto fix = [&](uint32_t res, uint32_t w, uint32_t e, int d) {
      const uint32_t m = perm_b32(e, e << 8, d ? 0x0B0B0909u : 0x0A0A0808u);
      const uint32_t sg = perm_b32(w, w, d ? 0x030C020Cu : 0x010C000Cu) & 0x80008000u;
      return (m & (sg | mp)) | (~m & res);
    };
    r.x = fix(r.x, w0, e0, 0);
    r.y = fix(r.y, w0, e0, 1);
    r.z = fix(r.z, w1, e1, 0);
    r.w = fix(r.w, w1, e1, 1);
  }
  return r;
}

// 16 two-bit codes (LSB-first in d) -> bf16 pairs (128 + q) in natural order, codes 0..7 in
// r0 and 8..15 in r1. Four masked shifts put codes k, k+4, k+8, k+12 in the bytes of one
// word; v_perm pairs code 2p with code 2p+1 between zero bytes, and the OR adds the 0x43
// high bytes (the same pairs as odd_run<2>, with fewer instructions).
MI_DEV void two_bit_runs(uint32_t d, u32x4_t& r0, u32x4_t& r1) {
  const uint32_t m = 0x03030303u, c43 = 0x43004300u;
  const uint32_t a = d & m, b = (d >> 2) & m, c = (d >> 4) & m, e = (d >> 6) & m;
  // [lo byte k, 0, hi byte k, 0]
  auto pr = [&](uint32_t hi, uint32_t lo, uint32_t k) {
    return perm_b32(hi, lo, 0x0C000C00u | k | ((4u + k) << 16)) | c43;
  };
  r0 = u32x4_t{pr(b, a, 0), pr(e, c, 0), pr(b, a, 1), pr(e, c, 1)};
  r1 = u32x4_t{pr(b, a, 2), pr(e, c, 2), pr(b, a, 3), pr(e, c, 3)};
}

// 8 codes of `OB` bits (LSB-first, starting `sh` bits into the 64-bit pair d1:d0) ->
// bf16 pairs (128 + q0, 128 + q1) .. (128 + q6, 128 + q7).
template <int OB>
MI_DEV u32x4_t odd_run(uint32_t d0, uint32_t d1, uint32_t sh) {
  const uint64_t v = ((((uint64_t)d1) << 32) | d0) >> sh;
  constexpr uint32_t mask = (1u << OB) - 1u;
  auto pr = [&](int p) {
    const uint32_t c0 = (uint32_t)(v >> (2 * p * OB)) & mask;
    const uint32_t c1 = (uint32_t)(v >> ((2 * p + 1) * OB)) & mask;
    return (c0 | (c1 << 16)) | 0x43004300u;
  };
  return u32x4_t{pr(0), pr(1), pr(2), pr(3)};
}

}  // namespace code_runs
}  // namespace mi
