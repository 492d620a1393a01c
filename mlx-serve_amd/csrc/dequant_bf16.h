// Dequantize helpers shared by the MFMA GEMM kernels that feed bf16 operands from packed
// 4-bit affine weights (prefill.hip, gmm.hip).
#pragma once
#include "mi_common.h"

namespace mi {
namespace dq {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

MI_DEV uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 8 nibbles q0..q7 (k order) -> four bf16 pairs (q0,q1)..(q6,q7) of s*q + b. The masks put
// each nibble in a byte of its own; a byte 0..15 read as an e4m3 code is exactly q * 2^-9
// (codes 0..7 are the subnormals q/8 * 2^-6, 8..15 the binade 1 + (q-8)/8 times 2^-6), so
// v_cvt_scalef32_pk_f32_fp8 with the power-of-two scale 2^9 gives q itself, two per
// instruction; then fma(s, q, b), one rounding to fp32, and one to bf16 (v_cvt_pk_bf16_f32).
MI_DEV u32x4_t dequant8(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const f32x2_t l0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, false);  // q0, q2
  const f32x2_t l1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, true);   // q4, q6
  const f32x2_t h0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, false);  // q1, q3
  const f32x2_t h1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, true);   // q5, q7
  u32x4_t o;
  o.x = pack_bf16x2(fmaf(s, l0.x, b), fmaf(s, h0.x, b));
  o.y = pack_bf16x2(fmaf(s, l0.y, b), fmaf(s, h0.y, b));
  o.z = pack_bf16x2(fmaf(s, l1.x, b), fmaf(s, h1.x, b));
  o.w = pack_bf16x2(fmaf(s, l1.y, b), fmaf(s, h1.y, b));
  return o;
}

}  // namespace dq
}  // namespace mi
