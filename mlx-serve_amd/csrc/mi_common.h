// Shared device helpers for the gfx950 quantized-matmul kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define MI_DEV __device__ __forceinline__

MI_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// acc + p[r0*stride] + p[(r0+1)*stride] + ... + p[(ks-1)*stride], added in that order (the
// fixed split order that keeps K-split results deterministic). The loads of U partials go
// out before their adds, so their memory latencies overlap instead of adding up one
// partial at a time (a runtime-count loop otherwise waits on each load before the next).
template <int U, typename T>
MI_DEV T add_splits(T acc, const T* __restrict__ p, int64_t stride, int r0, int ks) {
  for (int r = r0; r < ks; r += U) {
    T t[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (r + u < ks) t[u] = p[(int64_t)(r + u) * stride];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (r + u < ks) acc += t[u];
  }
  return acc;
}

// Round-to-nearest-even fp32 -> bf16 bits; NaN stays a quiet NaN.
MI_DEV uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// Eight bf16 values held in four dwords, as an MFMA A/B operand.
// bf16 x bf16 is exact in fp32; one rounding to bf16.
MI_DEV uint16_t bf16_mul(uint16_t a, uint16_t b) {
  return (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(a) * bf16_bits_to_f32(b));
}

// Sigmoid of a bf16 value, rounded once to fp32 from a double evaluation and then to
// bf16: the correctly rounded table value for all but astronomically rare inputs.
// Fast path: the fp32 evaluation 1/(1+expf(-v)) is within 3 fp32 ulp of that fp32
// rounding (expf <= 1 ulp, the add and the correctly rounded divide 0.5 ulp each), so both
// round to the same bf16 unless a bf16 rounding midpoint (low 16 bits 0x8000) lies within
// 8 ulp of it; those values, and v <= -80 (where expf(-v) overflows while the true value
// is still a representable fp32), take the double evaluation.
MI_DEV uint16_t sigmoid_bf16(uint16_t g) {
  const float vf = bf16_bits_to_f32(g);
  const float sf = 1.f / (1.f + expf(-vf));
  const uint32_t lo = __float_as_uint(sf) & 0xFFFFu;
  if (vf > -80.f && lo - (0x8000u - 8u) > 16u) return (uint16_t)f32_to_bf16_bits(sf);
  const double v = (double)vf;
  const float s = (float)(1.0 / (1.0 + exp(-v)));
  return (uint16_t)f32_to_bf16_bits(s);
}

// SwiGLU with the bf16 rounding points of the reference (src/transformer.zig:19846-19884):
// bf16(bf16(g * sigmoid(g)) * u).
MI_DEV uint16_t swiglu_bf16(uint16_t g, uint16_t u) {
  return bf16_mul(bf16_mul(g, sigmoid_bf16(g)), u);
}

MI_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// v_perm_b32: bytes 0-3 of the 64-bit pool are `lo`, bytes 4-7 are `hi`.
MI_DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

MI_DEV f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Inclusive wave scan (sum, or max when MAX) of 32-bit ints without LDS: Hillis-Steele
// over each 16-lane row with DPP row_shr 1/2/4/8 (lanes whose source is outside the row
// keep the identity), then each row adds the totals of the rows before it, read with
// v_readlane (scalar, no LDS round trip).
template <bool MAX>
MI_DEV int wave_scan_incl_i32(int v) {
  constexpr int id = MAX ? INT32_MIN : 0;
  auto op = [](int a, int b) { return MAX ? (a > b ? a : b) : a + b; };
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x111, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x112, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x114, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x118, 0xF, 0xF, false));
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = (int)(threadIdx.x & 63) >> 4;
  const int p01 = op(r0, r1), p012 = op(p01, r2);
  const int before = row == 0 ? id : row == 1 ? r0 : row == 2 ? p01 : p012;
  return op(v, before);
}
