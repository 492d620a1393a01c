// Shared device helpers for the gfx950 quantized-matmul kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "sigmoid_edges.h"

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

// Round-to-nearest-even fp32 -> bf16 bits; NaN stays a quiet NaN. One v_cvt_pk_bf16_f32
// (the integer form, add 0x7FFF + lsb with a NaN test, is ~5 VALU: the bf16 arithmetic of
// the slot reduce was VALU-bound on it).
MI_DEV uint32_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Eight bf16 values held in four dwords, as an MFMA A/B operand.
// bf16 x bf16 is exact in fp32; one rounding to bf16.
MI_DEV uint16_t bf16_mul(uint16_t a, uint16_t b) {
  return (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(a) * bf16_bits_to_f32(b));
}

// Sigmoid of a bf16 value v: bf16(fp32(1 / (1 + exp(-v)))), the inner expression in
// double, as the reference's table over every bf16 pattern. Fast path: e = 2^t with
// t = -v*log2(e) split Cody-Waite style into hi + lo (hi = fl(-v*L), lo the exact fma
// residual plus -v times L's own error), so e = exp2(hi) * (1 + lo*ln2) is within about
// 2 fp32 ulp (v_exp_f32 1 ulp, the correction fma 0.5 ulp); 1 + e adds 0.5 ulp and
// v_rcp_f32 1 ulp. Rounded to bf16 directly, that value is right unless a bf16 rounding
// midpoint (low 16 bits 0x8000) lies within a few ulp of it. So when it lies within 8 ulp
// of one, or v < -80 (the fp32 exponential overflows while the true value is a tiny fp32),
// the answer comes from the edge tables: kSigmoidEdgesNear holds every input whose
// correctly rounded fp32 sigmoid lies within kSigmoidEdgeUlp (48) ulp of a midpoint,
// kSigmoidEdgesTail every input below -80 with a nonzero result. An input in the window but not listed is > 48 ulp from a midpoint, so the
// fast value rounds right; one below -80 not listed has the result +0. The result depends
// on the bf16 input alone, so a pass over all 65536 inputs checks every case.
MI_DEV uint16_t sigmoid_bf16(uint16_t g) {
  const float vf = bf16_bits_to_f32(g);
  constexpr float kL = 1.44269502162933349609375f;  // fl(log2 e)
  constexpr float kLerr = 1.925963033500011e-08f;    // log2 e - kL
  constexpr float kLn2 = 0.693147182464599609375f;
  // |v| > 100 saturates (1 above; below -80 the table decides), and keeps hi finite
  const float nv = __builtin_fminf(__builtin_fmaxf(-vf, -100.f), 100.f);
  const float hi = nv * kL;
  const float lo = __builtin_fmaf(nv, kL, -hi) + nv * kLerr;
  const float e0 = __builtin_amdgcn_exp2f(hi);
  const float e = __builtin_fmaf(e0, lo * kLn2, e0);
  const float sf = __builtin_amdgcn_rcpf(1.f + e);
  const uint32_t lo16 = __float_as_uint(sf) & 0xFFFFu;
  if (vf >= -80.f && lo16 - (0x8000u - 8u) > 16u) return (uint16_t)f32_to_bf16_bits(sf);
  if (vf != vf) return (uint16_t)f32_to_bf16_bits(vf);  // NaN in, quiet NaN out
  // scans of the short tables: immediates and selects, no loads. Each entry is materialized
  // where it is used (an opaque copy): left as constants, the compiler hoists them out of
  // the caller's loops into ~36 registers held for the whole kernel.
  uint32_t r = vf < -80.f ? 0u : f32_to_bf16_bits(sf);
  if (vf < -80.f) {
#pragma unroll
    for (int i = 0; i < kSigmoidEdgeTailCount; ++i) {
      uint32_t e = kSigmoidEdgesTail[i];
      asm volatile("" : "+v"(e));
      r = (e >> 16) == (uint32_t)g ? (e & 0xFFFFu) : r;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSigmoidEdgeNearCount; ++i) {
      uint32_t e = kSigmoidEdgesNear[i];
      asm volatile("" : "+v"(e));
      r = (e >> 16) == (uint32_t)g ? (e & 0xFFFFu) : r;
    }
  }
  return (uint16_t)r;
}

// Block barrier ordering LDS only: waits for this wave's LDS operations, not for its global
// stores (__syncthreads' fence waits for those too). For the one-block glue kernels, whose
// global stores no other thread of the block reads.
MI_DEV void lds_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt untouched
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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
