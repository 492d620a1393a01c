// Decode GEMV for the weight formats without a fused matmul kernel, up to 8 activation rows,
// bf16 activations and outputs, fp32 accumulation: affine 2, 3, 5 and 6 bits, and the
// bias-less microscaling modes nvfp4 (e2m1 codes, 16-value groups, e4m3 scales), mxfp4
// (e2m1, 32, e8m0) and mxfp8 (e4m3, 32, e8m0).
//
// A row of K codes is one LSB-first bitstream over little-endian words: 32 codes are
// exactly BITS whole dwords, at dword c*BITS of the row for chunk c (the same stream as the
// reference's 8-code packs of BITS bytes, src/transformer.zig:516-578).
// Block = 4 waves and 16 weight rows; the block stages its activation rows in LDS once.
// Each wave streams its 4 weight rows together: lane l takes chunks l, l+64, ... and loads
// the chunk's BITS dwords of all 4 rows before using any, so 4*BITS loads are in flight per
// lane. Per chunk (inside one group, gs >= 32), row and activation row:
// acc += s * sum(x*q) + b * sum(x) (affine), acc += s * sum(x*element(q)) (fp modes; an
// nvfp4 chunk holds two groups). The wave's lanes are summed with shuffles in a fixed
// order. Element decoders build the fp32 bits directly (exact for every code): e2m1
// exponent e, mantissa f -> 2^(e-1) (1 + f/2), e = 0 -> f/2; e4m3 -> 2^(e-7) (1 + f/8),
// e = 0 -> f 2^-9, no NaN code; e8m0 -> 2^(b-127), b = 0 -> 2^-127 (the reference's
// constructions, src/transformer.zig:20126-20142, :18918-18924).
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {
namespace {

constexpr int kAnyRowsPerBlock = 16;

// Gathers: block column y is pair i, lhs(i) = lhs ? lhs[i] : i / lhs_div, expert
// rhs(i) = rhs ? rhs[i] : i; an lhs >= x_batch or an expert >= n_experts gives NaN rows.
// Dense calls are the single pair (0, 0).
struct AnyGather {
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t lhs_div, x_batch, n_experts;
};

MI_DEV float el_e2m1(uint32_t c) {
  const uint32_t m = c & 7u, e = m >> 1, f = m & 1u;
  const float mag = e ? __uint_as_float(((e + 126u) << 23) | (f << 22)) : 0.5f * (float)f;
  return (c & 8u) ? -mag : mag;
}
MI_DEV float el_e4m3(uint32_t b) {
  const uint32_t m = b & 0x7Fu, e = m >> 3, f = m & 7u;
  const float mag = e ? __uint_as_float(((e + 120u) << 23) | (f << 20)) : (float)f * 0.001953125f;
  return (b & 0x80u) ? -mag : mag;
}
MI_DEV float sc_e8m0(uint32_t b) { return b ? __uint_as_float(b << 23) : __uint_as_float(0x00400000u); }

// e2m1 codes to bf16 by byte tables: for 4 codes held one per byte (magnitude bits 0-2,
// sign bit 3), v_perm_b32 picks each magnitude's bf16 high byte (00 3F 3F 3F 40 40 40 40)
// and low byte (00 00 80 C0 00 40 80 C0) at once; the sign goes to bit 7 of the high byte.
// Two more permutes interleave them into bf16 pairs (bytes 0,1) and (bytes 2,3).
typedef __bf16 bf16x2a __attribute__((ext_vector_type(2)));
MI_DEV float dot2a(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2a, a),
                                         __builtin_bit_cast(bf16x2a, b), c, false);
}
MI_DEV void e2m1_pairs(uint32_t codes4, uint32_t& p01, uint32_t& p23) {
  const uint32_t m = codes4 & 0x07070707u;
  const uint32_t hb = perm_b32(0x40404040u, 0x3F3F3F00u, m) | ((codes4 & 0x08080808u) << 4);
  const uint32_t lb = perm_b32(0xC0804000u, 0xC0800000u, m);
  p01 = perm_b32(hb, lb, 0x05010400u);
  p23 = perm_b32(hb, lb, 0x07030602u);
}

MI_DEV float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
MI_DEV float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// FPM: -1 affine (bf16 scales and biases), 0 nvfp4, 1 mxfp4, 2 mxfp8 (uint8 scales).
template <int BITS, int MR, int FPM = -1>
__global__ void __launch_bounds__(256) qmv_any_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ w,
                                                      const void* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      uint16_t* __restrict__ y, int M, int N,
                                                      int K, int gs, AnyGather A) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  u32x4_t* xs = reinterpret_cast<u32x4_t*>(smem);  // [M][K/8] units of 8 bf16
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int np = K / 8;
  {
    const int64_t i = blockIdx.y;
    const int64_t li = A.lhs ? (int64_t)A.lhs[i] : i / A.lhs_div;
    const int64_t e = A.rhs ? (int64_t)A.rhs[i] : i;
    y += i * M * N;
    if (li >= A.x_batch || e >= A.n_experts) {  // block-uniform
      for (int o = tid; o < M * kAnyRowsPerBlock; o += blockDim.x) {
        const int m = o / kAnyRowsPerBlock, n = blockIdx.x * kAnyRowsPerBlock + o % kAnyRowsPerBlock;
        if (n < N) y[(int64_t)m * N + n] = 0x7FC0u;  // bf16 NaN
      }
      return;
    }
    const int64_t G0 = (int64_t)N * (K / gs);  // scale entries per expert
    x += li * M * K;
    w += e * N * ((int64_t)K * BITS / 32);
    s = reinterpret_cast<const uint8_t*>(s) + e * G0 * (FPM < 0 ? 2 : 1);
    if (b) b += e * G0;
  }
  constexpr bool FP4 = FPM == 0 || FPM == 1;  // e2m1 codes: byte-table decode, dot2
  for (int i = tid; i < M * np; i += blockDim.x) {
    const u32x4_t X = reinterpret_cast<const u32x4_t*>(x)[i];
    if constexpr (FP4) {  // pair order (x0,x2) (x4,x6) (x1,x3) (x5,x7): even / odd nibbles
      xs[i] = u32x4_t{perm_b32(X.y, X.x, 0x05040100u), perm_b32(X.w, X.z, 0x05040100u),
                      perm_b32(X.y, X.x, 0x07060302u), perm_b32(X.w, X.z, 0x07060302u)};
    } else {
      xs[i] = X;
    }
  }
  __syncthreads();
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int nch = K / 32;                   // 32-code chunks per row
  const int64_t wpr = (int64_t)nch * BITS;  // dwords per row
  const int G = K / gs;
  const int n0 = blockIdx.x * kAnyRowsPerBlock + wave * 4;
  if (n0 >= N) return;  // wave-uniform; no block barrier follows
  int nr[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) nr[rr] = min(n0 + rr, N - 1);
  float acc[4][MR];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[rr][m] = 0.f;
  for (int c = lane; c < nch; c += 64) {
    uint32_t wd[4][BITS];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int j = 0; j < BITS; ++j) wd[rr][j] = w[nr[rr] * wpr + (int64_t)c * BITS + j];
    const int g = (32 * c) / gs;
    float sc[4], sc2[4], bi[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      if constexpr (FPM < 0) {
        sc[rr] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(s)[(int64_t)nr[rr] * G + g]);
        bi[rr] = bf16_bits_to_f32(b[(int64_t)nr[rr] * G + g]);
      } else {
        const uint8_t* s8 = reinterpret_cast<const uint8_t*>(s) + (int64_t)nr[rr] * G + g;
        sc[rr] = FPM == 0 ? el_e4m3(s8[0]) : sc_e8m0(s8[0]);
        sc2[rr] = FPM == 0 ? el_e4m3(s8[1]) : sc[rr];  // nvfp4: codes 16..31 are the next group
        bi[rr] = 0.f;
      }
    }
    float sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sx[m] = 0.f;
      if (FPM < 0 && m < M) {  // the bias term: affine only
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4_t xv = xs[m * np + 4 * c + t];
          sx[m] += ((bf_lo(xv.x) + bf_hi(xv.x)) + (bf_lo(xv.y) + bf_hi(xv.y))) +
                   ((bf_lo(xv.z) + bf_hi(xv.z)) + (bf_lo(xv.w) + bf_hi(xv.w)));
        }
      }
    }
    if constexpr (FP4) {
      // all 4 rows' decoded weights first, so each staged activation read serves 4 rows
      uint32_t a[4][4][4];  // [row][dword t][(x0,x2) (x4,x6) (x1,x3) (x5,x7)]
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t wv = wd[rr][t];
          e2m1_pairs(wv & 0x0F0F0F0Fu, a[rr][t][0], a[rr][t][1]);
          e2m1_pairs((wv >> 4) & 0x0F0F0F0Fu, a[rr][t][2], a[rr][t][3]);
        }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m < M) {
          float d[4] = {0.f, 0.f, 0.f, 0.f}, dh[4];  // dh: nvfp4's first group of the chunk
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if (FPM == 0 && t == 2) {
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                dh[rr] = d[rr];
                d[rr] = 0.f;
              }
            }
            const u32x4_t xv = xs[m * np + 4 * c + t];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              d[rr] = dot2a(a[rr][t][0], xv.x, d[rr]);
              d[rr] = dot2a(a[rr][t][1], xv.y, d[rr]);
              d[rr] = dot2a(a[rr][t][2], xv.z, d[rr]);
              d[rr] = dot2a(a[rr][t][3], xv.w, d[rr]);
            }
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            if constexpr (FPM == 0) acc[rr][m] = fmaf(sc2[rr], d[rr], fmaf(sc[rr], dh[rr], acc[rr][m]));
            else acc[rr][m] = fmaf(sc[rr], d[rr], acc[rr][m]);
          }
        }
      }
      continue;
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float q[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const int o = j * BITS, wi = o >> 5, sh = o & 31;
        uint32_t v = wd[rr][wi] >> sh;
        if (sh + BITS > 32) v |= wd[rr][wi + 1] << (32 - sh);
        if constexpr (FPM == 2) q[j] = el_e4m3(v & MASK);
        else if constexpr (FPM >= 0) q[j] = el_e2m1(v & MASK);
        else q[j] = (float)(v & MASK);
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m < M) {
          float d = 0.f, dh = 0.f;  // dh: codes 16..31 of an nvfp4 chunk
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if (FPM == 0 && t == 2) {
              dh = d;
              d = 0.f;
            }
            const u32x4_t xv = xs[m * np + 4 * c + t];
            d = fmaf(bf_lo(xv.x), q[8 * t + 0], d);
            d = fmaf(bf_hi(xv.x), q[8 * t + 1], d);
            d = fmaf(bf_lo(xv.y), q[8 * t + 2], d);
            d = fmaf(bf_hi(xv.y), q[8 * t + 3], d);
            d = fmaf(bf_lo(xv.z), q[8 * t + 4], d);
            d = fmaf(bf_hi(xv.z), q[8 * t + 5], d);
            d = fmaf(bf_lo(xv.w), q[8 * t + 6], d);
            d = fmaf(bf_hi(xv.w), q[8 * t + 7], d);
          }
          if constexpr (FPM == 0) acc[rr][m] = fmaf(sc2[rr], d, fmaf(sc[rr], dh, acc[rr][m]));
          else if constexpr (FPM > 0) acc[rr][m] = fmaf(sc[rr], d, acc[rr][m]);
          else acc[rr][m] = fmaf(sc[rr], d, fmaf(bi[rr], sx[m], acc[rr][m]));
        }
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = acc[rr][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
      if (lane == 0 && m < M && n0 + rr < N) y[(int64_t)m * N + n0 + rr] = (uint16_t)f32_to_bf16_bits(v);
    }
}

template <int BITS, int FPM = -1>
void launch_mr(const uint16_t* x, const uint32_t* w, const void* s, const uint16_t* b,
               uint16_t* y, int M, int N, int K, int gs, size_t lds, const AnyGather& A,
               unsigned n_pairs, hipStream_t st) {
  const dim3 grid((unsigned)((N + kAnyRowsPerBlock - 1) / kAnyRowsPerBlock), n_pairs), block(256);
#define MI_ANY(MRV)                                                                             \
  do {                                                                                          \
    static const bool attr = hipFuncSetAttribute(                                               \
        reinterpret_cast<const void*>(&qmv_any_kernel<BITS, MRV, FPM>),                              \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;                  \
    (void)attr; /* a failure shows as a launch error above 64 KiB */                           \
    hipLaunchKernelGGL((qmv_any_kernel<BITS, MRV, FPM>), grid, block, lds, st, x, w, s, b, y, M, N, \
                       K, gs, A);                                                               \
  } while (0)
  if (M <= 1) MI_ANY(1);
  else if (M <= 2) MI_ANY(2);
  else if (M <= 4) MI_ANY(4);
  else MI_ANY(8);
#undef MI_ANY
}

}  // namespace

hipError_t launch_qmv_any_gather(const uint16_t* x, const uint32_t* w, const void* s,
                                 const uint16_t* b, uint16_t* y, int64_t M, int64_t N, int64_t K,
                                 int gs, int bits, int fp_mode, const uint32_t* lhs,
                                 const uint32_t* rhs, int64_t n_pairs, int64_t lhs_div,
                                 int64_t x_batch, int64_t n_experts, hipStream_t st) {
  const size_t lds = (size_t)M * K * 2;
  if (M < 1 || M > 8 || K % 32 || (fp_mode < 0 && gs < 32) || lds > 160 * 1024 ||
      N >= ((int64_t)1 << 31) || (uintptr_t)x % 16 || n_pairs < 1 || n_pairs > 65535 ||
      lhs_div < 1)
    return hipErrorNotSupported;
  const AnyGather A{lhs, rhs, lhs_div, x_batch, n_experts};
  const unsigned np = (unsigned)n_pairs;
  if (fp_mode >= 0) {
    switch (fp_mode) {
      case 0: launch_mr<4, 0>(x, w, s, b, y, (int)M, (int)N, (int)K, 16, lds, A, np, st); break;
      case 1: launch_mr<4, 1>(x, w, s, b, y, (int)M, (int)N, (int)K, 32, lds, A, np, st); break;
      case 2: launch_mr<8, 2>(x, w, s, b, y, (int)M, (int)N, (int)K, 32, lds, A, np, st); break;
      default: return hipErrorNotSupported;
    }
    return hipGetLastError();
  }
  switch (bits) {
    case 2: launch_mr<2>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, A, np, st); break;
    case 3: launch_mr<3>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, A, np, st); break;
    case 5: launch_mr<5>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, A, np, st); break;
    case 6: launch_mr<6>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, A, np, st); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

hipError_t launch_qmv_any(const uint16_t* x, const uint32_t* w, const void* s,
                          const uint16_t* b, uint16_t* y, int64_t M, int64_t N, int64_t K,
                          int gs, int bits, int fp_mode, hipStream_t st) {
  return launch_qmv_any_gather(x, w, s, b, y, M, N, K, gs, bits, fp_mode, nullptr, nullptr, 1, 1,
                               1, 1, st);
}

}  // namespace mi
