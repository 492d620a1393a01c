// Decode GEMV for the affine widths without a fused matmul kernel (2, 3, 5, 6 bits), up to
// 8 activation rows, bf16 activations and outputs, fp32 accumulation.
//
// A row of K codes is one LSB-first bitstream over little-endian words: 32 codes are
// exactly BITS whole dwords, at dword c*BITS of the row for chunk c (the same stream as the
// reference's 8-code packs of BITS bytes, src/transformer.zig:516-578).
// Block = 4 waves and 16 weight rows; the block stages its activation rows in LDS once.
// Each wave streams its 4 weight rows together: lane l takes chunks l, l+64, ... and loads
// the chunk's BITS dwords of all 4 rows before using any, so 4*BITS loads are in flight per
// lane. Per chunk (inside one group, gs >= 32), row and activation row:
// acc += s * sum(x*q) + b * sum(x). The wave's lanes are summed with shuffles in a fixed
// order.
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {
namespace {

constexpr int kAnyRowsPerBlock = 16;

MI_DEV float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
MI_DEV float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

template <int BITS, int MR>
__global__ void __launch_bounds__(256) qmv_any_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      uint16_t* __restrict__ y, int M, int N,
                                                      int K, int gs) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  u32x4_t* xs = reinterpret_cast<u32x4_t*>(smem);  // [M][K/8] units of 8 bf16
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int np = K / 8;
  for (int i = tid; i < M * np; i += blockDim.x) xs[i] = reinterpret_cast<const u32x4_t*>(x)[i];
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
    float sc[4], bi[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      sc[rr] = bf16_bits_to_f32(s[(int64_t)nr[rr] * G + g]);
      bi[rr] = bf16_bits_to_f32(b[(int64_t)nr[rr] * G + g]);
    }
    float sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sx[m] = 0.f;
      if (m < M) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4_t xv = xs[m * np + 4 * c + t];
          sx[m] += ((bf_lo(xv.x) + bf_hi(xv.x)) + (bf_lo(xv.y) + bf_hi(xv.y))) +
                   ((bf_lo(xv.z) + bf_hi(xv.z)) + (bf_lo(xv.w) + bf_hi(xv.w)));
        }
      }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float q[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const int o = j * BITS, wi = o >> 5, sh = o & 31;
        uint32_t v = wd[rr][wi] >> sh;
        if (sh + BITS > 32) v |= wd[rr][wi + 1] << (32 - sh);
        q[j] = (float)(v & MASK);
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m < M) {
          float d = 0.f;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
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
          acc[rr][m] = fmaf(sc[rr], d, fmaf(bi[rr], sx[m], acc[rr][m]));
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

template <int BITS>
void launch_mr(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
               uint16_t* y, int M, int N, int K, int gs, size_t lds, hipStream_t st) {
  const dim3 grid((unsigned)((N + kAnyRowsPerBlock - 1) / kAnyRowsPerBlock)), block(256);
#define MI_ANY(MRV)                                                                             \
  do {                                                                                          \
    static const bool attr = hipFuncSetAttribute(                                               \
        reinterpret_cast<const void*>(&qmv_any_kernel<BITS, MRV>),                              \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;                  \
    (void)attr; /* a failure shows as a launch error above 64 KiB */                           \
    hipLaunchKernelGGL((qmv_any_kernel<BITS, MRV>), grid, block, lds, st, x, w, s, b, y, M, N, \
                       K, gs);                                                                  \
  } while (0)
  if (M <= 1) MI_ANY(1);
  else if (M <= 2) MI_ANY(2);
  else if (M <= 4) MI_ANY(4);
  else MI_ANY(8);
#undef MI_ANY
}

}  // namespace

hipError_t launch_qmv_any(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, uint16_t* y, int64_t M, int64_t N, int64_t K,
                          int gs, int bits, hipStream_t st) {
  const size_t lds = (size_t)M * K * 2;
  if (M < 1 || M > 8 || K % 32 || gs < 32 || lds > 160 * 1024 || N >= ((int64_t)1 << 31) ||
      (uintptr_t)x % 16)
    return hipErrorNotSupported;
  switch (bits) {
    case 2: launch_mr<2>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, st); break;
    case 3: launch_mr<3>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, st); break;
    case 5: launch_mr<5>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, st); break;
    case 6: launch_mr<6>(x, w, s, b, y, (int)M, (int)N, (int)K, gs, lds, st); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace mi
