// Affine quantize / dequantize kernels, the sorted-gather work-list builder and the
// synthetic input generator.
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {

namespace {

// ---------------------------------------------------------------- dequantize --
// One thread per packed word: w = scale*q + bias (scale*q is exact in fp32).
// rounding 0: bf16(s*q + b); 1: bf16(bf16(s*q) + b) (a bf16 multiply then a bf16 add).
template <int BITS>
__global__ void dequant_kernel(void* __restrict__ out, const uint32_t* __restrict__ w,
                               const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                               int64_t n_words, int64_t K, int gs, int out_f32, int rounding) {
  constexpr int PF = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t wpr = K / PF;
  const int64_t G = K / gs;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / wpr;
    const int64_t k0 = (i - row * wpr) * PF;
    const int64_t gi = row * G + k0 / gs;
    const float sc = bf16_bits_to_f32(s[gi]);
    const float bi = bf16_bits_to_f32(b[gi]);
    const uint32_t word = w[i];
    float v[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const float sq = sc * (float)((word >> (j * BITS)) & MASK);
      v[j] = rounding ? bf16_bits_to_f32(f32_to_bf16_bits(sq)) + bi : sq + bi;
    }
    const int64_t o = row * K + k0;
    if (out_f32) {
      float* op = (float*)out + o;
#pragma unroll
      for (int j = 0; j < PF; j += 4) *(float4*)(op + j) = float4{v[j], v[j + 1], v[j + 2], v[j + 3]};
    } else {
      uint32_t* op = (uint32_t*)((uint16_t*)out + o);
#pragma unroll
      for (int j = 0; j < PF; j += 2)
        op[j / 2] = f32_to_bf16_bits(v[j]) | (f32_to_bf16_bits(v[j + 1]) << 16);
    }
  }
}

// Any affine width (2, 3, 5, 6 bits; 4 and 8 take the kernels around this one). A row of
// K codes is one LSB-first bitstream over its little-endian bytes; a pack of 8 codes is
// exactly `bits` bytes at byte 8*p*bits/8 of the row (the reference's unit of 8 values,
// src/transformer.zig:516-578). One thread per pack; gs >= 32, so a pack lies in one group.
__global__ void dequant_any_kernel(void* __restrict__ out, const uint32_t* __restrict__ w,
                                   const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                                   int64_t n_packs, int64_t K, int gs, int bits, int out_f32,
                                   int rounding) {
  const int64_t ppr = K / 8;                 // packs per row
  const int64_t row_bytes = K * bits / 8;    // a whole number of words
  const int64_t G = K / gs;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_packs;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / ppr, p = i - row * ppr;
    const uint8_t* pb = reinterpret_cast<const uint8_t*>(w) + row * row_bytes + p * bits;
    uint64_t r = 0;
    for (int j = 0; j < bits; ++j) r |= (uint64_t)pb[j] << (8 * j);
    const int64_t k0 = 8 * p;
    const int64_t gi = row * G + k0 / gs;
    const float sc = bf16_bits_to_f32(s[gi]);
    const float bi = bf16_bits_to_f32(b[gi]);
    const int64_t o = row * K + k0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sq = sc * (float)((uint32_t)(r >> (j * bits)) & mask);
      const float v = rounding ? bf16_bits_to_f32(f32_to_bf16_bits(sq)) + bi : sq + bi;
      if (out_f32) ((float*)out)[o + j] = v;
      else ((uint16_t*)out)[o + j] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

// Bias-less microscaling modes: w = element(q) * scale(s), exact in fp32 and in bf16.
// mode 0 nvfp4 (e2m1 codes, gs 16, e4m3 scales), 1 mxfp4 (e2m1, gs 32, e8m0), 2 mxfp8
// (e4m3 codes, gs 32, e8m0). Element decoders as the reference builds them from bits
// (src/transformer.zig:20126-20142 e2m1/e4m3 without a NaN code, :18918-18924 e8m0 with
// byte 0 = 2^-127), written as the values they produce. One thread per packed word.
MI_DEV float fp_e2m1(uint32_t c) {
  const uint32_t m = c & 7u, e = m >> 1, f = m & 1u;
  const float mag = e == 0 ? 0.5f * (float)f : __builtin_ldexpf(1.0f + 0.5f * (float)f, (int)e - 1);
  return (c & 8u) ? -mag : mag;
}
MI_DEV float fp_e4m3(uint32_t b) {
  const uint32_t m = b & 0x7Fu, e = m >> 3, f = m & 7u;
  const float mag =
      e == 0 ? __builtin_ldexpf((float)f, -9) : __builtin_ldexpf(1.0f + 0.125f * (float)f, (int)e - 7);
  return (b & 0x80u) ? -mag : mag;
}
MI_DEV float fp_e8m0(uint32_t b) { return __builtin_ldexpf(1.0f, b == 0 ? -127 : (int)b - 127); }

// gscale (nullable, nvfp4's optional fp32 global scale): element * scale is exact in fp32,
// the global scale multiplies that product with one rounding.
__global__ void dequant_fp_kernel(void* __restrict__ out, const uint32_t* __restrict__ w,
                                  const uint8_t* __restrict__ s, int64_t n_words, int64_t K,
                                  int mode, int out_f32, const float* __restrict__ gscale) {
  const int bits = mode == 2 ? 8 : 4, gs = mode == 0 ? 16 : 32, pf = 32 / bits;
  const float gsc = gscale ? *gscale : 1.f;
  const int64_t wpr = K / pf, G = K / gs;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / wpr, k0 = (i - row * wpr) * pf;
    const uint32_t word = w[i];
    for (int j = 0; j < pf; ++j) {
      const int64_t k = k0 + j;
      const uint32_t q = (word >> (j * bits)) & ((1u << bits) - 1u);
      const uint32_t sb = s[row * G + k / gs];
      float v = (mode == 2 ? fp_e4m3(q) : fp_e2m1(q)) * (mode == 0 ? fp_e4m3(sb) : fp_e8m0(sb));
      if (gscale) v *= gsc;
      if (out_f32) ((float*)out)[row * K + k] = v;
      else ((uint16_t*)out)[row * K + k] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

// 4-bit to bf16 with one rounding, gs in {32, 64, 128}. A block expands 1024 consecutive
// packed words: per step a wave reads 64 consecutive words (256 B) and writes their 512
// values as 1 KiB of consecutive bf16, so loads and stores are both contiguous per
// instruction. Word i of the flattened [rows, K/8] array belongs to group i >> log2(gs/8)
// of the flattened [rows, K/gs] scales (gs divides K), so no index division is needed.
// v_cvt_pk_bf16_f32 rounds to nearest even.
typedef __bf16 bf16x2q __attribute__((ext_vector_type(2)));
typedef float f32x2q __attribute__((ext_vector_type(2)));
MI_DEV uint32_t pk_bf16(float lo, float hi) {
  f32x2q v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2q));
}
template <int k>
MI_DEV float ubyte_f(uint32_t w) { return (float)((w >> (8 * k)) & 0xFFu); }

__global__ void __launch_bounds__(256) dequant4_bf16_kernel(u32x4_t* __restrict__ out,
                                                           const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b,
                                                           int64_t n_words, int wshift) {
  for (int64_t base = blockIdx.x * (int64_t)1024; base < n_words;
       base += (int64_t)gridDim.x * 1024) {
    uint32_t wd[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + j * 256 + threadIdx.x;
      wd[j] = i < n_words ? w[i] : 0u;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + j * 256 + threadIdx.x;
      if (i >= n_words) break;
      const int64_t gi = i >> wshift;
      const float sc = bf16_bits_to_f32(s[gi]), bi = bf16_bits_to_f32(b[gi]);
      const uint32_t lo = wd[j] & 0x0F0F0F0Fu, hi = (wd[j] >> 4) & 0x0F0F0F0Fu;
      u32x4_t o;
      o.x = pk_bf16(fmaf(sc, ubyte_f<0>(lo), bi), fmaf(sc, ubyte_f<0>(hi), bi));
      o.y = pk_bf16(fmaf(sc, ubyte_f<1>(lo), bi), fmaf(sc, ubyte_f<1>(hi), bi));
      o.z = pk_bf16(fmaf(sc, ubyte_f<2>(lo), bi), fmaf(sc, ubyte_f<2>(hi), bi));
      o.w = pk_bf16(fmaf(sc, ubyte_f<3>(lo), bi), fmaf(sc, ubyte_f<3>(hi), bi));
      out[i] = o;
    }
  }
}

// ------------------------------------------------------------------ quantize --
// One thread per group. Same fp32 steps as the MLX affine group quantizer:
// scale = max((max-min)/(2^bits-1), 1e-7) signed toward the larger-magnitude edge,
// q0 = rint(edge/scale); if q0 != 0: scale = edge/q0, bias = edge; else bias = 0.
// Codes clamp(rint((w-bias)/scale), 0, 2^bits-1) with the fp32 scale.
__global__ void quant_kernel(uint32_t* __restrict__ wq, uint16_t* __restrict__ so,
                             uint16_t* __restrict__ bo, const void* __restrict__ w, int w_f32,
                             int64_t n_groups, int gs, int bits) {
  const float n_bins = (float)((1 << bits) - 1);
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < n_groups;
       gi += (int64_t)gridDim.x * blockDim.x) {
    const int64_t base = gi * gs;
    auto ld = [&](int j) -> float {
      return w_f32 ? ((const float*)w)[base + j]
                   : bf16_bits_to_f32(((const uint16_t*)w)[base + j]);
    };
    float wmax = -INFINITY, wmin = INFINITY;
    for (int j = 0; j < gs; ++j) {
      const float v = ld(j);
      wmax = fmaxf(wmax, v);
      wmin = fminf(wmin, v);
    }
    const bool mask = fabsf(wmin) > fabsf(wmax);
    float scale = fmaxf(__fdiv_rn(wmax - wmin, n_bins), 1e-7f);
    scale = mask ? scale : -scale;
    const float edge = mask ? wmin : wmax;
    const float q0 = rintf(__fdiv_rn(edge, scale));
    float bias = 0.f;
    if (q0 != 0.f) {
      scale = __fdiv_rn(edge, q0);
      bias = edge;
    }
    // the group's codes as one LSB-first bitstream of gs*bits/32 whole words (any width)
    uint32_t* out = wq + gi * (gs * bits / 32);
    uint64_t acc = 0;
    int nb = 0, wo = 0;
    for (int j = 0; j < gs; ++j) {
      float qv = rintf(__fdiv_rn(__fsub_rn(ld(j), bias), scale));
      qv = fminf(fmaxf(qv, 0.f), n_bins);
      acc |= (uint64_t)(uint32_t)qv << nb;
      nb += bits;
      if (nb >= 32) {
        out[wo++] = (uint32_t)acc;
        acc >>= 32;
        nb -= 32;
      }
    }
    so[gi] = (uint16_t)f32_to_bf16_bits(scale);
    bo[gi] = (uint16_t)f32_to_bf16_bits(bias);
  }
}

// ----------------------------------------------------------------- generator --
__device__ uint64_t splitmix64(uint64_t seed, uint64_t counter) {
  uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void randn_kernel(void* out, int64_t n, uint64_t seed, float mean, float stddev,
                             int out_f32) {
  const int64_t pairs = (n + 1) / 2;
  for (int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < pairs;
       j += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t a = splitmix64(seed, 2 * j), b = splitmix64(seed, 2 * j + 1);
    const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    double sn, cs;
    sincos(6.283185307179586476925286766559 * u2, &sn, &cs);
    const float z0 = (float)(mean + stddev * (r * cs));
    const float z1 = (float)(mean + stddev * (r * sn));
    if (out_f32) {
      ((float*)out)[2 * j] = z0;
      if (2 * j + 1 < n) ((float*)out)[2 * j + 1] = z1;
    } else {
      ((uint16_t*)out)[2 * j] = (uint16_t)f32_to_bf16_bits(z0);
      if (2 * j + 1 < n) ((uint16_t*)out)[2 * j + 1] = (uint16_t)f32_to_bf16_bits(z1);
    }
  }
}

// ------------------------------------------------------------ sorted items --
// One 1024-thread block. For every run of equal rhs values (pairs [a, b)), the
// flattened positions [a*M, b*M) are cut into chunks of R rows; each chunk start
// becomes an item (expert, pos0, limit, 0) with limit = min(R, total - pos0). The
// consumer keeps a row only while its pair's rhs equals the item's expert, so the
// run end is never needed here. Pair j owns the chunk starts that fall in its own
// positions: ceil((o+1)M/R) - ceil(oM/R) with o = j - a.
constexpr int kBT = 1024;

// Inclusive block scan of 32-bit ints: DPP scans inside each wave, the 16 wave totals
// scanned by the first wave the same way.
template <bool MAX>
__device__ int block_scan_incl(int v, int* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = kBT / 64;
  constexpr int id = MAX ? INT32_MIN : 0;
  v = wave_scan_incl_i32<MAX>(v);
  if (lane == 63) sh[wave] = v;
  lds_sync();
  if (wave == 0) {
    const int t = lane < NW ? sh[lane] : id;
    const int w = wave_scan_incl_i32<MAX>(t);
    if (lane < NW) sh[NW + lane] = w;  // inclusive totals through wave `lane`
  }
  lds_sync();
  if (wave > 0) {
    const int p = sh[NW + wave - 1];
    v = MAX ? (p > v ? p : v) : v + p;
  }
  lds_sync();
  return v;
}

constexpr int kBPT = 4;  // pairs per thread per pass

__global__ void __launch_bounds__(kBT) build_items_kernel(const uint32_t* __restrict__ rhs,
                                                          int64_t n_pairs, int M, int R,
                                                          uint32_t* __restrict__ items,
                                                          uint32_t* __restrict__ count,
                                                          int64_t max_items) {
  __shared__ int sh[2 * (kBT / 64)];
  __shared__ int prev_a[kBT];
  __shared__ int carry_a, carry_n;
  if (threadIdx.x == 0) { carry_a = 0; carry_n = 0; }
  lds_sync();
  const int64_t total = n_pairs * M;
  const int rs = __builtin_ctz((unsigned)R);  // rows per item: a power of two
  // Each pass covers kBT * kBPT pairs; thread t owns pairs j0 .. j0 + kBPT - 1.
  for (int64_t base = 0; base < n_pairs; base += (int64_t)kBT * kBPT) {
    const int64_t j0 = base + (int64_t)threadIdx.x * kBPT;
    uint32_t cur[kBPT];
#pragma unroll
    for (int q = 0; q < kBPT; ++q) cur[q] = j0 + q < n_pairs ? rhs[j0 + q] : 0u;
    const uint32_t prv0 = j0 > 0 && j0 < n_pairs ? rhs[j0 - 1] : 0u;
    // run start of each owned pair, as far as this thread can see (-1: an earlier thread's)
    int amine[kBPT];
    int la = -1;
#pragma unroll
    for (int q = 0; q < kBPT; ++q) {
      const int64_t j = j0 + q;
      const bool start = j < n_pairs && (j == 0 || cur[q] != (q ? cur[q - 1] : prv0));
      if (start) la = (int)j;
      amine[q] = la;
    }
    const int incl_a = block_scan_incl<true>(la, sh);
    prev_a[threadIdx.x] = incl_a;
    lds_sync();
    int excl_a = threadIdx.x ? prev_a[threadIdx.x - 1] : -1;
    const int ca = carry_a;
    if (excl_a < ca) excl_a = ca;
    int a[kBPT], c[kBPT];
    int csum = 0;
#pragma unroll
    for (int q = 0; q < kBPT; ++q) {
      const int64_t j = j0 + q;
      a[q] = amine[q] >= 0 ? amine[q] : excl_a;
      c[q] = 0;
      if (j < n_pairs) {
        const int64_t o = j - a[q];
        c[q] = (int)((((o + 1) * M + R - 1) >> rs) - ((o * M + R - 1) >> rs));
      }
      csum += c[q];
    }
    const int incl = block_scan_incl<false>(csum, sh);
    int64_t off = (int64_t)carry_n + incl - csum;
#pragma unroll
    for (int q = 0; q < kBPT; ++q) {
      const int64_t o = j0 + q - a[q];
      const int64_t first = (o * M + R - 1) >> rs;
      for (int t = 0; t < c[q]; ++t) {
        const int64_t idx = off + t;
        if (idx < max_items) {
          const int64_t pos0 = (int64_t)a[q] * M + (first + t) * R;
          const int64_t lim = total - pos0 < R ? total - pos0 : R;
          items[4 * idx + 0] = cur[q];
          items[4 * idx + 1] = (uint32_t)pos0;
          items[4 * idx + 2] = (uint32_t)lim;
          items[4 * idx + 3] = 0u;
        }
      }
      off += c[q];
    }
    lds_sync();
    if (threadIdx.x == kBT - 1) {
      carry_a = incl_a > ca ? incl_a : ca;
      carry_n = (int)off;
    }
    lds_sync();
  }
  if (threadIdx.x == 0) {
    const int64_t n = carry_n < max_items ? carry_n : max_items;
    *count = (uint32_t)n;
  }
}

inline unsigned grid_for(int64_t n, int bs) {
  int64_t g = (n + bs - 1) / bs;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (unsigned)g;
}

}  // namespace

hipError_t launch_dequantize(void* out, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                             int64_t rows, int64_t K, int gs, int bits, int out_f32, int rounding,
                             hipStream_t st) {
  const int64_t n_words = rows * (K * bits / 32);
  if (n_words == 0) return hipSuccess;
  if (out_f32) rounding = 0;  // the fp32 result is exact; rounding applies to bf16 only
  const int bs = 256;
  if (bits == 4 && !out_f32 && rounding == 0 && (gs == 32 || gs == 64 || gs == 128) &&
      (uintptr_t)out % 16 == 0) {
    const int wshift = gs == 32 ? 2 : gs == 64 ? 3 : 4;  // log2(gs / 8)
    int64_t g = (n_words + 1023) / 1024;
    if (g > (int64_t)1 << 20) g = (int64_t)1 << 20;
    hipLaunchKernelGGL(dequant4_bf16_kernel, dim3((unsigned)g), dim3(bs), 0, st, (u32x4_t*)out,
                       w, s, b, n_words, wshift);
    return hipGetLastError();
  }
  if (bits != 4 && bits != 8) {
    const int64_t n_packs = rows * (K / 8);
    hipLaunchKernelGGL(dequant_any_kernel, dim3(grid_for(n_packs, bs)), dim3(bs), 0, st, out, w, s,
                       b, n_packs, K, gs, bits, out_f32, rounding);
    return hipGetLastError();
  }
  if (bits == 4)
    hipLaunchKernelGGL(dequant_kernel<4>, dim3(grid_for(n_words, bs)), dim3(bs), 0, st, out, w, s,
                       b, n_words, K, gs, out_f32, rounding);
  else
    hipLaunchKernelGGL(dequant_kernel<8>, dim3(grid_for(n_words, bs)), dim3(bs), 0, st, out, w, s,
                       b, n_words, K, gs, out_f32, rounding);
  return hipGetLastError();
}

hipError_t launch_dequantize_fp(void* out, const uint32_t* w, const uint8_t* s, int64_t rows,
                                int64_t K, int mode, int out_f32, const float* gscale,
                                hipStream_t st) {
  const int64_t n_words = rows * (K * (mode == 2 ? 8 : 4) / 32);
  if (n_words == 0) return hipSuccess;
  hipLaunchKernelGGL(dequant_fp_kernel, dim3(grid_for(n_words, 256)), dim3(256), 0, st, out, w, s,
                     n_words, K, mode, out_f32, gscale);
  return hipGetLastError();
}

hipError_t launch_quantize(uint32_t* wq, uint16_t* s, uint16_t* b, const void* w, int w_f32,
                           int64_t rows, int64_t K, int gs, int bits, hipStream_t st) {
  const int64_t ng = rows * (K / gs);
  if (ng == 0) return hipSuccess;
  const int bs = 256;
  hipLaunchKernelGGL(quant_kernel, dim3(grid_for(ng, bs)), dim3(bs), 0, st, wq, s, b, w, w_f32, ng,
                     gs, bits);
  return hipGetLastError();
}

hipError_t launch_randn(void* out, int64_t n, uint64_t seed, float mean, float stddev,
                        int out_f32, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int bs = 256;
  hipLaunchKernelGGL(randn_kernel, dim3(grid_for((n + 1) / 2, bs)), dim3(bs), 0, st, out, n, seed,
                     mean, stddev, out_f32);
  return hipGetLastError();
}

hipError_t launch_build_items(const uint32_t* rhs, int64_t n_pairs, int M, int rows_per_item,
                              uint32_t* items, uint32_t* item_count, int64_t max_items,
                              hipStream_t s) {
  // the block scans run on 32-bit ints: pair indices and item counts stay below 2^31
  if (n_pairs * (int64_t)M >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(build_items_kernel, dim3(1), dim3(kBT), 0, s, rhs, n_pairs, M, rows_per_item,
                     items, item_count, max_items);
  return hipGetLastError();
}

}  // namespace mi
