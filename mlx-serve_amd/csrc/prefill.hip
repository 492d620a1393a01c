// Prefill (large-M) 4-bit affine quantized GEMM for gfx950:
//   y[M,N] (bf16) = x[M,K] (bf16) @ dequant(w)[N,K]^T, fp32 accumulation.
// Replaces the reference's prefill route of qmatmulBits / prefillDqGemm
// (src/transformer.zig:20894-20983, :20987-21011), which expands the whole weight to a bf16
// copy in memory before a dense GEMM; here each weight tile is dequantized in registers on
// its way into the matrix cores and never exists in bf16 outside them.
//
// Block: 256 (M) x 256 (N) outputs, 4 waves, one per SIMD. Wave w owns weight rows
// [64w, 64w+64) of the tile (two 32-row MFMA tiles) against all 256 x rows (eight 32-row
// tiles): 16 accumulators of v_mfma_f32_32x32x16_bf16, D[n][m] = W[n][k] x[m][k].
// K advances in 64-wide steps through a 3-stage LDS ring. Every stage is filled by
// buffer_load ... lds (no VGPR round trip): the 256 x 64 x tile (32 KB, 16-byte slots XOR-
// swizzled by row so fragment reads are bank-conflict free), the 256 x 32 B packed weight
// tile (8 KB) and one dword of scales and of biases per weight row.
// Per 16-wide k-step a lane supplies 8 consecutive k of one weight row: word ks of the 16
// packed bytes it owns (k in [32h, 32h+32) of the step, h = lane/32), dequantized as
// bf16(s*q + b): q from a scaled fp8 conversion, fma(s, q, b), one rounding to bf16 by
// v_cvt_pk_bf16_f32, as MLX's GPU qmm rounds the weights it stages.
// The x fragment of the same k-step is the natural 16-byte slot 4h+ks of the row.
// One barrier per step, placed inside k-step 2 after the stage's last fragment reads: it
// publishes the next stage (its DMA waited on with an exact vmcnt) and frees this one for
// the DMA of step s+3. Loads past the last step repeat it, so the control flow is uniform
// and the compiler's wait counts stay exact.
#include <algorithm>
#include <cstdlib>

#include "mi_common.h"
#include "mi_internal.h"
#include "qmv_common.h"

namespace mi {
namespace {

using qmv_detail::mfma32;
using qmv_detail::vmcnt_imm;

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256, kRing = 3;
constexpr int kXBytes = kBM * kBK * 2;  // x tile: 256 rows x 128 B
constexpr int kWBytes = kBN * kBK / 2;  // packed 4-bit tile: 256 rows x 32 B
constexpr int kSBytes = kBN * 4;        // one dword of scales (or biases) per row
constexpr int kStage = kXBytes + kWBytes + 2 * kSBytes;
constexpr int kBufFlags = 0x00020000;   // raw dword access
constexpr int kLoadsPerStep = 12;       // DMA instructions per thread per step

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

#define MI_DMA_LDS(SIZE, rsrc, lds, voff, soff)                                            \
  __builtin_amdgcn_raw_ptr_buffer_load_lds((rsrc), (__attribute__((address_space(3))) void*)(lds), \
                                           SIZE, (voff), (soff), 0, 0)

// Scale dword of step st: the dword holding group g = (64 st + 32 h) / GS of the row.
template <int GS>
MI_DEV uint32_t sb_dword(int st) {
  return GS == 32 ? 4u * st : GS == 64 ? 4u * (st >> 1) : 4u * (st >> 2);
}
template <int GS>
MI_DEV bool sb_high(int st, int h) {
  return GS == 32 ? h != 0 : GS == 64 ? (st & 1) != 0 : ((st >> 1) & 1) != 0;
}

// SPLIT: this block covers K steps [split * sps, +sps) and writes fp32 partials.
template <int GS, bool SPLIT>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
prefill_kernel(PrefillParams P) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, h = lane >> 5;
  const int M = P.M, N = P.N, K = P.K, G = K / GS;
  const int mtiles = (M + kBM - 1) / kBM;
  // Consecutive blocks land on different XCDs: walking M fastest gives each XCD a fixed
  // set of x tiles while the weight tiles stream past.
  const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int split = blockIdx.y;
  const int s0 = split * P.sps;
  const int nsteps = min(P.sps, K / kBK - s0);
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);

  // Buffer resources based at the block's first rows; reads past them return 0.
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.x + (size_t)m0 * K), 0, mrows * K * 2, kBufFlags);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const unsigned char*)P.w + (size_t)n0 * (K / 2)), 0, nrows * (K / 2), kBufFlags);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.scales + (size_t)n0 * G), 0, nrows * G * 2, kBufFlags);
  const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.biases + (size_t)n0 * G), 0, nrows * G * 2, kBufFlags);
  // x: wave w moves tile rows 64w..64w+63 as 8 instructions of 8 rows x 128 B; LDS slot p
  // of row r holds k-slot p ^ ((r >> 1) & 7).
  uint32_t xo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xo[i] = (uint32_t)(min(r, mrows - 1) * K + 8 * c) * 2;
  }
  // packed w: wave w moves rows 64w..64w+63 as 2 instructions of 32 rows x 32 B; LDS half
  // p of row r holds 16-byte half p ^ ((r >> 3) & 1).
  uint32_t wo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 64 * wave + 32 * i + (lane >> 1);
    const int c = (lane & 1) ^ ((r >> 3) & 1);
    wo[i] = (uint32_t)(min(r, nrows - 1) * (K / 2) + 16 * c);
  }
  const uint32_t so = (uint32_t)min(64 * wave + lane, nrows - 1) * G * 2;
  auto issue = [&](int st, int stg) {
    unsigned char* base = smem + stg * kStage;
    const int k = s0 + st;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      MI_DMA_LDS(16, xres, base + 64 * wave * 128 + i * 1024, xo[i], k * kBK * 2);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      MI_DMA_LDS(16, wres, base + kXBytes + 64 * wave * 32 + i * 1024, wo[i], k * (kBK / 2));
    MI_DMA_LDS(4, sres, base + kXBytes + kWBytes + 256 * wave, so, sb_dword<GS>(k));
    MI_DMA_LDS(4, bres, base + kXBytes + kWBytes + kSBytes + 256 * wave, so, sb_dword<GS>(k));
  };

  f32x16_t acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // x fragment: tile row 32i + fr, k-slot 4h + ks of the stage.
  auto xfrag = [&](int stg, int i, int ks) -> u32x4_t {
    const int r = 32 * i + fr, c = 4 * h + ks;
    return *reinterpret_cast<const u32x4_t*>(smem + stg * kStage + r * 128 +
                                             ((c ^ ((r >> 1) & 7)) << 4));
  };
  struct WStep {
    u32x4_t q[2];
    uint32_t s[2], b[2];
  };
  // This wave's packed words and scale/bias dwords of weight rows 64w + 32j + fr.
  auto wread = [&](int stg, WStep& o) {
    const unsigned char* base = smem + stg * kStage + kXBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 64 * wave + 32 * j + fr;
      o.q[j] = *reinterpret_cast<const u32x4_t*>(base + r * 32 + ((h ^ ((r >> 3) & 1)) << 4));
      o.s[j] = *reinterpret_cast<const uint32_t*>(base + kWBytes + 4 * r);
      o.b[j] = *reinterpret_cast<const uint32_t*>(base + kWBytes + kSBytes + 4 * r);
    }
  };
  float sc[2], bp[2];
  auto scales_of = [&](const WStep& w, int st) {
    const bool hi = sb_high<GS>(s0 + st, h);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      sc[j] = __uint_as_float(hi ? (w.s[j] & 0xFFFF0000u) : (w.s[j] << 16));
      bp[j] = __uint_as_float(hi ? (w.b[j] & 0xFFFF0000u) : (w.b[j] << 16));
    }
  };

  // prologue: steps 0..2 in flight, step 0 published
  issue(0, 0);
  issue(min(1, nsteps - 1), 1);
  issue(min(2, nsteps - 1), 2);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kLoadsPerStep));
  __builtin_amdgcn_s_barrier();
  u32x4_t xb[2][8], a[2][2];
  WStep wc, wn;
  wread(0, wc);
  scales_of(wc, 0);
#pragma unroll
  for (int i = 0; i < 8; ++i) xb[0][i] = xfrag(0, i, 0);
#pragma unroll
  for (int j = 0; j < 2; ++j) a[0][j] = dequant8(wc.q[j][0], sc[j], bp[j]);

  auto mfmas = [&](int cur) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[cur][j], xb[cur][i], acc[i][j]);
  };
  // Interleave: one LDS read and three VALU ops (next k-step's operands) per MFMA.
  auto interleave = [&](int nds) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (m < nds) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto step = [&](int st, int stage) {
    const int ns = stage == kRing - 1 ? 0 : stage + 1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
#pragma unroll
      for (int i = 0; i < 8; ++i) xb[nxt][i] = xfrag(stage, i, ks + 1);
#pragma unroll
      for (int j = 0; j < 2; ++j) a[nxt][j] = dequant8(wc.q[j][ks + 1], sc[j], bp[j]);
      mfmas(cur);
      interleave(8);
    }
    {  // k-step 2: last fragments of this stage, barrier, DMA of step st+3, W of step st+1
#pragma unroll
      for (int i = 0; i < 8; ++i) xb[1][i] = xfrag(stage, i, 3);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kLoadsPerStep));
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(min(st + 3, nsteps - 1), stage);
      wread(ns, wn);
#pragma unroll
      for (int j = 0; j < 2; ++j) a[1][j] = dequant8(wc.q[j][3], sc[j], bp[j]);
      mfmas(0);
      interleave(6);
    }
    {  // k-step 3: first fragments and operands of step st+1
#pragma unroll
      for (int i = 0; i < 8; ++i) xb[0][i] = xfrag(ns, i, 0);
      scales_of(wn, st + 1);
#pragma unroll
      for (int j = 0; j < 2; ++j) a[0][j] = dequant8(wn.q[j][0], sc[j], bp[j]);
      mfmas(1);
      interleave(8);
      wc = wn;
    }
  };
  int st = 0;
  for (; st + 3 <= nsteps; st += 3) {
    step(st, 0);
    step(st + 1, 1);
    step(st + 2, 2);
  }
  if (st < nsteps) step(st, 0);
  if (st + 1 < nsteps) step(st + 1, 1);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may outlive the block

  // epilogue: acc[i][j] register r is D[n = 8(r/4) + 4h + r%4][m = fr] of tile (i, j)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + 32 * i + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 64 * wave + 32 * j + 8 * g + 4 * h;
        if (n >= N) continue;
        if constexpr (SPLIT) {
          f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                       acc[i][j][4 * g + 3]};
          *reinterpret_cast<f32x4_t*>(P.part + ((size_t)split * M + m) * N + n) = v;
        } else {
          u32x2_t o;
          o.x = pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
          o.y = pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          *reinterpret_cast<u32x2_t*>(P.y + (size_t)m * N + n) = o;
        }
      }
  }
}

// y = bf16(sum over splits in split order of part[split]); 4 outputs per thread.
__global__ void prefill_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ y,
                                      int64_t mn4, int ks) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn4;
       i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(part) + i;
    const f32x4_t acc = add_splits<8>(p4[0], p4, mn4, 1, ks);
    u32x2_t o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    reinterpret_cast<u32x2_t*>(y)[i] = o;
  }
}

template <int GS>
hipError_t launch_gs(const PrefillParams& P, hipStream_t s) {
  const int mtiles = (P.M + kBM - 1) / kBM, ntiles = (P.N + kBN - 1) / kBN;
  const size_t lds = (size_t)kRing * kStage;
  static bool attr = false;
  if (!attr) {
    for (auto k : {prefill_kernel<GS, true>, prefill_kernel<GS, false>}) {
      hipError_t e =
          hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    attr = true;
  }
  const dim3 grid((unsigned)(mtiles * ntiles), (unsigned)P.ks);
  if (P.ks > 1)
    hipLaunchKernelGGL((prefill_kernel<GS, true>), grid, dim3(kThreads), lds, s, P);
  else
    hipLaunchKernelGGL((prefill_kernel<GS, false>), grid, dim3(kThreads), lds, s, P);
  return hipGetLastError();
}

}  // namespace

bool prefill_supported(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  if (bits != 4 || (gs != 32 && gs != 64 && gs != 128)) return false;
  // 32-bit buffer offsets per block; 4-output stores; whole 64-wide steps and groups
  return M >= 1 && N >= 4 && N % 4 == 0 && K % kBK == 0 && K % gs == 0 &&
         (int64_t)kBM * K * 2 < ((int64_t)1 << 31) && (int64_t)kBN * K < ((int64_t)1 << 31) &&
         M < ((int64_t)1 << 30) && N < ((int64_t)1 << 30);
}

size_t prefill_plan(PrefillParams& P) {
  static const int forced_ks = [] {
    const char* v = std::getenv("MI_QMM_PREFILL_KS");
    return v ? std::atoi(v) : 0;
  }();
  const int steps = P.K / kBK;
  const int64_t tiles = (int64_t)((P.M + kBM - 1) / kBM) * ((P.N + kBN - 1) / kBN);
  // K splits: the fewest estimated microseconds over rounds of 256 blocks (one per CU) x
  // 64-wide steps a split (~2.15 us a step for a 256 x 256 tile), plus each split's fp32
  // partials written and read back once (~5 TB/s); at least 8 steps a split. Measured at
  // M=512: gate [14336,4096] 2 splits 27.5% of the bf16 peak (3 splits 20.5%), down
  // [4096,14336] 8 splits 29.2%.
  int ks = 1;
  if (forced_ks > 0) {
    ks = forced_ks;
  } else {
    double best = 1e30;
    for (int k = 1; k <= std::max(1, steps / 8); ++k) {
      const int64_t rounds = (tiles * k + 255) / 256;
      const int sps = (steps + k - 1) / k;
      const double part_us = k > 1 ? (double)k * P.M * P.N * 8 / 5e6 : 0.0;
      const double cost = (double)rounds * sps * 2.15 + part_us;
      if (cost < best - 1e-9) {
        best = cost;
        ks = k;
      }
    }
  }
  ks = std::max(1, std::min(ks, steps));
  P.sps = (steps + ks - 1) / ks;
  P.ks = (steps + P.sps - 1) / P.sps;
  return P.ks > 1 ? (size_t)P.ks * P.M * P.N * sizeof(float) : 0;
}

hipError_t launch_prefill(const PrefillParams& P, hipStream_t s) {
  if (!prefill_supported(P.M, P.N, P.K, 4, P.group_size)) return hipErrorNotSupported;
  if (P.ks > 1 && !P.part) return hipErrorInvalidValue;
  hipError_t e = P.group_size == 32 ? launch_gs<32>(P, s)
                 : P.group_size == 64 ? launch_gs<64>(P, s)
                                      : launch_gs<128>(P, s);
  if (e != hipSuccess || P.ks == 1) return e;
  const int64_t mn4 = (int64_t)P.M * P.N / 4;
  int64_t g = (mn4 + 255) / 256;
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(prefill_reduce_kernel, dim3((unsigned)g), dim3(256), 0, s, P.part, P.y, mn4,
                     P.ks);
  return hipGetLastError();
}

}  // namespace mi
