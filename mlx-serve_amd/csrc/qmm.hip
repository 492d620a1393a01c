// Prefill (large-M) affine quantized GEMM for gfx950:
//   y[M,N] (bf16) = x[M,K] (bf16) @ dequant(w)[N,K]^T, fp32 accumulation.
// Replaces the reference's prefill route of qmatmulBits / prefillDqGemm
// (src/transformer.zig:20894-20983, :20987-21011), which dequantizes the whole weight to
// bf16 in HBM and then runs a dense GEMM. Here dequantization is fused into the LDS stage:
// a block owns a BN x BM output tile and walks K in 64-wide steps:
//   - x (A operand): BM x 64 bf16 streamed HBM -> LDS by global_load_lds (no VGPR round
//     trip), 16-byte slots XOR-swizzled by row so MFMA fragment reads are conflict free.
//   - w (B operand): each thread owns half a row of the 256-row weight tile: its 16 (4-bit)
//     or 32 (8-bit) packed bytes and the group's scale/bias are prefetched into registers a
//     tile ahead, dequantized in fp32 as scale*q + bias, rounded once to bf16 (as MLX's GPU
//     qmm stages bf16 weights in threadgroup memory) and written to LDS.
//   - 8 waves in a 2 (M) x 4 (N) grid; each wave owns BM/2 x 64 outputs as 32x32 tiles of
//     v_mfma_f32_32x32x16_bf16.
// Double-buffered LDS (A and B) with one barrier per K step.
#include <cstdlib>

#include "mi_internal.h"
#include "qmv_common.h"

namespace mi {
namespace {

using qmv_detail::mfma32;
using qmv_detail::vmcnt_imm;
using qmv_detail::lds_barrier;

constexpr int kBN = 256;       // weight rows (output columns) per block
constexpr int kBK = 64;        // K per step
constexpr int kThreads = 256;  // 4 waves, one per SIMD
constexpr int kRowBytes = kBK * 2;  // one LDS row: 64 bf16 = 8 slots of 16 bytes
constexpr int kRing = 4;           // x tiles in the LDS ring (prefetch distance kRing - 1)

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

MI_DEV uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Byte k of a word as a float (selects v_cvt_f32_ubyte{k}).
template <int k>
MI_DEV float ubyte(uint32_t w) { return (float)((w >> (8 * k)) & 0xFFu); }

MI_DEV void dma16(const void* src, unsigned char* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// LDS byte offset of 16-byte slot `c` (0..7) of row `r` in a [rows][64 bf16] tile. A
// 16-byte read serves 16 lanes per pass over 64 banks (256 B); with slot c ^ ((r>>1)&7) the
// 16 consecutive rows a fragment read touches fall in 16 distinct bank quads.
MI_DEV int swz(int r, int c) { return r * kRowBytes + ((c ^ ((r >> 1) & 7)) << 4); }

// Sub-steps (64-wide K steps) per super-step: a lane's packed weights for one super-step
// are 64 contiguous bytes of one row.
template <int BITS>
constexpr int kSubSteps = BITS == 4 ? 4 : 2;

template <int BITS, int GS, int TN>
struct WRegs {
  static constexpr int SS = kSubSteps<BITS>;
  static constexpr int kWords = 16;                          // 64 bytes per row
  static constexpr int kGroups = (SS * 32) / GS > 0 ? (SS * 32) / GS : 1;
  uint32_t q[TN][kWords];
  uint32_t s[TN][kGroups], b[TN][kGroups];  // bf16 bits of scales / biases
};

// SPLIT: this launch is one of several K ranges and writes fp32 partials (a template
// parameter, so each instance has a single epilogue: a per-element branch there makes the
// 256-accumulator instance spill).
template <int BITS, int GS, int BM, bool SPLIT>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
qmm_kernel(QmmParams P) {
  constexpr int TM = BM / 32;  // 32-row MFMA tiles per wave (the wave covers all BM rows)
  constexpr int TN = 2;        // 32-column MFMA tiles per wave (64 weight rows)
  constexpr int PF = 32 / BITS;
  constexpr int SS = kSubSteps<BITS>;
  constexpr int SSK = SS * kBK;       // K per super-step
  constexpr int LV = SS * 32;         // values of one row a lane owns per super-step
  using R_t = WRegs<BITS, GS, TN>;
  constexpr int NG = R_t::kGroups;
  constexpr int ABYTES = BM * kRowBytes;
  constexpr int A_INSTR = ABYTES / (kThreads * 16);  // DMA instructions per thread per step
  constexpr int W_OPS = TN * 4 + 2 * TN * NG;         // vector-memory ops of one W prefetch
  extern __shared__ __align__(16) unsigned char smem[];  // [kRing][BM][128 B] x tiles

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int M = P.M, N = P.N, K = P.K;
  const int G = K / GS;
  const int mtiles = (M + BM - 1) / BM;
  // Consecutive blocks land on different XCDs; walking M fastest keeps each XCD on the
  // same x row block while the weight tiles stream past.
  const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
  const int m0 = mt * BM, n0 = nt * kBN;
  // This block's K range: super-steps [sup_base, sup_base + nsup).
  const int split = blockIdx.y;
  const int sup_base = split * P.sup_per_split;
  const int nsup = min(P.sup_per_split, K / SSK - sup_base);
  const int nsteps = nsup * SS;

  // K order. The MFMA k-slots [8*(l/32), +8) of lane l at k-step ks (0..3) of sub-step t of
  // super-step T stand for columns SSK*T + LV*(l/32) + 32*t + 8*ks .. +8, for both operands.
  // So a lane's B operands for a whole super-step are LV consecutive values of one weight
  // row (64 bytes), and x tile chunk c (h = c/4, ks = c%4) of sub-step t holds columns
  // SSK*T + LV*h + 32*t + 8*ks.
  // ---- x: a wave DMA instruction moves 8 rows x 128 B; slot s of row r holds chunk
  // s ^ ((r>>1)&7). 32-bit element offsets (x below 2^31 bytes, checked on host).
  uint32_t xo[A_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int r = (wave * A_INSTR + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xo[i] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + LV * (c >> 2) + 8 * (c & 3);
  }
  auto issue_a = [&](int step, int slot) {
    unsigned char* dst = smem + slot * ABYTES + wave * A_INSTR * 8 * kRowBytes;
    const uint32_t ko = (uint32_t)((sup_base + step / SS) * SSK + (step % SS) * 32);
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) dma16(P.x + (xo[i] + ko), dst + i * 8 * kRowBytes);
  };

  // ---- w: 32-bit word / group offsets from the uniform bases (sizes checked on host).
  const int fr = lane & 31, fk = lane >> 5;
  uint32_t wo[TN], so[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const uint32_t n = (uint32_t)min(n0 + wave * 64 + j * 32 + fr, N - 1);
    wo[j] = n * (uint32_t)(K / PF) + fk * (LV / PF);
    so[j] = n * (uint32_t)G;
  }
  auto load_w = [&](int sup, R_t& R) {
    const uint32_t g0 = (uint32_t)((sup_base + sup) * SSK + fk * LV) / GS;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const u32x4_t* p =
          reinterpret_cast<const u32x4_t*>(P.w + (wo[j] + (sup_base + sup) * (SSK / PF)));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4_t v = p[i];
        R.q[j][4 * i] = v.x; R.q[j][4 * i + 1] = v.y;
        R.q[j][4 * i + 2] = v.z; R.q[j][4 * i + 3] = v.w;
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        R.s[j][g] = P.scales[so[j] + g0 + g];
        R.b[j][g] = P.biases[so[j] + g0 + g];
      }
    }
  };
  // Dequantize the 8 values of sub-step t, k-step ks of tile j into one MFMA B operand.
  auto dequant = [&](const R_t& R, int j, int t, int ks) -> u32x4_t {
    constexpr int kPerGroup = GS / 32 > 0 ? GS / 32 : 1;  // sub-steps per group
    const int g = NG == 1 ? 0 : t / kPerGroup;
    const float sc = bf16_bits_to_f32(R.s[j][g]), bi = bf16_bits_to_f32(R.b[j][g]);
    u32x4_t o;
    if constexpr (BITS == 4) {
      const uint32_t w = R.q[j][4 * t + ks];
      const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
      o.x = pack_bf16x2(fmaf(sc, ubyte<0>(lo), bi), fmaf(sc, ubyte<0>(hi), bi));
      o.y = pack_bf16x2(fmaf(sc, ubyte<1>(lo), bi), fmaf(sc, ubyte<1>(hi), bi));
      o.z = pack_bf16x2(fmaf(sc, ubyte<2>(lo), bi), fmaf(sc, ubyte<2>(hi), bi));
      o.w = pack_bf16x2(fmaf(sc, ubyte<3>(lo), bi), fmaf(sc, ubyte<3>(hi), bi));
    } else {
      const uint32_t w0 = R.q[j][8 * t + 2 * ks], w1 = R.q[j][8 * t + 2 * ks + 1];
      o.x = pack_bf16x2(fmaf(sc, ubyte<0>(w0), bi), fmaf(sc, ubyte<1>(w0), bi));
      o.y = pack_bf16x2(fmaf(sc, ubyte<2>(w0), bi), fmaf(sc, ubyte<3>(w0), bi));
      o.z = pack_bf16x2(fmaf(sc, ubyte<0>(w1), bi), fmaf(sc, ubyte<1>(w1), bi));
      o.w = pack_bf16x2(fmaf(sc, ubyte<2>(w1), bi), fmaf(sc, ubyte<3>(w1), bi));
    }
    return o;
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Software pipeline over sub-steps. Barrier point B(u) makes x tile u visible and frees
  // the ring slot of tile u-1; it sits inside sub-step u-1, after the LDS reads of that
  // sub-step's last k-step were issued and before its last MFMAs, so the first A fragments
  // and B operands of sub-step u are produced under those MFMAs. Within a sub-step, k-step
  // ks runs its TM*TN MFMAs while k-step ks+1's fragments are read (front-loaded) and its
  // B operands dequantized (1 MFMA : 1 LDS read : 3-4 VALU).
  u32x4_t a[2][TM], bop[2][TN];
  auto read_a = [&](int step, int ks, u32x4_t (&dst)[TM]) {
    const unsigned char* A = smem + (step % kRing) * ABYTES;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      dst[i] = *reinterpret_cast<const u32x4_t*>(A + swz(i * 32 + fr, 4 * fk + ks));
  };
  auto mfmas = [&](const u32x4_t (&av)[TM], const u32x4_t (&bv)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(av[i], bv[j], acc[i][j]);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int m = 0; m < TM * TN; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
      if (m < TM) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
      } else {
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // B(u): wait for x tile u, barrier, then issue x tile u+kRing-1 into the slot tile u-1
  // used and (when u starts a super-step) the next super-step's weights into the free set.
  // After tile u's DMA (issued at B(u-kRing+1)) tiles u+1 .. u+kRing-2 and the w prefetches
  // issued at B(u-kRing+1) .. B(u-1) may still be in flight.
  auto barrier_point = [&](int u, int tu, R_t& Rfree) {
    int wv = 0;
#pragma unroll
    for (int d = 1; d < kRing; ++d) wv += ((tu - d) % SS + SS) % SS == 0 ? 1 : 0;
    __builtin_amdgcn_sched_barrier(0);
    if (wv == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kRing - 2) * A_INSTR));
    else if (wv == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kRing - 2) * A_INSTR + W_OPS));
    else if (wv == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kRing - 2) * A_INSTR + 2 * W_OPS));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm((kRing - 2) * A_INSTR + 3 * W_OPS));
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue_a(min(u + kRing - 1, nsteps - 1), (u + kRing - 1) % kRing);
    if (tu == 0) load_w(min(u / SS + 1, nsup - 1), Rfree);
  };
  // Sub-step `step` (t = step % SS) with weights Rc; Rn is the other weights set.
  auto sub_step = [&](int step, int t, R_t& Rc, R_t& Rn) {
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      read_a(step, ks + 1, a[nxt]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bop[nxt][j] = dequant(Rc, j, t, ks + 1);
      mfmas(a[cur], bop[cur]);
      interleave();
    }
    const int u = step + 1;
    // At a super-step end Rc's last values were dequantized above, so it takes the prefetch.
    if (t + 1 == SS) {
      barrier_point(u, 0, Rc);
      read_a(min(u, nsteps - 1), 0, a[0]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bop[0][j] = dequant(Rn, j, 0, 0);
    } else {
      barrier_point(u, t + 1, Rn);
      read_a(u, 0, a[0]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bop[0][j] = dequant(Rc, j, t + 1, 0);
    }
    mfmas(a[1], bop[1]);
    interleave();
  };

  // ---- prologue: w of super-step 0, x tiles 0 .. kRing-2, B(0) (issues the next x tile
  // and the w of super-step 1), first fragments.
  R_t R0, R1;
  load_w(0, R0);
#pragma unroll
  for (int u = 0; u < kRing - 1; ++u) issue_a(min(u, nsteps - 1), u);
  barrier_point(0, 0, R1);
  read_a(0, 0, a[0]);
#pragma unroll
  for (int j = 0; j < TN; ++j) bop[0][j] = dequant(R0, j, 0, 0);
  __builtin_amdgcn_sched_barrier(0);

  auto super_step = [&](int sup, R_t& Rc, R_t& Rn) {
#pragma unroll
    for (int t = 0; t < SS; ++t) sub_step(sup * SS + t, t, Rc, Rn);
  };
  int sup = 0;
  for (; sup + 1 < nsup; sup += 2) {
    super_step(sup, R0, R1);
    super_step(sup + 1, R1, R0);
  }
  if (sup < nsup) super_step(sup, R0, R1);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may outlive the block


  // ---- epilogue: C reg r of a 32x32 tile is row 8(r/4) + 4(lane/32) + r%4, col lane%32.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wave * 64 + j * 32 + fr;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        if (m >= M) continue;
        if constexpr (SPLIT) P.part[((int64_t)split * M + m) * N + n] = acc[i][j][r];
        else P.y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][r]);
      }
  }
}

template <int BITS, int GS, int BM>
hipError_t launch_bm(const QmmParams& P, hipStream_t s) {
  const int mtiles = (P.M + BM - 1) / BM, ntiles = (P.N + kBN - 1) / kBN;
  const size_t lds = kRing * (size_t)BM * kRowBytes;
  auto k = P.ks > 1 ? qmm_kernel<BITS, GS, BM, true> : qmm_kernel<BITS, GS, BM, false>;
  static bool attr = false;
  if (!attr) {
    for (auto kk : {qmm_kernel<BITS, GS, BM, true>, qmm_kernel<BITS, GS, BM, false>}) {
      hipError_t e = hipFuncSetAttribute((const void*)kk,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    attr = true;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)(mtiles * ntiles), (unsigned)P.ks), dim3(kThreads), lds, s,
                     P);
  return hipGetLastError();
}

template <int BITS, int GS>
hipError_t launch_gs(const QmmParams& P, hipStream_t s) {
  return P.bm == 256 ? launch_bm<BITS, GS, 256>(P, s) : launch_bm<BITS, GS, 128>(P, s);
}

// y[m, n] = bf16(sum over splits in order of part[split, m, n]).
__global__ void qmm_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ y,
                                  int64_t mn, int ks) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float acc = add_splits<8>(part[i], part + i, mn, 1, ks);
    y[i] = (uint16_t)f32_to_bf16_bits(acc);
  }
}

}  // namespace

bool qmm_supported(int M, int N, int K, int bits, int gs) {
  (void)N;
  if (bits != 4 && bits != 8) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  // 32-bit in-kernel offsets: x, packed w and scales must each stay below 2^31 bytes.
  if ((int64_t)M * K * 2 >= ((int64_t)1 << 31) || (int64_t)N * K * bits / 8 >= ((int64_t)1 << 31))
    return false;
  return M >= 1 && K % (kSubSteps<4> * kBK) == 0 && K % gs == 0;
}

size_t qmm_plan(QmmParams& P) {
  static const int forced_bm = [] {
    const char* v = std::getenv("MI_QMM_BM");
    return v ? std::atoi(v) : 0;
  }();
  static const int forced_ks = [] {
    const char* v = std::getenv("MI_QMM_KS");
    return v ? std::atoi(v) : 0;
  }();
  const int ss = P.bits == 4 ? kSubSteps<4> : kSubSteps<8>;
  const int nsup = P.K / (ss * kBK);
  const int ntiles = (P.N + kBN - 1) / kBN;
  // 256-row tiles when they fill the GPU; otherwise 128-row tiles.
  const int64_t big = (int64_t)((P.M + 255) / 256) * ntiles;
  P.bm = forced_bm ? (forced_bm == 256 ? 256 : 128) : (big >= 240 ? 256 : 128);
  const int64_t blocks = (int64_t)((P.M + P.bm - 1) / P.bm) * ntiles;
  // Split K when the tiles cannot fill the GPU, keeping >= 2 super-steps per split.
  int ks = 1;
  if (forced_ks > 0) ks = forced_ks;
  else if (blocks < 200) ks = (int)std::min<int64_t>((320 + blocks - 1) / blocks, nsup / 2);
  ks = std::max(1, std::min(ks, nsup));
  P.sup_per_split = (nsup + ks - 1) / ks;
  P.ks = (nsup + P.sup_per_split - 1) / P.sup_per_split;
  return P.ks > 1 ? (size_t)P.ks * P.M * P.N * sizeof(float) : 0;
}

hipError_t launch_qmm(const QmmParams& P, hipStream_t s) {
  if (!qmm_supported(P.M, P.N, P.K, P.bits, P.group_size)) return hipErrorNotSupported;
  if (P.ks > 1 && !P.part) return hipErrorInvalidValue;
  hipError_t e;
  if (P.bits == 4) {
    switch (P.group_size) {
      case 32: e = launch_gs<4, 32>(P, s); break;
      case 64: e = launch_gs<4, 64>(P, s); break;
      default: e = launch_gs<4, 128>(P, s); break;
    }
  } else {
    switch (P.group_size) {
      case 32: e = launch_gs<8, 32>(P, s); break;
      case 64: e = launch_gs<8, 64>(P, s); break;
      default: e = launch_gs<8, 128>(P, s); break;
    }
  }
  if (e != hipSuccess || P.ks == 1) return e;
  const int64_t mn = (int64_t)P.M * P.N;
  int64_t g = (mn + 255) / 256;
  if (g > 65535) g = 65535;
  hipLaunchKernelGGL(qmm_reduce_kernel, dim3((unsigned)g), dim3(256), 0, s, P.part, P.y, mn, P.ks);
  return hipGetLastError();
}

}  // namespace mi
