// Prefill (large-M) 4-bit affine quantized GEMM for gfx950:
//   y[M,N] (bf16) = x[M,K] (bf16) @ dequant(w)[N,K]^T, fp32 accumulation.
// Replaces the reference's prefill route of qmatmulBits / prefillDqGemm
// (src/transformer.zig:20894-20983, :20987-21011), which expands the whole weight to a bf16
// copy in memory before a dense GEMM; here each weight tile is dequantized in registers on
// its way into the matrix cores and never exists in bf16 outside them.
//
// Block: 256 (M) x 256 (N) outputs, 8 waves (two per SIMD), v_mfma_f32_32x32x16_bf16 with
// D[n][m] = W[n][k] x[m][k]. Per 16-wide k-step a lane supplies 8 consecutive k of one
// weight row (k in [32h, 32h+32) of the 64-wide step, h = lane/32), dequantized as
// bf16(s*q + b): q from a scaled fp8 conversion, fma(s, q, b), one rounding to bf16 by
// v_cvt_pk_bf16_f32, as MLX's GPU qmm rounds the weights it stages. The x fragment of the
// same k-step is the 16-byte slot 4h+ks of the row. All staging is buffer_load ... lds DMA
// (no VGPR round trip); the schedule is described at prefill_pp_kernel.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "mi_common.h"
#include "mi_internal.h"
#include "qmv_common.h"
#include "dequant_bf16.h"

namespace mi {
namespace {

using qmv_detail::mfma32;
using qmv_detail::vmcnt_imm;
using dq::dequant8;
using dq::pack_bf16x2;

constexpr int kBM = 256, kBN = 256, kBK = 64, kRing = 3;
constexpr int kXBytes = kBM * kBK * 2;  // x tile: 256 rows x 128 B
constexpr int kBufFlags = 0x00020000;   // raw dword access

#define MI_DMA_LDS(SIZE, rsrc, lds, voff, soff)                                            \
  __builtin_amdgcn_raw_ptr_buffer_load_lds((rsrc), (__attribute__((address_space(3))) void*)(lds), \
                                           SIZE, (voff), (soff), 0, 0)

// Ping-pong variant: 8 waves, two per SIMD. Wave w owns weight rows [32w, 32w + 32) (one
// 32-row tile) against all 256 x rows (eight 32-row tiles): 8 accumulators (128
// registers), so two waves fit a SIMD, and every weight of the block is dequantized by
// exactly one wave. (VALU work issued beside another wave's MFMAs delays them, so the
// dequantize count per MFMA is what this layout minimizes; the price is one 1 KB x
// fragment read per MFMA, half the LDS read bandwidth of a CU.) Each wave's work on a
// 64-wide step is two units: "mem" (its packed weights, scales and biases from LDS,
// dequantized to the 16 bf16 operand registers of the whole step, and the first x
// fragments) and "mfma" (the step's 32 MFMAs, the remaining x fragments read as they go).
// The two groups run the same units half a step apart on staggered barriers: while group
// 0 issues the matrix ops of step t, group 1 dequantizes step t, then the roles swap, so
// each SIMD always has one wave feeding the matrix core and one doing the VALU/LDS work.
// Timeline of half-steps h (a block barrier after each):
//   h = 2t:    group 0 mem(t),     group 1 mfma(t-1)
//   h = 2t+1:  group 0 mfma(t),    group 1 mem(t);  every wave issues the DMA of step t+2
//
// Staging is shaped by the number of memory requests, not bytes: the DMA path serves a
// bounded number of requests per CU per cycle, and a request per 4-byte scale was the
// largest cost. So LDS holds
//   - x: a 3-stage ring of 256 x 64 tiles (32 KB each; 128-byte rows, one request each),
//   - packed weights: 2 buffers of 2-step chunks (256 rows x 64 B: one request per row
//     per two steps, against one per step for 32-byte rows),
//   - scales and biases: 2 buffers of 8-group chunks (256 rows x 16 B each, moved as
//     4 dwords per row: one request per row per 8 groups).
// A chunk goes out with the x tile of its first step and lands one step ahead of use.
// Step t's x stage is last read in half 2t+2; the DMA that reuses it (step t+3) goes out
// in half 2t+3. Each wave waits (exact vmcnt) at the end of half 2t+1 for everything
// issued before the DMA of step t+2, so the barrier publishes step t+1 before group 0
// reads it in half 2t+2. The weight and scale buffers are reused two chunks later, after
// the last read of the chunk they held.
// 8-bit weights (BITS = 8) take the same path with one step per weight chunk (64 B of a row
// is one step's 64 codes), in 3 buffers: a 1-step chunk is last read in the half after its
// successor's DMA would go out, so two buffers would not do.
constexpr int kPPThreads = 512;
constexpr int kPPXStage = kXBytes;                   // 32 KB
constexpr int kPPWChunk = kBN * 64;                  // 256 rows x 64 B
constexpr int kPPSChunk = kBN * 16;                  // 256 rows x 16 B (scales or biases)
constexpr int kPPWOff = kRing * kPPXStage;           // 96 KB
// BITS = 16: weights already dequantized to bf16 (the other formats' large-M route). A
// lane's 64 bytes of its row per step are read straight into registers (a 3-step ring), so
// LDS holds only the x ring and the mem unit does no dequantize work.
template <int BITS>
constexpr int pp_wbufs() { return BITS == 4 ? 2 : BITS == 8 ? 3 : 0; }
template <int BITS>
constexpr int pp_soff() { return kPPWOff + pp_wbufs<BITS>() * kPPWChunk; }  // 128 / 144 KB
template <int BITS>
constexpr int pp_lds() { return BITS == 16 ? kPPWOff : pp_soff<BITS>() + 4 * kPPSChunk; }

// 8 bytes (codes q0..q7, k order) -> four bf16 pairs of s*q + b: each byte converts exactly
// (v_cvt_f32_ubyte), fma(s, q, b), one rounding to bf16.
MI_DEV u32x4_t dequant8_b8(uint32_t w0, uint32_t w1, float s, float b) {
  u32x4_t o;
  o.x = pack_bf16x2(fmaf(s, (float)(w0 & 0xFFu), b), fmaf(s, (float)((w0 >> 8) & 0xFFu), b));
  o.y = pack_bf16x2(fmaf(s, (float)((w0 >> 16) & 0xFFu), b), fmaf(s, (float)(w0 >> 24), b));
  o.z = pack_bf16x2(fmaf(s, (float)(w1 & 0xFFu), b), fmaf(s, (float)((w1 >> 8) & 0xFFu), b));
  o.w = pack_bf16x2(fmaf(s, (float)((w1 >> 16) & 0xFFu), b), fmaf(s, (float)(w1 >> 24), b));
  return o;
}

MI_DEV void wait_vm(int n) {  // s_waitcnt vmcnt(n) for the counts one step can issue
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4)); break;
    case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6)); break;
    case 8: __builtin_amdgcn_s_waitcnt(vmcnt_imm(8)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(10)); break;
  }
}

template <int BITS, int GS, bool SPLIT>
__global__ void __launch_bounds__(kPPThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_pp_kernel(PrefillParams P) {
  constexpr int RB = BITS * kBK / 8;  // bytes of a weight row per step: 32, 64 or 128
  constexpr bool W16 = BITS == 16;
  constexpr int kSOff = pp_soff<BITS>();
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // steps per scale chunk (8 groups): 4, 8 or 16
  constexpr int kSP = GS / 8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, nq = wave & 3;
  const int fr = lane & 31, h = lane >> 5;
  const int M = P.M, N = P.N, K = P.K, G = K / GS;
  const int mtiles = (M + kBM - 1) / kBM;
  const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int split = blockIdx.y;
  const int s0 = split * P.sps;
  const int nsteps = min(P.sps, K / kBK - s0);
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);

  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.x + (size_t)m0 * K), 0, mrows * K * 2, kBufFlags);
  const int rowb = K * BITS / 8;  // bytes of a weight row
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const unsigned char*)P.w + (size_t)n0 * rowb), 0, nrows * rowb, kBufFlags);
  // group 0 moves the scales, group 1 the biases
  const __amdgpu_buffer_rsrc_t sbres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((grp ? P.biases : P.scales) + (size_t)n0 * G), 0, nrows * G * 2, kBufFlags);
  // x: wave w moves tile rows 32w..32w+31 as 4 instructions of 8 rows x 128 B; LDS slot p
  // of row r holds k-slot p ^ ((r >> 1) & 7).
  uint32_t xo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 32 * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xo[i] = (uint32_t)(min(r, mrows - 1) * K + 8 * c) * 2;
  }
  // packed-weight chunk (2 steps at 4 bits, 1 at 8): wave w moves rows 32w..32w+31 as 2
  // instructions of 16 rows x 64 B; LDS part p (16 B) of row r holds part p ^ ((r >> 2) & 3)
  // of the row's 64 bytes.
  uint32_t wo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 32 * wave + 16 * i + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    wo[i] = (uint32_t)(min(r, nrows - 1) * rowb + 16 * c);
  }
  // scale (group 0) or bias (group 1) chunk: wave moves rows 64nq..64nq+63 as 4
  // instructions of 16 rows x 4 dwords; row-major 16 B per row in LDS.
  uint32_t so[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 64 * nq + 16 * i + (lane >> 2);
    so[i] = (uint32_t)(min(r, nrows - 1) * G * 2 + 4 * (lane & 3));
  }
  // bf16 weights: lane (fr, h) reads bytes 64h .. 64h+63 of its row's 128 per step
  u32x4_t wreg[W16 ? 3 : 1][4];
  const uint32_t w16o = (uint32_t)min(32 * wave + fr, nrows - 1) * (uint32_t)rowb + 64 * h;
  // DMA of local step st (x; the weight chunk when st is even; the scale chunk when st
  // starts one; bf16 weights into register slot `slot`). Returns the instructions issued
  // (0 past the last step).
  auto issue = [&](int st, auto slot_c) -> int {
    constexpr int slot = decltype(slot_c)::value;
    if (st >= nsteps) return 0;
    const int k = s0 + st;
    unsigned char* xb = smem + (st % kRing) * kPPXStage;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      MI_DMA_LDS(16, xres, xb + wave * 4096 + i * 1024, xo[i], k * kBK * 2);
    int n = 4;
    if constexpr (W16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        wreg[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(wres, w16o + 16 * i, k * RB, 0);
      return n + 4;
    }
    if (BITS == 8 || (st & 1) == 0) {
      unsigned char* wb = smem + kPPWOff + (BITS == 4 ? (st >> 1) & 1 : st % 3) * kPPWChunk;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        MI_DMA_LDS(16, wres, wb + wave * 2048 + i * 1024, wo[i], k * RB);
      n += 2;
    }
    if (st == 0 || k % kSP == 0) {
      const int c = k / kSP;
      unsigned char* sb = smem + kSOff + (c & 1) * 2 * kPPSChunk + grp * kPPSChunk;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        MI_DMA_LDS(4, sbres, sb + nq * 1024 + i * 256, so[i], c * 16);
      n += 4;
    }
    return n;
  };

  f32x16_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  // The accumulators go to AGPRs (the clobber makes AGPRs available to the allocator),
  // so the MFMA C/D traffic stays out of the VGPR file the other wave's VALU work uses.
  asm volatile("" ::: "a0");

  // x fragment of tile i: row 32 i + fr, k-slot 4h + ks.
  auto xfrag = [&](int stg, int i, int ks) -> u32x4_t {
    const int r = 32 * i + fr, c = 4 * h + ks;
    return *reinterpret_cast<const u32x4_t*>(smem + stg * kPPXStage + r * 128 +
                                             ((c ^ ((r >> 1) & 7)) << 4));
  };
  u32x4_t A[4], X[2][8];
  auto mem = [&](int st, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) X[0][i] = xfrag(st % kRing, i, 0);
    if constexpr (W16) return;  // the MFMAs read the weight registers in place
    const int k = s0 + st;
    const unsigned char* wb =
        smem + kPPWOff + (BITS == 4 ? (st >> 1) & 1 : st % 3) * kPPWChunk;
    const unsigned char* sb = smem + kSOff + ((k / kSP) & 1) * 2 * kPPSChunk;
    // group of this lane's 32 k within the chunk's 8
    const int gi = GS == 32 ? 2 * (k % 4) + h : GS == 64 ? k % 8 : (k >> 1) % 8;
    const int r = 32 * wave + fr;
    // the lane's 32 codes: 16 B (part 2(st%2) + h) at 4 bits, 32 B (parts 2h, 2h+1) at 8
    const int part = BITS == 4 ? 2 * (st & 1) + h : 2 * h;
    const u32x4_t q =
        *reinterpret_cast<const u32x4_t*>(wb + r * 64 + ((part ^ ((r >> 2) & 3)) << 4));
    u32x4_t q2 = q;
    if constexpr (BITS == 8)
      q2 = *reinterpret_cast<const u32x4_t*>(wb + r * 64 + (((part + 1) ^ ((r >> 2) & 3)) << 4));
    const uint16_t sv = *reinterpret_cast<const uint16_t*>(sb + r * 16 + 2 * gi);
    const uint16_t bv = *reinterpret_cast<const uint16_t*>(sb + kPPSChunk + r * 16 + 2 * gi);
    const float sc = __uint_as_float((uint32_t)sv << 16);
    const float bp = __uint_as_float((uint32_t)bv << 16);
    if constexpr (BITS == 4) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) A[ks] = dequant8(q[ks], sc, bp);
    } else {
      A[0] = dequant8_b8(q.x, q.y, sc, bp);
      A[1] = dequant8_b8(q.z, q.w, sc, bp);
      A[2] = dequant8_b8(q2.x, q2.y, sc, bp);
      A[3] = dequant8_b8(q2.z, q2.w, sc, bp);
    }
  };
  auto mfma = [&](int st, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int stg = st % kRing;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < 3) {
#pragma unroll
        for (int i = 0; i < 8; ++i) X[(ks + 1) & 1][i] = xfrag(stg, i, ks + 1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i] = mfma32(W16 ? wreg[slot][ks] : A[ks], X[ks & 1][i], acc[i]);
      // the next k-step's fragment reads go out ahead of this k-step's MFMAs, one read
      // per MFMA, so their latency hides under the matrix work
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (ks < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Both groups run the same unit sequence mem(t), mfma(t) with a barrier after each unit;
  // group 1 starts one half later (an extra barrier first), group 0 ends with an extra
  // barrier, so the barrier counts match. The DMA of step t+2 goes out in half 2t+1 for
  // both groups: after group 0's mfma(t) unit and after group 1's mem(t) unit.
  using c0 = std::integral_constant<int, 0>;
  using c1 = std::integral_constant<int, 1>;
  using c2 = std::integral_constant<int, 2>;
  issue(0, c0{});
  wait_vm(issue(1, c1{}));
  __builtin_amdgcn_s_barrier();
  if (grp) __builtin_amdgcn_s_barrier();
  // (ws: the register slot of step t's bf16 weights, wn: that of step t + 2)
  auto step = [&](int t, auto ws, auto wn) {
    mem(t, ws);
    __builtin_amdgcn_sched_barrier(0);
    if (grp) wait_vm(issue(t + 2, wn));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mfma(t, ws);
    __builtin_amdgcn_sched_barrier(0);
    if (!grp) wait_vm(issue(t + 2, wn));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (W16) {
    // unrolled by 3 so the weight registers of steps t, t+1, t+2 sit in static slots
    for (int t0 = 0; t0 < nsteps; t0 += 3) {
      step(t0, c0{}, c2{});
      if (t0 + 1 < nsteps) step(t0 + 1, c1{}, c0{});
      if (t0 + 2 < nsteps) step(t0 + 2, c2{}, c1{});
    }
  } else {
    for (int t = 0; t < nsteps; ++t) step(t, c0{}, c0{});
  }
  if (!grp) __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may outlive the block

  // epilogue: acc[i] register r is D[n = 32 wave + 8(r/4) + 4h + r%4][m = 32 i + fr]
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + 32 * i + fr;
    if (m >= M) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + 32 * wave + 8 * g + 4 * h;
      if (n >= N) continue;
      if constexpr (SPLIT) {
        f32x4_t v = {acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]};
        *reinterpret_cast<f32x4_t*>(P.part + ((size_t)split * M + m) * N + n) = v;
      } else {
        u32x2_t o;
        o.x = pack_bf16x2(acc[i][4 * g], acc[i][4 * g + 1]);
        o.y = pack_bf16x2(acc[i][4 * g + 2], acc[i][4 * g + 3]);
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

template <typename Kern>
hipError_t set_lds(Kern k, size_t lds) {
  return hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

template <int BITS, int GS>
hipError_t launch_gs(const PrefillParams& P, hipStream_t s) {
  const int mtiles = (P.M + kBM - 1) / kBM, ntiles = (P.N + kBN - 1) / kBN;
  constexpr int lds = pp_lds<BITS>();
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipSuccess;
    for (auto k : {prefill_pp_kernel<BITS, GS, true>, prefill_pp_kernel<BITS, GS, false>})
      if (e == hipSuccess) e = set_lds(k, lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const dim3 grid((unsigned)(mtiles * ntiles), (unsigned)P.ks);
  if (P.ks > 1)
    hipLaunchKernelGGL((prefill_pp_kernel<BITS, GS, true>), grid, dim3(kPPThreads), lds, s, P);
  else
    hipLaunchKernelGGL((prefill_pp_kernel<BITS, GS, false>), grid, dim3(kPPThreads), lds, s, P);
  return hipGetLastError();
}

template <int BITS>
hipError_t launch_bits(const PrefillParams& P, hipStream_t s) {
  if constexpr (BITS == 16)
    return launch_gs<16, 64>(P, s);  // no groups
  else
    return P.group_size == 32   ? launch_gs<BITS, 32>(P, s)
           : P.group_size == 64 ? launch_gs<BITS, 64>(P, s)
                                : launch_gs<BITS, 128>(P, s);
}

}  // namespace

bool prefill_supported(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  if (bits == 16)  // bf16 weights: no groups, no scale chunks
    return M >= 1 && N >= 4 && N % 4 == 0 && K % kBK == 0 &&
           (int64_t)kBM * K * 2 < ((int64_t)1 << 31) && (int64_t)kBN * K * 2 < ((int64_t)1 << 31) &&
           M < ((int64_t)1 << 30) && N < ((int64_t)1 << 30);
  if ((bits != 4 && bits != 8) || (gs != 32 && gs != 64 && gs != 128)) return false;
  // 32-bit buffer offsets per block; 4-output stores; whole 64-wide steps and groups; an
  // even group count, so every row's scales and biases start on a dword (the staging
  // moves them as dwords)
  return M >= 1 && N >= 4 && N % 4 == 0 && K % kBK == 0 && K % gs == 0 && (K / gs) % 2 == 0 &&
         (int64_t)kBM * K * 2 < ((int64_t)1 << 31) && (int64_t)kBN * K * bits / 8 < ((int64_t)1 << 31) &&
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
  if (!prefill_supported(P.M, P.N, P.K, P.bits, P.group_size)) return hipErrorNotSupported;
  if (P.ks > 1 && !P.part) return hipErrorInvalidValue;
  hipError_t e = P.bits == 16 ? launch_bits<16>(P, s)
                 : P.bits == 8 ? launch_bits<8>(P, s)
                               : launch_bits<4>(P, s);
  if (e != hipSuccess || P.ks == 1) return e;
  const int64_t mn4 = (int64_t)P.M * P.N / 4;
  int64_t g = (mn4 + 255) / 256;
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(prefill_reduce_kernel, dim3((unsigned)g), dim3(256), 0, s, P.part, P.y, mn4,
                     P.ks);
  return hipGetLastError();
}

}  // namespace mi
