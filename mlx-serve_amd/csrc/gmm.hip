// Grouped quantized GEMM over expert-sorted work items: the sorted gather_qmm of an MoE
// prefill (reference: the three gather_qmm(sorted_indices = true) calls over expert
// segments in src/transformer.zig:14961-15043, gather at :15011), 4-bit affine weights,
// group size 64, bf16 activations.
//
// A work item is a run of sorted pairs with one expert, cut at 32*MT rows (build_items in
// quant.hip). One block = one item x one 32*WV-row tile of the expert's weight: it streams
// that weight tile from HBM exactly once and multiplies it by all the item's rows, so an
// expert with up to 32*MT rows is read once per call whatever its segment length.
//
// Block: WV waves; wave w owns weight rows n0 + 32w .. +31 (one 32-row MFMA tile) against
// the item's 32*MT rows (MT tiles) of v_mfma_f32_32x32x16_bf16, D[n][m] = W[n][k] x[m][k],
// with two accumulator sets (even / odd k-steps) so consecutive MFMAs are independent.
// Per 64-wide step a lane (fr = lane % 32, h = lane / 32) holds 16 packed bytes of its
// weight row (k in [32h, 32h+32)), dequantized in registers as bf16(s*q + b)
// (dq::dequant8: no all-ones MFMA and no per-group epilogue); the x fragment of k-step ks
// is the 16-byte slot 4h+ks of the row.
// Pipeline, kD steps deep: a step's weight bytes go to a register ring, its gathered x rows
// to an LDS ring by buffer_load ... lds DMA (rows past the item's end read past the end of
// x: zeros, no memory traffic), and every 4 steps each lane loads 8 bytes (4 groups) of its
// row's scales (h = 0) or biases (h = 1), shared across the lane halves by a permlane swap.
// The loads of step t are issued kD - 1 steps ahead, the x DMA last, so before step t an
// exact vmcnt (the younger steps' loads only) publishes its x tile; the barrier waits on
// LDS traffic only. Chunked scale loads matter: one 2-byte load per lane per step made the
// L2 serve ~7.8 M requests per 113 MB projection and cost 10%.
// Occupancy: three 4-wave blocks per CU (<= 168 VGPRs, a 4-deep ring of 32 KB) so that a
// configs[3] T=512 projection's 768 (item, weight tile) blocks run in one round. With two
// blocks per CU (8-deep ring) the second round ran on half the chip, and every block's first
// step waited ~5 us behind the whole launch's initial loads (per-block s_memrealtime stamps);
// a 4-deep ring measured no slower than the 8-deep one. The dequantize of step t + 1 is
// interleaved with step t's MFMAs (it needs registers only).
#include <algorithm>
#include <type_traits>

#include "dequant_bf16.h"
#include "mi_common.h"
#include "mi_internal.h"
#include "qmv_common.h"

namespace mi {
namespace {

using dq::dequant8;
using dq::pack_bf16x2;
using qmv_detail::decode_item;
using qmv_detail::Item;
using qmv_detail::item_x_row;
using qmv_detail::mfma32;
using qmv_detail::vmcnt_imm;

constexpr int kOOB = 0x7FFFFFF0;  // buffer offset past any x: the load returns 0, no traffic
constexpr int kD = 4;        // steps in flight: LDS ring of x tiles, register ring of weights
constexpr int kBufFlags = 0x00020000;

MI_DEV u32x4_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t,
                            __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// 16 bytes per lane from the buffer into LDS at lds + 16 * lane (LDS DMA)
MI_DEV void dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           (int)voff, (int)soff, 0, 0);
}
MI_DEV u32x2_t ld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

MI_DEV uint32_t xor32_u32(uint32_t v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (lane & 32) ? r[0] : r[1];
}

// DUAL (P.dual): the first WV / 2 waves run the gate bank (w, scales, biases) and the others
// the up bank (w2, scales2, biases2) on the same rows of both and the same x tile; the
// epilogue writes y = SwiGLU(gate, up) through LDS (each product rounded to bf16 first).
template <int MT, int WV, bool DUAL>
__global__ void __launch_bounds__(64 * WV, 12 / WV) gmm_kernel(QmvParams P) {
  constexpr int kWT = DUAL ? WV / 2 : WV;  // waves per weight bank
  constexpr int R = 32 * MT, kNT = 32 * kWT, kThreads = 64 * WV;
  // Dynamic LDS: the x ring (kD stages of R rows x 128 B), then the row table. (With a
  // static array the compiler would drain every load before each LDS read that may alias
  // an LDS DMA; the waits here are exact and explicit.)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int kStage = R * 128;
  int64_t* rowtab = reinterpret_cast<int64_t*>(smem + kD * kStage);
  // x DMA instructions per thread per step: R rows x 128 B over kThreads lanes x 16 B
  constexpr int XU = R * 8 / kThreads;
  static_assert(XU >= 1 && XU * kThreads == R * 8, "x tile must split evenly over the lanes");
  constexpr int kN = XU + 1;  // VMEM instructions per step: x DMA and weights (+1 per chunk)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, h = lane >> 5;
  const int N = P.N, K = P.K, G = K / 64, nsteps = K / 64;
  const int n0 = blockIdx.x * kNT;
  const int n_items = (int)*P.item_count;
  const int mw = DUAL ? wave % kWT : wave;     // the wave's 32-row tile in its bank
  const bool up = DUAL && wave >= kWT;          // wave-uniform
  const uint32_t wrow = (uint32_t)min(n0 + 32 * mw + fr, N - 1);
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)P.x, 0, (int)(uint32_t)(P.x_batch * P.M * (int64_t)K * 2), kBufFlags);

  for (int it_i = blockIdx.y; it_i < n_items; it_i += gridDim.y) {
    const Item it = decode_item(P, it_i);
    if (it.cnt <= 0) continue;  // block-uniform
    const uint32_t e = __builtin_amdgcn_readfirstlane(it.expert_ok ? it.expert : 0u);
    const bool eok = it.expert_ok;
    if (tid < R) rowtab[tid] = item_x_row(P, it, tid);  // -1 skip, -2 NaN
    __syncthreads();

    const size_t mat = (size_t)e * (uint32_t)N;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((up ? P.w2 : P.w) + mat * (uint32_t)(K / 8)), 0, N * (K / 2), kBufFlags);
    const uint32_t wo = wrow * (uint32_t)(K / 2) + 16 * h;
    // lane h = 0 loads its row's scales, h = 1 its biases, 4 groups (8 bytes) at a time; a
    // lane-half swap shares them
    const uint16_t* sbp = (h ? (up ? P.biases2 : P.biases) : (up ? P.scales2 : P.scales)) +
                          (mat + wrow) * (uint32_t)G;
    const int nch = (nsteps + 3) / 4;
    // x: DMA instruction i of wave w moves rows 8 (XU w + i) .. +7 (8 x 128 B); LDS slot
    // p of row r holds k-slot p ^ ((r >> 1) & 7). Rows outside the item read past the
    // end of x (zeros, no memory traffic).
    uint32_t xo[XU];
#pragma unroll
    for (int i = 0; i < XU; ++i) {
      const int r = 8 * (XU * wave + i) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int64_t ro = rowtab[r];
      xo[i] = ro >= 0 ? (uint32_t)ro * 2u + 16u * c : (uint32_t)kOOB;
    }

    u32x4_t wq[kD];
    u32x2_t sbc[4];  // scale/bias chunks: chunk c (steps 4c..4c+3) in slot c % 4
    // Step t's loads: its scale chunk when t starts one, its weights, then (last, so the
    // wait before a step counts only younger loads) its x DMA.
    auto issue = [&](int t, int slot, int cslot) __attribute__((always_inline)) {
      const uint32_t tt = (uint32_t)min(t, nsteps - 1);
      if ((t & 3) == 0)
        sbc[cslot] = *reinterpret_cast<const u32x2_t*>(sbp + 4 * min(t >> 2, nch - 1));
      wq[slot] = ld16(wres, wo, tt * 32u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < XU; ++i)
        dma16(xres, smem + slot * kStage + (XU * wave + i) * 1024, xo[i], tt * 128u);
      __builtin_amdgcn_sched_barrier(0);
    };

    f32x16_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

    if (eok) {
      // step t: wait for its DMA (issued kD - 1 steps earlier) and for step t + 1's weights,
      // barrier, then the MFMAs of step t with step t + 1's dequantize interleaved (it needs
      // registers only: the weight ring and the scale chunk), then issue step t + kD - 1
      // into the stage step t - 1 freed. Unrolled by 16 (four scale chunks) so every
      // register slot is static.
#pragma unroll
      for (int j = 0; j < kD - 1; ++j) issue(j, j, (j >> 2) & 3);
      // step j's scale and bias (group j % 4 of chunk slot (j / 4) % 4)
      auto scale_bias = [&](int j, float& sc, float& bp) __attribute__((always_inline)) {
        const u32x2_t mine = sbc[(j >> 2) & 3];
        const uint32_t mw = (j & 2) ? mine.y : mine.x;
        const uint32_t ow = xor32_u32(mw, lane);
        const uint32_t sw = h ? ow : mw, bw = h ? mw : ow;
        sc = __uint_as_float((j & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
        bp = __uint_as_float((j & 1) ? (bw & 0xFFFF0000u) : (bw << 16));
      };
      u32x4_t A[4];
      {
        // step 0's weights and scale chunk: everything after them may stay in flight
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(XU + (kD - 2) * kN + (kD - 2) / 4));
        float sc, bp;
        scale_bias(0, sc, bp);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) A[ks] = dequant8(wq[0][ks], sc, bp);
      }
      for (int t0 = 0; t0 < nsteps; t0 += 16) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int t = t0 + j, js = j % kD;
          // Done: every load of step t and step t + 1's scale chunk and weights. In flight:
          // step t + 1's x DMA and steps t + 2 .. t + kD - 2 (kN each plus one per scale
          // chunk they start). The barrier waits on LDS traffic only.
          constexpr int kAfter0 = XU + (kD - 3) * kN;
          const int starts = ((j + kD - 2) >> 2) - ((j + 1) >> 2);  // multiples of 4 in j+2..j+kD-2
          switch (starts) {
            case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAfter0)); break;
            case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAfter0 + 1)); break;
            default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAfter0 + 2)); break;
          }
          qmv_detail::lds_barrier();
          if (t < nsteps) {
            u32x4_t X[4][MT], An[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
              for (int i = 0; i < MT; ++i) {
                const int r = 32 * i + fr, c = 4 * h + ks;
                X[ks][i] = *reinterpret_cast<const u32x4_t*>(
                    smem + js * kStage + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
              }
            float sc, bp;
            scale_bias(j + 1, sc, bp);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) An[ks] = dequant8(wq[(j + 1) % kD][ks], sc, bp);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
              for (int i = 0; i < MT; ++i)
                acc[i] = mfma32(A[ks], X[ks][i], acc[i]);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) A[ks] = An[ks];
            // fragment reads first, then each MFMA with a slice of the next dequantize
            __builtin_amdgcn_sched_group_barrier(0x100, 4 * MT, 0);
#pragma unroll
            for (int m = 0; m < 4 * MT; ++m) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 84 / (4 * MT), 0);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          issue(t + kD - 1, (j + kD - 1) % kD, ((j + kD - 1) >> 2) & 3);
        }
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may outlive its stage
    }

    // epilogue: acc[i] register r is D[n = 32 mw + 8(r/4) + 4h + r%4][m = 32 i + fr]
    if constexpr (DUAL) {
      // gate products in columns [0, kNT) of an LDS tile, up products in [kNT, 2 kNT) (row
      // stride padded by 4 halves), then every thread takes 4 adjacent outputs of a row
      constexpr int kTS = 2 * kNT + 4;
      uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
      __syncthreads();  // every wave is done reading the x ring
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2_t o;
          o.x = pack_bf16x2(acc[i][4 * g], acc[i][4 * g + 1]);
          o.y = pack_bf16x2(acc[i][4 * g + 2], acc[i][4 * g + 3]);
          *reinterpret_cast<u32x2_t*>(tile + (32 * i + fr) * kTS + (up ? kNT : 0) + 32 * mw +
                                      8 * g + 4 * h) = o;
        }
      __syncthreads();
      constexpr int kPerRow = kNT / 4, kRowsPerPass = kThreads / kPerRow;
      const int c4 = tid % kPerRow;
      const int n = n0 + 4 * c4;
#pragma unroll 1
      for (int m = tid / kPerRow; m < R; m += kRowsPerPass) {
        const int64_t ro = rowtab[m];
        if (ro == -1 || n >= N) continue;
        const int64_t pos = it.pos0 + m;
        u32x2_t gv = *reinterpret_cast<const u32x2_t*>(tile + m * kTS + 4 * c4);
        u32x2_t uv = *reinterpret_cast<const u32x2_t*>(tile + m * kTS + kNT + 4 * c4);
        if (ro == -2 || !eok) gv.x = gv.y = uv.x = uv.y = 0x7FC07FC0u;  // NaN rows
        const uint32_t gw[2] = {gv.x, gv.y}, uw[2] = {uv.x, uv.y};
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t lo = swiglu_bf16((uint16_t)(gw[q] & 0xFFFFu), (uint16_t)(uw[q] & 0xFFFFu));
          const uint32_t hi = swiglu_bf16((uint16_t)(gw[q] >> 16), (uint16_t)(uw[q] >> 16));
          o[q] = lo | (hi << 16);
        }
        u32x2_t ov;
        ov.x = o[0];
        ov.y = o[1];
        *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(P.y) + pos * N + n) = ov;
      }
    } else if (P.swiglu_gate) {
      // SwiGLU epilogue through LDS: the bf16 products go to a [R][kNT] tile in the x ring
      // (row stride kNT + 4 halves, so the 32 rows one store instruction covers fall in
      // distinct banks), the accumulators die, and every thread then takes 4 adjacent
      // outputs of a row: coalesced gate reads and output writes, and the SwiGLU math
      // runs with the loop's registers free.
      constexpr int kTS = kNT + 4;
      uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
      __syncthreads();  // every wave is done reading the x ring
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2_t o;
          o.x = pack_bf16x2(acc[i][4 * g], acc[i][4 * g + 1]);
          o.y = pack_bf16x2(acc[i][4 * g + 2], acc[i][4 * g + 3]);
          *reinterpret_cast<u32x2_t*>(tile + (32 * i + fr) * kTS + 32 * mw + 8 * g + 4 * h) = o;
        }
      __syncthreads();
      constexpr int kPerRow = kNT / 4, kRowsPerPass = kThreads / kPerRow;
      const int c4 = tid % kPerRow;
      const int n = n0 + 4 * c4;
#pragma unroll 1
      for (int m = tid / kPerRow; m < R; m += kRowsPerPass) {
        const int64_t ro = rowtab[m];
        if (ro == -1 || n >= N) continue;
        const int64_t pos = it.pos0 + m;
        const u32x2_t gt = *reinterpret_cast<const u32x2_t*>(P.swiglu_gate + pos * N + n);
        u32x2_t pv = *reinterpret_cast<const u32x2_t*>(tile + m * kTS + 4 * c4);
        if (ro == -2 || !eok) pv.x = pv.y = 0x7FC07FC0u;  // NaN rows, as the plain path
        const uint32_t gw[2] = {gt.x, gt.y}, pw[2] = {pv.x, pv.y};
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t lo = swiglu_bf16((uint16_t)(gw[q] & 0xFFFFu), (uint16_t)(pw[q] & 0xFFFFu));
          const uint32_t hi = swiglu_bf16((uint16_t)(gw[q] >> 16), (uint16_t)(pw[q] >> 16));
          o[q] = lo | (hi << 16);
        }
        u32x2_t ov;
        ov.x = o[0];
        ov.y = o[1];
        *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(P.y) + pos * N + n) = ov;
      }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = 32 * i + fr;
        const int64_t ro = rowtab[m];
        if (ro == -1) continue;
        const int64_t pos = it.pos0 + m;
        const bool nan = ro == -2 || !eok;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + 32 * mw + 8 * g + 4 * h;
          if (n >= N) continue;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = nan ? __builtin_nanf("") : acc[i][4 * g + q];
          u32x2_t o;
          o.x = pack_bf16x2(v[0], v[1]);
          o.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(P.y) + pos * N + n) = o;
        }
      }
    }
    __syncthreads();  // the row table and the x ring are reused by the next item
  }
}

// x-stationary variant for short K: the item's 64 x rows, all of K, fit in LDS, so the block
// moves them once by LDS DMA and then streams NS passes of 32 WV weight rows each (the
// wave's 32 rows of every pass, one after another through one register ring) with no
// barrier and no DMA inside the loop. Row r of x sits at r * S (S = 2K bytes rounded up to
// 1 KB, one DMA instruction's span, plus 128 B so that consecutive rows start half the banks
// apart), k-step t at + 128 t, and slot p of a step holds k-slot p ^ ((r >> 1) & 7), as in
// the ring layout of gmm_kernel.
__host__ __device__ constexpr int xs_row_stride(int K) { return (K * 2 + 1023) / 1024 * 1024 + 128; }
#ifndef MI_GMM_XS_DEPTH
#define MI_GMM_XS_DEPTH 8
#endif
constexpr int kXsD = MI_GMM_XS_DEPTH;  // weight ring depth of the x-stationary kernel
static_assert(kXsD == 4 || kXsD == 8 || kXsD == 16, "the step loop unrolls by 16");

template <int WV>
__global__ void __launch_bounds__(64 * WV, 1) gmm_xs_kernel(QmvParams P, int NS) {
  constexpr int MT = 2, R = 64, kNT = 32 * WV;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int N = P.N, K = P.K, G = K / 64, nsteps = K / 64;
  const int S = xs_row_stride(K);
  int64_t* rowtab = reinterpret_cast<int64_t*>(smem + R * S);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, h = lane >> 5;
  const int n_items = (int)*P.item_count;
  const int slice0 = blockIdx.x * kNT * NS;
  const int npass = min(NS, (N - slice0 + kNT - 1) / kNT);
  const int total = npass * nsteps;
  const int nchunk = (nsteps + 7) / 8;  // 1 KB DMA spans per x row
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)P.x, 0, (int)(uint32_t)(P.x_batch * P.M * (int64_t)K * 2), kBufFlags);

  for (int it_i = blockIdx.y; it_i < n_items; it_i += gridDim.y) {
    const Item it = decode_item(P, it_i);
    if (it.cnt <= 0) continue;  // block-uniform
    const uint32_t e = __builtin_amdgcn_readfirstlane(it.expert_ok ? it.expert : 0u);
    const bool eok = it.expert_ok;
    if (tid < R) rowtab[tid] = item_x_row(P, it, tid);  // -1 skip, -2 NaN
    __syncthreads();
    const size_t mat = (size_t)e * (uint32_t)N;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.w + mat * (uint32_t)(K / 8)), 0, N * (K / 2), kBufFlags);
    const uint16_t* const sbase = (h ? P.biases : P.scales) + mat * (uint32_t)G;
    auto row_of = [&](int p) __attribute__((always_inline)) {
      return (uint32_t)min(slice0 + p * kNT + 32 * wave + fr, N - 1);
    };
    // the epilogue of pass p: acc[i] register r is D[n = 32 wave + 8(r/4) + 4h + r%4][m = 32 i + fr]
    // one accumulator set, k-steps in order: the ring kernel's summation order, so both
    // instances give the same bits
    auto store = [&](int p, const f32x16_t (&acc)[MT], bool all_nan) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = 32 * i + fr;
        const int64_t ro = rowtab[m];
        if (ro == -1) continue;
        const int64_t pos = it.pos0 + m;
        const bool nan = all_nan || ro == -2;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = slice0 + p * kNT + 32 * wave + 8 * g + 4 * h;
          if (n >= N) continue;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = nan ? __builtin_nanf("") : acc[i][4 * g + q];
          u32x2_t o;
          o.x = pack_bf16x2(v[0], v[1]);
          o.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(P.y) + pos * N + n) = o;
        }
      }
    };
    f32x16_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    if (!eok) {
      for (int p = 0; p < npass; ++p) store(p, acc, true);
      __syncthreads();
      continue;
    }
    // the item's x rows: DMA span j of row r holds k-steps 8j .. 8j + 7 (lanes past the
    // row's end or the item's rows read past x: zeros, no traffic)
    for (int q = wave; q < R * nchunk; q += WV) {
      const int r = q / nchunk, j = q - r * nchunk;
      const int step = 8 * j + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int64_t ro = rowtab[r];
      const uint32_t src = ro >= 0 && step < nsteps
                               ? (uint32_t)ro * 2u + (uint32_t)step * 128u + 16u * c
                               : (uint32_t)kOOB;
      dma16(xres, smem + r * S + j * 1024, src, 0u);
    }
    u32x4_t wq[kXsD];
    constexpr int kCS = kXsD / 4 + 1;  // scale/bias chunk slots: chunks in use or in flight
    u32x2_t sbc[4];  // the chunk of steps 4c..4c+3 in slot c % 4
    // flat step u = p * nsteps + t; nsteps % 4 == 0, so a chunk starts when u % 4 == 0
    auto issue = [&](int u, int slot, int cslot) __attribute__((always_inline)) {
      const int uu = min(u, total - 1);
      const int p = uu / nsteps, t = uu - p * nsteps;
      const uint32_t wr = row_of(p);
      if ((u & 3) == 0)
        sbc[cslot] = *reinterpret_cast<const u32x2_t*>(sbase + wr * (uint32_t)G + t);
      wq[slot] = ld16(wres, wr * (uint32_t)(K / 2) + 16 * h, (uint32_t)t * 32u);
    };
    auto scale_bias = [&](int j, float& sc, float& bp) __attribute__((always_inline)) {
      const u32x2_t mine = sbc[(j >> 2) & 3];
      const uint32_t mw = (j & 2) ? mine.y : mine.x;
      const uint32_t ow = xor32_u32(mw, lane);
      const uint32_t sw = h ? ow : mw, bw = h ? mw : ow;
      sc = __uint_as_float((j & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
      bp = __uint_as_float((j & 1) ? (bw & 0xFFFF0000u) : (bw << 16));
    };
#pragma unroll
    for (int j = 0; j < kXsD - 1; ++j) issue(j, j, (j >> 2) & 3);
    static_assert(kCS <= 4, "scale chunk ring");
    // every DMA of this wave is older than the ring's loads; then all waves' rows are in
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((kXsD - 1) + (kXsD - 2) / 4 + 1));
    __syncthreads();
    for (int u0 = 0; u0 < total; u0 += 16) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int u = u0 + j;
        // step u's weights and scale chunk are in once only the younger steps' loads
        // (u+1 .. u+kXsD-2, one each plus one per scale chunk they start) are in flight
        const int starts = ((j + kXsD - 2) >> 2) - (j >> 2);
        switch (starts) {
          case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kXsD - 2)); break;
          case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kXsD - 1)); break;
          case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kXsD)); break;
          case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kXsD + 1)); break;
          default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kXsD + 2)); break;
        }
        if (u < total) {
          const int p = u / nsteps, t = u - p * nsteps;
          // the 32-row tiles that hold rows of the item (MTI = 1: rows 32..63 are padding)
          auto compute = [&](auto mt_c) __attribute__((always_inline)) {
            constexpr int MTI = decltype(mt_c)::value;
            u32x4_t X[4][MTI], A[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
              for (int i = 0; i < MTI; ++i) {
                const int r = 32 * i + fr, c = 4 * h + ks;
                X[ks][i] = *reinterpret_cast<const u32x4_t*>(smem + r * S + t * 128 +
                                                             ((c ^ ((r >> 1) & 7)) << 4));
              }
            float sc, bp;
            scale_bias(j, sc, bp);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) A[ks] = dequant8(wq[j % kXsD][ks], sc, bp);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
              for (int i = 0; i < MTI; ++i) acc[i] = mfma32(A[ks], X[ks][i], acc[i]);
          };
          compute(std::integral_constant<int, 2>{});
          if (t == nsteps - 1) {
            store(p, acc, false);
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
          }
        }
        issue(u + kXsD - 1, (j + kXsD - 1) % kXsD, ((j + kXsD - 1) >> 2) & 3);
      }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();  // the row table and the x rows are reused by the next item
  }
}

}  // namespace

bool gmm_supported(int64_t N, int64_t K, int bits, int gs, int x_f32, int64_t x_bytes) {
  // whole 64-wide steps; scale chunks of 4 groups on an 8-byte boundary; 4-output stores;
  // 32-bit buffer offsets
  return bits == 4 && gs == 64 && !x_f32 && K % 256 == 0 && N % 4 == 0 && N >= 4 &&
         N * (K / 2) < ((int64_t)1 << 31) && x_bytes + 2 * K < ((int64_t)1 << 31);
}

template <int MT, int WV, bool DUAL>
hipError_t launch_mt(const QmvParams& P, int grid_items, hipStream_t s) {
  const size_t lds = (size_t)kD * 32 * MT * 128 + 32 * MT * sizeof(int64_t);
  static bool attr = false;
  if (!attr) {
    auto k = gmm_kernel<MT, WV, DUAL>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  constexpr int kNT = 32 * (DUAL ? WV / 2 : WV);
  const dim3 grid((unsigned)((P.N + kNT - 1) / kNT), (unsigned)std::max(1, grid_items));
  hipLaunchKernelGGL((gmm_kernel<MT, WV, DUAL>), grid, dim3(64 * WV), lds, s, P);
  return hipGetLastError();
}

bool gmm_xs_fits(int64_t K) { return (int64_t)64 * xs_row_stride((int)K) + 512 <= 160 * 1024; }

hipError_t launch_gmm_xs(const QmvParams& P, int ns, int grid_items, hipStream_t s) {
  constexpr int WV = 8, kNT = 32 * WV;
  if (!P.items || !P.item_count || P.dual || P.swiglu_gate || !gmm_xs_fits(P.K) || ns < 1)
    return hipErrorInvalidValue;
  const size_t lds = (size_t)64 * xs_row_stride(P.K) + 64 * sizeof(int64_t);
  static size_t attr = 0;
  if (attr < lds) {
    hipError_t e = hipFuncSetAttribute((const void*)gmm_xs_kernel<WV>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr = lds;
  }
  const dim3 grid((unsigned)((P.N + kNT * ns - 1) / (kNT * ns)), (unsigned)std::max(1, grid_items));
  hipLaunchKernelGGL(gmm_xs_kernel<WV>, grid, dim3(64 * WV), lds, s, P, ns);
  return hipGetLastError();
}

hipError_t launch_gmm(const QmvParams& P, int mt, int grid_items, hipStream_t s) {
  if (!P.items || !P.item_count) return hipErrorInvalidValue;
  // 4 waves (128 weight rows) a block, three blocks a CU: 256-row blocks of 8 waves measured
  // 233 against 216 us per configs[3] T=512 layer (two blocks a CU then)
  if (P.dual && (!P.w2 || !P.scales2 || !P.biases2)) return hipErrorInvalidValue;
  switch (mt * 2 + (P.dual ? 1 : 0)) {
    case 2: return launch_mt<1, 4, false>(P, grid_items, s);
    case 3: return launch_mt<1, 4, true>(P, grid_items, s);
    case 4: return launch_mt<2, 4, false>(P, grid_items, s);
    case 5: return launch_mt<2, 4, true>(P, grid_items, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mi
