// Few-row decode GEMM, 4- or 8-bit affine gs 64, bf16 activations, on the 16x16x32 bf16 MFMA:
// dense quantized_matmul (2 <= M <= 64; above 32 rows in two 32-row passes over the
// weights held in registers) and gather_qmm work items of 2..32 rows (sorted expert runs). The weights stream straight into registers the way the one-row kernel
// streams them (no LDS copy of the weights).
//
// Bias-less fp4 modes (FPM 0 nvfp4: e2m1 codes, 16-value groups, e4m3 scales; FPM 1 mxfp4:
// 32-value groups, e8m0 scales) share the 4-bit chunk layout and transpose. Their group
// scale is exact in the product: each 8-code run converts to bf16 pairs of code x scale
// (v_cvt_scalef32_pk_bf16_fp4), so the MFMA accumulates across groups with no epilogue,
// no all-ones MFMA and no scale staging; the activations stay in natural order. A lane's
// scales come with its weight chunk (one dword per 128 codes for mxfp4, two for nvfp4).
//
// Affine 2/3/5/6-bit weights (FPM 100 + bits) keep the 4-bit instances' k mapping (step t
// = codes 32t..32t+31 of a 128-code chunk, lane block q = codes 32t + 8q..+7) and their
// affine epilogue; only the loads and the unpack differ. A row is one LSB-first bitstream,
// so a lane's 8 codes are `bits` bytes at byte 4t bits + q bits of the chunk: one 8-byte
// load from the dword below them covers them at every width, and the codes come out of
// a 64-bit shift as bf16 0x43qq (= 128 + q) pairs in natural order.
//
// Block = WR weight tiles of 16 rows x one K range (x one work item for gathers); its W
// waves are WR x WK: wave (rt, kp) owns tile rt and the kp-th run of NC 128-value chunks
// of the range. The block stages the range's activations (its rows, nibble-pair order)
// and the tiles' scale/bias pairs into LDS once; every wave reads them from there. A
// gather block first resolves its item's activation rows (sorted runs keep only the rows
// whose pair maps to the item's expert) into a small LDS table.
//
// Loads: lane l of a wave reads 16 B of weight row l%16 at byte 16*(l/16) of each
// 64-byte chunk (one b128 per chunk; 16 rows x 64 contiguous bytes per instruction),
// DEPTH chunks ahead. After two permlane swaps (a 4x4 dword transpose across the four
// 16-lane rows) lane l holds, in register t, dword l/16 of the 32-value run t of its row,
// so each MFMA step covers one run of 32 consecutive values, inside one group.
//
// MFMA (16x16x32 bf16) layout: lane l holds 8 k values of A row l%16 / B column l%16 for
// k block l/16; C lane l register r is row 4(l/16)+r, column l%16. A = weights as bf16
// 0x43qq (= 128+q exactly, v_perm against 0x43 bytes), k order [0,2,4,6,1,3,5,7] per 8;
// B = activations staged in that same order; C = sum x*(128+q) for one group, to which
// the group's affine terms are applied in fp32: s*C + (b - 128 s)*X, X = sum of x over
// the group, from a second MFMA of the same B against an all-ones A. Columns are
// activation rows (16 per MFMA; more than 16 rows run a second MFMA on rows 16..31).
// 8-bit weights: a 64-byte chunk is 64 values, exactly one group of 64, so no transpose is
// needed: step t takes words 2t, 2t+1 of the lane's 16 bytes as exact bf16 bytes q, the
// activations stay in natural order and the group adds s*C + b*X.
//
// The waves' partial sums of a tile are added in wave order through LDS; K ranges beyond
// one (activations too large for LDS) write fp32 partials that a second kernel sums in
// range order. Every sum has a fixed order: results are deterministic.
#pragma once
#include "qmv_common.h"
#include "code_runs.h"

#include <cstdint>
#include <type_traits>

namespace mi {
namespace qmvm_detail {

using qmv_detail::decode_item;
using qmv_detail::item_x_row;
using qmv_detail::Item;
using qmv_detail::lds_barrier;

using code_runs::bf16x2v;
using code_runs::f32x2v;
using code_runs::fp4_run;
using code_runs::fp4_run_e4m3;
using code_runs::fp_e4m3;
using code_runs::odd_run;
using code_runs::fp8_run;

typedef __bf16 bf16x8m __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2m __attribute__((ext_vector_type(2)));

constexpr int kChunkVals = 128;
constexpr int kBufFlags = 0x00020000;  // raw (untyped) dword buffer access on this target
constexpr uint32_t kOOB = 0x7FFFFFF0u;  // buffer offset past any resource: the load returns 0
constexpr int kMaxRows = 64;

MI_DEV f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8m, a),
                                                  __builtin_bit_cast(bf16x8m, b), c, 0, 0, 0);
}

// 8 nibbles -> bf16 pairs (128+q0, 128+q2), (q4, q6), (q1, q3), (q5, q7).
MI_DEV u32x4_t unpack8(uint32_t w) {
  constexpr uint32_t c43 = 0x43434343u;
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  return u32x4_t{perm_b32(c43, lo, 0x04010400u), perm_b32(c43, lo, 0x04030402u),
                 perm_b32(c43, hi, 0x04010400u), perm_b32(c43, hi, 0x04030402u)};
}

// 8 bytes (two words) -> bf16 pairs (q0, q1), (q2, q3), (q4, q5), (q6, q7), exact.
MI_DEV uint32_t pk_bf16(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2m));
}
template <int k>
MI_DEV float ubyte_f(uint32_t w) { return (float)((w >> (8 * k)) & 0xFFu); }
MI_DEV u32x4_t unpack8b(uint32_t w0, uint32_t w1) {
  return u32x4_t{pk_bf16(ubyte_f<0>(w0), ubyte_f<1>(w0)), pk_bf16(ubyte_f<2>(w0), ubyte_f<3>(w0)),
                 pk_bf16(ubyte_f<0>(w1), ubyte_f<1>(w1)), pk_bf16(ubyte_f<2>(w1), ubyte_f<3>(w1))};
}

// 4x4 transpose of dwords across the four 16-lane rows of the wave: on return, register
// t of row q holds what register q of row t held.
MI_DEV u32x4_t xpose4(u32x4_t v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  return u32x4_t{c[0], c[1], d[0], d[1]};
}

MI_DEV float lo_bf16(uint32_t v) { return __uint_as_float(v << 16); }
MI_DEV float hi_bf16(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// LDS plan of one block, shared by the kernel and the host.
struct QmvmLds {
  int xstride;  // bytes per staged activation row
  int xbytes, sbbytes, redbytes;
  __host__ __device__ int total() const {
    const int a = xbytes + sbbytes;
    return a > redbytes ? a : redbytes;
  }
};

// Row stride (in (group, row) entries) of the staged scale/bias table: padded past the
// block's rows so that the staging writes of one row's consecutive groups, 2 x stride words
// apart, fall in different banks (a multiple of 64 words put them all in one bank), while
// the 16-byte reads of 4 rows stay aligned.
__host__ __device__ inline int qmvm_sb_stride(int rows, bool sbf32) { return rows + (sbf32 ? 2 : 4); }

__host__ __device__ inline QmvmLds qmvm_lds(int M, int nvals, int gs, int rows, int waves, int mt,
                                            bool sbf32) {
  QmvmLds L;
  L.xstride = nvals * 2 + 16;  // +16 B: the 16 rows of a B read start in different banks
  L.xbytes = M * L.xstride;
  // per group and row: fp32 (s, b - 128 s), or the bf16 pair (s, b) when LDS is tight
  L.sbbytes = (nvals / gs) * qmvm_sb_stride(rows, sbf32) * (sbf32 ? 8 : 4);
  L.redbytes = waves * 16 * mt * 4;
  return L;
}

// G is read only by gathers (work items, index arrays, expert bank); dense calls pass
// their shapes in P.
template <int BITS, int GS, int NC, int XU, int DEPTH, int MT, bool SBF32, bool GATHER, int FPM = -1>
// MT 64 keeps four accumulator tiles and the second pass's activations in registers:
// blocks of up to 8 waves (256 VGPRs per lane) instead of 16.
__global__ void __launch_bounds__(MT == 64 ? 512 : 1024) qmvm_kernel(QmvmParams P, QmvParams Gp) {
  constexpr bool FP4 = FPM >= 0 && FPM < 100;  // any bias-less fp mode (the name predates mxfp8)
  constexpr bool ODD = FPM >= 100;             // affine 2/3/5/6 bits, 4-bit chunk layout
  constexpr int OB = ODD ? FPM - 100 : 0;
  static_assert(!FP4 || (BITS == (FPM == 2 ? 8 : 4) && MT <= 32),
                "fp modes: 4-bit (nvfp4, mxfp4) or 8-bit (mxfp8) codes, at most 32 rows");
  static_assert(!ODD || (BITS == 4 && MT <= 32 && (OB == 2 || OB == 3 || OB == 5 || OB == 6)),
                "odd widths: 2/3/5/6 bits on the 4-bit layout, at most 32 rows");
  constexpr int WB = ODD ? OB : BITS;  // stored bits per code
  constexpr int FGS = FPM == 0 ? 16 : 32;  // fp group size
  constexpr int CV = 512 / BITS;        // values per 64-byte chunk of a row
  constexpr int NSTEP = CV / 32;        // MFMA steps per chunk
  constexpr float BOFF = BITS == 4 ? -128.f : 0.f;  // 4-bit A holds 128 + q
  constexpr int SPG = GS / 32;  // 32-value MFMA steps per group
  // MT 64 loads every chunk up front: its pass loop then issues no loads
  constexpr int D = MT == 64 ? NC : DEPTH < NC ? DEPTH : NC;
  constexpr int GPC = CV / GS;  // groups per chunk (GS <= CV)
  constexpr int SBW = SBF32 ? 2 : 1;    // LDS words per (group, row)
  constexpr int SU = 4;                 // scale/bias loads per thread
  constexpr bool PAIRS = GS <= 64;      // scale/bias as dwords (two groups) or halves
  // MT 64: the activation rows are staged 32 at a time (two passes over the wave's
  // chunks, weights kept in registers), so LDS holds at most 32 rows.
  constexpr int MP = MT == 64 ? 32 : MT;  // rows per pass
  constexpr int NPASS = MT / MP;
  constexpr int NTP = MP / 16;            // 16-column MFMA tiles per pass
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int64_t rowtab[kMaxRows];  // gathers: element offset of each item row's x
  const int tid = threadIdx.x, BD = blockDim.x, W = BD >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int WR = P.wr;
  const int rt = wave % WR, kp = wave / WR;
  const int i = lane & 15, q = lane >> 4;
  const int N = P.N, K = P.K, G = K / (FP4 ? FGS : GS);
  const int kb0 = blockIdx.y * P.kr;
  const int nvals = min(K - kb0, P.kr);
  const int gr = nvals / GS, g0 = kb0 / GS;
  const int rows = 16 * WR;
  const int rs = qmvm_sb_stride(rows, SBF32);  // staged scale/bias row stride
  const int row0 = blockIdx.x * rows;
  const int upr = nvals / 8;  // staging units per activation row
  const int spr = PAIRS ? gr / 2 : gr;  // scale/bias loads per row
  const int c0 = kp * NC;     // first chunk of this wave within the range
  const int64_t PT = GATHER ? Gp.n_pairs * Gp.M : 0;
  const int n_items = GATHER ? (Gp.items ? (int)*Gp.item_count : Gp.n_items_fixed) : 1;

  for (int it_i = GATHER ? (int)blockIdx.z : 0; it_i < n_items;
       it_i += GATHER ? (int)gridDim.z : 1) {
    int M = P.M;
    uint32_t e = 0;
    bool eok = true;
    int64_t pos0 = 0;
    if constexpr (GATHER) {
      const Item it = decode_item(Gp, it_i);
      if (it.cnt <= 0) continue;  // block-uniform
      M = min(it.cnt, MT);
      e = __builtin_amdgcn_readfirstlane(it.expert_ok ? it.expert : 0u);
      eok = it.expert_ok;
      pos0 = it.pos0;
      if (wave == 0 && lane < M) rowtab[lane] = item_x_row(Gp, it, lane);  // -1 skip, -2 NaN
    }
    const int Mp0 = min(M, MP);  // rows of the first pass
    const QmvmLds L = qmvm_lds(Mp0, nvals, GS, rows, W, MT, SBF32);
    unsigned char* xs = smem;
    float* sb = reinterpret_cast<float*>(smem + L.xbytes);
    float* red = reinterpret_cast<float*>(smem);  // reused after the dot products

    const size_t mat = (size_t)e * (uint32_t)N;
    const uint32_t xbytes_all =
        GATHER ? (uint32_t)(Gp.x_batch * Gp.M * (int64_t)K * 2) : (uint32_t)(M * K * 2);
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void*)P.x, (short)0, xbytes_all, kBufFlags);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.w + mat * (uint32_t)(K * WB / 32)), (short)0, N * (K * WB / 8), kBufFlags);
    const __amdgpu_buffer_rsrc_t sres =
        FP4 ? __builtin_amdgcn_make_buffer_rsrc(
                  (void*)((const unsigned char*)P.scales + mat * (uint32_t)G), (short)0, N * G,
                  kBufFlags)
            : __builtin_amdgcn_make_buffer_rsrc((void*)(P.scales + mat * (uint32_t)G), (short)0,
                                                N * G * 2, kBufFlags);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.biases + mat * (uint32_t)G), (short)0, N * G * 2, kBufFlags);

    // 1. loads. Dense: activations, scale/bias, then the first D chunks (nothing waits
    //    before all are issued). Gather: the chunks and scale/bias first, then (after the
    //    row table is visible) the activations.
    u32x4_t xv[XU];
    auto load_x = [&](int pass) __attribute__((always_inline)) {
      const int mb = pass * MP, Mp = min(M - mb, MP);
#pragma unroll
      for (int t = 0; t < XU; ++t) {
        const int u = tid + t * BD;
        const int m = (int)__umulhi((uint32_t)u, P.upr_mr), k8 = u - m * upr;
        uint32_t off = kOOB;
        if constexpr (GATHER) {
          const int64_t ro = m < Mp ? rowtab[mb + m] : -1;
          if (ro >= 0) off = (uint32_t)(ro + kb0 + 8 * k8) * 2;
        } else {
          if (m < Mp) off = (uint32_t)((mb + m) * K + kb0 + 8 * k8) * 2;
        }
        xv[t] = __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0);
      }
    };
    if constexpr (!GATHER) load_x(0);
    uint32_t sv[SU], bv[SU];
#pragma unroll
    for (int t = 0; t < (FP4 ? 0 : SU); ++t) {
      const int v = tid + t * BD;
      const int rr = spr == 1 ? v : (int)__umulhi((uint32_t)v, P.spr_mr), gp = v - rr * spr;
      const bool ok = rr < rows && row0 + rr < N;
      if constexpr (PAIRS) {
        const uint32_t off = ok ? (uint32_t)((row0 + rr) * G + g0 + 2 * gp) * 2 : kOOB;
        sv[t] = __builtin_amdgcn_raw_buffer_load_b32(sres, off, 0, 0);
        bv[t] = __builtin_amdgcn_raw_buffer_load_b32(bres, off, 0, 0);
      } else {
        const uint32_t off = ok ? (uint32_t)((row0 + rr) * G + g0 + gp) * 2 : kOOB;
        sv[t] = __builtin_amdgcn_raw_buffer_load_b16(sres, off, 0, 0);
        bv[t] = __builtin_amdgcn_raw_buffer_load_b16(bres, off, 0, 0);
      }
    }
    const int wrow = min(row0 + rt * 16 + i, N - 1);
    const uint32_t wo = ODD ? (uint32_t)wrow * (uint32_t)(K * WB / 8) +
                                  (uint32_t)(kb0 + c0 * CV) * WB / 8 + ((uint32_t)(q * OB) & ~3u)
                            : (uint32_t)wrow * (uint32_t)(K * BITS / 8) +
                                  (uint32_t)(kb0 + c0 * CV) * BITS / 8 + 16 * q;
    const uint32_t osh = (uint32_t)(q * OB & 3) * 8;  // odd widths: bits below the lane's codes
    u32x4_t wv[NC], wv2[NC];  // odd widths: steps 0, 1 in wv and 2, 3 in wv2 (two dwords each)
    auto load_w = [&](int j) __attribute__((always_inline)) {
      if constexpr (ODD) {
        const uint32_t o = wo + 16 * OB * j;  // a chunk is 128 codes = 16 OB bytes
        auto ld = [&](int t) {
          return __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wres, o + 4 * OB * t, 0, 0));
        };
        const u32x2_t s0 = ld(0), s1 = ld(1), s2 = ld(2), s3 = ld(3);
        wv[j] = u32x4_t{s0.x, s0.y, s1.x, s1.y};
        wv2[j] = u32x4_t{s2.x, s2.y, s3.x, s3.y};
      } else {
        wv[j] = __builtin_amdgcn_raw_buffer_load_b128(wres, wo + 64 * j, 0, 0);
      }
    };
    // fp scales of the lane's row for chunk j: bytes (4 for mxfp4, 8 for nvfp4, 2 for mxfp8)
    constexpr int SPC = FPM == 0 ? 8 : FPM == 1 ? 4 : 2;
    const uint32_t fso = (uint32_t)wrow * (uint32_t)G + (uint32_t)(kb0 + c0 * CV) / FGS;
    u32x2_t fsw[NC];
    auto load_fs = [&](int j) __attribute__((always_inline)) {
      if constexpr (FPM == 0) {
        fsw[j] = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(sres, fso + SPC * j, 0, 0));
      } else if constexpr (FPM == 1) {
        fsw[j].x = __builtin_amdgcn_raw_buffer_load_b32(sres, fso + SPC * j, 0, 0);
      } else if constexpr (FPM == 2) {
        fsw[j].x = __builtin_amdgcn_raw_buffer_load_b16(sres, fso + SPC * j, 0, 0);
      }
    };
#pragma unroll
    for (int j = 0; j < D; ++j) {
      load_w(j);
      load_fs(j);
    }
    if constexpr (GATHER) {
      lds_barrier();  // the row table
      load_x(0);
    }

    // 2. stage activations (pair order) and scale/bias pairs.
    auto stage_x = [&](int Mp) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < XU; ++t) {
      const int u = tid + t * BD;
      const int m = (int)__umulhi((uint32_t)u, P.upr_mr), k8 = u - m * upr;
      const u32x4_t X = xv[t];
      if (m < Mp) {
        u32x4_t p = X;  // 8-bit, fp modes and odd widths: natural order
        if constexpr (BITS == 4 && !FP4 && !ODD) {
          p.x = perm_b32(X.y, X.x, 0x05040100u);  // (x0, x2)
          p.y = perm_b32(X.w, X.z, 0x05040100u);  // (x4, x6)
          p.z = perm_b32(X.y, X.x, 0x07060302u);  // (x1, x3)
          p.w = perm_b32(X.w, X.z, 0x07060302u);  // (x5, x7)
        }
        *reinterpret_cast<u32x4_t*>(xs + m * L.xstride + k8 * 16) = p;
      }
    }
    };
    stage_x(Mp0);
#pragma unroll
    for (int t = 0; t < (FP4 ? 0 : SU); ++t) {
      const int v = tid + t * BD;
      const int rr = spr == 1 ? v : (int)__umulhi((uint32_t)v, P.spr_mr), gp = v - rr * spr;
      if (rr < rows) {
        if constexpr (!SBF32) {
          uint32_t* sbu = reinterpret_cast<uint32_t*>(sb);
          if constexpr (PAIRS) {
            sbu[(2 * gp) * rs + rr] = perm_b32(bv[t], sv[t], 0x05040100u);
            sbu[(2 * gp + 1) * rs + rr] = perm_b32(bv[t], sv[t], 0x07060302u);
          } else {
            sbu[gp * rs + rr] = (sv[t] & 0xFFFFu) | (bv[t] << 16);
          }
        } else if constexpr (PAIRS) {
          const float s0 = lo_bf16(sv[t]), s1 = hi_bf16(sv[t]);
          *reinterpret_cast<f32x2_t*>(sb + 2 * ((2 * gp) * rs + rr)) =
              f32x2_t{s0, fmaf(BOFF, s0, lo_bf16(bv[t]))};
          *reinterpret_cast<f32x2_t*>(sb + 2 * ((2 * gp + 1) * rs + rr)) =
              f32x2_t{s1, fmaf(BOFF, s1, hi_bf16(bv[t]))};
        } else {
          const float s0 = lo_bf16(sv[t]);
          *reinterpret_cast<f32x2_t*>(sb + 2 * (gp * rs + rr)) =
              f32x2_t{s0, fmaf(BOFF, s0, lo_bf16(bv[t]))};
        }
      }
    }
    lds_barrier();

    // 3. MFMA over the wave's chunks as they land (pass 0); pass 1 of MT 64 reuses the
    //    weights held in registers against the next 32 staged rows.
    // 4-bit: lane block q of step t is values 32t + 8q.. of the chunk (after the
    // transpose); 8-bit: values 16q + 8t.. (two words of the lane's own 16 bytes)
    constexpr int QB = BITS == 4 ? 16 : 32;  // bytes between the lane blocks of a row
    // A operand of ones (bf16 1.0 = 0x3F80): ones x B puts each column's group sum X in
    // every row of C, i.e. in the accumulator layout of the outputs
    const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    f32x4_t acc[NTP];
    auto mfma_pass = [&](int Mp) __attribute__((always_inline)) {
#pragma unroll
      for (int tt = 0; tt < NTP; ++tt) acc[tt] = zero;
      const unsigned char* xrow[NTP];
#pragma unroll
      for (int tt = 0; tt < NTP; ++tt) xrow[tt] = xs + min(16 * tt + i, Mp - 1) * L.xstride + QB * q;
      // per-group pointer, stepped by one group at a time (no multiplies in the loop)
      const float* sbp = sb + SBW * ((c0 * GPC) * rs + rt * 16 + 4 * q);
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        if constexpr (D < NC) {
          if (j + D < NC) {
            load_w(j + D);
            load_fs(j + D);
          }
        }
        const u32x4_t tw = BITS == 4 && !ODD ? xpose4(wv[j]) : wv[j];
        const int kc = (c0 + j) * CV;  // chunk start within the range
        if constexpr (FPM == 2) {
          // step t: words 2t, 2t+1 of the lane's 16 bytes, codes 16q + 8t .. + 7 of the
          // chunk, all in group q/2 (byte q/2 of the chunk's two scale bytes)
          const float sc = __uint_as_float(((fsw[j].x >> (8 * (q >> 1))) & 0xFFu) << 23);
#pragma unroll
          for (int t = 0; t < NSTEP; ++t) {
            const uint32_t w0 = t == 0 ? tw.x : tw.z, w1 = t == 0 ? tw.y : tw.w;
            const u32x4_t a = fp8_run(w0, w1, sc);
            const int kb = (kc + 8 * t) * 2;
#pragma unroll
            for (int tt = 0; tt < NTP; ++tt) {
              const u32x4_t b = *reinterpret_cast<const u32x4_t*>(xrow[tt] + kb);
              acc[tt] = mfma16(a, b, acc[tt]);
            }
          }
          if constexpr (D < NC) __builtin_amdgcn_sched_barrier(0);
          continue;
        }
        if constexpr (FP4) {
          // run t holds codes 32t + 8q .. + 7 of the chunk: mxfp4 group t (byte t of the
          // dword), nvfp4 group 2t + q/2 (byte 2t + q/2 of the two dwords)
#pragma unroll
          for (int t = 0; t < NSTEP; ++t) {
            const uint32_t codes = t == 0 ? tw.x : t == 1 ? tw.y : t == 2 ? tw.z : tw.w;
            u32x4_t a;
            if constexpr (FPM == 0) {
              const uint32_t word = t < 2 ? fsw[j].x : fsw[j].y;
              a = fp4_run_e4m3(codes, fp_e4m3((word >> (8 * (2 * (t & 1) + (q >> 1)))) & 0xFFu));
            } else {
              a = fp4_run(codes, __uint_as_float(((fsw[j].x >> (8 * t)) & 0xFFu) << 23));
            }
            const int kb = (kc + 32 * t) * 2;
#pragma unroll
            for (int tt = 0; tt < NTP; ++tt) {
              const u32x4_t b = *reinterpret_cast<const u32x4_t*>(xrow[tt] + kb);
              acc[tt] = mfma16(a, b, acc[tt]);
            }
          }
          if constexpr (D < NC) __builtin_amdgcn_sched_barrier(0);
          continue;
        }
        f32x4_t c[NTP], cx[NTP];
#pragma unroll
        for (int tt = 0; tt < NTP; ++tt) c[tt] = cx[tt] = zero;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
          u32x4_t a;
          if constexpr (ODD) {
            const u32x4_t& h = t < 2 ? wv[j] : wv2[j];
            a = (t & 1) ? odd_run<OB>(h.z, h.w, osh) : odd_run<OB>(h.x, h.y, osh);
          } else if constexpr (BITS == 4) {
            a = unpack8(t == 0 ? tw.x : t == 1 ? tw.y : t == 2 ? tw.z : tw.w);
          } else {
            a = t == 0 ? unpack8b(tw.x, tw.y) : unpack8b(tw.z, tw.w);
          }
          const int kb = (kc + (BITS == 4 ? 32 : 8) * t) * 2;  // byte offset in a staged row
          // every column tile runs (rows past the pass's end repeat its last row and are
          // never written): no branches inside the unrolled chunk loop
#pragma unroll
          for (int tt = 0; tt < NTP; ++tt) {
            const u32x4_t b = *reinterpret_cast<const u32x4_t*>(xrow[tt] + kb);
            c[tt] = mfma16(a, b, t % SPG == 0 ? zero : c[tt]);
            cx[tt] = mfma16(ones, b, t % SPG == 0 ? zero : cx[tt]);
          }
          if (t % SPG == SPG - 1) {
            f32x4_t sb01, sb23;  // (s, b - 128 s) of rows 4q, 4q+1 and 4q+2, 4q+3
            if constexpr (SBF32) {
              sb01 = *reinterpret_cast<const f32x4_t*>(sbp);
              sb23 = *reinterpret_cast<const f32x4_t*>(sbp + 4);
            } else {
              const u32x4_t ev = *reinterpret_cast<const u32x4_t*>(sbp);
              sb01.x = lo_bf16(ev.x);
              sb01.y = fmaf(BOFF, sb01.x, hi_bf16(ev.x));
              sb01.z = lo_bf16(ev.y);
              sb01.w = fmaf(BOFF, sb01.z, hi_bf16(ev.y));
              sb23.x = lo_bf16(ev.z);
              sb23.y = fmaf(BOFF, sb23.x, hi_bf16(ev.z));
              sb23.z = lo_bf16(ev.w);
              sb23.w = fmaf(BOFF, sb23.z, hi_bf16(ev.w));
            }
            sbp += SBW * rs;
#pragma unroll
            for (int tt = 0; tt < NTP; ++tt) {
              f32x4_t& ac = acc[tt];
              const float X = cx[tt][0];
              ac[0] = fmaf(sb01.x, c[tt][0], fmaf(sb01.y, X, ac[0]));
              ac[1] = fmaf(sb01.z, c[tt][1], fmaf(sb01.w, X, ac[1]));
              ac[2] = fmaf(sb23.x, c[tt][2], fmaf(sb23.y, X, ac[2]));
              ac[3] = fmaf(sb23.z, c[tt][3], fmaf(sb23.w, X, ac[3]));
            }
          }
        }
        if constexpr (D < NC) __builtin_amdgcn_sched_barrier(0);  // keep the issue order
      }
    };
    // red[kp][rt][col][row16] : lane holds rows 4q..4q+3 of column i
    auto write_red = [&](const f32x4_t* a, int col0) __attribute__((always_inline)) {
#pragma unroll
      for (int tt = 0; tt < NTP; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[((kp * WR + rt) * MT + col0 + 16 * tt + i) * 16 + 4 * q + r] = a[tt][r];
    };
    if constexpr (NPASS == 1) {
      mfma_pass(Mp0);
      // 4. sum the WK waves of each tile in wave order, write y (or the range's partial).
      lds_barrier();  // LDS reads of step 3 are done: reuse it
      write_red(acc, 0);
    } else {
      // Two passes of 32 rows over the weights held in registers (a runtime branch, so
      // the compiler keeps no per-chunk state of the first pass for the second); the
      // second pass's activations are in flight while the first computes.
      const bool two = M > MP;  // block-uniform
      if (two) load_x(1);
      mfma_pass(Mp0);
      f32x4_t first[NTP];
#pragma unroll
      for (int tt = 0; tt < NTP; ++tt) first[tt] = acc[tt];
      if (two) {
        lds_barrier();  // the first pass's reads of the staged rows are done
        stage_x(M - MP);
        lds_barrier();
        mfma_pass(M - MP);
      }
      lds_barrier();  // LDS reads of step 3 are done: reuse it
      write_red(first, 0);
      if (two) write_red(acc, MP);
    }
    lds_barrier();
    const int WK = W / WR;
    const int nout = rows * M;
    for (int o = tid; o < nout; o += BD) {
      const int m = o / rows, rr = o - m * rows;  // consecutive threads: consecutive rows
      const int t2 = rr >> 4, r16 = rr & 15;
      const int n = row0 + rr;
      if (n >= N) continue;
      float v = 0.f;
      for (int k2 = 0; k2 < WK; ++k2) v += red[((k2 * WR + t2) * MT + m) * 16 + r16];
      int64_t pos = m;
      if constexpr (GATHER) {
        const int64_t ro = rowtab[m];
        if (ro == -1) continue;  // this row belongs to another item
        if (ro == -2 || !eok) v = __builtin_nanf("");
        pos = pos0 + m;
      }
      if (gridDim.y > 1) {
        const int64_t npos = GATHER ? PT : M;
        P.part[((int64_t)blockIdx.y * npos + pos) * N + n] = v;
      } else {
        uint16_t o = (uint16_t)f32_to_bf16_bits(v);
        if constexpr (GATHER) {
          if (Gp.swiglu_gate) o = swiglu_bf16(Gp.swiglu_gate[pos * N + n], o);
        }
        P.y[pos * N + n] = o;
      }
    }
    if constexpr (GATHER) lds_barrier();  // LDS and the row table are reused by the next item
  }
}

// Launches one instance family; explicitly instantiated per (MT, SBF32, GATHER) in
// qmvm.hip (dense) and qmvm_gather.hip (gathers) so the instances compile in parallel.
template <int BITS, int MT, bool SBF32, bool GATHER, int FPM = -1>
void launch_family(const QmvmParams& P, const QmvParams& G, const QmvmPlan& pl, dim3 grid,
                   hipStream_t s);

template <int BITS, int NC, int MT, bool SBF32, bool GATHER, int FPM = -1>
void launch_xd(const QmvmParams& P, const QmvParams& G, const QmvmPlan& pl, dim3 grid,
               hipStream_t s) {
  const dim3 block(64 * pl.waves);
  const size_t lds = (size_t)pl.lds;
#define MI_QMVM_LAUNCH(XU, DP)                                                              \
  do {                                                                                      \
    auto k = qmvm_kernel<BITS, 64, NC, XU, DP, MT, SBF32, GATHER, FPM>;                     \
    static bool attr = false; /* LDS above 64 KiB needs the attribute, once per kernel */ \
    if (!attr) {                                                                            \
      (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                160 * 1024 - 512);                                          \
      attr = true;                                                                          \
    }                                                                                       \
    hipLaunchKernelGGL(k, grid, block, lds, s, P, G);                                       \
  } while (0)
  // odd widths: the plans' two-chunk window only (fewer instances)
  bool d2 = FPM >= 100;
  if constexpr (NC > 2) d2 = d2 || pl.depth == 2;
  if (d2) {
    switch (pl.xu) {
      case 1: MI_QMVM_LAUNCH(1, 2); break;
      case 2: MI_QMVM_LAUNCH(2, 2); break;
      case 4: MI_QMVM_LAUNCH(4, 2); break;
      default: MI_QMVM_LAUNCH(8, 2); break;
    }
  } else if constexpr (FPM < 100) {
    switch (pl.xu) {
      case 1: MI_QMVM_LAUNCH(1, 4); break;
      case 2: MI_QMVM_LAUNCH(2, 4); break;
      case 4: MI_QMVM_LAUNCH(4, 4); break;
      default: MI_QMVM_LAUNCH(8, 4); break;
    }
  }
#undef MI_QMVM_LAUNCH
}

template <int BITS, int MT, bool SBF32, bool GATHER, int FPM>
void launch_family(const QmvmParams& P, const QmvParams& G, const QmvmPlan& pl, dim3 grid,
                   hipStream_t s) {
  switch (pl.nc) {
    case 1: launch_xd<BITS, 1, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 2: launch_xd<BITS, 2, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 3: launch_xd<BITS, 3, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 4: launch_xd<BITS, 4, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 5: launch_xd<BITS, 5, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 6: launch_xd<BITS, 6, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    case 7: launch_xd<BITS, 7, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
    default: launch_xd<BITS, 8, MT, SBF32, GATHER, FPM>(P, G, pl, grid, s); break;
  }
}

}  // namespace qmvm_detail
}  // namespace mi
