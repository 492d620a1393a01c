// Decode GEMV for work items of one activation row (dense M == 1, MoE decode pairs,
// sorted items of one row), 4-bit affine, bf16 activations: the HBM-streaming kernel.
//
// A block owns a 16-row weight tile and W waves split its K range. Lane l of a wave
// owns row l/4 and the 32-value slice l%4 of every 128-value chunk, so the 4 lanes of a
// row read its 64 contiguous bytes per chunk. A wave first issues its activation loads
// and its scale/bias loads, then its weight loads (16 B per chunk per lane): DEPTH
// chunks up front and one more as each chunk is consumed. Each wave stages the activations
// of its own chunks into LDS while the weights are in flight, so no block barrier precedes
// the dot products.
//
// Per 8 packed values: two masks split even/odd nibbles, v_perm builds bf16 pairs
// 0x43qq (= 128 + q exactly) and v_dot2_f32_bf16 multiplies them with the activations,
// which are staged in the same pair order ([x0,x2,x4,x6,x1,x3,x5,x7] per 8). The affine
// terms are applied per 32-value slice in fp32: s*sum(x*(128+q)) + (b - 128 s)*sum(x),
// with sum(x) per slice staged next to x. Scales/biases (gs 64/32) are loaded once per
// wave and row and handed to each chunk by DPP quad broadcasts. Rows reduce over their
// 4 lanes by shuffles and over the W waves through LDS in wave order (deterministic).
#pragma once
#include "mi_common.h"
#include "mi_internal.h"
#include "qmv_common.h"
#include "moe_route.h"
#include "code_runs.h"

#include <type_traits>


namespace mi {
namespace qmv1_detail {

using qmv_detail::decode_item;
using qmv_detail::item_x_row;
using qmv_detail::Item;
using qmv_detail::lds_barrier;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kChunkVals = 128;
// Buffer resource word 3 for raw (untyped) dword access on this target.
constexpr int kBufFlags = 0x00020000;

MI_DEV float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// One word of 8 nibbles against its 8 activations: masks split even / odd nibbles into
// bytes and v_perm pairs each byte with 0x43, giving bf16 0x43qq = 128 + q exactly (q < 16
// fits the 7-bit mantissa). x4 holds the activations staged in the matching pair order
// (x0, x2), (x4, x6), (x1, x3), (x5, x7), so acc += sum x_i (128 + q_i).
MI_DEV float dot8(uint32_t w, u32x4_t x4, float acc) {
  constexpr uint32_t c43 = 0x43434343u;
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  acc = dot2(perm_b32(c43, lo, 0x04010400u), x4.x, acc);  // (q0, q2)
  acc = dot2(perm_b32(c43, lo, 0x04030402u), x4.y, acc);  // (q4, q6)
  acc = dot2(perm_b32(c43, hi, 0x04010400u), x4.z, acc);  // (q1, q3)
  acc = dot2(perm_b32(c43, hi, 0x04030402u), x4.w, acc);  // (q5, q7)
  return acc;
}

// Quad broadcast of lane `src` (0..3) of each group of 4 lanes (DPP quad_perm); `src`
// is a constant once the chunk loop is unrolled.
MI_DEV uint32_t quad_bcast(uint32_t v, int src) {
  switch (src) {
    case 0: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x00, 0xF, 0xF, false);
    case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x55, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xAA, 0xF, 0xF, false);
    default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xFF, 0xF, 0xF, false);
  }
}

// Value of lane ^ 1 / lane ^ 2 within the quad (DPP quad_perm, no LDS round trip).
MI_DEV float quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
MI_DEV float quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// Lanes 0,1 of each quad take lane a, lanes 2,3 take lane a+1 (a = 0 or 2).
MI_DEV uint32_t quad_pairs(uint32_t v, int a) {
  return a == 0 ? (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x50, 0xF, 0xF, false)
                : (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xFA, 0xF, 0xF, false);
}

template <int GS>
constexpr int groups_per_chunk() {
  return kChunkVals / GS;
}

// Up to 16 waves per block when a wave holds <= 8 chunks (<= 128 VGPRs), else 8.
// FPM 0 / 1 / 2 (dense only): bias-less nvfp4 / mxfp4 / mxfp8 weights (mxfp8: one byte a
// code, a chunk is 128 bytes of a row), P.scales then uint8 [N, K / FGS] (e4m3 for nvfp4's
// 16-value groups, e8m0 for the mx modes' 32). Each 8-code
// word becomes exact bf16 pairs (mxfp4: code x scale; nvfp4: the code, its group's scale
// applied to the group's fp32 dot sum), dotted with the activations in natural order; no
// affine terms, so no per-slice sums.
template <int GS, int NC, int DEPTH, bool DENSE, bool DUAL = false, int FPM = -1>
__global__ void __launch_bounds__(NC <= 8 ? 1024 : 512) qmv1_kernel(QmvParams P) {
  constexpr bool FP = FPM >= 0 && FPM < 100;
  // FPM 100 + b: affine b = 2, 3, 5, 6 bits, one LSB-first bitstream per row; a lane's 32
  // codes of a chunk are 4b bytes at byte 4bg of the chunk's 16b (dword-aligned)
  // FPM 108: affine 8 bits at gs 64, one byte a code (a chunk is 128 bytes of a row); each
  // code converts exactly to bf16 (v_cvt_f32_ubyte, v_cvt_pk_bf16_f32) and the epilogue adds
  // b * sum(x) (no 128 offset)
  constexpr bool B8 = FPM == 108;
  constexpr bool ODD = FPM >= 100 && !B8;
  constexpr int OB = ODD ? FPM - 100 : 4;
  static_assert(!FP || (DENSE && !DUAL && FPM <= 2), "fp modes: dense calls");
  constexpr bool FP8 = FPM == 2;
  static_assert(!B8 || (DENSE && !DUAL && GS == 64), "8-bit one-row: dense calls at gs 64");
  constexpr bool BYTES = FP8 || B8;  // one byte a code: two 16-byte loads per lane and chunk
  static_assert(!ODD || (DENSE && !DUAL && GS == 64 && (OB == 2 || OB == 3 || OB == 5 || OB == 6)),
                "odd widths: dense calls at group size 64");
  constexpr int FGS = FPM == 0 ? 16 : 32;
  constexpr int GPC = groups_per_chunk<GS>();
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, BD = blockDim.x, W = BD >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane >> 2, g = lane & 3;
  const int K = P.K, N = P.N, G = K / GS;
  const int tile = blockIdx.x, ks = blockIdx.y;
  // Block K range (whole chunks) and this wave's chunks.
  // (the plan gives every wave NC chunks; only the last split can be shorter)
  const int kb0 = ks * P.gps * GS;
  const int kb1 = min(K, kb0 + P.gps * GS);
  const int nchb = (kb1 - kb0) / kChunkVals;
  // A wave whose range starts past the end (rounded-up plans) loads a valid chunk but
  // weighs everything 0.
  const int c0 = min(wave * NC, nchb - 1);
  const int nmine = wave * NC < nchb ? min(NC, nchb - c0) : 0;
  const int nload = max(1, nmine);
  const int nvals = kb1 - kb0, nunits = nvals / 8;
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);               // nvals bf16, dot8 order
  float* xsum = reinterpret_cast<float*>(smem + nvals * 2);        // nvals/32 slice sums
  float* red = xsum + nvals / 32;                                  // [W][16]
  const int n = tile * 16 + r;
  const uint32_t nn = (uint32_t)min(n, N - 1);
  const int64_t PT = P.n_pairs * P.M;

  // DUAL: gate (bank 0) and up (bank 1) for the same item. Both banks' loads go out
  // before either is consumed (one memory round trip per item, not two); the gate sums
  // wait in gsave and the up pass writes swiglu(gate, up) with the reference's rounding
  // points.
  __shared__ float gsave[16];
  constexpr int ND = GPC >= 2 ? NC * GPC / 2 : 1;
  constexpr int NSL = (ND + 3) / 4;
  constexpr int D = DEPTH < NC ? DEPTH : NC;
  // Each wave stages the activations of its own chunks (ceil(NC/4) 16-byte units per lane)
  // and waits only for its own LDS writes, not for the whole block's.
  constexpr int XN = (NC + 3) / 4;
  struct BankLoads {
    __amdgpu_buffer_rsrc_t wres;
    uint32_t wo;
    uint32_t sd[GPC >= 2 ? NSL : NC], bd[GPC >= 2 ? NSL : NC];
    u32x2_t fs[FP ? NC : 1];  // fp modes: the row's scale bytes of each chunk
    u32x4_t wv[NC];
    u32x2_t wv2[ODD ? NC : 1];  // odd widths: dwords 4, 5 of a lane's 5- or 6-dword slice
    u32x4_t wv8[BYTES ? NC : 1];  // one byte a code: bytes 16..31 of a lane's 32-byte slice
  };
  // One chunk's weights of this lane: 16 B at 4 bits, OB dwords at the odd widths.
  auto load_chunk = [&](BankLoads& L, int j) __attribute__((always_inline)) {
    if constexpr (ODD) {
      const uint32_t o = L.wo + 16 * OB * j;
      if constexpr (OB == 2) {
        const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(L.wres, o, 0, 0));
        L.wv[j] = u32x4_t{v.x, v.y, 0u, 0u};
      } else if constexpr (OB == 3) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(L.wres, o, 0, 0);
        L.wv[j] = u32x4_t{v[0], v[1], v[2], 0u};
      } else {
        L.wv[j] = __builtin_amdgcn_raw_buffer_load_b128(L.wres, o, 0, 0);
        if constexpr (OB == 5) {
          L.wv2[j] = u32x2_t{__builtin_amdgcn_raw_buffer_load_b32(L.wres, o + 16, 0, 0), 0u};
        } else {
          L.wv2[j] = __builtin_bit_cast(u32x2_t,
                                        __builtin_amdgcn_raw_buffer_load_b64(L.wres, o + 16, 0, 0));
        }
      }
    } else if constexpr (BYTES) {
      L.wv[j] = __builtin_amdgcn_raw_buffer_load_b128(L.wres, L.wo + 128 * j, 0, 0);
      L.wv8[j] = __builtin_amdgcn_raw_buffer_load_b128(L.wres, L.wo + 128 * j + 16, 0, 0);
    } else {
      L.wv[j] = __builtin_amdgcn_raw_buffer_load_b128(L.wres, L.wo + 64 * j, 0, 0);
    }
  };
  // 1. every global load of this item, before anything waits, as buffer loads from
  //    per-matrix resources: 32-bit lane offsets, chunk / slot strides folded into the
  //    instructions' immediate offsets. Reads past a wave's range only feed chunks that
  //    weigh 0, and reads past a resource's end return 0.
  auto issue_x = [&](int64_t xr, u32x4_t (&xv)[XN]) {
    const uint16_t* xb = reinterpret_cast<const uint16_t*>(P.x) + (xr < 0 ? 0 : xr) + kb0;
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, nvals * 2, kBufFlags);
#pragma unroll
    for (int i = 0; i < XN; ++i)
      xv[i] = __builtin_amdgcn_raw_buffer_load_b128(
          xres, (c0 * 16 + lane + 64 * i) * 16, 0, 0);
  };
  auto issue_bank = [&](const Item& it, auto bank_c, BankLoads& L) {
    constexpr int BANK = decltype(bank_c)::value;
    const uint32_t* Pw = BANK ? P.w2 : P.w;
    const uint16_t* Ps = BANK ? P.scales2 : P.scales;
    const uint16_t* Pb = BANK ? P.biases2 : P.biases;
    const uint32_t e = __builtin_amdgcn_readfirstlane(it.expert_ok ? it.expert : 0u);
    const size_t mat = (size_t)e * (uint32_t)N;
    L.wres = ODD ? __builtin_amdgcn_make_buffer_rsrc(
                       (void*)((const unsigned char*)Pw + mat * (uint32_t)(K / 8 * OB)), (short)0,
                       N * (K / 8 * OB), kBufFlags)
                 : BYTES ? __builtin_amdgcn_make_buffer_rsrc((void*)(Pw + mat * (uint32_t)(K / 4)),
                                                           (short)0, N * K, kBufFlags)
                 : __builtin_amdgcn_make_buffer_rsrc((void*)(Pw + mat * (uint32_t)(K / 8)), (short)0,
                                                     N * (K / 2), kBufFlags);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(Ps + mat * (uint32_t)G), (short)0, N * G * 2, kBufFlags);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(Pb + mat * (uint32_t)G), (short)0, N * G * 2, kBufFlags);
    L.wo = ODD   ? nn * (uint32_t)(K / 8 * OB) + (uint32_t)(kb0 + c0 * kChunkVals) / 8 * OB + 4 * OB * g
           : BYTES ? nn * (uint32_t)K + (uint32_t)(kb0 + c0 * kChunkVals) + 32 * g
                 : nn * (uint32_t)(K / 2) + (uint32_t)(kb0 + c0 * kChunkVals) / 2 + 16 * g;
    // Scales/biases. gs 64/32: the wave's groups of a row are contiguous dwords; lane g
    // of the row's quad loads dwords g, g+4, ... and chunks take theirs by a quad
    // broadcast. gs 128: one bf16 per chunk.
    const uint32_t so = nn * (uint32_t)(G * 2) + (uint32_t)((kb0 + c0 * kChunkVals) / GS) * 2;
    if constexpr (FP) {
      // the chunk's 8 (nvfp4) or 4 (mxfp4) scale bytes of the row; the row's 4 lanes read
      // the same bytes and each takes its own slice's
      const int Gf = K / FGS;
      const __amdgpu_buffer_rsrc_t fres = __builtin_amdgcn_make_buffer_rsrc(
          (void*)((const unsigned char*)Ps + mat * (uint32_t)Gf), (short)0, N * Gf, kBufFlags);
      const uint32_t fo = nn * (uint32_t)Gf + (uint32_t)(kb0 + c0 * kChunkVals) / FGS;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        if constexpr (FPM == 0)
          L.fs[j] = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(fres, fo + 8 * j, 0, 0));
        else
          L.fs[j].x = __builtin_amdgcn_raw_buffer_load_b32(fres, fo + 4 * j, 0, 0);
      }
    } else if constexpr (GPC >= 2) {
#pragma unroll
      for (int i = 0; i < NSL; ++i) {
        L.sd[i] = __builtin_amdgcn_raw_buffer_load_b32(sres, so + 4 * g + 16 * i, 0, 0);
        L.bd[i] = __builtin_amdgcn_raw_buffer_load_b32(bres, so + 4 * g + 16 * i, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        L.sd[j] = __builtin_amdgcn_raw_buffer_load_b16(sres, so + 2 * j, 0, 0);
        L.bd[j] = __builtin_amdgcn_raw_buffer_load_b16(bres, so + 2 * j, 0, 0);
      }
    }
    // Weights: the first D chunks now, then one more as each chunk is consumed, so a
    // wave's data arrives in the order it is used.
#pragma unroll
    for (int j = 0; j < D; ++j) load_chunk(L, j);
  };
  // 2. stage the activations in dot8's pair order, with per-32-value sums.
  auto stage_x = [&](const u32x4_t (&xv)[XN]) {
#pragma unroll
    for (int i = 0; i < XN; ++i) {
      const int u = c0 * 16 + lane + 64 * i;  // 16-byte unit of the block range
      const u32x4_t X = xv[i];
      float s8 = ((bf16_bits_to_f32(X.x & 0xFFFFu) + bf16_bits_to_f32(X.x >> 16)) +
                  (bf16_bits_to_f32(X.y & 0xFFFFu) + bf16_bits_to_f32(X.y >> 16))) +
                 ((bf16_bits_to_f32(X.z & 0xFFFFu) + bf16_bits_to_f32(X.z >> 16)) +
                  (bf16_bits_to_f32(X.w & 0xFFFFu) + bf16_bits_to_f32(X.w >> 16)));
      s8 += quad_xor1(s8);
      s8 += quad_xor2(s8);
      // (a wave whose range was clamped onto the last chunk writes the same values as that
      // chunk's own wave)
      if (u < nunits && u < (c0 + NC) * 16) {
        if constexpr (FP || ODD || B8) {  // natural order: these decoders emit (q0, q1), (q2, q3), ..
          *reinterpret_cast<u32x4_t*>(xs + u * 4) = X;
          if ((ODD || B8) && (u & 3) == 0) xsum[u >> 2] = s8;
        } else {
          u32x4_t o;
          o.x = perm_b32(X.y, X.x, 0x05040100u);  // (x0, x2)
          o.y = perm_b32(X.w, X.z, 0x05040100u);  // (x4, x6)
          o.z = perm_b32(X.y, X.x, 0x07060302u);  // (x1, x3)
          o.w = perm_b32(X.w, X.z, 0x07060302u);  // (x5, x7)
          *reinterpret_cast<u32x4_t*>(xs + u * 4) = o;
          if ((u & 3) == 0) xsum[u >> 2] = s8;
        }
      }
    }
    // The wave reads only what its own lanes wrote: a wave-level fence, no block barrier
    // (the weight loads stay in flight).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // 3. dot products, chunk by chunk as the loads land (chunks past the range weigh 0),
  // 4. reduce the row's 4 lanes, then the waves in order, and write.
  auto compute = [&](const Item& it, int64_t xr, auto bank_c, BankLoads& L) {
    constexpr int BANK = decltype(bank_c)::value;
    const bool ok = it.expert_ok && xr >= 0;
    float y = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      if constexpr (D < NC) {
        if (j + D < NC) load_chunk(L, j + D);
      }
      const int jj = min(j, nload - 1);
      const int off = (c0 + jj) * kChunkVals + 32 * g;  // within the block range
      const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(xs + off / 2);
      if constexpr (FP) {
        // lane slice g of chunk j: codes 32g .. 32g + 31, word t = codes 32g + 8t ..
        // mxfp4 / mxfp8: one e8m0 scale (byte g) for the slice, applied in the conversion.
        // nvfp4: two e4m3 scales (bytes 2g, 2g+1), one per 16 codes: the codes convert
        // exactly (scale 1), each group's dot sum is scaled in fp32, the groups in order.
        float acc = 0.f, grp = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e8 = __uint_as_float(((L.fs[j].x >> (8 * g)) & 0xFFu) << 23);
          u32x4_t a;
          if constexpr (FP8) {  // codes 8t .. 8t+7: two dwords of the lane's 32 bytes
            const u32x4_t h = t < 2 ? L.wv[j] : L.wv8[j];
            a = (t & 1) ? code_runs::fp8_run(h.z, h.w, e8) : code_runs::fp8_run(h.x, h.y, e8);
          } else {
            const uint32_t codes = t == 0 ? L.wv[j].x : t == 1 ? L.wv[j].y : t == 2 ? L.wv[j].z
                                                                                : L.wv[j].w;
            a = code_runs::fp4_run(codes, FPM == 1 ? e8 : 1.f);
          }
          const u32x4_t xv4 = xp[t];
          float& d = FPM == 0 ? grp : acc;
          d = dot2(a.x, xv4.x, d);
          d = dot2(a.y, xv4.y, d);
          d = dot2(a.z, xv4.z, d);
          d = dot2(a.w, xv4.w, d);
          if constexpr (FPM == 0) {
            if (t & 1) {  // a 16-code group is complete
              const int b = 2 * g + (t >> 1);
              const uint32_t wd = b < 4 ? L.fs[j].x : L.fs[j].y;
              acc = fmaf(code_runs::fp_e4m3((wd >> (8 * (b & 3))) & 0xFFu), grp, acc);
              grp = 0.f;
            }
          }
          // one word's pairs live at a time (the compiler otherwise decodes ahead and
          // spills)
          asm volatile("" : "+v"(acc), "+v"(grp));
          __builtin_amdgcn_sched_barrier(0);
        }
        y = fmaf(j < nmine ? 1.f : 0.f, acc, y);
        if constexpr (D < NC) __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      float acc = 0.f;
      if constexpr (ODD) {
        // run t (codes 8t .. 8t+7 of the slice) starts at byte t*OB of the lane's dwords
        auto dw = [&](int i) -> uint32_t {
          return i == 0 ? L.wv[j].x : i == 1 ? L.wv[j].y : i == 2 ? L.wv[j].z : i == 3 ? L.wv[j].w
                 : i == 4 ? L.wv2[j].x : i == 5 ? L.wv2[j].y : 0u;
        };
        if constexpr (OB == 2) {  // a dword is two runs
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4_t a0, a1;
            code_runs::two_bit_runs(dw(h), a0, a1);
            const u32x4_t x0 = xp[2 * h], x1 = xp[2 * h + 1];
            acc = dot2(a0.x, x0.x, acc);
            acc = dot2(a0.y, x0.y, acc);
            acc = dot2(a0.z, x0.z, acc);
            acc = dot2(a0.w, x0.w, acc);
            acc = dot2(a1.x, x1.x, acc);
            acc = dot2(a1.y, x1.y, acc);
            acc = dot2(a1.z, x1.z, acc);
            acc = dot2(a1.w, x1.w, acc);
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int i = (t * OB) >> 2, sh = 8 * ((t * OB) & 3);
            const u32x4_t a = code_runs::odd_run<OB>(dw(i), i + 1 < OB ? dw(i + 1) : 0u, sh);
            const u32x4_t xv4 = xp[t];
            acc = dot2(a.x, xv4.x, acc);
            acc = dot2(a.y, xv4.y, acc);
            acc = dot2(a.z, xv4.z, acc);
            acc = dot2(a.w, xv4.w, acc);
          }
        }
      } else if constexpr (B8) {
        // codes 8t .. 8t+7 of the slice: two dwords of the lane's 32 bytes, each byte an
        // exact bf16 (0..255 needs 8 significant bits)
        auto pk = [](uint32_t d, int b) {
          const float lo = (float)((d >> (8 * b)) & 0xFFu), hi = (float)((d >> (8 * b + 8)) & 0xFFu);
          return __builtin_bit_cast(uint32_t, __builtin_convertvector((code_runs::f32x2v){lo, hi}, bf16x2_t));
        };
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4_t h = t < 2 ? L.wv[j] : L.wv8[j];
          const uint32_t d0 = (t & 1) ? h.z : h.x, d1 = (t & 1) ? h.w : h.y;
          const u32x4_t xv4 = xp[t];
          acc = dot2(pk(d0, 0), xv4.x, acc);
          acc = dot2(pk(d0, 2), xv4.y, acc);
          acc = dot2(pk(d1, 0), xv4.z, acc);
          acc = dot2(pk(d1, 2), xv4.w, acc);
        }
      } else {
        acc = dot8(L.wv[j].x, xp[0], acc);
        acc = dot8(L.wv[j].y, xp[1], acc);
        acc = dot8(L.wv[j].z, xp[2], acc);
        acc = dot8(L.wv[j].w, xp[3], acc);
      }
      const float use = j < nmine ? 1.f : 0.f;
      float s, b;
      if constexpr (GPC == 2) {
        // chunk j's groups are dword j: lane j % 4, slot j / 4 of the quad
        const uint32_t sw = quad_bcast(L.sd[j >> 2], j & 3);
        const uint32_t bw = quad_bcast(L.bd[j >> 2], j & 3);
        s = bf16_bits_to_f32(g >= 2 ? sw >> 16 : sw & 0xFFFFu);
        b = bf16_bits_to_f32(g >= 2 ? bw >> 16 : bw & 0xFFFFu);
      } else if constexpr (GPC == 4) {
        // chunk j's groups are dwords 2j, 2j+1: lanes g<2 take lane (2j)%4, g>=2 the next
        const int a = (2 * j) & 3;
        const uint32_t sw = quad_pairs(L.sd[(2 * j) >> 2], a);
        const uint32_t bw = quad_pairs(L.bd[(2 * j) >> 2], a);
        s = bf16_bits_to_f32((g & 1) ? sw >> 16 : sw & 0xFFFFu);
        b = bf16_bits_to_f32((g & 1) ? bw >> 16 : bw & 0xFFFFu);
      } else {
        s = bf16_bits_to_f32(L.sd[j] & 0xFFFFu);
        b = bf16_bits_to_f32(L.bd[j] & 0xFFFFu);
      }
      s *= use;
      b *= use;
      y = fmaf(s, acc, y);
      y = fmaf(fmaf(B8 ? 0.f : -128.f, s, b), xsum[off >> 5], y);
      if constexpr (D < NC) __builtin_amdgcn_sched_barrier(0);  // keep the issue order
    }
    y += quad_xor1(y);
    y += quad_xor2(y);
    if (g == 0) red[wave * 16 + r] = y;
    lds_barrier();
    if (tid < 16 && tile * 16 + tid < N) {
      float v = 0.f;
      for (int w2 = 0; w2 < W; ++w2) v += red[w2 * 16 + tid];
      const int64_t p = it.pos0;
      const int nout = tile * 16 + tid;
      if (!DUAL && P.ks > 1) {
        P.part[((int64_t)ks * PT + p) * N + nout] = v;
      } else {
        if (!ok) v = __builtin_nanf("");
        if (DUAL && BANK == 0) {
          gsave[tid] = v;
        } else {
          uint16_t o = (uint16_t)f32_to_bf16_bits(v);
          if (DUAL) o = swiglu_bf16((uint16_t)f32_to_bf16_bits(gsave[tid]), o);
          else if (P.swiglu_gate) o = swiglu_bf16(P.swiglu_gate[p * N + nout], o);
          ((uint16_t*)P.y)[p * N + nout] = o;
        }
      }
    }
  };
  using bank0_t = std::integral_constant<int, 0>;
  using bank1_t = std::integral_constant<int, 1>;
  auto process = [&](const Item& it, int64_t xr, u32x4_t (&xv)[XN]) {
    BankLoads L0;
    issue_bank(it, bank0_t{}, L0);
    if constexpr (DUAL) {
      BankLoads L1;
      issue_bank(it, bank1_t{}, L1);
      stage_x(xv);
      compute(it, xr, bank0_t{}, L0);
      lds_barrier();  // gsave written, the reduction buffer free again
      compute(it, xr, bank1_t{}, L1);
    } else {
      stage_x(xv);
      compute(it, xr, bank0_t{}, L0);
    }
  };
  if constexpr (DENSE) {
    // one pair, no indices: straight-line, no work-item decode
    Item it;
    it.pos0 = 0;
    it.cnt = 1;
    it.expert = 0;
    it.expert_ok = true;
    u32x4_t xv[XN];
    issue_x(0, xv);
    process(it, 0, xv);
  } else {
    const int n_items = P.items ? (int)*P.item_count : P.n_items_fixed;
    __shared__ uint32_t route_expert;
    for (int it_i = blockIdx.z; it_i < n_items; it_i += gridDim.z) {
      Item it = decode_item(P, it_i);
      if (it.cnt <= 0) continue;
      // the activation row does not depend on the expert: its loads go out first
      const int64_t xr = item_x_row(P, it, 0);
      if (xr == -1) continue;  // block-uniform
      u32x4_t xv[XN];
      issue_x(xr, xv);
      if constexpr (DUAL) {
        if (P.route_logits) {
          // unsorted one-row items: item it_i is pair it_i = (token, slot)
          const int t = it_i / P.route_k, slot = it_i - t * P.route_k;
          if (wave == 0) {
            uint32_t sel;
            float w;
            const float* lg = P.route_logits + (int64_t)t * P.route_E;
            route_token<4>(lg, P.route_E, P.route_k, lane, sel, w);
            if (lane == slot) {
              route_expert = sel;
              if (tile == 0 && ks == 0) {
                P.route_inds[it_i] = sel;
                P.route_scores[it_i] = (uint16_t)f32_to_bf16_bits(w);
              }
            }
          }
          lds_barrier();
          it.expert = route_expert;
          it.expert_ok = route_expert < (uint32_t)P.n_experts;
        }
      }
      process(it, xr, xv);
      lds_barrier();  // LDS is reused by the next item
    }
  }
}

template <int GS, int NC, int DEPTH, bool DENSE>
void launch_k(const QmvParams& P, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  // gate + up + SwiGLU in one launch: group size 64 work items only
  if constexpr (GS == 64 && !DENSE) {
    if (P.dual) {
      hipLaunchKernelGGL((qmv1_kernel<GS, NC, DEPTH, false, true>), grid, block, lds, s, P);
      return;
    }
  }
  hipLaunchKernelGGL((qmv1_kernel<GS, NC, DEPTH, DENSE, false>), grid, block, lds, s, P);
}

template <int GS, int NC, bool DENSE>
void launch_depth(const QmvParams& P, dim3 grid, dim3 block, int depth, size_t lds,
                  hipStream_t s) {
  // depth 4 covers "all loads up front" for NC <= 4; NC <= 2 has a single schedule
  if (NC > 2 && depth == 2) launch_k<GS, NC, 2, DENSE>(P, grid, block, lds, s);
  else launch_k<GS, NC, 4, DENSE>(P, grid, block, lds, s);
}

template <int GS, int NC>
hipError_t launch_nc(const QmvParams& P, dim3 grid, int waves, int depth, size_t lds,
                     hipStream_t s) {
  const dim3 block(64 * waves);
  const bool dense = !P.items && !P.lhs && !P.rhs && P.n_pairs == 1 && P.M == 1;
  if (dense) launch_depth<GS, NC, true>(P, grid, block, depth, lds, s);
  else launch_depth<GS, NC, false>(P, grid, block, depth, lds, s);
  return hipGetLastError();
}

// Dense one-row launches of the other weight formats (fp4 modes, odd widths): the
// instances for one format, dispatched on the plan's chunks per wave and depth.
template <int NC, int FPM>
void launch_nc_fmt(const QmvParams& P, dim3 grid, dim3 block, int depth, size_t lds,
                   hipStream_t s) {
  if (NC > 2 && depth == 2)
    hipLaunchKernelGGL((qmv1_kernel<64, NC, 2, true, false, FPM>), grid, block, lds, s, P);
  else
    hipLaunchKernelGGL((qmv1_kernel<64, NC, 4, true, false, FPM>), grid, block, lds, s, P);
}

template <int FPM>
void launch_fmt(const QmvParams& P, const Qmv1Plan& pl, hipStream_t s) {
  const dim3 grid((unsigned)pl.tiles, (unsigned)P.ks, 1), block(64 * pl.waves);
  switch (pl.nc) {
    case 1: launch_nc_fmt<1, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 2: launch_nc_fmt<2, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 3: launch_nc_fmt<3, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 4: launch_nc_fmt<4, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 5: launch_nc_fmt<5, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 6: launch_nc_fmt<6, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 7: launch_nc_fmt<7, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 8: launch_nc_fmt<8, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 10: launch_nc_fmt<10, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 12: launch_nc_fmt<12, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    case 14: launch_nc_fmt<14, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
    default: launch_nc_fmt<16, FPM>(P, grid, block, pl.depth, pl.lds, s); break;
  }
}

}  // namespace qmv1_detail

// Launch for one group size; each group size is instantiated in its own translation unit
// (qmv1_g32.hip, qmv1_g64.hip, qmv1_g128.hip) so the kernel instances compile in parallel.
template <int GS>
hipError_t launch_qmv1_gs(const QmvParams& P, dim3 grid, int waves, int nc, int depth,
                          size_t lds, hipStream_t s) {
  using namespace qmv1_detail;
  switch (nc) {
    case 1: return launch_nc<GS, 1>(P, grid, waves, depth, lds, s);
    case 2: return launch_nc<GS, 2>(P, grid, waves, depth, lds, s);
    case 3: return launch_nc<GS, 3>(P, grid, waves, depth, lds, s);
    case 4: return launch_nc<GS, 4>(P, grid, waves, depth, lds, s);
    case 5: return launch_nc<GS, 5>(P, grid, waves, depth, lds, s);
    case 6: return launch_nc<GS, 6>(P, grid, waves, depth, lds, s);
    case 7: return launch_nc<GS, 7>(P, grid, waves, depth, lds, s);
    case 8: return launch_nc<GS, 8>(P, grid, waves, depth, lds, s);
    case 10: return launch_nc<GS, 10>(P, grid, waves, depth, lds, s);
    case 12: return launch_nc<GS, 12>(P, grid, waves, depth, lds, s);
    case 14: return launch_nc<GS, 14>(P, grid, waves, depth, lds, s);
    default: return launch_nc<GS, 16>(P, grid, waves, depth, lds, s);
  }
}

}  // namespace mi
