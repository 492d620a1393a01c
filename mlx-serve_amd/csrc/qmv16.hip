// Decode-width (M <= 16 rows per item) affine quantized matmul on the gfx950
// 16x16x32 bf16 MFMA: dense qmv and gather_qmm work items.
//
// Block = W waves on one 16-row weight tile of one item. The waves split the K
// range between them and each streams its part in 256-byte-per-row chunks:
//   * the block first stages the activations of its K range into LDS (fragment
//     order, per-group sums) -- all of its LDS writes before any DMA starts;
//   * each wave DMAs chunk c+1 (16 rows x 256 B of packed weights, 4 instructions of
//     4 rows x 256 contiguous bytes, plus one instruction for the 16-byte scale and
//     bias runs of the chunk's groups) straight into LDS while it runs the MFMAs of
//     chunk c; 16-byte slot s of row r lands at s ^ (r & 15) so fragment reads of
//     the 16 rows hit distinct banks;
//   * once every DMA has landed, the waves' partial sums are added through LDS in
//     wave order and written. Fixed summation order: deterministic.
//
// MFMA layout (16x16x32): lane l holds 8 k values of A row l%16 / B column l%16 for
// k block l/16; C lane l register r is row 4(l/16)+r, column l%16. A lane's k blocks
// of one group are its VPL consecutive packed words, so step j of a group uses word
// j (4-bit) or words 2j, 2j+1 (8-bit) of them; the activations are staged in the
// same order (and nibble-permuted for 4-bit, see a_perm / b_frag).
#include "qmv_common.h"

namespace mi {

namespace {

using namespace qmv_detail;

typedef __bf16 bf16x8q __attribute__((ext_vector_type(8)));

MI_DEV f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8q, a),
                                                  __builtin_bit_cast(bf16x8q, b), c, 0, 0, 0);
}

constexpr int kChunk = 16 * 256;  // LDS bytes of one chunk of one tile
constexpr int kSbuf = 1024;       // LDS bytes of one chunk's scale/bias runs

// MP = activation rows staged (1, 2, 4 or 16); MR = C registers kept per lane.
template <int BITS, int GS, int MP, bool XF32>
__global__ void __launch_bounds__(512) qmv16_kernel(QmvParams P) {
  constexpr int PF = 32 / BITS;
  constexpr int WPG = GS / PF;      // packed words per group per row
  constexpr int GSB = WPG * 4;      // bytes per group per row
  constexpr int UG = 256 / GSB;     // groups per chunk
  constexpr int STEPS = GS / 32;    // MFMA steps per group
  constexpr int WPS = 8 / PF;       // packed words per lane per step
  constexpr int VPL = WPG / 4;      // packed words per lane per group
  constexpr int MR = MP < 4 ? MP : 4;
  constexpr int PLANES = XF32 ? 2 : 1;
  constexpr int FB = 2;             // staging fragments per thread per pass
  constexpr int SPG = STEPS * 4;    // staged fragments per (group, row)

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int64_t srow[16];

  const int tid = threadIdx.x;
  const int BD = blockDim.x, W = BD >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int l16 = lane & 15, q = lane >> 4;
  const int K = P.K, N = P.N;
  const int G = K / GS;
  const uint32_t wrow_b = (uint32_t)(K / PF) * 4u;  // bytes per packed weight row
  const int tile = blockIdx.x, ks = blockIdx.y;
  const int g0 = ks * P.gps;
  const int g1 = min(G, g0 + P.gps);
  const int GB = g1 - g0;
  const int NF = GB * SPG * MP;  // staged A fragments

  unsigned char* wbuf = smem + (size_t)wave * 2 * kChunk;
  unsigned char* sbuf = smem + (size_t)W * 2 * kChunk + (size_t)wave * 2 * kSbuf;
  u32x4_t* sx = (u32x4_t*)(smem + (size_t)W * 2 * (kChunk + kSbuf));  // [GB][STEPS][4][MP]
  float* sxs = (float*)(sx + (size_t)NF * PLANES);                     // [GB][16]
  float* sred = sxs + (size_t)GB * 16;                                 // [W][MR][64]

  // This wave's groups: whole chunks, so chunk starts stay multiples of UG.
  const int gpw = ((GB + W - 1) / W + UG - 1) / UG * UG;
  const int gw0 = min(g1, g0 + wave * gpw);
  const int gw1 = min(g1, gw0 + gpw);
  const int nch = (gw1 - gw0 + UG - 1) / UG;
  const int arow = l16 & (MP - 1);  // A rows >= MP feed C rows that are never written
  const int sw = l16 & 15;
  const uint32_t c43 = 0x43434343u;
  const bool sdma = UG <= 8 && (G % 8) == 0;  // 16-byte aligned scale/bias runs

  const int n_items = P.item_count ? (int)*P.item_count : P.n_items_fixed;
  for (int itx = blockIdx.z; itx < n_items; itx += gridDim.z) {
    const Item it = decode_item(P, itx);
    const uint32_t ex = it.expert_ok ? it.expert : 0u;
    if (tid < 16) srow[tid] = item_x_row(P, it, tid);
    lds_barrier();

    // ---- stage the activations of [g0, g1) -------------------------------------
    for (int base = 0; base < NF; base += FB * BD) {
      u32x4_t v[FB][PLANES];
      float sum[FB];
#pragma unroll
      for (int i = 0; i < FB; ++i) {
        const int f = base + i * BD + tid;
        const int s = f % SPG, m = (f / SPG) % MP, u = f / (SPG * MP);
        const int j = s >> 2, qq = s & 3;
        const int64_t xr = (f < NF) ? srow[m] : -1;
        const bool ok = xr >= 0;
        const int64_t k0 = ok ? xr + (int64_t)(g0 + u) * GS + (qq * VPL + j * WPS) * PF : 0;
        if constexpr (XF32) {
          const u32x4_t* xp = (const u32x4_t*)((const float*)P.x + k0);
          const u32x4_t a = xp[0], b = xp[1];
          float e[8];
          *(u32x4_t*)&e[0] = ok ? a : u32x4_t{0u, 0u, 0u, 0u};
          *(u32x4_t*)&e[4] = ok ? b : u32x4_t{0u, 0u, 0u, 0u};
          uint32_t hi[8], lo[8];
          float sm = 0.f;
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            hi[t] = f32_to_bf16_bits(e[t]);
            lo[t] = f32_to_bf16_bits(e[t] - bf16_bits_to_f32(hi[t]));
            sm += e[t];
          }
          v[i][0] = u32x4_t{hi[0] | hi[1] << 16, hi[2] | hi[3] << 16, hi[4] | hi[5] << 16,
                            hi[6] | hi[7] << 16};
          v[i][PLANES - 1] = u32x4_t{lo[0] | lo[1] << 16, lo[2] | lo[3] << 16,
                                     lo[4] | lo[5] << 16, lo[6] | lo[7] << 16};
          sum[i] = sm;
        } else {
          const u32x4_t a = *(const u32x4_t*)((const uint16_t*)P.x + k0);
          v[i][0] = ok ? a : u32x4_t{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int i = 0; i < FB; ++i) {
        const int f = base + i * BD + tid;
        const int s = f % SPG, m = (f / SPG) % MP, u = f / (SPG * MP);
        const int j = s >> 2, qq = s & 3;
        float sm;
        if constexpr (XF32) {
          sm = sum[i];
        } else {
          const u32x4_t a = v[i][0];
          sm = (bf16_bits_to_f32(a.x & 0xFFFFu) + bf16_bits_to_f32(a.x >> 16)) +
               (bf16_bits_to_f32(a.y & 0xFFFFu) + bf16_bits_to_f32(a.y >> 16)) +
               (bf16_bits_to_f32(a.z & 0xFFFFu) + bf16_bits_to_f32(a.z >> 16)) +
               (bf16_bits_to_f32(a.w & 0xFFFFu) + bf16_bits_to_f32(a.w >> 16));
        }
        // Group sum over the SPG consecutive lanes holding one (u, m).
#pragma unroll
        for (int d = 1; d < SPG; d <<= 1) sm += __shfl_xor(sm, d, 64);
        if (f < NF) {
          const int idx = ((u * STEPS + j) * 4 + qq) * MP + m;
          sx[idx] = a_perm<BITS>(v[i][0]);
          if constexpr (XF32) sx[NF + idx] = a_perm<BITS>(v[i][PLANES - 1]);
          if (s == 0) sxs[u * 16 + m] = sm;
        }
      }
    }
    if constexpr (MP < 16) {
      for (int t = tid; t < GB * (16 - MP); t += BD)
        sxs[(t / (16 - MP)) * 16 + MP + t % (16 - MP)] = 0.f;
    }
    lds_barrier();

    // ---- stream this wave's groups ----------------------------------------------
    const unsigned char* tbase = (const unsigned char*)P.w + ((int64_t)ex * N) * wrow_b;
    const int n_own = min(tile * 16 + l16, N - 1);
    const uint16_t* srp = P.scales + ((int64_t)ex * N + n_own) * G;
    const uint16_t* brp = P.biases + ((int64_t)ex * N + n_own) * G;
    auto issue = [&](int c, int b, uint32_t (&sv)[UG], uint32_t (&bv)[UG]) {
      const int gc = gw0 + c * UG;
      const int nslots = min(UG, gw1 - gc) * GSB / 16;  // valid 16-byte slots per row
      const int s = lane & 15;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + (lane >> 4);
        const int sl = s ^ r;
        const uint32_t nr = (uint32_t)min(tile * 16 + r, N - 1);
        const unsigned char* src =
            tbase + nr * wrow_b + (uint32_t)gc * GSB + (sl < nslots ? sl * 16 : 0);
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void*)(wbuf + b * kChunk + i * 1024), 16,
            0, 0);
      }
      if (sdma) {
        // Lanes 0-15: scale run of row l16, 16-31: bias run (32-63 repeat them).
        const uint32_t nr = (uint32_t)min(tile * 16 + l16, N - 1);
        const uint16_t* run =
            ((q & 1) ? P.biases : P.scales) + ((int64_t)ex * N + nr) * G + (gc & ~7);
        __builtin_amdgcn_global_load_lds(
            run, (__attribute__((address_space(3))) void*)(sbuf + b * kSbuf), 16, 0, 0);
      } else {
#pragma unroll
        for (int u = 0; u < UG; ++u) {
          const int g = min(gc + u, gw1 - 1);
          sv[u] = srp[g];
          bv[u] = brp[g];
        }
      }
    };
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    auto compute = [&](int c, int b, const uint32_t (&sv)[UG], const uint32_t (&bv)[UG]) {
      const int gc = gw0 + c * UG;
      const int ng = min(UG, gw1 - gc);
      const unsigned char* myrow = wbuf + b * kChunk + l16 * 256;
      auto load_words = [&](int u, uint32_t (&words)[VPL]) {
        const int byte0 = u * GSB + q * VPL * 4;
        if constexpr (VPL >= 4) {
#pragma unroll
          for (int t = 0; t < VPL / 4; ++t) {
            const int slot = (byte0 >> 4) + t;
            const u32x4_t v = *(const u32x4_t*)(myrow + ((slot ^ sw) << 4));
            words[4 * t] = v.x; words[4 * t + 1] = v.y; words[4 * t + 2] = v.z;
            words[4 * t + 3] = v.w;
          }
        } else if constexpr (VPL == 2) {
          const u32x2_t v = *(const u32x2_t*)(myrow + (((byte0 >> 4) ^ sw) << 4) + (byte0 & 15));
          words[0] = v.x; words[1] = v.y;
        } else {
          words[0] = *(const uint32_t*)(myrow + (((byte0 >> 4) ^ sw) << 4) + (byte0 & 15));
        }
      };
      auto epilogue = [&](int u, const f32x4_t& accg) {
        const int ul = gc + u - g0;
        const f32x4_t xs = *(const f32x4_t*)&sxs[ul * 16 + 4 * q];
        uint32_t sbits, bbits;
        if (sdma) {
          const int gi = ((gc & 7) + u) * 2;
          sbits = *(const uint16_t*)(sbuf + b * kSbuf + l16 * 16 + gi);
          bbits = *(const uint16_t*)(sbuf + b * kSbuf + 256 + l16 * 16 + gi);
        } else {
          sbits = sv[u];
          bbits = bv[u];
        }
        const float sc = bf16_bits_to_f32(sbits);
        const float bi = bf16_bits_to_f32(bbits);
        const float bb = (BITS == 4) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r] = fmaf(bb, xs[r], fmaf(sc, accg[r], acc[r]));
      };
      auto mma = [&](int u, const uint32_t (&words)[VPL], f32x4_t& a) {
        const int ul = gc + u - g0;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
          const int idx = ((ul * STEPS + j) * 4 + q) * MP + arow;
          const u32x4_t B = b_frag<BITS>(words, j, c43);
          a = mfma16(sx[idx], B, j == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : a);
          if constexpr (XF32) a = mfma16(sx[NF + idx], B, a);
        }
      };
#pragma unroll
      for (int u = 0; u < UG; u += 2) {
        if (u + 1 < ng) {
          uint32_t w0[VPL], w1[VPL];
          load_words(u, w0);
          load_words(u + 1, w1);
          f32x4_t a0, a1;
          mma(u, w0, a0);
          mma(u + 1, w1, a1);
          epilogue(u, a0);
          epilogue(u + 1, a1);
        } else if (u < ng) {
          uint32_t w0[VPL];
          load_words(u, w0);
          f32x4_t a0;
          mma(u, w0, a0);
          epilogue(u, a0);
        }
      }
    };

    if (nch > 0) {
      uint32_t sA[UG], bA[UG], sB[UG], bB[UG];
      auto wait_prev = [&]() {  // chunk c landed: only chunk c+1's loads may pend
        if (sdma) __builtin_amdgcn_s_waitcnt(vmcnt_imm(5));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 + 2 * UG));
      };
      issue(0, 0, sA, bA);
      int c = 0;
      for (; c + 2 < nch; c += 2) {
        issue(c + 1, 1, sB, bB);
        wait_prev();
        compute(c, 0, sA, bA);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // buffer 0 reads done before reuse
        issue(c + 2, 0, sA, bA);
        wait_prev();
        compute(c + 1, 1, sB, bB);
        __builtin_amdgcn_s_waitcnt(0xC07F);
      }
      if (c + 1 < nch) {
        issue(c + 1, 1, sB, bB);
        wait_prev();
        compute(c, 0, sA, bA);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        compute(c + 1, 1, sB, bB);
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        compute(c, 0, sA, bA);
      }
    }

    // ---- reduce the waves (every DMA has landed), write -------------------------
#pragma unroll
    for (int r = 0; r < MR; ++r) sred[(wave * MR + r) * 64 + lane] = acc[r];
    lds_barrier();
    const int64_t PT = P.n_pairs * P.M;
    for (int t = tid; t < MR * 64; t += BD) {
      const int r = t >> 6, l2 = t & 63;
      const int li = 4 * (l2 >> 4) + r;
      const int nn = tile * 16 + (l2 & 15);
      const int64_t xr = li < 16 ? srow[li] : -1;
      if (nn >= N || li >= it.cnt || xr == -1) continue;
      float v = 0.f;
      for (int w2 = 0; w2 < W; ++w2) v += sred[(w2 * MR + r) * 64 + l2];
      const int64_t p = it.pos0 + li;
      if (P.ks > 1) {
        P.part[((int64_t)ks * PT + p) * N + nn] = v;
      } else {
        if (xr < 0 || !it.expert_ok) v = __builtin_nanf("");
        if constexpr (XF32) ((float*)P.y)[p * N + nn] = v;
        else ((uint16_t*)P.y)[p * N + nn] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
    lds_barrier();
  }
}

template <int BITS, int GS, int MP, bool XF32>
hipError_t launch_t(const QmvParams& P, dim3 grid, int waves, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv16_kernel<BITS, GS, MP, XF32>), grid, dim3(64 * waves), lds, s, P);
  return hipGetLastError();
}

template <int BITS, int GS, bool XF32>
hipError_t launch_m(const QmvParams& P, dim3 grid, int waves, size_t lds, int mp,
                    hipStream_t s) {
  switch (mp) {
    case 1: return launch_t<BITS, GS, 1, XF32>(P, grid, waves, lds, s);
    case 2: return launch_t<BITS, GS, 2, XF32>(P, grid, waves, lds, s);
    case 4: return launch_t<BITS, GS, 4, XF32>(P, grid, waves, lds, s);
    default: return launch_t<BITS, GS, 16, XF32>(P, grid, waves, lds, s);
  }
}

template <int BITS, bool XF32>
hipError_t launch_gs(const QmvParams& P, dim3 grid, int waves, size_t lds, int mp,
                     hipStream_t s) {
  switch (P.group_size) {
    case 32: return launch_m<BITS, 32, XF32>(P, grid, waves, lds, mp, s);
    case 64: return launch_m<BITS, 64, XF32>(P, grid, waves, lds, mp, s);
    default: return launch_m<BITS, 128, XF32>(P, grid, waves, lds, mp, s);
  }
}

}  // namespace

int qmv16_mp_for_rows(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 16; }

int qmv16_groups_per_chunk(int bits, int gs) { return 256 / (gs * bits / 8); }

size_t qmv16_lds_bytes(int groups, int gs, int mp, int x_f32, int waves) {
  const int mr = mp < 4 ? mp : 4;
  return (size_t)waves * 2 * (kChunk + kSbuf) +
         (size_t)groups * (gs / 32) * 4 * mp * 16 * (x_f32 ? 2 : 1) + (size_t)groups * 16 * 4 +
         (size_t)waves * mr * 64 * 4;
}

hipError_t launch_qmv16(const QmvParams& P, const QmvConfig& C, hipStream_t s) {
  dim3 grid((unsigned)P.row_blocks, (unsigned)P.ks, (unsigned)C.grid_z);
  const int mp = qmv16_mp_for_rows(C.rows);
  const size_t lds = qmv16_lds_bytes(P.gps, P.group_size, mp, P.x_f32, C.waves);
  hipError_t e = (P.bits == 4)
                     ? (P.x_f32 ? launch_gs<4, true>(P, grid, C.waves, lds, mp, s)
                                : launch_gs<4, false>(P, grid, C.waves, lds, mp, s))
                     : (P.x_f32 ? launch_gs<8, true>(P, grid, C.waves, lds, mp, s)
                                : launch_gs<8, false>(P, grid, C.waves, lds, mp, s));
  if (e != hipSuccess || P.ks == 1) return e;
  return launch_reduce_splits(P, s);
}

}  // namespace mi
