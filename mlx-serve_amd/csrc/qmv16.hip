// Decode-width (M <= 16 rows per item) affine quantized matmul on the gfx950
// 16x16x32 bf16 MFMA: dense qmv and gather_qmm work items.
//
// Block = W waves on one 16-row weight tile of one item; the waves split the K range.
// Each wave works alone until the final reduction -- no LDS writes and no barriers
// before it, so nothing forces the DMA queue to drain:
//   * it DMAs (global_load_lds dwordx4, 64 lanes x 16 contiguous bytes per
//     instruction) its activation slice, the scale and bias runs of its groups, and
//     its first 16-row x 256-byte weight chunk straight into its own LDS area;
//   * it then streams the weight chunks double-buffered (chunk c+1 in flight while
//     chunk c runs on the MFMAs);
//   * after every DMA has landed, the waves' partial sums are added through LDS in
//     wave order and written. Fixed summation order: deterministic.
// 16-byte slot s of LDS row r is stored at s ^ (r & 15) (weights: within the row;
// activations: within each 64-slot block of the row) so the fragment reads of 16
// rows hit distinct banks.
//
// Arithmetic per quantization group g and output (m, n):
//   4-bit: nibble q -> bf16 0x43qq = 128+q (v_perm against a 0x43 byte pool), so the
//          MFMA gives A_g = sum_k x*(128+q) and the group adds s*A_g + (b - 128 s)*X_g;
//   8-bit: byte -> bf16(q) exactly; the group adds s*A_g + b*X_g;
//   X_g = sum_k x over the group = the same MFMA against an all-ones B operand, which
//   lands already in the C layout of the output rows.
// MFMA layout (16x16x32): lane l holds 8 k values of A row l%16 / B column l%16 for
// k block l/16; C lane l register r is row 4(l/16)+r, column l%16. A lane's k blocks
// of one group are its VPL consecutive packed words; step j of a group uses word j
// (4-bit) or words 2j, 2j+1 (8-bit) of them, and the activation fragment for that
// step is the matching 8 values, nibble-permuted for 4-bit as it is read.
#include "qmv_common.h"

namespace mi {

namespace {

using namespace qmv_detail;

typedef __bf16 bf16x8q __attribute__((ext_vector_type(8)));

MI_DEV f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8q, a),
                                                  __builtin_bit_cast(bf16x8q, b), c, 0, 0, 0);
}

MI_DEV void dma16(const void* src, unsigned char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16,
                                   0, 0);
}

constexpr int kChunk = 16 * 256;  // LDS bytes of one weight chunk (16 rows x 256 B)

// Per-wave LDS plan, shared by the kernel and the host.
struct Qmv16Lds {
  int xs_row;  // 16-byte slots per staged activation row (multiple of 64)
  int xbytes;  // MP rows of activations
  int spr;     // 16-byte scale slots per weight row
  int sbytes;  // scale + bias runs (whole 64-slot DMA instructions)
  int wave;    // LDS bytes per wave
};

__host__ __device__ inline Qmv16Lds qmv16_lds(int gpw, int gs, int mp, int xbytes_per_val) {
  Qmv16Lds L;
  L.xs_row = ((gpw * gs * xbytes_per_val + 15) / 16 + 63) / 64 * 64;
  L.xbytes = mp * L.xs_row * 16;
  L.spr = (gpw + 7) / 8;
  L.sbytes = (2 * 16 * L.spr + 63) / 64 * 64 * 16;
  L.wave = 2 * kChunk + L.sbytes + L.xbytes;
  return L;
}

// MP = activation rows staged (1, 2, 4 or 16); MR = C registers kept per lane.
template <int BITS, int GS, int MP, bool XF32>
__global__ void __launch_bounds__(512) qmv16_kernel(QmvParams P) {
  constexpr int PF = 32 / BITS;
  constexpr int WPG = GS / PF;    // packed words per group per row
  constexpr int GSB = WPG * 4;    // bytes per group per row
  constexpr int UG = 256 / GSB;   // groups per chunk
  constexpr int STEPS = GS / 32;  // MFMA steps per group
  constexpr int WPS = 8 / PF;     // packed words per lane per step
  constexpr int VPL = WPG / 4;    // packed words per lane per group
  constexpr int MR = MP < 4 ? MP : 4;
  constexpr int XB = XF32 ? 4 : 2;  // activation bytes per value
  constexpr uint32_t kOnes = 0x3F803F80u;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

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
  // This wave's groups: whole chunks, so chunk starts stay multiples of UG.
  const int gpw = ((GB + W - 1) / W + UG - 1) / UG * UG;
  const int gw0 = min(g1, g0 + wave * gpw);
  const int gw1 = min(g1, gw0 + gpw);
  const int nch = (gw1 - gw0 + UG - 1) / UG;
  const Qmv16Lds L = qmv16_lds(gpw, GS, MP, XB);
  unsigned char* base = smem + (size_t)wave * L.wave;
  unsigned char* wbuf = base;               // [2][16 rows][256 B]
  unsigned char* sbuf = base + 2 * kChunk;  // [scales|biases][16 rows][spr][16 B]
  unsigned char* xbuf = sbuf + L.sbytes;    // [MP rows][xs_row slots][16 B]
  float* sred = (float*)(smem + (size_t)W * L.wave);  // [W][MR][64]
  const int arow = l16 & (MP - 1);  // A rows >= MP feed C rows that are never written
  const uint32_t c43 = 0x43434343u;

  const int n_items = P.item_count ? (int)*P.item_count : P.n_items_fixed;
  for (int itx = blockIdx.z; itx < n_items; itx += gridDim.z) {
    const Item it = decode_item(P, itx);
    const uint32_t ex = it.expert_ok ? it.expert : 0u;
    const unsigned char* tbase = (const unsigned char*)P.w + ((int64_t)ex * N) * wrow_b;

    // ---- DMA: activations, scale/bias runs, first weight chunk ------------------
    // Activations: row m, slot s (16 B of the wave's k range) -> slot-block b*64,
    // position (s % 64) ^ (m & 15). Rows without data read row 0 (don't-care).
    if (nch > 0) {
      const int nxi = MP * L.xs_row / 64;  // instructions
      for (int i = 0; i < nxi; ++i) {
        const int m = (i * 64) / L.xs_row;
        const int blk = (i * 64) % L.xs_row;            // first slot of this block
        const int sl = blk + ((lane ^ (m & 15)) & 63);  // logical slot fetched by lane
        const int64_t xr = item_x_row(P, it, m);
        const int64_t xo = (xr >= 0 ? xr : 0) + (int64_t)gw0 * GS;
        const int lim = (gw1 - gw0) * GS * XB / 16;  // valid slots
        const int64_t off = (int64_t)(sl < lim ? sl : 0) * (16 / XB);
        dma16((const unsigned char*)P.x + (xo + off) * XB, xbuf + (size_t)i * 1024);
      }
      // Scale/bias runs: slot sl of row r holds the 8 groups from
      // min(gw0 + 8 sl, G - 8) (clamped so the last row never reads past its end).
      const int nsl = 2 * 16 * L.spr;
      for (int i0 = 0; i0 < nsl; i0 += 64) {
        const int f = min(i0 + lane, nsl - 1);
        const int a = f / (16 * L.spr), r = (f / L.spr) % 16, sl = f % L.spr;
        const uint32_t nr = (uint32_t)min(tile * 16 + r, N - 1);
        const int st = min(gw0 + 8 * sl, G - 8);
        dma16((a ? P.biases : P.scales) + ((int64_t)ex * N + nr) * G + st, sbuf + i0 * 16);
      }
    }
    auto issue = [&](int c, int b) {
      const int gc = gw0 + c * UG;
      const int nslots = min(UG, gw1 - gc) * GSB / 16;  // valid 16-byte slots per row
      const int s = lane & 15;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + (lane >> 4);
        const int sl = s ^ r;
        const uint32_t nr = (uint32_t)min(tile * 16 + r, N - 1);
        dma16(tbase + nr * wrow_b + (uint32_t)gc * GSB + (sl < nslots ? sl * 16 : 0),
              wbuf + b * kChunk + i * 1024);
      }
    };

    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    const unsigned char* xrow = xbuf + (size_t)arow * L.xs_row * 16;
    const int xsw = arow & 15;
    // Activation fragment (hi, lo for fp32) for group ul (relative to gw0), step j.
    auto a_frag = [&](int ul, int j, u32x4_t& hi, u32x4_t& lo) {
      const int kk = ul * GS + (q * VPL + j * WPS) * PF;  // k offset in the wave range
      const int c = kk * XB / 16;                         // logical 16-byte slot
      const int pc = (c & ~63) + ((c & 63) ^ xsw);
      if constexpr (XF32) {
        const int pc1 = ((c + 1) & ~63) + (((c + 1) & 63) ^ xsw);
        float v[8];
        *(u32x4_t*)&v[0] = *(const u32x4_t*)(xrow + pc * 16);
        *(u32x4_t*)&v[4] = *(const u32x4_t*)(xrow + pc1 * 16);
        uint32_t h[8], l[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          h[t] = f32_to_bf16_bits(v[t]);
          l[t] = f32_to_bf16_bits(v[t] - bf16_bits_to_f32(h[t]));
        }
        hi = a_perm<BITS>(u32x4_t{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16,
                                  h[6] | h[7] << 16});
        lo = a_perm<BITS>(u32x4_t{l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16,
                                  l[6] | l[7] << 16});
      } else {
        hi = a_perm<BITS>(*(const u32x4_t*)(xrow + pc * 16));
      }
    };
    auto compute = [&](int c, int b) {
      const int gc = gw0 + c * UG;
      const int ng = min(UG, gw1 - gc);
      const unsigned char* myrow = wbuf + b * kChunk + l16 * 256;
      auto load_words = [&](int u, uint32_t (&words)[VPL]) {
        const int byte0 = u * GSB + q * VPL * 4;
        if constexpr (VPL >= 4) {
#pragma unroll
          for (int t = 0; t < VPL / 4; ++t) {
            const int slot = (byte0 >> 4) + t;
            const u32x4_t v = *(const u32x4_t*)(myrow + ((slot ^ l16) << 4));
            words[4 * t] = v.x; words[4 * t + 1] = v.y; words[4 * t + 2] = v.z;
            words[4 * t + 3] = v.w;
          }
        } else if constexpr (VPL == 2) {
          const u32x2_t v =
              *(const u32x2_t*)(myrow + (((byte0 >> 4) ^ l16) << 4) + (byte0 & 15));
          words[0] = v.x; words[1] = v.y;
        } else {
          words[0] = *(const uint32_t*)(myrow + (((byte0 >> 4) ^ l16) << 4) + (byte0 & 15));
        }
      };
      auto group = [&](int u, const uint32_t (&words)[VPL], f32x4_t& a, f32x4_t& xs) {
        const int ul = gc + u - gw0;
        const u32x4_t ones = {kOnes, kOnes, kOnes, kOnes};
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
          u32x4_t Ah, Al;
          a_frag(ul, j, Ah, Al);
          const u32x4_t B = b_frag<BITS>(words, j, c43);
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
          a = mfma16(Ah, B, j == 0 ? z : a);
          xs = mfma16(Ah, ones, j == 0 ? z : xs);
          if constexpr (XF32) {
            a = mfma16(Al, B, a);
            xs = mfma16(Al, ones, xs);
          }
        }
      };
      auto epilogue = [&](int u, const f32x4_t& a, const f32x4_t& xs) {
        const int g = gc + u, sl = (g - gw0) >> 3;
        const int gi = (sl * 8 + (g - min(gw0 + 8 * sl, G - 8))) * 2;  // byte in row run
        const float sc = bf16_bits_to_f32(*(const uint16_t*)(sbuf + (l16 * L.spr) * 16 + gi));
        const float bi =
            bf16_bits_to_f32(*(const uint16_t*)(sbuf + ((16 + l16) * L.spr) * 16 + gi));
        const float bb = (BITS == 4) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r] = fmaf(bb, xs[r], fmaf(sc, a[r], acc[r]));
      };
#pragma unroll
      for (int u = 0; u < UG; u += 2) {
        if (u + 1 < ng) {
          uint32_t w0[VPL], w1[VPL];
          load_words(u, w0);
          load_words(u + 1, w1);
          f32x4_t a0, a1, x0, x1;
          group(u, w0, a0, x0);
          group(u + 1, w1, a1, x1);
          epilogue(u, a0, x0);
          epilogue(u + 1, a1, x1);
        } else if (u < ng) {
          uint32_t w0[VPL];
          load_words(u, w0);
          f32x4_t a0, x0;
          group(u, w0, a0, x0);
          epilogue(u, a0, x0);
        }
      }
    };

    if (nch > 0) {
      // Chunk c (and, for c = 0, everything issued before it) has landed once only
      // chunk c+1's 4 DMAs may still be pending.
      issue(0, 0);
      int c = 0;
      for (; c + 2 < nch; c += 2) {
        issue(c + 1, 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        compute(c, 0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // buffer 0 reads done before reuse
        issue(c + 2, 0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        compute(c + 1, 1);
        __builtin_amdgcn_s_waitcnt(0xC07F);
      }
      if (c + 1 < nch) {
        issue(c + 1, 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        compute(c, 0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        compute(c + 1, 1);
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        compute(c, 0);
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
      if (nn >= N || li >= it.cnt) continue;
      const int64_t xr = item_x_row(P, it, li);
      if (xr == -1) continue;
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

// Scale/bias runs are 8-group (16-byte) DMAs from even group offsets.
bool qmv16_supported(int K, int gs, int bits) {
  const int G = K / gs;
  return qmv16_groups_per_chunk(bits, gs) <= 8 && G >= 8 && G % 2 == 0;
}

size_t qmv16_lds_bytes(int groups, int gs, int bits, int mp, int x_f32, int waves) {
  const int ug = qmv16_groups_per_chunk(bits, gs);
  const int gpw = ((groups + waves - 1) / waves + ug - 1) / ug * ug;
  const Qmv16Lds L = qmv16_lds(gpw, gs, mp, x_f32 ? 4 : 2);
  const int mr = mp < 4 ? mp : 4;
  return (size_t)waves * L.wave + (size_t)waves * mr * 64 * 4;
}

hipError_t launch_qmv16(const QmvParams& P, const QmvConfig& C, hipStream_t s) {
  dim3 grid((unsigned)P.row_blocks, (unsigned)P.ks, (unsigned)C.grid_z);
  const int mp = qmv16_mp_for_rows(C.rows);
  const size_t lds = qmv16_lds_bytes(P.gps, P.group_size, P.bits, mp, P.x_f32, C.waves);
  hipError_t e = (P.bits == 4)
                     ? (P.x_f32 ? launch_gs<4, true>(P, grid, C.waves, lds, mp, s)
                                : launch_gs<4, false>(P, grid, C.waves, lds, mp, s))
                     : (P.x_f32 ? launch_gs<8, true>(P, grid, C.waves, lds, mp, s)
                                : launch_gs<8, false>(P, grid, C.waves, lds, mp, s));
  if (e != hipSuccess || P.ks == 1) return e;
  return launch_reduce_splits(P, s);
}

}  // namespace mi
