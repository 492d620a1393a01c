// Small-M affine quantized matmul on gfx950 MFMA: dense qmv (decode, M <= 32 rows
// per pass) and gather_qmm over (expert, row-chunk) work items.
//
// Semantics: y[p, n] = sum_k x[row(p), k] * (scale[e,n,g] * q[e,n,k] + bias[e,n,g])
// with fp32 accumulation (MLX quantized_matmul / gather_qmm, transpose=true, affine).
//
// Arithmetic, per quantization group g of GS values and per output (m, n):
//   4-bit: each nibble q becomes the bf16 value 128+q with one v_and_or_b32 per pair
//          (0x4300 | q is exactly 128+q), so the MFMA computes
//          A_g = sum_k x*(128+q) and the group contributes s*A_g + (b - 128 s)*X_g.
//   8-bit: each byte becomes bf16(q) exactly; contribution s*A_g + b*X_g.
//   X_g = sum_k x over the group comes from the same MFMA against an all-ones B.
// The 16x16x32 bf16 MFMA contracts 32 k per instruction: lane l holds 8 k values of
// A row (l%16) and of B column (l%16) for k-block (l/16); C lane l holds rows
// 4*(l/16)+r, column l%16. Within a k-block the order of the 8 k values is free as
// long as A and B agree, which is what lets the nibble unpack skip shuffles: the
// activation fragment is permuted once per group and shared by every weight tile.
//
// Work decomposition: block = W waves splitting the group range of K (split-K inside
// the block, reduced through LDS, deterministic); each wave covers RT tiles of 16
// output rows (weights streamed once) and MT tiles of 16 activation rows.
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {

namespace {

constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;

template <int VPL>
MI_DEV void load_words(const uint32_t* __restrict__ p, uint32_t (&out)[VPL]) {
  if constexpr (VPL == 1) {
    out[0] = __builtin_nontemporal_load(p);
  } else if constexpr (VPL == 2) {
    u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < VPL / 4; ++i) {
      u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p) + i);
      out[4 * i + 0] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  }
}

// A fragment for one 8-value k-block of activations (bf16 bits, natural order).
template <int BITS>
MI_DEV u32x4_t a_frag(u32x4_t X) {
  if constexpr (BITS == 4) {
    // Nibble unpack yields k order [0,4,1,5,2,6,3,7]; permute x to match.
    u32x4_t A;
    A.x = perm_b32(X.z, X.x, 0x05040100u);
    A.y = perm_b32(X.z, X.x, 0x07060302u);
    A.z = perm_b32(X.w, X.y, 0x05040100u);
    A.w = perm_b32(X.w, X.y, 0x07060302u);
    return A;
  } else {
    return X;
  }
}

// B fragment for k-block j of a lane's packed words.
template <int BITS>
MI_DEV u32x4_t b_frag(const uint32_t* words, int j) {
  u32x4_t B;
  if constexpr (BITS == 4) {
    const uint32_t w = words[j];
    B.x = (w & 0x000F000Fu) | 0x43004300u;
    B.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    B.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    B.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  } else {
    const uint32_t w0 = words[2 * j], w1 = words[2 * j + 1];
    // Bytes are exact in bf16, so the fp32 value's upper half is the bf16 value.
    const uint32_t f0 = __float_as_uint((float)(w0 & 0xFFu));
    const uint32_t f1 = __float_as_uint((float)((w0 >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((w0 >> 16) & 0xFFu));
    const uint32_t f3 = __float_as_uint((float)(w0 >> 24));
    const uint32_t f4 = __float_as_uint((float)(w1 & 0xFFu));
    const uint32_t f5 = __float_as_uint((float)((w1 >> 8) & 0xFFu));
    const uint32_t f6 = __float_as_uint((float)((w1 >> 16) & 0xFFu));
    const uint32_t f7 = __float_as_uint((float)(w1 >> 24));
    B.x = perm_b32(f1, f0, 0x07060302u);
    B.y = perm_b32(f3, f2, 0x07060302u);
    B.z = perm_b32(f5, f4, 0x07060302u);
    B.w = perm_b32(f7, f6, 0x07060302u);
  }
  return B;
}

// Split an fp32 8-vector into bf16 hi + bf16 lo (x = hi + lo to ~2^-16 relative).
MI_DEV void split_f32(const float* v, u32x4_t& hi, u32x4_t& lo) {
  uint32_t h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = f32_to_bf16_bits(v[i]);
    l[i] = f32_to_bf16_bits(v[i] - bf16_bits_to_f32(h[i]));
  }
  hi = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  lo = u32x4_t{l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16)};
}

struct RowMap {
  int64_t pos0;  // first flattened (pair, m) position of the item
  int cnt;       // valid positions in the item (<= 16*MT)
  uint32_t expert;
  bool expert_ok;
};

MI_DEV RowMap decode_item(const QmvParams& P, int it) {
  RowMap r;
  if (P.items) {
    const uint32_t* e = P.items + 4 * (int64_t)it;
    r.expert = e[0];
    r.pos0 = (int64_t)e[1];
    r.cnt = (int)e[2];
  } else {
    const int64_t pair = it / P.items_per_pair;
    const int c = it - (int)(pair * P.items_per_pair);
    r.pos0 = pair * P.M + (int64_t)c * P.rows_per_item;
    r.cnt = min(P.rows_per_item, P.M - c * P.rows_per_item);
    r.expert = P.rhs ? P.rhs[pair] : (uint32_t)pair;
  }
  r.expert_ok = r.expert < (uint32_t)P.n_experts;
  return r;
}

// Row li of an item is real when inside the item's limit and, for sorted work
// items, while its pair still belongs to the item's expert run.
MI_DEV bool row_valid(const QmvParams& P, const RowMap& rm, int li) {
  if (li >= rm.cnt) return false;
  if (P.items) return P.rhs[(rm.pos0 + li) / P.M] == rm.expert;
  return true;
}

// x row for flattened position p, or -1 when the lhs index is out of range.
MI_DEV int64_t x_row_of(const QmvParams& P, int64_t p) {
  const int64_t pair = p / P.M;
  const int64_t m = p - pair * P.M;
  const int64_t l = P.lhs ? (int64_t)P.lhs[pair] : pair / P.lhs_div;
  return (l < P.x_batch) ? l * P.M + m : -1;
}

template <int BITS, int GS, int MT, int R4, int RT, bool XF32>
__global__ void __launch_bounds__(512) qmv_kernel(QmvParams P) {
  constexpr int WPG = GS * BITS / 32;  // packed words per group per row
  constexpr int VPL = WPG / 4;         // words per lane per group
  constexpr int STEPS = GS / 32;       // MFMA k-blocks per group
  constexpr int CH = GS / 4;           // activation values per lane per group
  constexpr int SLOTS = RT * MT * R4;
  extern __shared__ float red[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int W = blockDim.x >> 6;
  const int ln = lane & 15, q = lane >> 4;
  const int K = P.K, N = P.N;
  const int G = K / GS;
  const int64_t wrow = (int64_t)K * BITS / 32;  // words per weight row
  const int g0 = (int)((int64_t)wave * G / W), g1 = (int)((int64_t)(wave + 1) * G / W);
  const int n_base = blockIdx.x * (RT * 16);

  const int n_items = P.item_count ? (int)*P.item_count : P.n_items_fixed;
  for (int it = blockIdx.y; it < n_items; it += gridDim.y) {
    const RowMap rm = decode_item(P, it);
    const uint32_t ex = rm.expert_ok ? rm.expert : 0u;

    // Per-lane activation row pointers (A rows = ln of each m-tile).
    const char* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int li = mt * 16 + ln;
      int64_t xr = -1;
      if (row_valid(P, rm, li)) xr = x_row_of(P, rm.pos0 + li);
      xrow[mt] = (xr >= 0) ? (const char*)P.x + xr * (int64_t)K * (XF32 ? 4 : 2) : nullptr;
    }
    // Per-lane weight rows (B columns = ln of each row tile).
    const uint32_t* wp[RT];
    const uint16_t* sp[RT];
    const uint16_t* bp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = min(n_base + rt * 16 + ln, N - 1);
      const int64_t row = (int64_t)ex * N + n;
      wp[rt] = P.w + row * wrow + q * VPL;
      sp[rt] = P.scales + row * G;
      bp[rt] = P.biases + row * G;
    }

    float acc[RT][MT][R4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < R4; ++r) acc[rt][mt][r] = 0.f;

    uint32_t wcur[RT][VPL];
    uint32_t scur[RT], bcur[RT];
    if (g0 < g1) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        load_words<VPL>(wp[rt] + (int64_t)g0 * WPG, wcur[rt]);
        scur[rt] = sp[rt][g0];
        bcur[rt] = bp[rt][g0];
      }
    }
    for (int g = g0; g < g1; ++g) {
      uint32_t wnext[RT][VPL];
      uint32_t snext[RT], bnext[RT];
      if (g + 1 < g1) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          load_words<VPL>(wp[rt] + (int64_t)(g + 1) * WPG, wnext[rt]);
          snext[rt] = sp[rt][g + 1];
          bnext[rt] = bp[rt][g + 1];
        }
      }
      // Activation fragments for this group (shared by all RT weight tiles).
      f32x4_t xs[MT];
      f32x4_t accg[RT][MT];
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        u32x4_t Ahi[MT], Alo[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          u32x4_t X = {0u, 0u, 0u, 0u}, Xl = {0u, 0u, 0u, 0u};
          if (xrow[mt]) {
            const int64_t k0 = (int64_t)g * GS + q * CH + j * 8;
            if constexpr (XF32) {
              const float* xp = (const float*)xrow[mt] + k0;
              float v[8];
              *(float4*)&v[0] = *(const float4*)xp;
              *(float4*)&v[4] = *(const float4*)(xp + 4);
              split_f32(v, X, Xl);
            } else {
              X = *(const u32x4_t*)((const uint16_t*)xrow[mt] + k0);
            }
          }
          Ahi[mt] = a_frag<BITS>(X);
          if constexpr (XF32) Alo[mt] = a_frag<BITS>(Xl);
        }
        const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4_t c0 = (j == 0) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : xs[mt];
          xs[mt] = mfma16x16x32(as_bf16x8(Ahi[mt]), as_bf16x8(ones), c0);
          if constexpr (XF32) xs[mt] = mfma16x16x32(as_bf16x8(Alo[mt]), as_bf16x8(ones), xs[mt]);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const u32x4_t B = b_frag<BITS>(wcur[rt], j);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x4_t c0 = (j == 0) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : accg[rt][mt];
            accg[rt][mt] = mfma16x16x32(as_bf16x8(Ahi[mt]), as_bf16x8(B), c0);
            if constexpr (XF32)
              accg[rt][mt] = mfma16x16x32(as_bf16x8(Alo[mt]), as_bf16x8(B), accg[rt][mt]);
          }
        }
      }
      // Group epilogue: acc += s * A_g + b' * X_g.
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float s = bf16_bits_to_f32(scur[rt]);
        const float b = bf16_bits_to_f32(bcur[rt]);
        const float bb = (BITS == 4) ? fmaf(-128.f, s, b) : b;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < R4; ++r)
            acc[rt][mt][r] = fmaf(bb, xs[mt][r], fmaf(s, accg[rt][mt][r], acc[rt][mt][r]));
      }
      if (g + 1 < g1) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
          for (int v = 0; v < VPL; ++v) wcur[rt][v] = wnext[rt][v];
          scur[rt] = snext[rt];
          bcur[rt] = bnext[rt];
        }
      }
    }

    // Split-K reduction across the block's waves, then write.
    if (W > 1) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < R4; ++r)
            red[(wave * SLOTS + (rt * MT + mt) * R4 + r) * 64 + lane] = acc[rt][mt][r];
      __syncthreads();
    }
    for (int idx = threadIdx.x; idx < SLOTS * 64; idx += blockDim.x) {
      const int slot = idx >> 6, l2 = idx & 63;
      float v;
      if (W > 1) {
        v = 0.f;
        for (int w2 = 0; w2 < W; ++w2) v += red[(w2 * SLOTS + slot) * 64 + l2];
      } else {
        // W == 1: the thread owns its own slots (blockDim == 64, idx == slot*64+lane).
        const int rt = slot / (MT * R4), rem = slot % (MT * R4);
        v = 0.f;
#pragma unroll
        for (int rt2 = 0; rt2 < RT; ++rt2)
#pragma unroll
          for (int mt2 = 0; mt2 < MT; ++mt2)
#pragma unroll
            for (int r2 = 0; r2 < R4; ++r2)
              if (rt2 == rt && mt2 * R4 + r2 == rem) v = acc[rt2][mt2][r2];
      }
      const int rt = slot / (MT * R4), rem = slot % (MT * R4);
      const int mt = rem / R4, r = rem % R4;
      const int li = mt * 16 + 4 * (l2 >> 4) + r;
      const int n = n_base + rt * 16 + (l2 & 15);
      if (n < N && row_valid(P, rm, li)) {
        const int64_t p = rm.pos0 + li;
        const bool ok = rm.expert_ok && x_row_of(P, p) >= 0;
        if (!ok) v = __builtin_nanf("");
        if constexpr (XF32)
          ((float*)P.y)[p * N + n] = v;
        else
          ((uint16_t*)P.y)[p * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
    if (W > 1) __syncthreads();
  }
}

template <int BITS, int GS, int MT, int R4, int RT, bool XF32>
hipError_t launch_t(const QmvParams& P, dim3 grid, int W, hipStream_t s) {
  constexpr int SLOTS = RT * MT * R4;
  const size_t lds = (W > 1) ? (size_t)W * SLOTS * 64 * sizeof(float) : 0;
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, MT, R4, RT, XF32>), grid, dim3(64 * W), lds, s, P);
  return hipGetLastError();
}

template <int BITS, int GS, int MT, int R4, bool XF32>
hipError_t launch_rt(const QmvParams& P, dim3 grid, int W, int RT, hipStream_t s) {
  switch (RT) {
    case 1: return launch_t<BITS, GS, MT, R4, 1, XF32>(P, grid, W, s);
    case 2: return launch_t<BITS, GS, MT, R4, 2, XF32>(P, grid, W, s);
    default: return launch_t<BITS, GS, MT, R4, 4, XF32>(P, grid, W, s);
  }
}

template <int BITS, int GS, bool XF32>
hipError_t launch_m(const QmvParams& P, dim3 grid, int W, int RT, int rows, hipStream_t s) {
  if (rows <= 1) return launch_rt<BITS, GS, 1, 1, XF32>(P, grid, W, RT, s);
  if (rows <= 2) return launch_rt<BITS, GS, 1, 2, XF32>(P, grid, W, RT, s);
  if (rows <= 16) return launch_rt<BITS, GS, 1, 4, XF32>(P, grid, W, RT, s);
  return launch_rt<BITS, GS, 2, 4, XF32>(P, grid, W, RT, s);
}

template <int BITS, bool XF32>
hipError_t launch_gs(const QmvParams& P, dim3 grid, int W, int RT, int rows, int gs,
                     hipStream_t s) {
  switch (gs) {
    case 32: return launch_m<BITS, 32, XF32>(P, grid, W, RT, rows, s);
    case 64: return launch_m<BITS, 64, XF32>(P, grid, W, RT, rows, s);
    default: return launch_m<BITS, 128, XF32>(P, grid, W, RT, rows, s);
  }
}

}  // namespace

hipError_t launch_qmv(const QmvParams& P, const QmvConfig& C, hipStream_t s) {
  dim3 grid((unsigned)C.row_groups, (unsigned)C.grid_y);
  if (P.bits == 4)
    return P.x_f32 ? launch_gs<4, true>(P, grid, C.waves, C.rt, C.rows, P.group_size, s)
                   : launch_gs<4, false>(P, grid, C.waves, C.rt, C.rows, P.group_size, s);
  return P.x_f32 ? launch_gs<8, true>(P, grid, C.waves, C.rt, C.rows, P.group_size, s)
                 : launch_gs<8, false>(P, grid, C.waves, C.rt, C.rows, P.group_size, s);
}

}  // namespace mi
