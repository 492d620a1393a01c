// Small-M affine quantized matmul on gfx950: dense qmv (decode) and gather_qmm over
// (expert, <=32-row) work items, on the 32x32x16 bf16 MFMA.
//
// Semantics: y[p, n] = sum_k x[row(p), k] * (scale[e,n,g] * q[e,n,k] + bias[e,n,g]),
// fp32 accumulation (MLX quantized_matmul / gather_qmm, transpose=true, affine).
//
// Arithmetic per quantization group g (GS values of k) and output (m, n):
//   4-bit: a nibble q becomes the bf16 value 128+q (bits 0x43qq, built with v_perm
//          from the masked word), the MFMA gives A_g = sum_k x*(128+q), and
//          the group adds s*A_g + (b - 128 s)*X_g.
//   8-bit: a byte becomes bf16(q) exactly; the group adds s*A_g + b*X_g.
//   X_g = sum_k x over the group, computed once per block while staging x.
// 32x32x16 layout: lane l holds 8 k values of A row (l%32) / B column (l%32) for
// k-half (l/32); C lane l register r is row 8(r/4)+4(l/32)+r%4, column l%32. A lane's
// share of one group of one weight row is contiguous (GS/2 values), so weights
// stream as 16-byte loads. Inside a k-half the order of the 8 values is free as long
// as A and B agree: x is permuted once, at staging, to the nibble-unpack order.
//
// Work decomposition: grid (32-row weight tile, K range, item). A block's W waves
// share one weight tile and split its K range; the activations of the range are
// staged once into LDS (fragment order + group sums); the waves' partials are
// summed through LDS in wave order. K ranges beyond one per block (activations too
// large for LDS) are summed by a second, elementwise kernel in range order. Every
// sum has a fixed order, so results are deterministic.
#include "mi_common.h"
#include "mi_internal.h"

// Packed words per lane per load chunk (one chunk is in flight while one computes).
#ifndef MI_QMV_CW
#define MI_QMV_CW 32
#endif

namespace mi {

namespace {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

MI_DEV f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                  __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
}

template <int N>
MI_DEV void load_u32(const uint32_t* __restrict__ p, uint32_t (&out)[N]) {
  if constexpr (N == 2) {
    u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p) + i);
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  }
}

// 4-bit unpack: lo = w & 0x0F0F0F0F holds nibbles 0,2,4,6 in its bytes, hi the odd
// ones; v_perm pairs each nibble byte with a 0x43 byte, giving bf16 0x43qq = 128+q.
// Fragment k order is therefore [0,2,4,6,1,3,5,7]; activations are permuted to match.
template <int BITS>
MI_DEV u32x4_t a_perm(u32x4_t X) {
  if constexpr (BITS == 4) {
    return u32x4_t{perm_b32(X.y, X.x, 0x05040100u), perm_b32(X.w, X.z, 0x05040100u),
                   perm_b32(X.y, X.x, 0x07060302u), perm_b32(X.w, X.z, 0x07060302u)};
  } else {
    return X;
  }
}

// B fragment (8 k values of one weight row) for MFMA step j of a lane's words.
template <int BITS>
MI_DEV u32x4_t b_frag(const uint32_t* words, int j, uint32_t c43) {
  if constexpr (BITS == 4) {
    const uint32_t w = words[j];
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    return u32x4_t{perm_b32(c43, lo, 0x04010400u), perm_b32(c43, lo, 0x04030402u),
                   perm_b32(c43, hi, 0x04010400u), perm_b32(c43, hi, 0x04030402u)};
  } else {
    const uint32_t w0 = words[2 * j], w1 = words[2 * j + 1];
    // Bytes are exact in bf16: the fp32 value's upper half is the bf16 value.
    const uint32_t f0 = __float_as_uint((float)(w0 & 0xFFu));
    const uint32_t f1 = __float_as_uint((float)((w0 >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((w0 >> 16) & 0xFFu));
    const uint32_t f3 = __float_as_uint((float)(w0 >> 24));
    const uint32_t f4 = __float_as_uint((float)(w1 & 0xFFu));
    const uint32_t f5 = __float_as_uint((float)((w1 >> 8) & 0xFFu));
    const uint32_t f6 = __float_as_uint((float)((w1 >> 16) & 0xFFu));
    const uint32_t f7 = __float_as_uint((float)(w1 >> 24));
    return u32x4_t{perm_b32(f1, f0, 0x07060302u), perm_b32(f3, f2, 0x07060302u),
                   perm_b32(f5, f4, 0x07060302u), perm_b32(f7, f6, 0x07060302u)};
  }
}

struct Item {
  int64_t pos0;  // first flattened (pair, m) position
  int cnt;       // positions in this item (<= 32)
  uint32_t expert;
  bool expert_ok;
};

MI_DEV Item decode_item(const QmvParams& P, int it) {
  Item r;
  if (P.items) {
    const uint32_t* e = P.items + 4 * (int64_t)it;
    r.expert = e[0];
    r.pos0 = (int64_t)e[1];
    r.cnt = (int)e[2];
  } else {
    const int64_t pair = it / P.items_per_pair;
    const int c = it - (int)(pair * P.items_per_pair);
    r.pos0 = pair * P.M + (int64_t)c * 32;
    r.cnt = min(32, P.M - c * 32);
    r.expert = P.rhs ? P.rhs[pair] : (uint32_t)pair;
  }
  r.expert_ok = r.expert < (uint32_t)P.n_experts;
  return r;
}

// Element offset of x's row for item row li; -1: not a row of this item; -2: the
// row exists but its lhs index is out of range (NaN output). Sorted items keep a
// row only while its pair's rhs is the item's expert.
MI_DEV int64_t item_x_row(const QmvParams& P, const Item& it, int li) {
  if (li >= it.cnt) return -1;
  const int64_t p = it.pos0 + li;
  const int64_t pair = p / P.M;
  if (P.items && P.rhs[pair] != it.expert) return -1;
  const int64_t m = p - pair * P.M;
  const int64_t l = P.lhs ? (int64_t)P.lhs[pair] : pair / P.lhs_div;
  if (l >= P.x_batch) return -2;
  return (l * P.M + m) * (int64_t)P.K;
}

// One block = W waves on one 32-row weight tile of one item over one K range.
// The K range's activations are staged into LDS once (fragment order, group sums),
// the waves split the range's groups between them, stream their weights as 16-byte
// loads one chunk ahead, and the block sums the waves' partials through LDS in wave
// order. With a single K range the block writes y; otherwise it writes an fp32
// partial that reduce_splits_kernel sums in split order.
template <int BITS, int GS, int MR, bool XF32>
__global__ void __launch_bounds__(512) qmv_kernel(QmvParams P) {
  constexpr int PF = 32 / BITS;
  constexpr int WPG = GS / PF;    // packed words per group per row
  constexpr int VPL = WPG / 2;    // words per lane per group (one k-half)
  constexpr int STEPS = GS / 16;  // MFMA steps per group
  constexpr int UG = VPL >= MI_QMV_CW ? 1 : MI_QMV_CW / VPL;  // groups per chunk
  constexpr int MPAD = MR == 1 ? 1 : MR == 2 ? 2 : MR == 4 ? 8 : MR == 8 ? 16 : 32;
  constexpr int MXS = MPAD < 8 ? 8 : MPAD;  // group-sum row stride (b128 reads)
  constexpr int PLANES = XF32 ? 2 : 1;
  constexpr int FB = 4;                     // staging fragments per thread per pass

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int64_t srow[32];

  const int tid = threadIdx.x;
  const int BD = blockDim.x, W = BD >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int l32 = lane & 31, hh = lane >> 5;
  const int K = P.K, N = P.N;
  const int G = K / GS;
  const int64_t wrow = (int64_t)K / PF;
  const int rb = blockIdx.x, ks = blockIdx.y;
  const int g0 = ks * P.gps;
  const int g1 = min(G, g0 + P.gps);
  const int GB = g1 - g0;                        // groups staged by this block
  const int NF = GB * STEPS * 2 * MPAD;          // A fragments staged
  u32x4_t* sx = (u32x4_t*)smem;                  // [GB][STEPS][2][MPAD] (+ lo plane)
  float* sxs = (float*)(sx + (size_t)NF * PLANES);  // [GB][MXS]
  float* sred = (float*)smem;                    // reused after the main loop
  const uint32_t c43 = 0x43434343u;  // byte pool for the 4-bit unpack
  // This wave's share of the block's groups.
  const int gw0 = g0 + (int)((int64_t)GB * wave / W);
  const int gw1 = g0 + (int)((int64_t)GB * (wave + 1) / W);

  const int n_items = P.item_count ? (int)*P.item_count : P.n_items_fixed;
  for (int itx = blockIdx.z; itx < n_items; itx += gridDim.z) {
    const Item it = decode_item(P, itx);
    const uint32_t ex = it.expert_ok ? it.expert : 0u;
    if (tid < 32) srow[tid] = item_x_row(P, it, tid);

    // Uniform (SGPR) expert bases plus 32-bit per-lane byte offsets, so loads use
    // the saddr form and per-group addresses are scalar adds.
    const int n = min(rb * 32 + l32, N - 1);
    const uint32_t* wbase = P.w + (int64_t)ex * N * wrow;
    const uint16_t* sbase = P.scales + (int64_t)ex * N * G;
    const uint16_t* bbase = P.biases + (int64_t)ex * N * G;
    const uint32_t woff = (uint32_t)(((int64_t)n * wrow + hh * VPL) * 4);
    const uint32_t soff = (uint32_t)((int64_t)n * G * 2);

    uint32_t wcur[UG][VPL], scur[UG], bcur[UG];
    auto load_chunk = [&](int gc, uint32_t (&wv)[UG][VPL], uint32_t (&sv)[UG],
                          uint32_t (&bv)[UG]) {
#pragma unroll
      for (int u = 0; u < UG; ++u) {
        const int g = min(gc + u, gw1 - 1);
        load_u32<VPL>((const uint32_t*)((const char*)(wbase + (int64_t)g * WPG) + woff), wv[u]);
        sv[u] = *(const uint16_t*)((const char*)(sbase + g) + soff);
        bv[u] = *(const uint16_t*)((const char*)(bbase + g) + soff);
      }
    };
    // First chunk's weights go out before the staging so both latencies overlap.
    if (gw0 < gw1) load_chunk(gw0, wcur, scur, bcur);
    __syncthreads();  // srow visible

    // ---- stage x[rows][g0*GS, g1*GS) into LDS ---------------------------------
    for (int base = 0; base < NF; base += FB * BD) {
      u32x4_t v[FB][PLANES];
      float sum[FB];
#pragma unroll
      for (int i = 0; i < FB; ++i) {
        const int f = base + i * BD + tid;
        const int s = f % (2 * STEPS), m = (f / (2 * STEPS)) % MPAD;
        const int u = f / (2 * STEPS * MPAD);
        const int64_t xr = (f < NF) ? srow[m] : -1;
        const bool ok = xr >= 0;
        const int64_t k0 =
            ok ? xr + (int64_t)(g0 + u) * GS + (s & 1) * (GS / 2) + 8 * (s >> 1) : 0;
        if constexpr (XF32) {
          const u32x4_t* xp = (const u32x4_t*)((const float*)P.x + k0);
          const u32x4_t a = xp[0], b = xp[1];
          float e[8];
          *(u32x4_t*)&e[0] = ok ? a : u32x4_t{0u, 0u, 0u, 0u};
          *(u32x4_t*)&e[4] = ok ? b : u32x4_t{0u, 0u, 0u, 0u};
          uint32_t hi[8], lo[8];
          float sm = 0.f;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            hi[q] = f32_to_bf16_bits(e[q]);
            lo[q] = f32_to_bf16_bits(e[q] - bf16_bits_to_f32(hi[q]));
            sm += e[q];
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
        const int s = f % (2 * STEPS), m = (f / (2 * STEPS)) % MPAD;
        const int u = f / (2 * STEPS * MPAD);
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
        // Group sum over the 2*STEPS consecutive lanes holding one (u, m).
#pragma unroll
        for (int d = 1; d < 2 * STEPS; d <<= 1) sm += __shfl_xor(sm, d, 64);
        if (f < NF) {
          const int idx = ((u * STEPS + (s >> 1)) * 2 + (s & 1)) * MPAD + m;
          sx[idx] = a_perm<BITS>(v[i][0]);
          if constexpr (XF32) sx[NF + idx] = a_perm<BITS>(v[i][PLANES - 1]);
          if (s == 0) sxs[u * MXS + m] = sm;
        }
      }
    }
    if constexpr (MPAD < MXS) {
      for (int t = tid; t < GB * (MXS - MPAD); t += BD)
        sxs[(t / (MXS - MPAD)) * MXS + MPAD + t % (MXS - MPAD)] = 0.f;
    }
    __syncthreads();

    // ---- this wave's groups -----------------------------------------------------
    // A rows >= MPAD read row (l32 % MPAD): those C rows are never written, so the
    // values are don't-care and the LDS reads need no mask.
    const int arow = l32 & (MPAD - 1);
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    auto group_mfma = [&](int ul, const uint32_t* words, f32x16_t& accg) {
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        const int idx = ((ul * STEPS + j) * 2 + hh) * MPAD + arow;
        const u32x4_t B = b_frag<BITS>(words, j, c43);
        accg = mfma32(sx[idx], B, j == 0 ? f32x16_t{} : accg);
        if constexpr (XF32) accg = mfma32(sx[NF + idx], B, accg);
      }
    };
    auto group_epilogue = [&](int ul, uint32_t sbits, uint32_t bbits, const f32x16_t& accg) {
      float xs[MR];
#pragma unroll
      for (int r4 = 0; r4 < (MR + 3) / 4; ++r4) {
        const f32x4_t v4 = *(const f32x4_t*)&sxs[ul * MXS + 8 * r4 + 4 * hh];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * r4 + e < MR) xs[4 * r4 + e] = v4[e];
      }
      const float sc = bf16_bits_to_f32(sbits);
      const float bi = bf16_bits_to_f32(bbits);
      const float bb = (BITS == 4) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] = fmaf(bb, xs[r], fmaf(sc, accg[r], acc[r]));
    };
    for (int gc = gw0; gc < gw1; gc += UG) {
      const bool more = gc + UG < gw1;
      uint32_t wnx[UG][VPL], snx[UG], bnx[UG];
      if (more) load_chunk(gc + UG, wnx, snx, bnx);
      // Two groups at a time: their MFMA chains are independent and interleave.
#pragma unroll
      for (int u = 0; u < UG; u += 2) {
        const int ul = gc + u - g0;
        if (gc + u + 1 < gw1 && u + 1 < UG) {
          f32x16_t a0, a1;
#pragma unroll
          for (int j = 0; j < STEPS; ++j) {
            const int i0 = ((ul * STEPS + j) * 2 + hh) * MPAD + arow;
            const int i1 = (((ul + 1) * STEPS + j) * 2 + hh) * MPAD + arow;
            const u32x4_t B0 = b_frag<BITS>(wcur[u], j, c43);
            const u32x4_t B1 = b_frag<BITS>(wcur[u + 1 < UG ? u + 1 : u], j, c43);
            a0 = mfma32(sx[i0], B0, j == 0 ? f32x16_t{} : a0);
            a1 = mfma32(sx[i1], B1, j == 0 ? f32x16_t{} : a1);
            if constexpr (XF32) {
              a0 = mfma32(sx[NF + i0], B0, a0);
              a1 = mfma32(sx[NF + i1], B1, a1);
            }
          }
          group_epilogue(ul, scur[u], bcur[u], a0);
          group_epilogue(ul + 1, scur[u + 1 < UG ? u + 1 : u], bcur[u + 1 < UG ? u + 1 : u], a1);
        } else if (gc + u < gw1) {
          f32x16_t a0;
          group_mfma(ul, wcur[u], a0);
          group_epilogue(ul, scur[u], bcur[u], a0);
        }
      }
      if (more) {
#pragma unroll
        for (int u = 0; u < UG; ++u) {
#pragma unroll
          for (int q = 0; q < VPL; ++q) wcur[u][q] = wnx[u][q];
          scur[u] = snx[u];
          bcur[u] = bnx[u];
        }
      }
    }

    // ---- reduce the waves' partials (wave order), write --------------------------
    __syncthreads();  // staging area is reused
#pragma unroll
    for (int r = 0; r < MR; ++r) sred[(wave * MR + r) * 64 + lane] = acc[r];
    __syncthreads();
    const int64_t PT = P.n_pairs * P.M;
    for (int t = tid; t < MR * 64; t += BD) {
      const int r = t >> 6, l2 = t & 63;
      const int li = 8 * (r / 4) + 4 * (l2 >> 5) + (r % 4);
      const int nn = rb * 32 + (l2 & 31);
      const int64_t xr = li < 32 ? srow[li] : -1;
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
    __syncthreads();
  }
}

// Sums the K-split partials in split order and applies the NaN rule for rows whose
// indices were out of range (recomputed from the item list).
template <bool XF32>
__global__ void reduce_splits_kernel(QmvParams P) {
  const int64_t PT = P.n_pairs * P.M;
  const int64_t total = PT * P.N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = i / P.N;
    const int64_t pair = p / P.M;
    float v = 0.f;
    for (int k2 = 0; k2 < P.ks; ++k2) v += P.part[(int64_t)k2 * total + i];
    const uint32_t e = P.rhs ? P.rhs[pair] : (uint32_t)pair;
    const int64_t l = P.lhs ? (int64_t)P.lhs[pair] : pair / P.lhs_div;
    if (e >= (uint32_t)P.n_experts || l >= P.x_batch) v = __builtin_nanf("");
    if constexpr (XF32) ((float*)P.y)[i] = v;
    else ((uint16_t*)P.y)[i] = (uint16_t)f32_to_bf16_bits(v);
  }
}

template <int BITS, int GS, int MR, bool XF32>
hipError_t launch_t(const QmvParams& P, dim3 grid, int waves, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, MR, XF32>), grid, dim3(64 * waves), lds, s, P);
  return hipGetLastError();
}

template <int BITS, int GS, bool XF32>
hipError_t launch_m(const QmvParams& P, dim3 grid, int waves, size_t lds, int mr,
                    hipStream_t s) {
  switch (mr) {
    case 1: return launch_t<BITS, GS, 1, XF32>(P, grid, waves, lds, s);
    case 2: return launch_t<BITS, GS, 2, XF32>(P, grid, waves, lds, s);
    case 4: return launch_t<BITS, GS, 4, XF32>(P, grid, waves, lds, s);
    case 8: return launch_t<BITS, GS, 8, XF32>(P, grid, waves, lds, s);
    default: return launch_t<BITS, GS, 16, XF32>(P, grid, waves, lds, s);
  }
}

template <int BITS, bool XF32>
hipError_t launch_gs(const QmvParams& P, dim3 grid, int waves, size_t lds, int mr,
                     hipStream_t s) {
  switch (P.group_size) {
    case 32: return launch_m<BITS, 32, XF32>(P, grid, waves, lds, mr, s);
    case 64: return launch_m<BITS, 64, XF32>(P, grid, waves, lds, mr, s);
    default: return launch_m<BITS, 128, XF32>(P, grid, waves, lds, mr, s);
  }
}

}  // namespace

int qmv_mr_for_rows(int rows) {
  return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 8 ? 4 : rows <= 16 ? 8 : 16;
}

// LDS bytes of one block: staged fragments + group sums, or the wave reduction.
size_t qmv_lds_bytes(int groups, int gs, int mr, int x_f32, int waves) {
  const int mpad = mr == 1 ? 1 : mr == 2 ? 2 : mr == 4 ? 8 : mr == 8 ? 16 : 32;
  const int mxs = mpad < 8 ? 8 : mpad;
  const size_t stage = (size_t)groups * (gs / 16) * 2 * mpad * 16 * (x_f32 ? 2 : 1) +
                       (size_t)groups * mxs * 4;
  const size_t red = (size_t)waves * mr * 64 * 4;
  return stage > red ? stage : red;
}

hipError_t launch_qmv(const QmvParams& P, const QmvConfig& C, hipStream_t s) {
  dim3 grid((unsigned)P.row_blocks, (unsigned)P.ks, (unsigned)C.grid_z);
  const int mr = qmv_mr_for_rows(C.rows);
  const size_t lds = qmv_lds_bytes(P.gps, P.group_size, mr, P.x_f32, C.waves);
  hipError_t e = (P.bits == 4)
                     ? (P.x_f32 ? launch_gs<4, true>(P, grid, C.waves, lds, mr, s)
                                : launch_gs<4, false>(P, grid, C.waves, lds, mr, s))
                     : (P.x_f32 ? launch_gs<8, true>(P, grid, C.waves, lds, mr, s)
                                : launch_gs<8, false>(P, grid, C.waves, lds, mr, s));
  if (e != hipSuccess || P.ks == 1) return e;
  const int64_t total = P.n_pairs * P.M * P.N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (P.x_f32)
    hipLaunchKernelGGL(reduce_splits_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, P);
  else
    hipLaunchKernelGGL(reduce_splits_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace mi
