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
#include "qmv_common.h"


namespace mi {

namespace {

using namespace qmv_detail;

// One block = W waves sharing one K range [g0, g1) of one item; wave w owns the
// 32-row weight tile blockIdx.x*W + w and streams it over the K range in chunks of
// UG groups (256 bytes of each row). Flow:
//   1. the block stages the range's activations into LDS (fragment order, group
//      sums) -- all LDS writes happen here, before any weight DMA is in flight;
//   2. each wave DMAs chunk c+1 of its tile straight into LDS (global_load_lds
//      dwordx4: every instruction reads 4 rows x 256 contiguous bytes; 16-byte slot
//      s of row r lands at slot s ^ (r & 15), so fragment reads hit distinct banks)
//      while it runs the MFMAs of chunk c from the other buffer;
//   3. each wave writes its finished rows (y, or an fp32 partial per K range that
//      reduce_splits_kernel sums in range order).
template <int BITS, int GS, int MR, bool XF32>
__global__ void __launch_bounds__(64 * kQmvMaxWaves) qmv_kernel(QmvParams P) {
  constexpr int PF = 32 / BITS;
  constexpr int WPG = GS / PF;    // packed words per group per row
  constexpr int VPL = WPG / 2;    // words per lane per group (one k-half)
  constexpr int STEPS = GS / 16;  // MFMA steps per group
  constexpr int GSB = WPG * 4;    // bytes per group per row
  constexpr int UG = 256 / GSB;   // groups per chunk (256 bytes per row)
  constexpr int MPAD = MR == 1 ? 1 : MR == 2 ? 2 : MR == 4 ? 8 : MR == 8 ? 16 : 32;
  constexpr int MXS = MPAD < 8 ? 8 : MPAD;  // group-sum row stride (b128 reads)
  constexpr int PLANES = XF32 ? 2 : 1;
  constexpr int FB = 2;                     // staging fragments per thread per pass
  constexpr int CHUNK = 32 * 256;           // LDS bytes of one chunk of one tile

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int64_t srow[32];

  const int tid = threadIdx.x;
  const int BD = blockDim.x, W = BD >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int l32 = lane & 31, hh = lane >> 5;
  const int K = P.K, N = P.N;
  const int G = K / GS;
  const uint32_t wrow_b = (uint32_t)(K / PF) * 4u;  // bytes per packed weight row
  const int ks = blockIdx.y;
  const int g0 = ks * P.gps;
  const int g1 = min(G, g0 + P.gps);
  const int GB = g1 - g0;                        // groups in this K range
  const int NF = GB * STEPS * 2 * MPAD;          // A fragments staged
  const int nch = (GB + UG - 1) / UG;            // chunks per tile
  unsigned char* swt = smem;                     // [W][2][32 rows][256 B]
  unsigned char* ssb = smem + (size_t)W * 2 * CHUNK;  // [W][2][scales 32x16 B, biases]
  u32x4_t* sx = (u32x4_t*)(ssb + (size_t)W * 2 * 1024);  // [GB][STEPS][2][MPAD] (+lo)
  float* sxs = (float*)(sx + (size_t)NF * PLANES);          // [GB][MXS]
  const uint32_t c43 = 0x43434343u;  // byte pool for the 4-bit unpack
  const int arow = l32 & (MPAD - 1);  // A rows >= MPAD: don't-care C rows, no mask
  const int tile = blockIdx.x * W + wave;
  const bool active = tile * 32 < N;
  unsigned char* wbuf = swt + wave * 2 * CHUNK;
  unsigned char* sbuf = ssb + wave * 2 * 1024;
  const unsigned char* myrow0 = wbuf + l32 * 256;
  // Scales/biases come by DMA (16-byte runs of 8 groups per row) when the packing
  // allows 16-byte aligned runs; otherwise each lane loads its own.
  constexpr bool kSdmaOk = UG <= 8;
  const bool sdma = kSdmaOk && (G % 8) == 0;
  const int sw = l32 & 15;

  const int n_items = P.item_count ? (int)*P.item_count : P.n_items_fixed;
  for (int itx = blockIdx.z; itx < n_items; itx += gridDim.z) {
    const Item it = decode_item(P, itx);
    const uint32_t ex = it.expert_ok ? it.expert : 0u;
    if (tid < 32) srow[tid] = item_x_row(P, it, tid);
    lds_barrier();

    // ---- 1. stage x[rows][g0*GS, g1*GS) into LDS ---------------------------------
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
    lds_barrier();

    if (active) {
      // ---- 2. stream the tile over the K range ---------------------------------
      const unsigned char* tbase = (const unsigned char*)P.w + ((int64_t)ex * N) * wrow_b;
      const int n = min(tile * 32 + l32, N - 1);
      const uint16_t* srp = P.scales + ((int64_t)ex * N + n) * G;
      const uint16_t* brp = P.biases + ((int64_t)ex * N + n) * G;
      // DMA chunk c (groups g0 + c*UG ...) into buffer b; scales/biases to registers.
      auto issue = [&](int c, int b, uint32_t (&sv)[UG], uint32_t (&bv)[UG]) {
        const int gc = g0 + c * UG;
        const int nslots = min(UG, g1 - gc) * GSB / 16;  // valid slots per row
        const int s = lane & 15;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 4 * i + (lane >> 4);
          const int sl = s ^ (r & 15);
          const uint32_t nr = (uint32_t)min(tile * 32 + r, N - 1);
          const unsigned char* src =
              tbase + nr * wrow_b + (uint32_t)gc * GSB + (sl < nslots ? sl * 16 : 0);
          __builtin_amdgcn_global_load_lds(
              src, (__attribute__((address_space(3))) void*)(wbuf + b * CHUNK + i * 1024),
              16, 0, 0);
        }
        if (sdma) {
          // One instruction: lanes 0-31 fetch the scale run, 32-63 the bias run, of
          // row l32 for the 8 groups [gc & ~7, +8) that hold this chunk.
          const uint32_t nr = (uint32_t)min(tile * 32 + l32, N - 1);
          const uint16_t* run = (hh ? P.biases : P.scales) + ((int64_t)ex * N + nr) * G + (gc & ~7);
          __builtin_amdgcn_global_load_lds(
              run, (__attribute__((address_space(3))) void*)(sbuf + b * 1024), 16, 0, 0);
        } else {
#pragma unroll
          for (int u = 0; u < UG; ++u) {
            const int g = min(gc + u, g1 - 1);
            sv[u] = srp[g];
            bv[u] = brp[g];
          }
        }
      };
      float acc[MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] = 0.f;
      // MFMAs of chunk c from buffer b (two groups interleaved).
      auto compute = [&](int c, int b, const uint32_t (&sv)[UG], const uint32_t (&bv)[UG]) {
        const unsigned char* myrow = myrow0 + b * CHUNK;
        const int gc = g0 + c * UG;
        const int ng = min(UG, g1 - gc);
        auto load_words = [&](int u, uint32_t (&words)[VPL]) {
          const int byte0 = u * GSB + hh * (GSB / 2);
          if constexpr (VPL >= 4) {
#pragma unroll
            for (int q = 0; q < VPL / 4; ++q) {
              const int slot = (byte0 >> 4) + q;
              const u32x4_t t = *(const u32x4_t*)(myrow + ((slot ^ sw) << 4));
              words[4 * q] = t.x; words[4 * q + 1] = t.y; words[4 * q + 2] = t.z;
              words[4 * q + 3] = t.w;
            }
          } else {
            const int slot = byte0 >> 4;
            const u32x2_t t = *(const u32x2_t*)(myrow + ((slot ^ sw) << 4) + (byte0 & 15));
            words[0] = t.x; words[1] = t.y;
          }
        };
        auto epilogue = [&](int u, int ul, const f32x16_t& accg) {
          float xs[MR];
#pragma unroll
          for (int r4 = 0; r4 < (MR + 3) / 4; ++r4) {
            const f32x4_t v4 = *(const f32x4_t*)&sxs[ul * MXS + 8 * r4 + 4 * hh];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (4 * r4 + e < MR) xs[4 * r4 + e] = v4[e];
          }
          uint32_t sbits, bbits;
          if (sdma) {
            const int gi = ((gc & 7) + u) * 2;  // byte of group gc+u inside the run
            sbits = *(const uint16_t*)(sbuf + b * 1024 + l32 * 16 + gi);
            bbits = *(const uint16_t*)(sbuf + b * 1024 + 512 + l32 * 16 + gi);
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
#pragma unroll
        for (int u = 0; u < UG; u += 2) {
          const int ul = gc + u - g0;
          if (u + 1 < ng) {
            uint32_t w0[VPL], w1[VPL];
            load_words(u, w0);
            load_words(u + 1, w1);
            f32x16_t a0, a1;
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
              const int i0 = ((ul * STEPS + j) * 2 + hh) * MPAD + arow;
              const int i1 = i0 + STEPS * 2 * MPAD;
              const u32x4_t B0 = b_frag<BITS>(w0, j, c43);
              const u32x4_t B1 = b_frag<BITS>(w1, j, c43);
              a0 = mfma32(sx[i0], B0, j == 0 ? f32x16_t{} : a0);
              a1 = mfma32(sx[i1], B1, j == 0 ? f32x16_t{} : a1);
              if constexpr (XF32) {
                a0 = mfma32(sx[NF + i0], B0, a0);
                a1 = mfma32(sx[NF + i1], B1, a1);
              }
            }
            epilogue(u, ul, a0);
            epilogue(u + 1, ul + 1, a1);
          } else if (u < ng) {
            uint32_t w0[VPL];
            load_words(u, w0);
            f32x16_t a0;
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
              const int i0 = ((ul * STEPS + j) * 2 + hh) * MPAD + arow;
              const u32x4_t B0 = b_frag<BITS>(w0, j, c43);
              a0 = mfma32(sx[i0], B0, j == 0 ? f32x16_t{} : a0);
              if constexpr (XF32) a0 = mfma32(sx[NF + i0], B0, a0);
            }
            epilogue(u, ul, a0);
          }
        }
      };

      uint32_t sA[UG], bA[UG], sB[UG], bB[UG];
      issue(0, 0, sA, bA);
      // Steady state, two chunks per trip so the scale registers ping-pong without
      // copies; every issue is unconditional so vmcnt accounting stays exact.
      // "chunk c landed" = at most one chunk's loads (issued later) still pending.
      auto wait_prev = [&]() {
        if (sdma) __builtin_amdgcn_s_waitcnt(vmcnt_imm(9));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 + 2 * UG));
      };
      int c = 0;
      for (; c + 2 < nch; c += 2) {
        issue(c + 1, 1, sB, bB);
        wait_prev();                          // chunk c landed
        compute(c, 0, sA, bA);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // buffer 0 reads done
        issue(c + 2, 0, sA, bA);
        wait_prev();                          // chunk c+1 landed
        compute(c + 1, 1, sB, bB);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // buffer 1 reads done
      }
      if (c + 1 < nch) {
        issue(c + 1, 1, sB, bB);
        wait_prev();
        compute(c, 0, sA, bA);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        compute(c + 1, 1, sB, bB);
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        compute(c, 0, sA, bA);
      }

      // ---- 3. write this wave's rows ---------------------------------------------
      const int64_t PT = P.n_pairs * P.M;
      const int nn = tile * 32 + l32;
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const int li = 8 * (r / 4) + 4 * hh + (r % 4);
        const int64_t xr = li < 32 ? srow[li] : -1;
        if (nn < N && li < it.cnt && xr != -1) {
          float v = acc[r];
          const int64_t p = it.pos0 + li;
          if (P.ks > 1) {
            P.part[((int64_t)ks * PT + p) * N + nn] = v;
          } else {
            if (xr < 0 || !it.expert_ok) v = __builtin_nanf("");
            if constexpr (XF32) ((float*)P.y)[p * N + nn] = v;
            else ((uint16_t*)P.y)[p * N + nn] = (uint16_t)f32_to_bf16_bits(v);
          }
        }
      }
    }
    lds_barrier();  // LDS is restaged for the next item
  }
}

// Sums the K-split partials in split order and applies the NaN rule for rows whose
// indices were out of range. One thread per output element, 32-bit index math.
template <bool XF32>
__global__ void reduce_splits_kernel(QmvParams P) {
  const uint32_t PT = (uint32_t)(P.n_pairs * P.M);
  const uint32_t N = (uint32_t)P.N;
  const uint32_t total = PT * N;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += gridDim.x * blockDim.x) {
    float v = add_splits<8>(0.f, P.part + i, (int64_t)total, 0, P.ks);
    const uint32_t p = i / N;
    const uint32_t pair = P.M == 1 ? p : p / (uint32_t)P.M;
    const uint32_t e = P.rhs ? P.rhs[pair] : pair;
    const uint32_t l = P.lhs ? P.lhs[pair] : pair / (uint32_t)P.lhs_div;
    if (e >= (uint32_t)P.n_experts || (int64_t)l >= P.x_batch) v = __builtin_nanf("");
    if constexpr (XF32) {
      ((float*)P.y)[i] = v;
    } else {
      uint16_t o = (uint16_t)f32_to_bf16_bits(v);
      if (P.swiglu_gate) o = swiglu_bf16(P.swiglu_gate[i], o);
      ((uint16_t*)P.y)[i] = o;
    }
  }
}

}  // namespace

hipError_t launch_reduce_splits(const QmvParams& P, hipStream_t s) {
  const int64_t total = P.n_pairs * P.M * P.N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (P.x_f32)
    hipLaunchKernelGGL(reduce_splits_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, P);
  else
    hipLaunchKernelGGL(reduce_splits_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, P);
  return hipGetLastError();
}

namespace {

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

// Groups in one wave's weight slice (256 bytes of each row).
int qmv_groups_per_wave(int bits, int gs) { return 256 / (gs * bits / 8); }

// Dynamic LDS bytes of one block: double-buffered weight chunks of every wave +
// staged fragments + group sums.
size_t qmv_lds_bytes(int groups, int gs, int mr, int x_f32, int waves) {
  const int mpad = mr == 1 ? 1 : mr == 2 ? 2 : mr == 4 ? 8 : mr == 8 ? 16 : 32;
  const int mxs = mpad < 8 ? 8 : mpad;
  return (size_t)waves * 2 * (32 * 256 + 1024) +
         (size_t)groups * (gs / 16) * 2 * mpad * 16 * (x_f32 ? 2 : 1) +
         (size_t)groups * mxs * 4;
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
  return launch_reduce_splits(P, s);
}

}  // namespace mi
