// Decode MoE down projection fused with the score-weighted sum over the k slots of a token
// (the reference's gatherQmvDownReduce, src/transformer.zig:20675-20761): one launch
// instead of a gather and a reduce, same results bit for bit.
//
// Block = 16 output rows of one token; its waves are k slots x WS waves per slot. Each
// wave of slot s stages its own chunks of that pair's activation row into the slot's LDS
// region (a wave-level fence, no block barrier, before its dot products) and streams
// the 16-row tile of expert inds[t*k + s] over K (WS x NC chunks of 128 values), with
// the one-row kernel's arithmetic (bf16 0x43qq nibbles, v_dot2_f32_bf16, affine terms per
// 32-value slice). The 16 writer threads then take the slots in ascending order:
// total = bf16(total + bf16(bf16(v_s) * score_s)) from bf16 zero, a NaN v_s for an expert
// id out of range, exactly as the separate gather + down_reduce do.
#include "qmv1_kernel.h"

namespace mi {
namespace {

using namespace qmv1_detail;

struct MoeDownParams {
  const uint16_t* act;     // [T*k, K] bf16, one row per (token, slot)
  const uint32_t* w;       // [E, N, K/8]
  const uint16_t* scales;  // [E, N, K/64] bf16
  const uint16_t* biases;
  const uint32_t* inds;    // [T*k]
  const uint16_t* scores;  // [T*k] bf16
  uint16_t* y;             // [T, N] bf16
  int N, K, E, k, ws;
};

MI_DEV uint16_t bf16_add_bits(uint16_t a, uint16_t b) {
  return (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(a) + bf16_bits_to_f32(b));
}

template <int NC>
__global__ void __launch_bounds__(1024) moe_down_kernel(MoeDownParams P) {
  constexpr int GS = 64;
  constexpr int XN = (NC + 3) / 4;  // 16-byte activation units per lane (its own chunks)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int okf[16];
  __shared__ uint16_t score_l[16];
  __shared__ uint16_t prod[16][16];  // [slot][row]: bf16(bf16(v_s) * score_s)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = blockDim.x >> 6;
  const int WS = P.ws;
  const int s = wave / WS, kp = wave - s * WS;
  const int r = lane >> 2, g = lane & 3;
  const int tile = blockIdx.x, t = blockIdx.y;
  const int N = P.N, K = P.K, G = K / GS, k = P.k;
  const int64_t pair = (int64_t)t * k + s;
  const uint32_t e_raw = __builtin_amdgcn_readfirstlane(P.inds[pair]);
  const bool ok = e_raw < (uint32_t)P.E;
  const uint32_t e = ok ? e_raw : 0u;
  const int xstride = K * 2 + (K / 32) * 4;  // per slot: K bf16 (dot8 order), K/32 sums
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem + s * xstride);
  float* xsum = reinterpret_cast<float*>(smem + s * xstride + K * 2);
  float* red = reinterpret_cast<float*>(smem + k * xstride);  // [W][16]
  const int n = tile * 16 + r;
  const uint32_t nn = (uint32_t)min(n, N - 1);
  const int c0 = kp * NC;

  // 1. loads: the token's scores, this slot's activation row, scale/bias dwords, then the
  //    weights. Everything is in flight before the first wait.
  const uint16_t my_score = tid < k ? P.scores[(int64_t)t * k + tid] : (uint16_t)0;
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.act + pair * K), (short)0, K * 2, kBufFlags);
  const size_t mat = (size_t)e * (uint32_t)N;
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.w + mat * (uint32_t)(K / 8)), (short)0, N * (K / 2), kBufFlags);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.scales + mat * (uint32_t)G), (short)0, N * G * 2, kBufFlags);
  const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.biases + mat * (uint32_t)G), (short)0, N * G * 2, kBufFlags);
  const int nunits = K / 8;
  u32x4_t xv[XN];
#pragma unroll
  for (int i = 0; i < XN; ++i)
    xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xres, (c0 * 16 + lane + 64 * i) * 16, 0, 0);
  constexpr int NSL = (NC + 3) / 4;  // gs 64: a dword holds the two groups of a chunk
  const uint32_t so = nn * (uint32_t)(G * 2) + (uint32_t)c0 * 4;
  uint32_t sd[NSL], bd[NSL];
#pragma unroll
  for (int i = 0; i < NSL; ++i) {
    sd[i] = __builtin_amdgcn_raw_buffer_load_b32(sres, so + 4 * g + 16 * i, 0, 0);
    bd[i] = __builtin_amdgcn_raw_buffer_load_b32(bres, so + 4 * g + 16 * i, 0, 0);
  }
  const uint32_t wo = nn * (uint32_t)(K / 2) + (uint32_t)c0 * 64 + 16 * g;
  u32x4_t wv[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) wv[j] = __builtin_amdgcn_raw_buffer_load_b128(wres, wo + 64 * j, 0, 0);

  // 2. stage the wave's activations in dot8's pair order with per-32-value sums.
#pragma unroll
  for (int i = 0; i < XN; ++i) {
    const int u = c0 * 16 + lane + 64 * i;
    const u32x4_t X = xv[i];
    float s8 = ((bf16_bits_to_f32(X.x & 0xFFFFu) + bf16_bits_to_f32(X.x >> 16)) +
                (bf16_bits_to_f32(X.y & 0xFFFFu) + bf16_bits_to_f32(X.y >> 16))) +
               ((bf16_bits_to_f32(X.z & 0xFFFFu) + bf16_bits_to_f32(X.z >> 16)) +
                (bf16_bits_to_f32(X.w & 0xFFFFu) + bf16_bits_to_f32(X.w >> 16)));
    s8 += quad_xor1(s8);
    s8 += quad_xor2(s8);
    if (u < nunits && u < (c0 + NC) * 16) {
      u32x4_t o;
      o.x = perm_b32(X.y, X.x, 0x05040100u);  // (x0, x2)
      o.y = perm_b32(X.w, X.z, 0x05040100u);  // (x4, x6)
      o.z = perm_b32(X.y, X.x, 0x07060302u);  // (x1, x3)
      o.w = perm_b32(X.w, X.z, 0x07060302u);  // (x5, x7)
      *reinterpret_cast<u32x4_t*>(xs + u * 4) = o;
      if ((u & 3) == 0) xsum[u >> 2] = s8;
    }
  }
  if (kp == 0 && lane == 0) okf[s] = ok;  // read after the reduction barrier below
  if (tid < k) score_l[tid] = my_score;
  // the wave reads only what its own lanes staged
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 3. dot products of the wave's chunks.
  float yv = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int off = (c0 + j) * kChunkVals + 32 * g;
    const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(xs + off / 2);
    float acc = 0.f;
    acc = dot8(wv[j].x, xp[0], acc);
    acc = dot8(wv[j].y, xp[1], acc);
    acc = dot8(wv[j].z, xp[2], acc);
    acc = dot8(wv[j].w, xp[3], acc);
    // chunk j's two groups are dword j of the quad: lane j % 4, slot j / 4
    const uint32_t sw = quad_bcast(sd[j >> 2], j & 3);
    const uint32_t bw = quad_bcast(bd[j >> 2], j & 3);
    const float sc = bf16_bits_to_f32(g >= 2 ? sw >> 16 : sw & 0xFFFFu);
    const float bi = bf16_bits_to_f32(g >= 2 ? bw >> 16 : bw & 0xFFFFu);
    yv = fmaf(sc, acc, yv);
    yv = fmaf(fmaf(-128.f, sc, bi), xsum[off >> 5], yv);
  }

  // 4. reduce the row's 4 lanes, then per slot over its waves (one thread per slot and
  //    row), then the slots in ascending order.
  yv += quad_xor1(yv);
  yv += quad_xor2(yv);
  if (g == 0) red[wave * 16 + r] = yv;
  lds_barrier();
  if (tid < 16 * k) {
    const int s2 = tid >> 4, row = tid & 15;
    float v = 0.f;
    for (int w2 = 0; w2 < WS; ++w2) v += red[(s2 * WS + w2) * 16 + row];
    if (!okf[s2]) v = __builtin_nanf("");
    prod[s2][row] = bf16_mul((uint16_t)f32_to_bf16_bits(v), score_l[s2]);
  }
  lds_barrier();
  if (tid < 16 && tile * 16 + tid < N) {
    uint16_t total = 0;  // bf16 zero
    for (int s2 = 0; s2 < k; ++s2) total = bf16_add_bits(total, prod[s2][tid]);
    P.y[(int64_t)t * N + tile * 16 + tid] = total;
  }
  (void)W;
}

template <int NC>
void launch_one(const MoeDownParams& P, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  static const bool big_lds = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&moe_down_kernel<NC>),
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024) == hipSuccess;
  (void)big_lds;  // a failure shows as a launch error for plans above 64 KiB
  hipLaunchKernelGGL((moe_down_kernel<NC>), grid, block, lds, s, P);
}

}  // namespace

// The caller passes the one-row gather plan's factorization (WS waves per slot x NC chunks
// per wave == K / 128, no K split), so every fp32 sum is formed in the same order as in the
// gather kernel and the result matches gather + down_reduce bit for bit.
bool moe_down_supported(int64_t T, int k, int64_t N, int64_t K, int gs, int bits, int ws, int nc) {
  if (bits != 4 || gs != 64 || K % 128 || k < 1 || T < 1 || T > 65535 || ws < 1) return false;
  if (N * (K / 2) >= ((int64_t)1 << 31) || k * ws > 16 || ws * nc != K / 128) return false;
  if (!((nc >= 1 && nc <= 8) || nc == 10 || nc == 12 || nc == 14 || nc == 16)) return false;
  const size_t lds = (size_t)k * (K * 2 + (K / 32) * 4) + (size_t)k * ws * 16 * 4;
  return lds <= 160 * 1024 - 1024;
}

hipError_t launch_moe_down(uint16_t* y, const uint16_t* act, const uint32_t* w,
                           const uint16_t* scales, const uint16_t* biases, const uint32_t* inds,
                           const uint16_t* scores, int64_t T, int k, int64_t N, int64_t K,
                           int64_t E, int ws, int nc, hipStream_t s) {
  if (!moe_down_supported(T, k, N, K, 64, 4, ws, nc)) return hipErrorInvalidValue;
  MoeDownParams P{act, w, scales, biases, inds, scores, y, (int)N, (int)K, (int)E, k, ws};
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)T);
  const dim3 block(64 * k * ws);
  const size_t lds = (size_t)k * (K * 2 + (K / 32) * 4) + (size_t)k * ws * 16 * 4;
  switch (nc) {
    case 1: launch_one<1>(P, grid, block, lds, s); break;
    case 2: launch_one<2>(P, grid, block, lds, s); break;
    case 3: launch_one<3>(P, grid, block, lds, s); break;
    case 4: launch_one<4>(P, grid, block, lds, s); break;
    case 5: launch_one<5>(P, grid, block, lds, s); break;
    case 6: launch_one<6>(P, grid, block, lds, s); break;
    case 7: launch_one<7>(P, grid, block, lds, s); break;
    case 8: launch_one<8>(P, grid, block, lds, s); break;
    case 10: launch_one<10>(P, grid, block, lds, s); break;
    case 12: launch_one<12>(P, grid, block, lds, s); break;
    case 14: launch_one<14>(P, grid, block, lds, s); break;
    default: launch_one<16>(P, grid, block, lds, s); break;
  }
  return hipGetLastError();
}

}  // namespace mi

