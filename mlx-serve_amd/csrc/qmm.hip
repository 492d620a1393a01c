// Prefill (large-M) affine quantized GEMM for gfx950:
//   y[M,N] (bf16) = x[M,K] (bf16) @ dequant(w)[N,K]^T, fp32 accumulation.
// Replaces the reference's prefill route of qmatmulBits / prefillDqGemm
// (src/transformer.zig:20894-20983, :20987-21011), which dequantizes the whole weight to
// bf16 in HBM and then runs a dense GEMM. Here dequantization is fused into the LDS stage:
// a block owns a BN x BM output tile and walks K in 64-wide steps:
//   - x (A operand): BM x 64 bf16 streamed HBM -> LDS by global_load_lds (no VGPR round
//     trip), 16-byte slots XOR-swizzled by row so MFMA fragment reads are conflict free.
//   - w (B operand): each thread owns half a row of the 256-row weight tile: its 16 (4-bit)
//     or 32 (8-bit) packed bytes and the group's scale/bias are prefetched into registers a
//     tile ahead, dequantized in fp32 as scale*q + bias, rounded once to bf16 (as MLX's GPU
//     qmm stages bf16 weights in threadgroup memory) and written to LDS.
//   - 8 waves in a 2 (M) x 4 (N) grid; each wave owns BM/2 x 64 outputs as 32x32 tiles of
//     v_mfma_f32_32x32x16_bf16.
// Double-buffered LDS (A and B) with one barrier per K step.
#include "mi_internal.h"
#include "qmv_common.h"

namespace mi {
namespace {

using qmv_detail::mfma32;

constexpr int kBN = 256;       // weight rows (output columns) per block
constexpr int kBK = 64;        // K per step
constexpr int kThreads = 512;  // 8 waves
constexpr int kRowBytes = kBK * 2;  // one LDS row: 64 bf16 = 8 slots of 16 bytes

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

MI_DEV uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Byte k of a word as a float (selects v_cvt_f32_ubyte{k}).
template <int k>
MI_DEV float ubyte(uint32_t w) { return (float)((w >> (8 * k)) & 0xFFu); }

MI_DEV void dma16(const void* src, unsigned char* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// LDS byte offset of 16-byte slot `c` (0..7) of row `r` in a [rows][64 bf16] tile.
MI_DEV int swz(int r, int c) { return r * kRowBytes + ((c ^ (r & 7)) << 4); }

template <int BITS>
struct WRegs {
  static constexpr int kWords = 32 * BITS / 32;  // packed words for 32 values
  uint32_t q[kWords];
  uint32_t s, b;  // bf16 bits of the scale and bias
};

template <int BITS, int GS, int BM>
__global__ void __launch_bounds__(kThreads) qmm_kernel(QmmParams P) {
  constexpr int WM = BM / 2;       // wave tile rows (M)
  constexpr int TM = WM / 32;      // 32-row MFMA tiles per wave
  constexpr int TN = 2;            // 32-col MFMA tiles per wave (wave tile 64 wide)
  constexpr int PF = 32 / BITS;
  constexpr int ABYTES = BM * kRowBytes;
  constexpr int BBYTES = kBN * kRowBytes;
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* abuf = smem;                 // [2][BM][128 B]
  unsigned char* bbuf = smem + 2 * ABYTES;    // [2][256][128 B]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int M = P.M, N = P.N, K = P.K;
  const int G = K / GS;
  const int mtiles = (M + BM - 1) / BM;
  // Consecutive blocks land on different XCDs; walking M fastest keeps each XCD on the
  // same x row block while the weight tiles stream past.
  const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
  const int m0 = mt * BM, n0 = nt * kBN;
  const int nsteps = K / kBK;

  // ---- A (x) DMA plan: a wave instruction moves 8 rows x 128 B.
  constexpr int A_INSTR = BM * kRowBytes / (kThreads * 16);  // per thread per step
  const uint16_t* xa[A_INSTR];
  int a_lds[A_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int r = (wave * A_INSTR + i) * 8 + (lane >> 3);
    const int slot = lane & 7;
    const int c = slot ^ (r & 7);  // logical chunk that lands in this slot
    const int gm = min(m0 + r, M - 1);
    xa[i] = P.x + (int64_t)gm * K + c * 8;
    a_lds[i] = (wave * A_INSTR + i) * 8 * kRowBytes;  // wave-uniform base of the 1 KiB run
  }
  auto issue_a = [&](int step, int buf) {
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      dma16(xa[i] + step * kBK, abuf + buf * ABYTES + a_lds[i]);
  };

  // ---- B (w) plan: thread -> (row, half of the 64-wide step).
  const int wr = tid >> 1, half = tid & 1;
  const int gn = min(n0 + wr, N - 1);
  const uint32_t* wrow = P.w + (int64_t)gn * (K / PF) + half * (32 / PF);
  const uint16_t* srow = P.scales + (int64_t)gn * G;
  const uint16_t* brow = P.biases + (int64_t)gn * G;
  auto load_w = [&](int step, WRegs<BITS>& R) {
    const uint32_t* p = wrow + step * (kBK / PF);
#pragma unroll
    for (int i = 0; i < R.kWords / 4; ++i) {
      u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p) + i);
      R.q[4 * i] = v.x; R.q[4 * i + 1] = v.y; R.q[4 * i + 2] = v.z; R.q[4 * i + 3] = v.w;
    }
    const int g = (step * kBK + half * 32) / GS;
    R.s = srow[g];
    R.b = brow[g];
  };
  auto store_w = [&](const WRegs<BITS>& R, int buf) {
    const float s = bf16_bits_to_f32(R.s), b = bf16_bits_to_f32(R.b);
    uint32_t o[16];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = R.q[i] & 0x0F0F0F0Fu, hi = (R.q[i] >> 4) & 0x0F0F0F0Fu;
        // values 8i..8i+7 are lo.b0, hi.b0, lo.b1, hi.b1, ...
        o[4 * i + 0] = pack_bf16x2(fmaf(s, ubyte<0>(lo), b),
                                   fmaf(s, ubyte<0>(hi), b));
        o[4 * i + 1] = pack_bf16x2(fmaf(s, ubyte<1>(lo), b),
                                   fmaf(s, ubyte<1>(hi), b));
        o[4 * i + 2] = pack_bf16x2(fmaf(s, ubyte<2>(lo), b),
                                   fmaf(s, ubyte<2>(hi), b));
        o[4 * i + 3] = pack_bf16x2(fmaf(s, ubyte<3>(lo), b),
                                   fmaf(s, ubyte<3>(hi), b));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = R.q[i];
        o[2 * i + 0] = pack_bf16x2(fmaf(s, ubyte<0>(w), b),
                                   fmaf(s, ubyte<1>(w), b));
        o[2 * i + 1] = pack_bf16x2(fmaf(s, ubyte<2>(w), b),
                                   fmaf(s, ubyte<3>(w), b));
      }
    }
    unsigned char* dst = bbuf + buf * BBYTES;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t v = {o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
      *reinterpret_cast<u32x4_t*>(dst + swz(wr, half * 4 + j)) = v;
    }
  };

  // ---- MFMA plan: wave (wm, wn) owns rows [wm*WM, +WM) x cols [wn*64, +64) of the tile.
  const int wm = wave >> 2, wn = wave & 3;
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int fr = lane & 31, fk = lane >> 5;  // fragment row, k half (8 values)
  auto compute = [&](int buf) {
    const unsigned char* A = abuf + buf * ABYTES;
    const unsigned char* B = bbuf + buf * BBYTES;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int c = 2 * ks + fk;
      u32x4_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + i * 32 + fr;
        a[i] = *reinterpret_cast<const u32x4_t*>(A + swz(r, c));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * 64 + j * 32 + fr;
        b[j] = *reinterpret_cast<const u32x4_t*>(B + swz(r, c));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
  };

  // ---- pipeline
  WRegs<BITS> R;
  load_w(0, R);
  issue_a(0, 0);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) & lgkmcnt(0)
  store_w(R, 0);
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const bool more = step + 1 < nsteps;
    if (more) {
      load_w(step + 1, R);
      issue_a(step + 1, buf ^ 1);
    }
    compute(buf);
    if (more) store_w(R, buf ^ 1);  // waits for the loads (and the DMA) of step + 1
    __syncthreads();
  }

  // ---- epilogue: C reg r of a 32x32 tile is row 8(r/4) + 4(lane/32) + r%4, col lane%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * 64 + j * 32 + fr;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        if (m < M) P.y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][r]);
      }
    }
}

template <int BITS, int GS, int BM>
hipError_t launch_bm(const QmmParams& P, hipStream_t s) {
  const int mtiles = (P.M + BM - 1) / BM, ntiles = (P.N + kBN - 1) / kBN;
  const size_t lds = 2 * (size_t)BM * kRowBytes + 2 * (size_t)kBN * kRowBytes;
  auto k = qmm_kernel<BITS, GS, BM>;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)(mtiles * ntiles)), dim3(kThreads), lds, s, P);
  return hipGetLastError();
}

template <int BITS, int GS>
hipError_t launch_gs(const QmmParams& P, hipStream_t s) {
  // 128-row tiles when 256-row tiles would leave CUs idle.
  const int64_t big = (int64_t)((P.M + 255) / 256) * ((P.N + kBN - 1) / kBN);
  return big >= 240 ? launch_bm<BITS, GS, 256>(P, s) : launch_bm<BITS, GS, 128>(P, s);
}

}  // namespace

bool qmm_supported(int M, int N, int K, int bits, int gs) {
  (void)N;
  if (bits != 4 && bits != 8) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  return M >= 1 && K % kBK == 0 && K % gs == 0;
}

hipError_t launch_qmm(const QmmParams& P, hipStream_t s) {
  if (!qmm_supported(P.M, P.N, P.K, P.bits, P.group_size)) return hipErrorNotSupported;
  if (P.bits == 4) {
    switch (P.group_size) {
      case 32: return launch_gs<4, 32>(P, s);
      case 64: return launch_gs<4, 64>(P, s);
      default: return launch_gs<4, 128>(P, s);
    }
  }
  switch (P.group_size) {
    case 32: return launch_gs<8, 32>(P, s);
    case 64: return launch_gs<8, 64>(P, s);
    default: return launch_gs<8, 128>(P, s);
  }
}

}  // namespace mi
