// MoE glue around gather_qmm, on the GPU so the grouped launch needs no host sync:
//   route_topk      softmax top-k routing           (src/transformer.zig:17022-17072)
//   sort_dispatch   argsort / inverse / lhs = order//k (src/transformer.zig:14965-14993)
//   take_rows       row gather (mlx_take_axis 0)    (src/transformer.zig:15037)
//   swiglu          table SwiGLU, bf16 rounding     (src/transformer.zig:19846-19884)
//   down_reduce     bf16 score product + ascending bf16 sum over slots
//                                                   (src/transformer.zig:20577-20623)
#include "mi_common.h"
#include "mi_internal.h"
#include "moe_route.h"

namespace mi {
namespace {

MI_DEV uint16_t bf16_add(uint16_t a, uint16_t b) {
  return (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(a) + bf16_bits_to_f32(b));
}


// One wave per token (route_token in moe_route.h).
template <int NV>
__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits,
                                                         int64_t T, int E, int k,
                                                         uint32_t* __restrict__ inds,
                                                         void* __restrict__ scores,
                                                         int scores_bf16) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  uint32_t sel_i;
  float sc;
  route_token<NV>(logits + t * E, E, k, lane, sel_i, sc);
  if (lane < k) {
    inds[t * k + lane] = sel_i;
    if (scores_bf16) ((uint16_t*)scores)[t * k + lane] = (uint16_t)f32_to_bf16_bits(sc);
    else ((float*)scores)[t * k + lane] = sc;
  }
}

// Group-limited routing (groupLimitedRouting, src/transformer.zig:17242-17347, with the
// group mask of groupLimitMask :17138-17236), one wave per token, fp32 throughout:
// score = sigmoid(logit); biased = score + bias[e]; a group's score is the sum of its two
// largest biased values; the topk_group best groups survive (ties to the lower group id)
// and every other expert's key becomes -1e4; the k best keys are selected in descending
// order (ties to the lower id); the weights are the UNBIASED scores of the selected,
// divided by (their sum in slot order + 1e-20) when route_norm and k > 1, then times
// route_scale. E <= 64 * NV, n_group <= 64.
constexpr int kGroupedMaxE = 1024;
template <int NV>
__global__ void __launch_bounds__(256) route_grouped_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t T, int E, int k,
    int n_group, int topk_group, int route_norm, float route_scale, uint32_t* __restrict__ inds,
    float* __restrict__ scores) {
  __shared__ float biased_s[4][kGroupedMaxE];
  __shared__ float gscore_s[4][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  if (t >= T) return;
  using namespace route_detail;
  const float* row = logits + t * E;
  float* biased = biased_s[wv];
  float sc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      sc[j] = 1.f / (1.f + expf(-row[e]));
      biased[e] = sc[j] + bias[e];
    } else {
      sc[j] = 0.f;
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0xC07F);
  // group scores: lane g scans its group for the two largest biased values
  const int gsz = E / n_group;
  if (lane < n_group) {
    float m1 = -INFINITY, m2 = -INFINITY;
    for (int i = 0; i < gsz; ++i) {
      const float v = biased[lane * gsz + i];
      if (v > m1) {
        m2 = m1;
        m1 = v;
      } else if (v > m2) {
        m2 = v;
      }
    }
    gscore_s[wv][lane] = m1 + m2;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0xC07F);
  // a group survives when fewer than topk_group groups beat it (ties to the lower id)
  bool keep_g = false;
  if (lane < n_group) {
    const float mine = gscore_s[wv][lane];
    int rank = 0;
    for (int g2 = 0; g2 < n_group; ++g2) {
      const float o = gscore_s[wv][g2];
      rank += (o > mine || (o == mine && g2 < lane)) ? 1 : 0;
    }
    keep_g = rank < topk_group;
  }
  const uint64_t keep_mask = __ballot(keep_g);
  uint64_t key[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      const float kv = ((keep_mask >> (e / gsz)) & 1) ? biased[e] : -1.0e4f;
      key[j] = kv == kv ? ((uint64_t)ord_f32(kv) << 32) | (uint32_t)~e : 0;
    } else {
      key[j] = 0;
    }
  }
  uint32_t sel_i = 0;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) best = key[j] > best ? key[j] : best;
    best = wave_max_u64(best, lane);
    const uint32_t bi = best ? ~(uint32_t)best : (uint32_t)r;
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (best && (uint32_t)(lane + 64 * j) == bi) key[j] = 0;  // taken
    if (lane == r) sel_i = bi;
  }
  // weights: the unbiased score of each selected expert, slot r in lane r
  float w = 0.f;
  if (lane < k) {
    const float v = row[sel_i < (uint32_t)E ? sel_i : 0];
    w = sel_i < (uint32_t)E ? 1.f / (1.f + expf(-v)) : NAN;
  }
  if (route_norm && k > 1) {
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum += __shfl(w, r, 64);  // ascending slot order
    w = w / (sum + 1e-20f);
  }
  if (route_scale != 1.f) w = w * route_scale;
  if (lane < k) {
    inds[t * k + lane] = sel_i;
    scores[t * k + lane] = w;
  }
}

// Stable counting sort of expert ids by one 1024-thread block. Ids >= E share the
// last bucket (kept in index order). seg may be null; otherwise seg[e] is the first
// sorted position of expert e and seg[E] the number of in-range ids.
constexpr int kSortThreads = 1024;

// WAVE_COUNTS: the scatter of a 1024-id chunk takes 3 barriers: each wave's per-bucket
// counts go to an LDS table wc[16][E+1] (16-bit) and an id's position adds the counts of
// the waves before its own. Otherwise the 16 waves take turns (16 barriers per chunk),
// for expert counts whose table does not fit in LDS.
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortMaxWaveCountE = 4000;

template <bool WAVE_COUNTS>
__global__ void __launch_bounds__(kSortThreads) sort_dispatch_kernel(
    const uint32_t* __restrict__ flat, int64_t n, int k, int E, uint32_t* __restrict__ order,
    uint32_t* __restrict__ inv, uint32_t* __restrict__ sorted, uint32_t* __restrict__ lhs,
    uint32_t* __restrict__ seg, int stage) {
  // cnt[E+1], part[kSortThreads], then wc[16][E+1] u16; stage: then order[n], sorted[n]
  extern __shared__ uint32_t sh[];
  uint32_t* cnt = sh;
  uint32_t* part = sh + (E + 1);
  uint16_t* wc = reinterpret_cast<uint16_t*>(part + kSortThreads);
  uint32_t* s_order = part + kSortThreads + (WAVE_COUNTS ? (kSortWaves * (E + 1) + 1) / 2 : 0);
  uint32_t* s_sorted = s_order + n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NB = E + 1;
  const int nbits = 32 - __builtin_clz((unsigned)E);  // bits of the largest bucket id, E
  for (int b = tid; b < NB; b += kSortThreads) cnt[b] = 0;
  if constexpr (WAVE_COUNTS)
    for (int b = tid; b < kSortWaves * NB; b += kSortThreads) wc[b] = 0;
  lds_sync();
  // 8 loads in flight per thread before the first atomic. Up to 8 chunks of 1024 ids the
  // thread's ids stay in registers for the scatter below (no second round of loads).
  const bool keep = n <= 8 * kSortThreads;
  uint32_t vk[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  for (int64_t i0 = tid; i0 < n; i0 += 8 * kSortThreads) {
    uint32_t v[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int64_t i = i0 + (int64_t)p * kSortThreads;
      v[p] = i < n ? flat[i] : 0xFFFFFFFFu;
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      vk[p] = v[p];
      if (i0 + (int64_t)p * kSortThreads < n)
        atomicAdd(&cnt[v[p] < (uint32_t)E ? v[p] : (uint32_t)E], 1u);
    }
  }
  lds_sync();
  // Exclusive scan of cnt: each thread owns a contiguous run of buckets.
  const int per = (NB + kSortThreads - 1) / kSortThreads;
  const int b0 = min(tid * per, NB), b1 = min(b0 + per, NB);
  uint32_t local = 0;
  for (int b = b0; b < b1; ++b) local += cnt[b];
  // Block exclusive scan of `local`: DPP scan within each wave, then the 16 wave totals
  // scanned by the first wave.
  const uint32_t incl = (uint32_t)wave_scan_incl_i32<false>((int)local);
  if (lane == 63) part[wave] = incl;
  lds_sync();
  if (wave == 0) {
    const uint32_t wt = lane < kSortWaves ? part[lane] : 0u;
    const uint32_t wi = (uint32_t)wave_scan_incl_i32<false>((int)wt);
    if (lane < kSortWaves) part[kSortWaves + lane] = wi - wt;  // exclusive
  }
  lds_sync();
  uint32_t run = part[kSortThreads / 64 + wave] + incl - local;
  for (int b = b0; b < b1; ++b) {
    const uint32_t c = cnt[b];
    cnt[b] = run;  // cnt now holds the next free position of each bucket
    if (seg) seg[b] = run;
    run += c;
  }
  lds_sync();
  // Stable scatter, 1024 ids at a time; waves of a chunk take their turn in order.
  auto scatter = [&](int64_t base, uint32_t loaded) {
    const int64_t i = base + tid;
    const bool valid = i < n;
    const uint32_t raw = valid ? loaded : 0u;
    const uint32_t b = valid ? (raw < (uint32_t)E ? raw : (uint32_t)E) : 0xFFFFFFFFu;
    // Lanes of this wave holding the same bucket: one ballot per bit of the bucket id,
    // each lane keeping the lanes that agree with it on every bit (invalid lanes removed).
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool one = (b >> bit) & 1u;
      const uint64_t m = __ballot(one);
      peers &= one ? m : ~m;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    const bool lead = rank == 0;
    if constexpr (WAVE_COUNTS) {
      const uint32_t nb = (uint32_t)__popcll(peers);
      if (valid && lead) wc[wave * NB + b] = (uint16_t)nb;
      lds_sync();
      if (valid) {
        // all 16 reads issued back to back (a loop bounded by `wave` waited on each in turn:
        // ~2 us a 1024-id chunk)
        uint32_t pos = cnt[b] + (uint32_t)rank;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
          const uint32_t c = wc[w * NB + b];
          pos += w < wave ? c : 0u;
        }
        if (stage) {
          s_order[pos] = (uint32_t)i;
          s_sorted[pos] = raw;
        } else {
          order[pos] = (uint32_t)i;
          sorted[pos] = raw;
          lhs[pos] = (uint32_t)i / (uint32_t)k;
        }
        inv[i] = pos;
      }
      lds_sync();  // every read of cnt / wc for this chunk is done
      if (valid && lead) {
        atomicAdd(&cnt[b], nb);
        wc[wave * NB + b] = 0;
      }
      lds_sync();
      return;
    }
    for (int w = 0; w < kSortThreads / 64; ++w) {
      if (wave == w && valid) {
        const uint32_t start = cnt[b];
        const uint32_t pos = start + (uint32_t)rank;
        if (stage) {
          s_order[pos] = (uint32_t)i;
          s_sorted[pos] = raw;
        } else {
          order[pos] = (uint32_t)i;
          sorted[pos] = raw;
          lhs[pos] = (uint32_t)i / (uint32_t)k;
        }
        inv[i] = pos;
        if (lead) cnt[b] = start + (uint32_t)__popcll(peers);
      }
      lds_sync();
    }
  };
  if (keep) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if ((int64_t)c * kSortThreads >= n) break;  // block-uniform
      scatter((int64_t)c * kSortThreads, vk[c]);
    }
    if (stage) {
      // the sorted arrays leave LDS in order: coalesced stores instead of three scattered
      // ones per id (4096 ids: 11.6 -> 10.8 us a launch)
      lds_sync();
      for (int j = tid; j < n; j += kSortThreads) {
        const uint32_t o = s_order[j];
        order[j] = o;
        sorted[j] = s_sorted[j];
        lhs[j] = o / (uint32_t)k;
      }
    }
    return;
  }
  // longer lists: the next chunk's id is loaded while this chunk is scattered
  uint32_t next = tid < n ? flat[tid] : 0u;
  for (int64_t base = 0; base < n; base += kSortThreads) {
    const uint32_t cur = next;
    next = base + kSortThreads + tid < n ? flat[base + kSortThreads + tid] : 0u;
    scatter(base, cur);
  }
}

__global__ void take_rows_kernel(void* __restrict__ out, const void* __restrict__ in,
                                 const uint32_t* __restrict__ idx, int64_t n_src,
                                 int64_t row_bytes) {
  const int64_t r = blockIdx.y;
  const uint32_t src = idx[r];
  const bool ok = (int64_t)src < n_src;
  if ((row_bytes & 15) == 0) {
    const int64_t nv = row_bytes >> 4;
    u32x4_t* o = (u32x4_t*)((char*)out + r * row_bytes);
    const u32x4_t* s = (const u32x4_t*)((const char*)in + (int64_t)src * row_bytes);
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < nv;
         j += (int64_t)gridDim.x * blockDim.x) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      o[j] = ok ? s[j] : z;
    }
  } else {
    unsigned char* o = (unsigned char*)out + r * row_bytes;
    const unsigned char* s = (const unsigned char*)in + (int64_t)src * row_bytes;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < row_bytes;
         j += (int64_t)gridDim.x * blockDim.x)
      o[j] = ok ? s[j] : 0;
  }
}

// 8 values per thread with 16-byte loads and stores (n % 8 == 0, 16-byte aligned).
__global__ void swiglu8_kernel(u32x4_t* __restrict__ y, const u32x4_t* __restrict__ g,
                               const u32x4_t* __restrict__ u, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    const u32x4_t gv = g[i], uv = u[i];
    u32x4_t o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = swiglu_bf16((uint16_t)(gv[c] & 0xFFFFu), (uint16_t)(uv[c] & 0xFFFFu));
      const uint32_t hi = swiglu_bf16((uint16_t)(gv[c] >> 16), (uint16_t)(uv[c] >> 16));
      o[c] = lo | (hi << 16);
    }
    y[i] = o;
  }
}

__global__ void swiglu_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ g,
                              const uint16_t* __restrict__ u, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint16_t gv = g[i];
    y[i] = swiglu_bf16(gv, u[i]);
  }
}

// y[t, n] = sum over slots s ascending of bf16(v[t*k+s, n] * score[t*k+s]), each add
// rounded to bf16, starting from bf16 zero.
// rows (nullable): v's row of pair p is rows[p] (the inverse of the expert sort), so the
// unsort rides in the reduce; a row index >= n_rows reads as zeros, as take_rows returns.
// The bf16 score product and the slot sum are those of down_reduce_kernel, so the result is
// bit-equal to take_rows followed by the plain reduce.
__global__ void down_reduce_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ v,
                                   const uint16_t* __restrict__ scores,
                                   const uint32_t* __restrict__ rows, int64_t n_rows,
                                   int64_t T, int k, int64_t N) {
  const int64_t t = blockIdx.y;
  for (int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; n < N;
       n += (int64_t)gridDim.x * blockDim.x) {
    uint16_t total = 0;
    for (int s = 0; s < k; ++s) {
      const int64_t p = t * k + s;
      const int64_t src = rows ? (int64_t)rows[p] : p;
      const uint16_t x = src < n_rows ? v[src * N + n] : (uint16_t)0;
      total = bf16_add(total, bf16_mul(x, scores[p]));
    }
    y[t * N + n] = total;
  }
}

// 8 outputs per thread with 16-byte loads (N % 8 == 0, 16-byte aligned rows).
__global__ void down_reduce8_kernel(u32x4_t* __restrict__ y, const u32x4_t* __restrict__ v,
                                    const uint16_t* __restrict__ scores,
                                    const uint32_t* __restrict__ rows, int64_t n_rows,
                                    int64_t T, int k, int64_t N8) {
  const int64_t t = blockIdx.y;
  for (int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; n < N8;
       n += (int64_t)gridDim.x * blockDim.x) {
    u32x4_t total = {0u, 0u, 0u, 0u};
    int s = 0;
    // 8 slots at a time: every row index, score and row segment of the group is loaded
    // before the first add (one memory round trip a group, not one a slot)
    for (; s + 8 <= k; s += 8) {
      const int64_t p0 = t * k + s;
      int64_t src[8];
      if (rows) {
#pragma unroll
        for (int q = 0; q < 8; ++q) src[q] = (int64_t)rows[p0 + q];
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) src[q] = p0 + q;
      }
      u32x4_t xs[8];
      uint16_t scs[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        xs[q] = src[q] < n_rows ? v[src[q] * N8 + n] : zero;  // out of range: a zero row
        scs[q] = scores[p0 + q];
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t lo = bf16_add((uint16_t)(total[c] & 0xFFFFu), bf16_mul((uint16_t)(xs[q][c] & 0xFFFFu), scs[q]));
          const uint32_t hi = bf16_add((uint16_t)(total[c] >> 16), bf16_mul((uint16_t)(xs[q][c] >> 16), scs[q]));
          total[c] = lo | (hi << 16);
        }
      }
    }
    for (; s < k; ++s) {
      const int64_t p = t * k + s;
      const int64_t src = rows ? (int64_t)rows[p] : p;
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      const u32x4_t x = src < n_rows ? v[src * N8 + n] : zero;
      const uint16_t sc = scores[p];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t lo = bf16_add((uint16_t)(total[c] & 0xFFFFu), bf16_mul((uint16_t)(x[c] & 0xFFFFu), sc));
        const uint32_t hi = bf16_add((uint16_t)(total[c] >> 16), bf16_mul((uint16_t)(x[c] >> 16), sc));
        total[c] = lo | (hi << 16);
      }
    }
    y[t * N8 + n] = total;
  }
}

unsigned grid_for(int64_t n, int threads) {
  int64_t b = (n + threads - 1) / threads;
  return (unsigned)(b < 1 ? 1 : b > 65535 ? 65535 : b);
}

}  // namespace

hipError_t launch_route_topk(const float* logits, int64_t T, int E, int k, uint32_t* inds,
                             void* scores, int scores_bf16, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const unsigned grid = (unsigned)((T + 3) / 4);
  const int nv = (E + 63) / 64;
#define MI_ROUTE(NVV)                                                                      \
  hipLaunchKernelGGL(route_topk_kernel<NVV>, dim3(grid), dim3(256), 0, s, logits, T, E, k, \
                     inds, scores, scores_bf16)
  if (nv <= 1) MI_ROUTE(1);
  else if (nv <= 2) MI_ROUTE(2);
  else if (nv <= 4) MI_ROUTE(4);
  else if (nv <= 8) MI_ROUTE(8);
  else MI_ROUTE(16);
#undef MI_ROUTE
  return hipGetLastError();
}

hipError_t launch_route_grouped(const float* logits, const float* bias, int64_t T, int E, int k,
                                int n_group, int topk_group, int route_norm, float route_scale,
                                uint32_t* inds, float* scores, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const unsigned grid = (unsigned)((T + 3) / 4);
  const int nv = (E + 63) / 64;
#define MI_ROUTEG(NVV)                                                                       \
  hipLaunchKernelGGL(route_grouped_kernel<NVV>, dim3(grid), dim3(256), 0, s, logits, bias, T, \
                     E, k, n_group, topk_group, route_norm, route_scale, inds, scores)
  if (nv <= 2) MI_ROUTEG(2);
  else if (nv <= 4) MI_ROUTEG(4);
  else if (nv <= 8) MI_ROUTEG(8);
  else MI_ROUTEG(16);
#undef MI_ROUTEG
  return hipGetLastError();
}

size_t sort_dispatch_lds_bytes(int E) {
  const size_t base = ((size_t)E + 1 + kSortThreads) * 4;
  return E <= kSortMaxWaveCountE ? base + ((size_t)kSortWaves * (E + 1) + 1) / 2 * 4 : base;
}

namespace {
// Lists of up to 8 chunks whose sorted order / id arrays fit LDS beside the tables are
// scattered into LDS and written out in order.
bool sort_stage(int64_t n, int E) {
  return n <= 8 * kSortThreads && sort_dispatch_lds_bytes(E) + (size_t)n * 8 <= 160 * 1024;
}
}  // namespace

hipError_t launch_sort_dispatch(const uint32_t* flat, int64_t n, int k, int E, uint32_t* order,
                                uint32_t* inv, uint32_t* sorted, uint32_t* lhs, uint32_t* seg,
                                hipStream_t s) {
  const int stage = sort_stage(n, E) ? 1 : 0;
  const size_t lds = sort_dispatch_lds_bytes(E) + (stage ? (size_t)n * 8 : 0);
  if (E <= kSortMaxWaveCountE) {
    static const bool attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&sort_dispatch_kernel<true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    (void)attr;  // a failure shows as a launch error for tables above 64 KiB
    hipLaunchKernelGGL(sort_dispatch_kernel<true>, dim3(1), dim3(kSortThreads), lds, s, flat, n,
                       k, E, order, inv, sorted, lhs, seg, stage);
  } else {
    static const bool attr2 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&sort_dispatch_kernel<false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    (void)attr2;
    hipLaunchKernelGGL(sort_dispatch_kernel<false>, dim3(1), dim3(kSortThreads), lds, s, flat, n,
                       k, E, order, inv, sorted, lhs, seg, stage);
  }
  return hipGetLastError();
}

hipError_t launch_take_rows(void* out, const void* in, const uint32_t* idx, int64_t n,
                            int64_t n_src, int64_t row_bytes, hipStream_t s) {
  if (n == 0 || row_bytes == 0) return hipSuccess;
  const int64_t units = (row_bytes & 15) == 0 ? row_bytes / 16 : row_bytes;
  hipLaunchKernelGGL(take_rows_kernel, dim3(grid_for(units, 256), (unsigned)n), dim3(256), 0, s,
                     out, in, idx, n_src, row_bytes);
  return hipGetLastError();
}

hipError_t launch_swiglu(uint16_t* y, const uint16_t* g, const uint16_t* u, int64_t n,
                         hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (n % 8 == 0 && ((uintptr_t)y | (uintptr_t)g | (uintptr_t)u) % 16 == 0) {
    hipLaunchKernelGGL(swiglu8_kernel, dim3(grid_for(n / 8, 256)), dim3(256), 0, s, (u32x4_t*)y,
                       (const u32x4_t*)g, (const u32x4_t*)u, n / 8);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, y, g, u, n);
  return hipGetLastError();
}

hipError_t launch_down_reduce(uint16_t* y, const uint16_t* v, const uint16_t* scores, int64_t T,
                              int k, int64_t N, hipStream_t s, const uint32_t* rows,
                              int64_t n_rows) {
  if (!rows) n_rows = T * k;
  if (T == 0 || N == 0) return hipSuccess;
  if (N % 8 == 0 && ((uintptr_t)y | (uintptr_t)v) % 16 == 0) {
    hipLaunchKernelGGL(down_reduce8_kernel, dim3(grid_for(N / 8, 256), (unsigned)T), dim3(256), 0,
                       s, (u32x4_t*)y, (const u32x4_t*)v, scores, rows, n_rows, T, k, N / 8);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(down_reduce_kernel, dim3(grid_for(N, 256), (unsigned)T), dim3(256), 0, s, y,
                     v, scores, rows, n_rows, T, k, N);
  return hipGetLastError();
}

}  // namespace mi
