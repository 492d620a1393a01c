// Softmax top-k routing of one token by one wave (moeRoutingChain,
// src/transformer.zig:17022-17072), shared by the routing kernel and the launches that
// route inside themselves. Plus the wave-wide reductions it uses.
#pragma once
#include "mi_common.h"

namespace mi {
namespace route_detail {

// Wave-wide reductions without LDS: DPP quad_perm (lane ^ 1, ^ 2), row_half_mirror and
// row_mirror (pair the two completed halves of each 8 and 16 lanes), then permlane16/32
// swaps (rows ^ 1, halves). Every lane ends with the result; the combine order is fixed.
template <int CTRL>
MI_DEV uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
MI_DEV uint32_t xor16_u32(uint32_t v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (lane & 16) ? r[0] : r[1];
}
MI_DEV uint32_t xor32_u32(uint32_t v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (lane & 32) ? r[0] : r[1];
}
struct U64Max {
  MI_DEV static uint64_t op(uint64_t a, uint64_t b) { return a > b ? a : b; }
};
template <int CTRL>
MI_DEV uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}
MI_DEV uint64_t wave_max_u64(uint64_t k, int lane) {
  k = U64Max::op(k, dpp_u64<0xB1>(k));   // lane ^ 1
  k = U64Max::op(k, dpp_u64<0x4E>(k));   // lane ^ 2
  k = U64Max::op(k, dpp_u64<0x141>(k));  // other quad of the 8
  k = U64Max::op(k, dpp_u64<0x140>(k));  // other half of the 16
  k = U64Max::op(k, ((uint64_t)xor16_u32((uint32_t)(k >> 32), lane) << 32) |
                        xor16_u32((uint32_t)k, lane));
  k = U64Max::op(k, ((uint64_t)xor32_u32((uint32_t)(k >> 32), lane) << 32) |
                        xor32_u32((uint32_t)k, lane));
  return k;
}
template <bool MAX>
MI_DEV float wave_reduce_f32(float v, int lane) {
  auto comb = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = comb(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v))));
  v = comb(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v))));
  v = comb(v, __uint_as_float(dpp_u32<0x141>(__float_as_uint(v))));
  v = comb(v, __uint_as_float(dpp_u32<0x140>(__float_as_uint(v))));
  v = comb(v, __uint_as_float(xor16_u32(__float_as_uint(v), lane)));
  v = comb(v, __uint_as_float(xor32_u32(__float_as_uint(v), lane)));
  return v;
}

// Order-preserving key of a non-NaN logit (-0 counts as +0): larger value, larger key.
MI_DEV uint32_t ord_f32(float v) {
  const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
MI_DEV float unord_f32(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}


}  // namespace route_detail

// Wave maximum of a 32-bit key, the same butterfly as wave_reduce_f32.
MI_DEV uint32_t wave_max_u32(uint32_t v, int lane) {
  using namespace route_detail;
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = mx(v, dpp_u32<0xB1>(v));
  v = mx(v, dpp_u32<0x4E>(v));
  v = mx(v, dpp_u32<0x141>(v));
  v = mx(v, dpp_u32<0x140>(v));
  v = mx(v, xor16_u32(v, lane));
  v = mx(v, xor32_u32(v, lane));
  return v;
}

// k rounds of selection over order-preserving 32-bit keys of the ids lane + 64 j (key 0:
// not a candidate). Each round takes the wave's largest key and, among the ids holding
// it, the lowest (ids ascend with j, then with the lane: one ballot per j); that id's key
// becomes 0. A round with no candidate takes id r and key 0. Lane r < k ends with round
// r's id and key. Every lane of the wave must call it.
template <int NV>
MI_DEV void select_topk(uint32_t (&key)[NV], int k, int lane, uint32_t& sel_i,
                        uint32_t& sel_key) {
  sel_i = 0;
  sel_key = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t lb = key[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) lb = key[j] > lb ? key[j] : lb;
    const uint32_t m = __builtin_amdgcn_readfirstlane(wave_max_u32(lb, lane));
    uint32_t bi = (uint32_t)r;
    if (m) {
      bi = 0xFFFFFFFFu;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const uint64_t b = __builtin_amdgcn_ballot_w64(key[j] == m);
        if (bi == 0xFFFFFFFFu && b) bi = 64u * j + (uint32_t)__builtin_ctzll(b);
      }
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if ((uint32_t)(lane + 64 * j) == bi) key[j] = 0;  // taken
    }
    if (lane == r) {
      sel_i = bi;
      sel_key = m;
    }
  }
}

// Softmax over the E logits of `row`, top-k, weights renormalized over the k selected.
// Lane r < k ends with slot r: its expert id and its weight (slots in descending logit
// order, ties to the lower id). NaN logits never win; a round with no candidate takes id
// r with a NaN weight, as an all-NaN row does. NV = ceil(E / 64) values per lane. Every
// lane of the wave must call it.
template <int NV>
MI_DEV void route_token(const float* __restrict__ row, int E, int k, int lane, uint32_t& sel_i,
                        float& weight) {
  using namespace route_detail;
  float v[NV];
  uint32_t key[NV];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? row[e] : -INFINITY;
    mx = fmaxf(mx, v[j]);
    key[j] = (e < E && v[j] == v[j]) ? ord_f32(v[j]) : 0u;  // never 0 for a non-NaN
  }
  mx = wave_reduce_f32<true>(mx, lane);
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (lane + 64 * j < E) den += expf(v[j] - mx);
  den = wave_reduce_f32<false>(den, lane);

  uint32_t sel_key;
  select_topk<NV>(key, k, lane, sel_i, sel_key);
  const float sel_v = sel_key ? unord_f32(sel_key) : NAN;
  // Renormalized softmax weights of the selected experts; slot r lives in lane r.
  const float w = lane < k ? expf(sel_v - mx) / den : 0.f;
  float sum = 0.f;
  for (int r = 0; r < k; ++r)  // ascending slot order
    sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w), r));
  weight = w / sum;
}

}  // namespace mi
