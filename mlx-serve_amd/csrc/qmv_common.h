// Device helpers shared by the small-M quantized matmul kernels (qmv*.hip).
#pragma once
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {
namespace qmv_detail {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

MI_DEV f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                  __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
}

template <int N>
MI_DEV void load_u32(const uint32_t* __restrict__ p, uint32_t (&out)[N]) {
  if constexpr (N == 2) {
    u32x2_t v = *reinterpret_cast<const u32x2_t*>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      u32x4_t v = *(reinterpret_cast<const u32x4_t*>(p) + i);
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
    const uint32_t pair = (uint32_t)it / (uint32_t)P.items_per_pair;
    const int c = it - (int)(pair * P.items_per_pair);
    r.pos0 = (int64_t)pair * P.M + (int64_t)c * P.rpi;
    r.cnt = min(P.rpi, P.M - c * P.rpi);
    r.expert = P.rhs ? P.rhs[pair] : pair;
  }
  r.expert_ok = r.expert < (uint32_t)P.n_experts;
  return r;
}

// Element offset of x's row for item row li; -1: not a row of this item; -2: the
// row exists but its lhs index is out of range (NaN output). Sorted items keep a
// row only while its pair's rhs is the item's expert. Positions are < 2^32.
MI_DEV int64_t item_x_row(const QmvParams& P, const Item& it, int li) {
  if (li >= it.cnt) return -1;
  const uint32_t p = (uint32_t)(it.pos0 + li);
  const uint32_t pair = P.M == 1 ? p : p / (uint32_t)P.M;
  if (P.items && P.rhs[pair] != it.expert) return -1;
  const uint32_t m = p - pair * (uint32_t)P.M;
  const uint32_t l = P.lhs ? P.lhs[pair] : (P.lhs_div == 1 ? pair : pair / (uint32_t)P.lhs_div);
  if ((int64_t)l >= P.x_batch) return -2;
  return ((int64_t)l * P.M + m) * (int64_t)P.K;
}

// Block barrier for LDS traffic only: waits for this wave's LDS operations, not for
// its outstanding global loads (a __syncthreads fence would drain those too).
MI_DEV void lds_barrier() { lds_sync(); }

// s_waitcnt immediate for vmcnt(n) (gfx9 split field), expcnt/lgkmcnt untouched.
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

}  // namespace qmv_detail
}  // namespace mi
