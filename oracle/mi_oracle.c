/*
 * mi_oracle.c -- CPU restatement of MLX affine quantized matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Parity status per function (what pins it; tests/test_oracle.py holds the checks):
 *   mo_pack/mo_unpack        known bit patterns + round trip; reference restatement
 *                            src/transformer.zig:20098-20108 (nibble order), :522-525 (bytes).
 *   mo_quantize_bf16         invariants (code range, exact edge, |w-deq| <= |s|/2, exact zero)
 *                            and hand-computed groups: exact .5 ties of the codes and of
 *                            edge/scale (rint, ties to even), the edge refit, negative-edge
 *                            groups, the q0 == 0 branch under the 1e-7 scale floor, codes
 *                            straddling words at 2/3/5/6 bits. Bit-parity with real
 *                            mx.quantize is PARITY UNPINNED (MLX is an un-vendored submodule,
 *                            no MLX here): these checks fix this restatement, not MLX.
 *   mo_dequantize            closed forms (s*q exact in fp32), hand-computed values; which
 *                            bf16 rounding mx.dequantize applies is PARITY UNPINNED, both kept.
 *   mo_qmm_f64 / gather      numpy float64 matmul on independently dequantized weights,
 *                            one-hot / all-ones / integer special cases.
 *   mo_route_softmax_topk    numpy softmax + lexsort top-k.
 *   mo_route_grouped_f64     reduces to a plain sigmoid top-k when one group or every group
 *                            survives (numpy lexsort); a hand-built group mask case.
 *   mo_sort_dispatch         numpy stable argsort; inverse-permutation identity.
 *   mo_swiglu / down_reduce  exhaustive sigmoid table vs fp64 sigmoid; composition checks.
 *                            The table is the correctly rounded sigmoid; the reference builds
 *                            it with mlx_sigmoid on bf16 values (src/transformer.zig:19876-
 *                            19880), whose rounding is PARITY UNPINNED (no MLX here).
 *   mo_affine_params...      the reference's own test cases for the geometry solve.
 */
#include "mi_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- bf16 --- */
float mo_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t mo_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
    return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  }
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

void mo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mo_f32_to_bf16(in[i]);
}

void mo_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mo_bf16_to_f32(in[i]);
}

/* ----------------------------------------------------------- generator --- */
uint64_t mo_splitmix64(uint64_t seed, uint64_t counter) {
  uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void mo_uniform_f64(double* out, int64_t n, uint64_t seed) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = (double)(mo_splitmix64(seed, (uint64_t)i) >> 11) * (1.0 / 9007199254740992.0);
}

void mo_randn_f32(float* out, int64_t n, uint64_t seed, double mean, double stddev) {
  const double two_pi = 6.283185307179586476925286766559;
  int64_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < pairs; ++j) {
    uint64_t a = mo_splitmix64(seed, (uint64_t)(2 * j));
    uint64_t b = mo_splitmix64(seed, (uint64_t)(2 * j + 1));
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double r = sqrt(-2.0 * log(u1));
    double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
    out[2 * j] = (float)(mean + stddev * z0);
    if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + stddev * z1);
  }
}

/* ------------------------------------------------------------- packing --- */
/* Affine widths MLX packs: 2, 3, 4, 5, 6 and 8 bits. A row of K codes is one LSB-first
 * bitstream, code j at bit j*bits of the row's little-endian bytes (uint32 words, K*bits a
 * multiple of 32). For 2/4/8 bits this is "value j of a word = (word >> (j*bits)) & mask"
 * (src/transformer.zig:20098-20108); 5 bits puts 8 codes in 5 bytes and 6 bits 4 codes in
 * 3 bytes (src/transformer.zig:516-578, the byte reads of vqmmColumnLoad / vqmmColumnChain). */
static int valid_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

static uint32_t get_code(const uint32_t* row, int64_t j, int bits) {
  const int64_t o = j * bits;
  const int64_t w = o >> 5;
  const int sh = (int)(o & 31);
  uint64_t v = row[w] >> sh;
  if (sh + bits > 32) v |= (uint64_t)row[w + 1] << (32 - sh);
  return (uint32_t)(v & ((1u << bits) - 1u));
}

/* the row's words must start at zero */
static void put_code(uint32_t* row, int64_t j, int bits, uint32_t code) {
  const int64_t o = j * bits;
  const int64_t w = o >> 5;
  const int sh = (int)(o & 31);
  code &= (1u << bits) - 1u;
  row[w] |= code << sh;
  if (sh + bits > 32) row[w + 1] |= code >> (32 - sh);
}

int mo_pack(const uint8_t* q, int64_t rows, int64_t K, int bits, uint32_t* wq) {
  if (!valid_bits(bits) || (K * bits) % 32) return -1;
  int64_t wc = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t* row = wq + r * wc;
    for (int64_t c = 0; c < wc; ++c) row[c] = 0;
    for (int64_t j = 0; j < K; ++j) put_code(row, j, bits, q[r * K + j]);
  }
  return 0;
}

int mo_unpack(const uint32_t* wq, int64_t rows, int64_t K, int bits, uint8_t* q) {
  if (!valid_bits(bits) || (K * bits) % 32) return -1;
  int64_t wc = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < K; ++j) q[r * K + j] = (uint8_t)get_code(wq + r * wc, j, bits);
  return 0;
}

/* ------------------------------------------------------------ quantize --- */
/* Restates MLX's affine group quantizer (mx.quantize, mode "affine"): per group
 * of gs values along K, in fp32: scale = max((max-min)/(2^bits-1), 1e-7), signed
 * toward the larger-magnitude edge; edge = that extreme; q0 = rint(edge/scale);
 * when q0 != 0 the scale is refit to edge/q0 and bias = edge (so 0.0 lands on an
 * integer code), else bias = 0; codes = clamp(rint((w-bias)/scale), 0, 2^bits-1).
 * Scales and biases are stored rounded to bf16; codes use the fp32 scale.
 * Reference call sites: src/mlx.zig:275 (mlx_quantize), src/transformer.zig:24853-24872
 * (bf16 weight quantized at bits/gs). */
int mo_quantize_bf16(const uint16_t* w, int64_t rows, int64_t K, int gs, int bits,
                     uint32_t* wq, uint16_t* scales, uint16_t* biases) {
  if (!valid_bits(bits) || gs <= 0 || K % gs || (gs * bits) % 32) return -1;
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  int64_t wc = K * bits / 32, ng = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < ng; ++g) {
      const uint16_t* src = w + r * K + g * gs;
      float wmax = -INFINITY, wmin = INFINITY;
      for (int j = 0; j < gs; ++j) {
        float v = mo_bf16_to_f32(src[j]);
        wmax = fmaxf(wmax, v);
        wmin = fminf(wmin, v);
      }
      int mask = fabsf(wmin) > fabsf(wmax);
      volatile float span = wmax - wmin; /* keep each fp32 op rounded on its own */
      float scale = fmaxf(span / n_bins, eps);
      scale = mask ? scale : -scale;
      float edge = mask ? wmin : wmax;
      float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      uint32_t* gw = wq + r * wc + g * (gs * bits / 32);  /* the group's whole words */
      for (int c = 0; c < gs * bits / 32; ++c) gw[c] = 0;
      for (int j = 0; j < gs; ++j) {
        volatile float d = mo_bf16_to_f32(src[j]) - bias;
        float qv = rintf(d / scale);
        qv = fminf(fmaxf(qv, 0.0f), n_bins);
        put_code(gw, j, bits, (uint32_t)qv);
      }
      scales[r * ng + g] = mo_f32_to_bf16(scale);
      biases[r * ng + g] = mo_f32_to_bf16(bias);
    }
  }
  return 0;
}

/* ---------------------------------------------------------- dequantize --- */
/* w = scale * q + bias per element (src/transformer.zig:20099-20104 restates it;
 * src/mlx.zig:271 is the mlx_dequantize binding). float(bf16 s) * q is exact in
 * fp32, so the fp32 result is one rounding of s*q+b. For bf16 output:
 *   MO_DQ_BF16_FUSED  : bf16(s*q + b)                       (one rounding)
 *   MO_DQ_BF16_OPWISE : bf16(float(bf16(s*q)) + b)          (MLX op-by-op: multiply
 *                       then add, each a bf16 op; the composed fallback of mx.dequantize) */
int mo_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                  int64_t rows, int64_t K, int gs, int bits, int kind, void* out) {
  if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32) return -1;
  int64_t wc = K * bits / 32, ng = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < K; ++k) {
      float q = (float)get_code(wq + r * wc, k, bits);
      float s = mo_bf16_to_f32(scales[r * ng + k / gs]);
      float b = mo_bf16_to_f32(biases[r * ng + k / gs]);
      volatile float sq = s * q; /* exact */
      float v;
      if (kind == MO_DQ_BF16_OPWISE) {
        float sqr = mo_bf16_to_f32(mo_f32_to_bf16(sq));
        volatile float t = sqr + b;
        v = t;
      } else {
        volatile float t = sq + b;
        v = t;
      }
      if (kind == MO_DQ_F32)
        ((float*)out)[r * K + k] = v;
      else
        ((uint16_t*)out)[r * K + k] = mo_f32_to_bf16(v);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ qmm --- */
static double x_at(const void* x, int x_f32, int64_t i) {
  return x_f32 ? (double)((const float*)x)[i] : (double)mo_bf16_to_f32(((const uint16_t*)x)[i]);
}

/* Exact dequantized row n (fp64: s*q+b has no rounding in double). */
static void deq_row_f64(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                        int64_t n, int64_t K, int gs, int bits, double* row) {
  int64_t wc = K * bits / 32, ng = K / gs;
  for (int64_t k = 0; k < K; ++k) {
    double q = (double)get_code(wq + n * wc, k, bits);
    row[k] = (double)mo_bf16_to_f32(scales[n * ng + k / gs]) * q +
             (double)mo_bf16_to_f32(biases[n * ng + k / gs]);
  }
}

/* y = x @ dequant(W)^T, transpose=true (src/transformer.zig:20970-20981 calls
 * mlx_quantized_matmul with transpose=true, "affine"). Truth = fp64 over exactly
 * dequantized weights, as the reference tests' ground truth (:24881-24893). */
int mo_qmm_f64(const void* x, int x_f32, const uint32_t* wq, const uint16_t* scales,
               const uint16_t* biases, int64_t M, int64_t N, int64_t K, int gs, int bits,
               double* y) {
  if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32) return -1;
#pragma omp parallel
  {
    double* row = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      deq_row_f64(wq, scales, biases, n, K, gs, bits, row);
      for (int64_t m = 0; m < M; ++m) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += x_at(x, x_f32, m * K + k) * row[k];
        y[m * N + n] = acc;
      }
    }
    free(row);
  }
  return 0;
}

/* The timed CPU baseline: fp32 accumulation, dequant on the fly, threads over N.
 * Per group: acc += s * sum(x*q) + b * sum(x), the same algebra MLX's qmv uses. */
int mo_qmm_f32(const uint16_t* x_bf16, const uint32_t* wq, const uint16_t* scales,
               const uint16_t* biases, int64_t M, int64_t N, int64_t K, int gs, int bits,
               float* y, int threads) {
  if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32) return -1;
  int64_t wc = K * bits / 32, ng = K / gs;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  float* xs = (float*)malloc(sizeof(float) * (size_t)(M * ng));
  for (int64_t i = 0; i < M * K; ++i) xf[i] = mo_bf16_to_f32(x_bf16[i]);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < ng; ++g) {
      float s = 0.f;
      for (int j = 0; j < gs; ++j) s += xf[m * K + g * gs + j];
      xs[m * ng + g] = s;
    }
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel
  {
    float* qrow = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      for (int64_t k = 0; k < K; ++k) qrow[k] = (float)get_code(wq + n * wc, k, bits);
      for (int64_t m = 0; m < M; ++m) {
        float acc = 0.f;
        const float* xr = xf + m * K;
        for (int64_t g = 0; g < ng; ++g) {
          float d = 0.f;
          for (int j = 0; j < gs; ++j) d += xr[g * gs + j] * qrow[g * gs + j];
          acc += mo_bf16_to_f32(scales[n * ng + g]) * d + mo_bf16_to_f32(biases[n * ng + g]) * xs[m * ng + g];
        }
        y[m * N + n] = acc;
      }
    }
    free(qrow);
  }
  free(xf);
  free(xs);
  return 0;
}

/* --------------------------------------------------------- gather_qmm --- */
/* out[i] = x[lhs(i)] @ dequant(W[rhs(i)])^T. MLX gather_qmm semantics with
 * transpose=true (src/mlx.zig:265; call site src/transformer.zig:20782). A null
 * lhs means MLX's default (arange over x's batch, broadcast against rhs): the
 * reference's decode call broadcasts one token over its top-k slots
 * (src/transformer.zig:15098, x [B,S,1,1,D] vs inds [B,S,K] -> lhs(i) = i / K)
 * and the sorted call passes one row per pair (:15011 -> lhs(i) = i). */
int mo_gather_qmm_f64(const void* x, int x_f32, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint32_t* lhs, const uint32_t* rhs,
                      int64_t n_idx, int64_t lhs_div, int64_t M, int64_t N, int64_t K,
                      int64_t x_batch, int64_t n_experts, int gs, int bits, double* out) {
  if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32 || lhs_div <= 0) return -1;
  int64_t wc = K * bits / 32, ng = K / gs;
  for (int64_t i = 0; i < n_idx; ++i) {
    int64_t li = lhs ? (int64_t)lhs[i] : i / lhs_div;
    int64_t ri = rhs ? (int64_t)rhs[i] : i;
    if (li < 0 || li >= x_batch || ri < 0 || ri >= n_experts) return -2;
  }
#pragma omp parallel
  {
    double* row = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(dynamic, 1)
    for (int64_t i = 0; i < n_idx; ++i) {
      int64_t li = lhs ? (int64_t)lhs[i] : i / lhs_div;
      int64_t ri = rhs ? (int64_t)rhs[i] : i;
      const uint32_t* we = wq + ri * N * wc;
      const uint16_t* se = scales + ri * N * ng;
      const uint16_t* be = biases + ri * N * ng;
      for (int64_t n = 0; n < N; ++n) {
        deq_row_f64(we, se, be, n, K, gs, bits, row);
        for (int64_t m = 0; m < M; ++m) {
          double acc = 0.0;
          for (int64_t k = 0; k < K; ++k) acc += x_at(x, x_f32, (li * M + m) * K + k) * row[k];
          out[(i * M + m) * N + n] = acc;
        }
      }
    }
    free(row);
  }
  return 0;
}

/* ------------------------------------------------------------- routing --- */
/* moeRoutingChain (src/transformer.zig:17022-17072): argpartition(-logits, k-1)
 * selects the top-k set; softmax(precise) over all experts; take the selected
 * weights; divide by their sum. argpartition leaves the order inside the top-k
 * unspecified, so this restatement fixes it: descending logit, ties by index.
 * The weight sum runs in that slot order. */
/* Descending selection of k of n keys, ties to the lower index (the reference test's
 * routerRefRow, src/transformer.zig:23263-23282). */
static void ref_row_topk(const double* keys, int n, int k, int* out) {
  char taken[1024] = {0};
  for (int r = 0; r < k; ++r) {
    int bidx = 0, found = 0;
    double best = -INFINITY;
    for (int i = 0; i < n; ++i) {
      if (taken[i]) continue;
      if (!found || keys[i] > best) {
        best = keys[i];
        bidx = i;
        found = 1;
      }
    }
    taken[bidx] = 1;
    out[r] = bidx;
  }
}

/* Group-limited routing (groupLimitedRouting, src/transformer.zig:17242-17347, group mask
 * groupLimitMask :17138-17236) in float64, as the reference's own test computes its
 * reference (:23390-23515): sigmoid, + bias, group score = sum of the group's two largest
 * keys, the topk_group best groups kept, other keys -1e4, top-k; weights = unbiased
 * sigmoid of the selected, / (sum + 1e-20) when route_norm and k > 1, * route_scale. */
int mo_route_grouped_f64(const float* logits, const float* bias, int64_t T, int64_t E, int k,
                         int n_group, int topk_group, int route_norm, double route_scale,
                         uint32_t* inds, double* w) {
  if (k <= 0 || k > E || E > 1024 || n_group <= 0 || n_group > 64 || E % n_group ||
      topk_group <= 0 || topk_group > n_group)
    return -1;
  const int gsz = (int)(E / n_group);
  double sig[1024], keys[1024], gscore[64];
  int gsel[64], ids[64];
  for (int64_t t = 0; t < T; ++t) {
    for (int i = 0; i < E; ++i) {
      sig[i] = 1.0 / (1.0 + exp(-(double)logits[t * E + i]));
      keys[i] = sig[i] + (double)bias[i];
    }
    for (int g = 0; g < n_group; ++g) {
      double m1 = -INFINITY, m2 = -INFINITY;
      for (int i = 0; i < gsz; ++i) {
        const double v = keys[g * gsz + i];
        if (v > m1) {
          m2 = m1;
          m1 = v;
        } else if (v > m2) {
          m2 = v;
        }
      }
      gscore[g] = m1 + m2;
    }
    ref_row_topk(gscore, n_group, topk_group, gsel);
    char kept[64] = {0};
    for (int j = 0; j < topk_group; ++j) kept[gsel[j]] = 1;
    for (int i = 0; i < E; ++i)
      if (!kept[i / gsz]) keys[i] = -1.0e4;
    ref_row_topk(keys, (int)E, k, ids);
    double sum = 0.0;
    for (int j = 0; j < k; ++j) sum += sig[ids[j]];
    for (int j = 0; j < k; ++j) {
      double v = sig[ids[j]];
      if (route_norm && k > 1) v = v / (sum + 1e-20);
      inds[t * k + j] = (uint32_t)ids[j];
      w[t * k + j] = v * route_scale;
    }
  }
  return 0;
}

int mo_route_softmax_topk(const float* logits, int64_t T, int64_t E, int k,
                          uint32_t* inds, float* scores) {
  if (k <= 0 || k > E) return -1;
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    float mx = -INFINITY;
    for (int64_t e = 0; e < E; ++e) mx = fmaxf(mx, l[e]);
    float den = 0.f;
    for (int64_t e = 0; e < E; ++e) den += expf(l[e] - mx);
    uint32_t* ti = inds + t * k;
    for (int j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        int taken = 0;
        for (int p = 0; p < j; ++p) taken |= (ti[p] == (uint32_t)e);
        if (taken) continue;
        if (best < 0 || l[e] > l[best]) best = e;
      }
      ti[j] = (uint32_t)best;
    }
    float w[1024];
    float sum = 0.f;
    for (int j = 0; j < k; ++j) {
      w[j] = expf(l[ti[j]] - mx) / den;
      sum += w[j];
    }
    for (int j = 0; j < k; ++j) scores[t * k + j] = w[j] / sum;
  }
  return 0;
}

/* ---------------------------------------------------- sorted dispatch --- */
/* moeMLP2 sorted path (src/transformer.zig:14961-15005): order = argsort(flat),
 * inv = argsort(order), sorted = take(flat, order), lhs = order // K. A stable
 * counting sort; ties keep pair order (MLX argsort's tie order does not change
 * the permuted-back result, since every pair is computed independently). */
int mo_sort_dispatch(const uint32_t* flat, int64_t n, int k, uint32_t* order,
                     uint32_t* inv, uint32_t* sorted, uint32_t* lhs) {
  if (k <= 0) return -1;
  uint32_t maxv = 0;
  for (int64_t i = 0; i < n; ++i) maxv = flat[i] > maxv ? flat[i] : maxv;
  int64_t nb = (int64_t)maxv + 2;
  int64_t* cnt = (int64_t*)calloc((size_t)nb, sizeof(int64_t));
  for (int64_t i = 0; i < n; ++i) cnt[flat[i] + 1]++;
  for (int64_t b = 1; b < nb; ++b) cnt[b] += cnt[b - 1];
  for (int64_t i = 0; i < n; ++i) order[cnt[flat[i]]++] = (uint32_t)i;
  free(cnt);
  for (int64_t j = 0; j < n; ++j) {
    inv[order[j]] = (uint32_t)j;
    sorted[j] = flat[order[j]];
    lhs[j] = order[j] / (uint32_t)k;
  }
  return 0;
}

/* ---------------------------------------------------- fused contracts --- */
/* Table SwiGLU (src/transformer.zig:19855-19884 builds sigmoid over every bf16
 * pattern; :19846-19849 applies g*sig then *up, each a bf16 multiply). The table value
 * is the sigmoid evaluated in double, rounded to fp32 and then to bf16 (MLX's own
 * sigmoid rounding is not available here; this is the correctly rounded value). */
void mo_sigmoid_table_bf16(uint16_t* table) {
  for (uint32_t i = 0; i < 65536u; ++i) {
    double v = (double)mo_bf16_to_f32((uint16_t)i);
    float s = (float)(1.0 / (1.0 + exp(-v)));
    table[i] = mo_f32_to_bf16(s);
  }
}

void mo_swiglu_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* y) {
  static uint16_t table[65536];
  static int init = 0;
  if (!init) {
    mo_sigmoid_table_bf16(table);
    init = 1;
  }
  for (int64_t i = 0; i < n; ++i) {
    float gv = mo_bf16_to_f32(g[i]);
    float sig = mo_bf16_to_f32(table[g[i]]);
    float act = mo_bf16_to_f32(mo_f32_to_bf16(gv * sig));
    y[i] = mo_f32_to_bf16(act * mo_bf16_to_f32(u[i]));
  }
}

/* Composed down-projection tail (src/transformer.zig:20613-20621): per slot a
 * bf16 product with the slot score, then an ascending bf16 accumulate. */
void mo_down_reduce_bf16(const uint16_t* v, const uint16_t* scores, int64_t topk,
                         int64_t N, uint16_t* y) {
  for (int64_t n = 0; n < N; ++n) {
    float total = 0.f;
    for (int64_t s = 0; s < topk; ++s) {
      float p = mo_bf16_to_f32(mo_f32_to_bf16(mo_bf16_to_f32(v[s * N + n]) * mo_bf16_to_f32(scores[s])));
      total = mo_bf16_to_f32(mo_f32_to_bf16(total + p));
    }
    y[n] = mo_f32_to_bf16(total);
  }
}

/* ------------------------------------------------------ geometry solve --- */
/* affineParamsFromGeometry (src/transformer.zig:16763-16782). */
int mo_affine_params_from_geometry(int64_t w_cols, int64_t s_cols, int64_t in_dim,
                                   int* bits, int* gs) {
  if (in_dim <= 0 || w_cols <= 0 || s_cols <= 0) return -1;
  if ((w_cols * 32) % in_dim != 0 || in_dim % s_cols != 0) return -1;
  int64_t b = (w_cols * 32) / in_dim, g = in_dim / s_cols;
  if (!(b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8)) return -1;
  if (!(g == 32 || g == 64 || g == 128)) return -1;
  *bits = (int)b;
  *gs = (int)g;
  return 0;
}

/* ------------------------------------------------ microscaling fp modes --- */
/* Bias-less modes (mlx_quantized_matmul / mlx_dequantize with mode "nvfp4", "mxfp4",
 * "mxfp8"; the reference routes them at src/transformer.zig:20905-20921 and names the
 * (bits, group_size) of each at :16846-16854): w = element(q) * scale(s), with
 *   nvfp4: 4-bit e2m1 codes, gs 16, e4m3 scale bytes;
 *   mxfp4: 4-bit e2m1 codes, gs 32, e8m0 scale bytes;
 *   mxfp8: 8-bit e4m3 codes, gs 32, e8m0 scale bytes.
 * The element decoders follow the reference's bit constructions (:20126-20142 for e2m1 and
 * e4m3 with no NaN code, :18918-18924 for e8m0 with byte 0 = 2^-127), restated as the
 * values they produce. Every product is exact in fp32 and in bf16. */
float mo_e2m1(uint32_t c) {
  const uint32_t m = c & 7u, e = m >> 1, f = m & 1u;
  const float mag = e == 0 ? 0.5f * (float)f : ldexpf(1.0f + 0.5f * (float)f, (int)e - 1);
  return (c & 8u) ? -mag : mag;
}

float mo_e4m3(uint32_t b) {
  const uint32_t m = b & 0x7Fu, e = m >> 3, f = m & 7u;
  const float mag = e == 0 ? ldexpf((float)f, -9) : ldexpf(1.0f + (float)f / 8.0f, (int)e - 7);
  return (b & 0x80u) ? -mag : mag;
}

float mo_e8m0(uint32_t b) { return ldexpf(1.0f, b == 0 ? -127 : (int)b - 127); }

/* mode: 0 nvfp4, 1 mxfp4, 2 mxfp8. out_bf16: 0 fp32, 1 bf16 (exact either way). */
int mo_dequantize_fp(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                     int mode, int out_bf16, void* out) {
  return mo_dequantize_fp_gs(wq, scales, rows, K, mode, out_bf16, 0, 1.0f, out);
}

/* nvfp4's optional global scale (mlx_dequantize's global_scale, src/mlx.zig:271): the
 * element * scale product (exact in fp32) times the fp32 global scale, one rounding. */
int mo_dequantize_fp_gs(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                        int mode, int out_bf16, int has_gscale, float gscale, void* out) {
  if (has_gscale && mode != 0) return -1;
  if (mode < 0 || mode > 2) return -1;
  const int bits = mode == 2 ? 8 : 4, gs = mode == 0 ? 16 : 32;
  if (K % gs) return -1;
  const int64_t wc = K * bits / 32, ng = K / gs;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k) {
      const uint32_t q = get_code(wq + r * wc, k, bits);
      const uint32_t sb = scales[r * ng + k / gs];
      const float el = mode == 2 ? mo_e4m3(q) : mo_e2m1(q);
      const float sc = mode == 0 ? mo_e4m3(sb) : mo_e8m0(sb);
      volatile float v = el * sc;
      if (has_gscale) v = v * gscale;
      if (out_bf16) ((uint16_t*)out)[r * K + k] = mo_f32_to_bf16(v);
      else ((float*)out)[r * K + k] = v;
    }
  return 0;
}
