// Tests of the C++ host mirror (mlx-serve_amd/host), named after the reference tests they
// mirror (src/transformer.zig). The C oracle (oracle/liboracle.so) is the checker.
//   test_host --cpu   cases that need no GPU
//   test_host --gpu   cases that run on the GPU (through libmi_qmm.so)
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "mi_host.hpp"
#include "mi_qmm.h"
extern "C" {
#include "mi_oracle.h"
}

using namespace mi::host;

namespace {

struct Case {
  const char* name;
  bool gpu;
  std::function<void()> fn;
};
std::vector<Case>& registry() {
  static std::vector<Case> r;
  return r;
}
struct Reg {
  Reg(const char* n, bool g, std::function<void()> f) { registry().push_back({n, g, f}); }
};
struct Fail : std::runtime_error {
  using std::runtime_error::runtime_error;
};
#define EXPECT(c)                                                                          \
  do {                                                                                     \
    if (!(c)) throw Fail(std::string(__FILE__ ":") + std::to_string(__LINE__) + " " #c); \
  } while (0)
#define CASE(name, gpu, fn) static Reg reg_##fn(name, gpu, fn)

const hipStream_t S = nullptr;

// Host bf16 helpers shared with the oracle.
std::vector<uint16_t> to_bf16(const std::vector<float>& f) {
  std::vector<uint16_t> h(f.size());
  mo_f32_to_bf16_array(f.data(), h.data(), (int64_t)f.size());
  return h;
}
float bf(uint16_t h) { return mo_bf16_to_f32(h); }

struct HostQuant {
  std::vector<uint32_t> wq;
  std::vector<uint16_t> s, b;
};
// W ~ N(0, 0.02) fp32 -> bf16 -> affine quantize, rows x K.
HostQuant make_weight(int64_t rows, int64_t K, uint64_t seed, int bits = 4, int gs = 64) {
  std::vector<float> w((size_t)(rows * K));
  mo_randn_f32(w.data(), rows * K, seed, 0.0, 0.02);
  std::vector<uint16_t> wb = to_bf16(w);
  HostQuant q{std::vector<uint32_t>((size_t)(rows * K * bits / 32)),
              std::vector<uint16_t>((size_t)(rows * K / gs)),
              std::vector<uint16_t>((size_t)(rows * K / gs))};
  EXPECT(mo_quantize_bf16(wb.data(), rows, K, gs, bits, q.wq.data(), q.s.data(), q.b.data()) == 0);
  return q;
}
std::vector<uint16_t> make_x(int64_t M, int64_t K, uint64_t seed) {
  std::vector<float> x((size_t)(M * K));
  mo_randn_f32(x.data(), M * K, seed, 0.0, 1.0);
  return to_bf16(x);
}

template <class T>
Array dev(const std::vector<T>& h, std::vector<int64_t> shape, Dtype dt) {
  Array a(shape, dt);
  EXPECT(a.nbytes() == h.size() * sizeof(T));
  a.upload(h.data());
  return a;
}
template <class T>
std::vector<T> host(const Array& a) {
  std::vector<T> h(a.nbytes() / sizeof(T));
  a.download(h.data());
  return h;
}

double max_err_ratio(const std::vector<uint16_t>& y, const std::vector<double>& truth) {
  double m = 0, d = 0;
  for (size_t i = 0; i < truth.size(); ++i) {
    m = std::max(m, std::fabs(truth[i]));
    d = std::max(d, std::fabs((double)bf(y[i]) - truth[i]));
  }
  return d / (m > 0 ? m : 1.0);
}

// ------------------------------------------------------------------- CPU --
void geometry_solve() {
  // src/transformer.zig:22930 "affineParamsFromGeometry: exact per-weight solve for
  // off-config sidecar quants": q_proj [8192,320] / scales [8192,16] at H=2048 -> 5-bit
  // gs 128; v_proj [512,384] / [512,16] -> 6-bit gs 128; switch experts
  // [256,512,256] / [256,512,32] -> 4-bit gs 64; q_proj geometry at 3000 -> null.
  const uint32_t H = 2048;
  auto q = affineParamsFromGeometry(Array::shape_only({8192, 320}, Dtype::uint32),
                                    Array::shape_only({8192, 16}, Dtype::bfloat16), H);
  EXPECT(q && q->bits == 5 && q->group_size == 128);
  auto v = affineParamsFromGeometry(Array::shape_only({512, 384}, Dtype::uint32),
                                    Array::shape_only({512, 16}, Dtype::bfloat16), H);
  EXPECT(v && v->bits == 6 && v->group_size == 128);
  auto e = affineParamsFromGeometry(Array::shape_only({256, 512, 256}, Dtype::uint32),
                                    Array::shape_only({256, 512, 32}, Dtype::bfloat16), H);
  EXPECT(e && e->bits == 4 && e->group_size == 64);
  EXPECT(!affineParamsFromGeometry(Array::shape_only({8192, 320}, Dtype::uint32),
                                   Array::shape_only({8192, 16}, Dtype::bfloat16), 3000));
}
CASE("affineParamsFromGeometry: exact per-weight solve for off-config sidecar quants", false,
     geometry_solve);

void decline_non_affine_cpu() {
  // A non-affine mode is refused before any device work (no GPU needed).
  Array x = Array::view((void*)16, {1, 256}, Dtype::bfloat16);
  Array w = Array::view((void*)16, {64, 32}, Dtype::uint32);
  Array sb = Array::view((void*)16, {64, 4}, Dtype::bfloat16);
  bool threw = false;
  try {
    qmatmulBits(x, w, sb, sb, 4, 64, QuantMode::nvfp4, S);
  } catch (const Unsupported&) {
    threw = true;
  }
  EXPECT(threw);
}
CASE("qmatmulBits declines non-affine modes (the reference falls back to stock MLX)", false,
     decline_non_affine_cpu);

// ------------------------------------------------------------------- GPU --
void routing_chain() {
  // src/transformer.zig:25626 "moeRoutingChain produces top-K indices and renormalized
  // softmax weights": row 0 -> experts {0, 3}, row 1 -> {1, 4}; logits sum 15; weights
  // sum to 1.
  const std::vector<float> data = {10, 0, 0, 5, 0, 0, 0, 10, 0, 0, 5, 0};
  Array logits = dev(data, {2, 6}, Dtype::float32);
  MoeRouting r = moeRoutingChain(logits, 2, S, Dtype::float32);
  EXPECT(r.inds.shape() == std::vector<int64_t>({2, 2}));
  EXPECT(r.norm_scores.shape() == std::vector<int64_t>({2, 2}));
  auto inds = host<uint32_t>(r.inds);
  auto sc = host<float>(r.norm_scores);
  for (int row = 0; row < 2; ++row) {
    float gsum = 0, ssum = 0;
    for (int j = 0; j < 2; ++j) {
      gsum += data[row * 6 + inds[row * 2 + j]];
      ssum += sc[row * 2 + j];
    }
    EXPECT(std::fabs(gsum - 15.f) < 1e-3f);
    EXPECT(std::fabs(ssum - 1.f) < 1e-3f);
  }
  EXPECT(inds[0] == 0 && inds[1] == 3 && inds[2] == 1 && inds[3] == 4);
}
CASE("moeRoutingChain produces top-K indices and renormalized softmax weights", true,
     routing_chain);

void qmatmul_vs_truth() {
  for (int bits : {4, 8}) {
    for (int64_t M : {1, 5, 300}) {
      const int64_t N = 320, K = 1024;
      HostQuant q = make_weight(N, K, 100 + M, bits);
      auto x = make_x(M, K, 200 + M);
      Array y = qmatmulBits(dev(x, {M, K}, Dtype::bfloat16),
                            dev(q.wq, {N, K * bits / 32}, Dtype::uint32),
                            dev(q.s, {N, K / 64}, Dtype::bfloat16),
                            dev(q.b, {N, K / 64}, Dtype::bfloat16), bits, 64, QuantMode::affine, S);
      EXPECT(y.shape() == std::vector<int64_t>({M, N}));
      std::vector<double> truth((size_t)(M * N));
      EXPECT(mo_qmm_f64(x.data(), 0, q.wq.data(), q.s.data(), q.b.data(), M, N, K, 64, bits,
                        truth.data()) == 0);
      EXPECT(max_err_ratio(host<uint16_t>(y), truth) <= 1e-2);
    }
  }
}
CASE("qmatmulBits matches dequantize+matmul reference (affine, decode and prefill widths)",
     true, qmatmul_vs_truth);

void gather_decode_and_prefill() {
  // Per-expert ground truth for the decode call (x [B,S,1,1,D], inds [B,S,K], no lhs)
  // and the sorted prefill call (lhs = order // K).
  const int64_t E = 8, N = 96, D = 512, B = 2, Sq = 3, Kt = 2;
  HostQuant q = make_weight(E * N, D, 7);
  Array W = dev(q.wq, {E, N, D / 8}, Dtype::uint32), Sc = dev(q.s, {E, N, D / 64}, Dtype::bfloat16),
        Bi = dev(q.b, {E, N, D / 64}, Dtype::bfloat16);
  auto x = make_x(B * Sq, D, 8);
  std::vector<uint32_t> inds = {1, 7, 0, 0, 5, 2, 3, 6, 4, 4, 7, 1};
  Array res;
  gatherExpertMm(&res, dev(x, {B, Sq, 1, 1, D}, Dtype::bfloat16), W, Sc, Bi, Array(),
                 dev(inds, {B, Sq, Kt}, Dtype::uint32), 4, 64, QuantMode::affine, false, S);
  EXPECT(res.shape() == std::vector<int64_t>({B, Sq, Kt, 1, N}));
  std::vector<double> truth((size_t)(B * Sq * Kt * N));
  EXPECT(mo_gather_qmm_f64(x.data(), 0, q.wq.data(), q.s.data(), q.b.data(), nullptr, inds.data(),
                           B * Sq * Kt, Kt, 1, N, D, B * Sq, E, 64, 4, truth.data()) == 0);
  EXPECT(max_err_ratio(host<uint16_t>(res), truth) <= 1e-2);

  const int64_t n = B * Sq * Kt;
  std::vector<uint32_t> order(n), inv(n), srt(n), lhs(n);
  EXPECT(mo_sort_dispatch(inds.data(), n, (int)Kt, order.data(), inv.data(), srt.data(),
                          lhs.data()) == 0);
  Array res2;
  gatherExpertMm(&res2, dev(x, {B * Sq, 1, D}, Dtype::bfloat16), W, Sc, Bi,
                 dev(lhs, {n}, Dtype::uint32), dev(srt, {n}, Dtype::uint32), 4, 64,
                 QuantMode::affine, true, S);
  std::vector<double> t2((size_t)(n * N));
  EXPECT(mo_gather_qmm_f64(x.data(), 0, q.wq.data(), q.s.data(), q.b.data(), lhs.data(),
                           srt.data(), n, 1, 1, N, D, B * Sq, E, 64, 4, t2.data()) == 0);
  EXPECT(max_err_ratio(host<uint16_t>(res2), t2) <= 1e-2);
}
CASE("gatherExpertMm matches per-expert ground truth (decode + prefill shapes)", true,
     gather_decode_and_prefill);

MoeMlpWeights make_moe(int64_t E, int64_t D, int64_t I, uint64_t seed) {
  MoeMlpWeights mw;
  HostQuant g = make_weight(E * I, D, seed), u = make_weight(E * I, D, seed + 1),
            d = make_weight(E * D, I, seed + 2);
  mw.switch_gate_w = dev(g.wq, {E, I, D / 8}, Dtype::uint32);
  mw.switch_gate_s = dev(g.s, {E, I, D / 64}, Dtype::bfloat16);
  mw.switch_gate_b = dev(g.b, {E, I, D / 64}, Dtype::bfloat16);
  mw.switch_up_w = dev(u.wq, {E, I, D / 8}, Dtype::uint32);
  mw.switch_up_s = dev(u.s, {E, I, D / 64}, Dtype::bfloat16);
  mw.switch_up_b = dev(u.b, {E, I, D / 64}, Dtype::bfloat16);
  mw.switch_down_w = dev(d.wq, {E, D, I / 8}, Dtype::uint32);
  mw.switch_down_s = dev(d.s, {E, D, I / 64}, Dtype::bfloat16);
  mw.switch_down_b = dev(d.b, {E, D, I / 64}, Dtype::bfloat16);
  return mw;
}

void moe_sorted_equals_decode() {
  // The sorted (prefill) and in-place (decode) expert paths agree on the same tokens.
  const int64_t E = 16, D = 512, I = 256, Kt = 4;
  MoeMlpWeights mw = make_moe(E, D, I, 31);
  for (int64_t B : {1, 3}) {
    auto x = make_x(B, D, 32 + B);
    std::vector<float> logits((size_t)(B * E));
    mo_randn_f32(logits.data(), B * E, 33 + B, 0.0, 1.0);
    MoeRouting r = moeRoutingChain(dev(logits, {B, 1, E}, Dtype::float32), (int)Kt, S);
    Array xd = dev(x, {B, 1, D}, Dtype::bfloat16);
    auto yd = host<uint16_t>(moeExperts(xd, r, mw, S, false));
    auto ys = host<uint16_t>(moeExperts(xd, r, mw, S, true));
    std::vector<double> t(ys.size());
    for (size_t i = 0; i < ys.size(); ++i) t[i] = bf(ys[i]);
    EXPECT(max_err_ratio(yd, t) <= 2e-2);
  }
}
CASE("moeExperts: sorted prefill path matches the fused decode path", true,
     moe_sorted_equals_decode);

void fused_gate_up_bit_identical() {
  // src/transformer.zig:24081 "fused gate+up+SwiGLU expert kernel is bit-identical to the
  // split gatherQmv path": two independent banks, top-K 3.
  const int64_t E = 8, N = 64, K = 256, TOPK = 3;
  HostQuant g = make_weight(E * N, K, 41), u = make_weight(E * N, K, 42);
  auto x = make_x(1, K, 43);
  std::vector<uint32_t> inds = {5, 0, 7};
  Array xd = dev(x, {1, K}, Dtype::bfloat16), id = dev(inds, {1, TOPK}, Dtype::uint32);
  Array Wg = dev(g.wq, {E, N, K / 8}, Dtype::uint32), Sg = dev(g.s, {E, N, K / 64}, Dtype::bfloat16),
        Bg = dev(g.b, {E, N, K / 64}, Dtype::bfloat16);
  Array Wu = dev(u.wq, {E, N, K / 8}, Dtype::uint32), Su = dev(u.s, {E, N, K / 64}, Dtype::bfloat16),
        Bu = dev(u.b, {E, N, K / 64}, Dtype::bfloat16);
  Array fused({TOPK, N}, Dtype::bfloat16);
  const mi_optional_int gs{64, true}, bits{4, true};
  EXPECT(mi_gather_qmv_gate_up_swiglu(fused.data(), xd.data(), (uint32_t*)Wg.data(), Sg.data(),
                                      Bg.data(), (uint32_t*)Wu.data(), Su.data(), Bu.data(),
                                      (uint32_t*)id.data(), 1, (int)TOPK, N, K, E, gs, bits,
                                      "affine", S) == MI_OK);
  Array gs_out, us_out;
  const Array x5 = xd.reshape({1, 1, K});
  gatherExpertMm(&gs_out, x5, Wg, Sg, Bg, Array(), id, 4, 64, QuantMode::affine, false, S);
  gatherExpertMm(&us_out, x5, Wu, Su, Bu, Array(), id, 4, 64, QuantMode::affine, false, S);
  Array split({TOPK, N}, Dtype::bfloat16);
  EXPECT(mi_swiglu(split.data(), gs_out.data(), us_out.data(), TOPK * N, MI_DTYPE_BFLOAT16, S) ==
         MI_OK);
  EXPECT(host<uint16_t>(fused) == host<uint16_t>(split));
}
CASE("fused gate+up+SwiGLU expert kernel is bit-identical to the split gatherQmv path", true,
     fused_gate_up_bit_identical);

}  // namespace

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  int failed = 0, ran = 0;
  for (const Case& c : registry()) {
    if (c.gpu != gpu) continue;
    ++ran;
    std::printf("CASE %s\n", c.name);
    std::fflush(stdout);
    try {
      c.fn();
      std::printf("  ok\n");
    } catch (const std::exception& e) {
      ++failed;
      std::printf("  FAILED: %s\n", e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%d/%d passed\n", ran - failed, ran);
  return failed ? 1 : 0;
}
