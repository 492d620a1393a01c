// C++ host-side mirror of the reference's wrappers over libmi_qmm's C ABI.
#include "mi_host.hpp"

#include <numeric>

#include "mi_qmm.h"

namespace mi::host {

namespace {

void check(int rc) {
  if (rc == MI_OK) return;
  const std::string msg = mi_last_error();
  if (rc == MI_ERR_UNSUPPORTED) throw Unsupported(rc, msg);
  throw MlxError(rc, msg);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw MlxError(MI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

mi_optional_int some(uint32_t v) { return mi_optional_int{(int)v, true}; }

void require(bool ok, const std::string& msg) {
  if (!ok) throw MlxError(MI_ERR_INVALID, msg);
}

}  // namespace

size_t dtype_size(Dtype d) {
  switch (d) {
    case Dtype::uint32:
    case Dtype::float32: return 4;
    case Dtype::float16:
    case Dtype::bfloat16: return 2;
  }
  return 0;
}

const char* cstr(QuantMode m) {
  switch (m) {
    case QuantMode::affine: return "affine";
    case QuantMode::nvfp4: return "nvfp4";
    case QuantMode::mxfp4: return "mxfp4";
    case QuantMode::mxfp8: return "mxfp8";
  }
  return "affine";
}

Array::Array(std::vector<int64_t> shape, Dtype dt) : shape_(std::move(shape)), dtype_(dt) {
  const size_t n = nbytes();
  void* p = nullptr;
  if (n) hip_check(hipMalloc(&p, n), "hipMalloc");
  buf_ = std::shared_ptr<void>(p, [](void* q) {
    if (q) (void)hipFree(q);
  });
  data_ = p;
}

Array Array::view(void* data, std::vector<int64_t> shape, Dtype dt) {
  Array a;
  a.data_ = data;
  a.shape_ = std::move(shape);
  a.dtype_ = dt;
  return a;
}

Array Array::shape_only(std::vector<int64_t> shape, Dtype dt) { return view(nullptr, shape, dt); }

int64_t Array::size() const {
  return std::accumulate(shape_.begin(), shape_.end(), (int64_t)1, std::multiplies<int64_t>());
}

Array Array::reshape(std::vector<int64_t> shape) const {
  Array a = *this;
  a.shape_ = std::move(shape);
  require(a.size() == size(), "reshape changes the element count");
  return a;
}

void Array::upload(const void* host) {
  hip_check(hipMemcpy(data_, host, nbytes(), hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void Array::download(void* host) const {
  hip_check(hipMemcpy(host, data_, nbytes(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

std::optional<QuantParams> affineParamsFromGeometry(const Array& w, const Array& sc,
                                                    uint32_t in_dim) {
  if (in_dim == 0 || w.ndim() < 2 || sc.ndim() < 2) return std::nullopt;
  int bits = 0, gs = 0;
  if (mi_affine_params_from_geometry(w.dim(-1), sc.dim(-1), in_dim, &bits, &gs) != MI_OK)
    return std::nullopt;
  return QuantParams{(uint32_t)bits, (uint32_t)gs, QuantMode::affine};
}

Array qmatmulBits(const Array& x, const Array& w, const Array& sc, const Array& bi, uint32_t bits,
                  uint32_t group_size, QuantMode mode, hipStream_t s) {
  // This library serves the affine mode only; other modes are declined before any device
  // work, as the reference's kernel wrappers return null for modes they do not handle.
  if (mode != QuantMode::affine)
    throw Unsupported(MI_ERR_UNSUPPORTED, std::string("mode ") + cstr(mode) + " not supported");
  require(x.ndim() >= 1 && w.ndim() == 2, "qmatmulBits: x [..., K], w [N, K*bits/32]");
  const int64_t K = x.dim(-1), N = w.dim(0), M = x.size() / (K ? K : 1);
  std::vector<int64_t> yshape = x.shape();
  yshape.back() = N;
  Array y(yshape, x.dtype());
  check(mi_quantized_matmul(y.data(), x.data(), (const uint32_t*)w.data(), sc.data(), bi.data(), M,
                            N, K, true, some(group_size), some(bits), cstr(mode), (int)x.dtype(),
                            (int)sc.dtype(), s));
  return y;
}

void gatherExpertMm(Array* res, const Array& x, const Array& w, const Array& sc, const Array& bi,
                    const Array& lhs_idx, const Array& rhs_idx, uint32_t bits, uint32_t group_size,
                    QuantMode mode, bool sorted, hipStream_t s) {
  require(x.ndim() >= 2 && w.ndim() == 3, "gatherExpertMm: x [..., M, K], w [E, N, Kp]");
  const int64_t K = x.dim(-1), M = x.dim(-2), E = w.dim(0), N = w.dim(1);
  const int64_t n_idx = rhs_idx.size();
  const int64_t x_batch = x.size() / (M * K);
  int64_t lhs_div = 1;
  if (lhs_idx) {
    require(lhs_idx.size() == n_idx, "lhs/rhs index counts differ");
  } else if (x_batch != n_idx) {
    // MLX broadcast of x's batch over trailing index dims (the decode call: x
    // [B,S,1,1,D] against inds [B,S,K]).
    require(x_batch > 0 && n_idx % x_batch == 0, "x batch does not broadcast against indices");
    lhs_div = n_idx / x_batch;
  }
  std::vector<int64_t> shape = rhs_idx.shape();
  shape.push_back(M);
  shape.push_back(N);
  *res = Array(shape, x.dtype());
  check(mi_gather_qmm(res->data(), x.data(), (const uint32_t*)w.data(), sc.data(), bi.data(),
                      (const uint32_t*)lhs_idx.data(), (const uint32_t*)rhs_idx.data(), n_idx,
                      lhs_div, x_batch, M, N, K, E, true, some(group_size), some(bits),
                      cstr(mode), sorted, (int)x.dtype(), (int)sc.dtype(), s));
}

MoeRouting moeRoutingChain(const Array& router_logits, int k, hipStream_t s, Dtype scores_dtype) {
  require(router_logits.dtype() == Dtype::float32, "router logits must be float32");
  const int64_t E = router_logits.dim(-1), T = router_logits.size() / E;
  std::vector<int64_t> shape = router_logits.shape();
  shape.back() = k;
  MoeRouting r{Array(shape, Dtype::uint32), Array(shape, scores_dtype)};
  check(mi_moe_route_topk((uint32_t*)r.inds.data(), r.norm_scores.data(),
                          (const float*)router_logits.data(), T, E, k, (int)scores_dtype, s));
  return r;
}

Array moeExperts(const Array& x, const MoeRouting& routing, const MoeMlpWeights& mw, hipStream_t s,
                 bool force_sorted) {
  require(x.ndim() == 3 && x.dtype() == Dtype::bfloat16, "moeExperts: x [B, S, D] bf16");
  require(routing.norm_scores.dtype() == Dtype::bfloat16, "moeExperts: bf16 scores");
  const int64_t B = x.dim(0), S = x.dim(1), D = x.dim(2);
  const int64_t K = routing.inds.dim(-1);
  const int64_t T = B * S, total = T * K;
  const int64_t E = mw.switch_gate_w.dim(0), I = mw.switch_gate_w.dim(1);
  const QuantParams& g = mw.gate_qp;
  const QuantParams& d = mw.down_qp;
  require(mw.up_qp.bits == g.bits && mw.up_qp.group_size == g.group_size,
          "gate and up banks must share their quantization");
  Array out({B, S, D}, Dtype::bfloat16);
  const bool do_sort = force_sorted || S > 1 || total >= 64;  // src/transformer.zig:14951
  if (!do_sort) {
    // Decode: in-place expert-bank reads, fused gate+up+SwiGLU then down+score-reduce.
    Array act({T, K, I}, Dtype::bfloat16);
    check(mi_gather_qmv_gate_up_swiglu(
        act.data(), x.data(), (const uint32_t*)mw.switch_gate_w.data(), mw.switch_gate_s.data(),
        mw.switch_gate_b.data(), (const uint32_t*)mw.switch_up_w.data(), mw.switch_up_s.data(),
        mw.switch_up_b.data(), (const uint32_t*)routing.inds.data(), T, (int)K, I, D, E,
        some(g.group_size), some(g.bits), cstr(g.mode), s));
    check(mi_gather_qmv_down_reduce(
        out.data(), act.data(), (const uint32_t*)mw.switch_down_w.data(), mw.switch_down_s.data(),
        mw.switch_down_b.data(), (const uint32_t*)routing.inds.data(),
        routing.norm_scores.data(), T, (int)K, D, I, E, some(d.group_size), some(d.bits),
        cstr(d.mode), s));
    return out;
  }
  // Sorted prefill path: order = argsort(flat), inv = argsort(order), sorted ids,
  // lhs = order // K. The reference gathers x rows into x_rep; lhs indices make the
  // grouped gather read them in place.
  Array order({total}, Dtype::uint32), inv({total}, Dtype::uint32);
  Array sorted_inds({total}, Dtype::uint32), lhs_idx({total}, Dtype::uint32);
  check(mi_moe_sort_dispatch((uint32_t*)order.data(), (uint32_t*)inv.data(),
                             (uint32_t*)sorted_inds.data(), (uint32_t*)lhs_idx.data(), nullptr,
                             (const uint32_t*)routing.inds.data(), total, (int)K, E, s));
  const Array xt = x.reshape({T, 1, D});
  Array gate_out, up_out, down_out;
  gatherExpertMm(&gate_out, xt, mw.switch_gate_w, mw.switch_gate_s, mw.switch_gate_b, lhs_idx,
                 sorted_inds, g.bits, g.group_size, g.mode, true, s);
  gatherExpertMm(&up_out, xt, mw.switch_up_w, mw.switch_up_s, mw.switch_up_b, lhs_idx,
                 sorted_inds, g.bits, g.group_size, g.mode, true, s);
  Array act({total, 1, I}, Dtype::bfloat16);
  check(mi_swiglu(act.data(), gate_out.data(), up_out.data(), total * I, (int)Dtype::bfloat16, s));
  gatherExpertMm(&down_out, act, mw.switch_down_w, mw.switch_down_s, mw.switch_down_b, Array(),
                 sorted_inds, d.bits, d.group_size, d.mode, true, s);
  // Inverse permute to (token, slot) order, then the score-weighted slot sum.
  Array unsorted({total, D}, Dtype::bfloat16);
  check(mi_take_rows(unsorted.data(), down_out.data(), (const uint32_t*)inv.data(), total, total,
                     D * 2, s));
  check(mi_moe_down_reduce(out.data(), unsorted.data(), routing.norm_scores.data(), T, (int)K, D,
                           (int)Dtype::bfloat16, s));
  return out;
}

}  // namespace mi::host
