// C++ host side above the C ABI, mirroring the reference's Zig wrappers for this path
// (src/transformer.zig) with the same names, argument meaning and error behaviour:
//   affineParamsFromGeometry  :16763-16782
//   qmatmulBits               :20894-20983 (affine)
//   gatherExpertMm            :20768-20784
//   moeRoutingChain           :17022-17072
//   moeExperts                the routed-expert part of moeMLP2 :14944-15140
// Arrays are refcounted device buffers (like mlx_array handles); every op is asynchronous
// on the given HIP stream. Failures throw MlxError (the reference's error.MlxError from
// mlx.check, src/mlx.zig:547-550); a request the library declines throws Unsupported.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace mi::host {

// mlx_dtype values (src/mlx.zig:20-35) for the dtypes this path uses.
enum class Dtype : int { uint32 = 3, float16 = 9, float32 = 10, bfloat16 = 12 };
size_t dtype_size(Dtype d);

// QuantMode (src/model.zig:19-43); only affine is served by this library.
enum class QuantMode { affine, nvfp4, mxfp4, mxfp8 };
const char* cstr(QuantMode m);

struct MlxError : std::runtime_error {
  int code;
  MlxError(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};
struct Unsupported : MlxError {
  using MlxError::MlxError;
};

class Array {
 public:
  Array() = default;
  // New device buffer (hipMalloc), owned and freed with the last handle.
  Array(std::vector<int64_t> shape, Dtype dt);
  // Non-owning view of caller memory.
  static Array view(void* data, std::vector<int64_t> shape, Dtype dt);
  // Shape-only handle (no data), enough for geometry queries.
  static Array shape_only(std::vector<int64_t> shape, Dtype dt);

  void* data() const { return data_; }
  const std::vector<int64_t>& shape() const { return shape_; }
  int64_t dim(int i) const { return shape_[i < 0 ? (int)shape_.size() + i : i]; }
  int ndim() const { return (int)shape_.size(); }
  Dtype dtype() const { return dtype_; }
  int64_t size() const;
  size_t nbytes() const { return (size_t)size() * dtype_size(dtype_); }
  explicit operator bool() const { return data_ != nullptr; }
  Array reshape(std::vector<int64_t> shape) const;  // same buffer

  // Synchronous copies (tests and set-up; not for the hot path).
  void upload(const void* host);
  void download(void* host) const;

 private:
  std::shared_ptr<void> buf_;
  void* data_ = nullptr;
  std::vector<int64_t> shape_;
  Dtype dtype_ = Dtype::float32;
};

struct QuantParams {
  uint32_t bits = 4, group_size = 64;
  QuantMode mode = QuantMode::affine;
};

// bits = w_cols*32/in_dim, gs = in_dim/s_cols; nullopt when that is not an affine layout.
std::optional<QuantParams> affineParamsFromGeometry(const Array& w, const Array& sc,
                                                    uint32_t in_dim);

// y[..., N] = x[..., K] @ dequantize(w)^T (mlx_quantized_matmul, transpose=true).
Array qmatmulBits(const Array& x, const Array& w, const Array& sc, const Array& bi, uint32_t bits,
                  uint32_t group_size, QuantMode mode, hipStream_t s);

// res = gather_qmm(x, w, sc, bi, lhs_idx, rhs_idx, transpose=true, gs, bits, mode, sorted).
// lhs_idx may be a null Array (MLX's arange, broadcast over trailing index dims).
// res shape = rhs_idx.shape ++ [M, N].
void gatherExpertMm(Array* res, const Array& x, const Array& w, const Array& sc, const Array& bi,
                    const Array& lhs_idx, const Array& rhs_idx, uint32_t bits, uint32_t group_size,
                    QuantMode mode, bool sorted, hipStream_t s);

struct MoeRouting {
  Array inds;         // uint32 [..., k]
  Array norm_scores;  // [..., k], renormalized softmax weights
};
// Softmax top-k routing over fp32 logits [..., E].
MoeRouting moeRoutingChain(const Array& router_logits, int k, hipStream_t s,
                           Dtype scores_dtype = Dtype::bfloat16);

struct MoeMlpWeights {
  Array switch_gate_w, switch_gate_s, switch_gate_b;
  Array switch_up_w, switch_up_s, switch_up_b;
  Array switch_down_w, switch_down_s, switch_down_b;
  QuantParams gate_qp, up_qp, down_qp;
};
// Routed experts of one MoE layer: x [B, S, D] bf16, routing over k slots ->
// sum_k score_k * down(swiglu(gate(x), up(x))) as [B, S, D] bf16. Like moeMLP2 (:14951)
// it takes the sorted path when S > 1 or B*S*k >= 64 (argsort by expert, grouped
// gather_qmm, inverse permute) and otherwise the fused decode path (gate+up+SwiGLU,
// down+score-reduce). `force_sorted` picks the sorted path regardless.
Array moeExperts(const Array& x, const MoeRouting& routing, const MoeMlpWeights& mw, hipStream_t s,
                 bool force_sorted = false);

}  // namespace mi::host
