// C ABI (include/mi_qmm.h): argument validation, dispatch to the gfx950 kernels,
// per-stream workspace, error reporting.
#include "../../include/mi_qmm.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "mi_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Resolve MLX defaults and check the affine / transpose=true scope shared by all
// matmul entry points. Returns MI_OK or an error/decline code.
int resolve_common(mi_optional_int gs_in, mi_optional_int bits_in, const char* mode,
                   bool transpose, int64_t K, int* gs, int* bits) {
  *gs = gs_in.has_value ? gs_in.value : 64;
  *bits = bits_in.has_value ? bits_in.value : 4;
  if (mode && std::strcmp(mode, "affine") != 0)
    return fail(MI_ERR_UNSUPPORTED, "mode '%s' not supported (affine only)", mode);
  if (!transpose) return fail(MI_ERR_UNSUPPORTED, "transpose=false not supported");
  if (*bits != 4 && *bits != 8) return fail(MI_ERR_UNSUPPORTED, "bits=%d not supported", *bits);
  if (*gs != 32 && *gs != 64 && *gs != 128)
    return fail(MI_ERR_UNSUPPORTED, "group_size=%d not supported", *gs);
  if (K <= 0 || K % *gs != 0)
    return fail(MI_ERR_INVALID, "K=%lld must be a positive multiple of group_size=%d",
                (long long)K, *gs);
  if (K > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "K too large");
  return MI_OK;
}

// Per-device scratch for sorted work lists and K-split partials. Calls on one
// stream are ordered, so reuse by later calls is safe; calls that overlap on
// different streams of one device must not both use it. It only grows outside
// stream capture (mi_workspace_reserve sizes it up front).
struct Workspace {
  void* data = nullptr;
  size_t size = 0;
};
std::mutex g_ws_mu;
std::map<int, Workspace> g_ws;

int workspace(hipStream_t s, size_t bytes, void** data) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Workspace& w = g_ws[dev];
  if (w.size < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(MI_ERR_WORKSPACE, "workspace too small during stream capture "
                  "(call mi_workspace_reserve before capturing)");
    if (w.data) {
      e = hipDeviceSynchronize();  // queued work may still use the old buffer
      if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
      (void)hipFree(w.data);
      w.data = nullptr;
      w.size = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4;
    e = hipMalloc(&w.data, want);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
    w.size = want;
  }
  *data = w.data;
  return MI_OK;
}

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

// Launch shape for the small-M kernel: one block per (32-row tile, K range, item).
// K ranges: as few as keep the staged activations within the LDS budget. Waves per
// block: enough to keep ~16 waves per CU streaming, at least 2 groups per wave.
struct QmvPlan {
  mi::QmvConfig cfg;
  int row_blocks, ks, gps;
};

QmvPlan qmv_plan(int N, int K, int gs, int rows, int64_t n_items, int x_f32) {
  static const int env_w = env_int("MI_QMM_QMV_WAVES", 0);
  static const int env_ks = env_int("MI_QMM_QMV_KS", 0);
  static const int env_target = env_int("MI_QMM_QMV_TARGET_WAVES", 4096);
  const size_t lds_max = 64 * 1024;
  QmvPlan p;
  p.cfg.rows = rows;
  p.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
  p.row_blocks = ceil_div(N, 32);
  const int G = K / gs;
  const int mr = mi::qmv_mr_for_rows(rows);
  int ks = 1;
  while (ks < G && mi::qmv_lds_bytes(ceil_div(G, ks), gs, mr, x_f32, 1) > lds_max) ++ks;
  if (env_ks > 0) ks = env_ks < G ? env_ks : G;
  p.gps = ceil_div(G, ks);
  p.ks = ceil_div(G, p.gps);
  const int64_t blocks = (int64_t)p.row_blocks * p.cfg.grid_z * p.ks;
  int w = 4;
  while (w < 8 && blocks * w < env_target && p.gps / (2 * w) >= 1) w <<= 1;
  if (env_w >= 1 && env_w <= 8) w = env_w;
  while (w > 1 && mi::qmv_lds_bytes(p.gps, gs, mr, x_f32, w) > lds_max) w >>= 1;
  p.cfg.waves = w;
  return p;
}

bool valid_x_dtype(int d) { return d == MI_DTYPE_BFLOAT16 || d == MI_DTYPE_FLOAT32; }

}  // namespace

extern "C" {

const char* mi_last_error(void) { return g_err.c_str(); }

int mi_workspace_reserve(int64_t bytes, void* stream) {
  if (bytes < 0) return fail(MI_ERR_INVALID, "negative size");
  void* d = nullptr;
  return workspace((hipStream_t)stream, (size_t)bytes, &d);
}

const char* mi_version(void) { return "mi_qmm 0.1 gfx950"; }

int mi_affine_params_from_geometry(int64_t w_cols, int64_t s_cols, int64_t in_dim, int* bits,
                                   int* group_size) {
  if (!bits || !group_size) return fail(MI_ERR_INVALID, "null output pointer");
  if (in_dim <= 0 || w_cols <= 0 || s_cols <= 0)
    return fail(MI_ERR_INVALID, "non-positive geometry");
  if ((w_cols * 32) % in_dim != 0 || in_dim % s_cols != 0)
    return fail(MI_ERR_INVALID, "geometry is not an affine packing");
  const int64_t b = (w_cols * 32) / in_dim, g = in_dim / s_cols;
  if (!(b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8))
    return fail(MI_ERR_INVALID, "bits=%lld not an affine width", (long long)b);
  if (!(g == 32 || g == 64 || g == 128))
    return fail(MI_ERR_INVALID, "group_size=%lld not an affine group", (long long)g);
  *bits = (int)b;
  *group_size = (int)g;
  return MI_OK;
}

int mi_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales,
                  const void* biases, const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                  int64_t n_idx, int64_t lhs_div, int64_t x_batch, int64_t M, int64_t N, int64_t K,
                  int64_t n_experts, bool transpose, mi_optional_int group_size,
                  mi_optional_int bits, const char* mode, bool sorted_indices, int x_dtype,
                  int sb_dtype, void* stream) {
  int gs = 0, nb = 0;
  int rc = resolve_common(group_size, bits, mode, transpose, K, &gs, &nb);
  if (rc) return rc;
  if (!valid_x_dtype(x_dtype)) return fail(MI_ERR_UNSUPPORTED, "x dtype %d not supported", x_dtype);
  if (sb_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
  if (n_idx < 0 || M < 0 || N < 0 || x_batch < 0 || n_experts < 0 || lhs_div <= 0)
    return fail(MI_ERR_INVALID, "negative size or lhs_div <= 0");
  if (n_idx == 0 || M == 0 || N == 0) return MI_OK;
  if (!y || !x || !w || !scales || !biases) return fail(MI_ERR_INVALID, "null tensor pointer");
  if (x_batch == 0 || n_experts == 0) return fail(MI_ERR_INVALID, "empty x or weight bank");
  if (N > (int64_t)1 << 30 || M > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "N or M too large");
  if (n_idx * M >= ((int64_t)1 << 32)) return fail(MI_ERR_INVALID, "n_idx*M exceeds 2^32");
  hipStream_t s = (hipStream_t)stream;

  mi::QmvParams P{};
  P.w = w;
  P.scales = (const uint16_t*)scales;
  P.biases = (const uint16_t*)biases;
  P.x = x;
  P.y = y;
  P.lhs = lhs_indices;
  P.rhs = rhs_indices;
  P.n_pairs = n_idx;
  P.lhs_div = lhs_div;
  P.x_batch = x_batch;
  P.n_experts = n_experts;
  P.M = (int)M;
  P.N = (int)N;
  P.K = (int)K;
  P.bits = nb;
  P.group_size = gs;
  P.x_f32 = x_dtype == MI_DTYPE_FLOAT32;

  const bool use_items = sorted_indices && rhs_indices != nullptr && n_idx > 1;
  const int64_t PT = n_idx * M;
  const int rows = M <= 32 ? (int)M : 32;
  int64_t n_items, max_items = 0;
  if (!use_items) {
    P.items_per_pair = ceil_div(M, 32);
    n_items = n_idx * P.items_per_pair;
    if (n_items > INT32_MAX) return fail(MI_ERR_INVALID, "too many work items");
    P.n_items_fixed = (int)n_items;
  } else {
    // Runs of equal rhs, cut into 32-row chunks; bound valid for any input order.
    max_items = (PT + 31) / 32 + n_idx;
    const int64_t runs_bound = n_idx < n_experts ? n_idx : n_experts;
    n_items = (PT + 31) / 32 + runs_bound;
    P.items_per_pair = 1;
    P.n_items_fixed = 0;
  }
  QmvPlan plan = qmv_plan(P.N, P.K, gs, use_items ? 32 : rows, n_items, P.x_f32);
  P.ks = plan.ks;
  P.gps = plan.gps;
  P.row_blocks = plan.row_blocks;
  size_t items_bytes = use_items ? (size_t)max_items * 16 + 256 : 0;
  size_t part_bytes = P.ks > 1 ? (size_t)P.ks * PT * N * 4 : 0;
  if (items_bytes || part_bytes) {
    void* data = nullptr;
    rc = workspace(s, ((items_bytes + 255) / 256) * 256 + part_bytes, &data);
    if (rc) return rc;
    P.part = (float*)((char*)data + ((items_bytes + 255) / 256) * 256);
    if (use_items) {
      uint32_t* count = (uint32_t*)data;
      uint32_t* items = (uint32_t*)((char*)data + 256);
      hipError_t e = mi::launch_build_items(rhs_indices, n_idx, (int)M, 32, items, count,
                                            max_items, s);
      if (e != hipSuccess) return hip_fail(e, "build_items launch");
      P.items = items;
      P.item_count = count;
    }
  }
  hipError_t e = mi::launch_qmv(P, plan.cfg, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "qmv launch");
}

int mi_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, bool transpose,
                        mi_optional_int group_size, mi_optional_int bits, const char* mode,
                        int x_dtype, int sb_dtype, void* stream) {
  int gs = 0, nb = 0;
  int rc = resolve_common(group_size, bits, mode, transpose, K, &gs, &nb);
  if (rc) return rc;
  if (!valid_x_dtype(x_dtype)) return fail(MI_ERR_UNSUPPORTED, "x dtype %d not supported", x_dtype);
  if (sb_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
  if (M < 0 || N < 0) return fail(MI_ERR_INVALID, "negative size");
  if (M == 0 || N == 0) return MI_OK;
  if (!y || !x || !w || !scales || !biases) return fail(MI_ERR_INVALID, "null tensor pointer");
  if (N > (int64_t)1 << 30 || M > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "N or M too large");
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == MI_DTYPE_BFLOAT16 && M > 32 && mi::qmm_supported((int)M, (int)N, (int)K, nb, gs)) {
    mi::QmmParams Q{w, (const uint16_t*)scales, (const uint16_t*)biases, (const uint16_t*)x,
                    (uint16_t*)y, (int)M, (int)N, (int)K, nb, gs};
    hipError_t e = mi::launch_qmm(Q, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmm launch");
  }
  // Dense = gather with a single pair on expert 0; M rows ride in one x batch.
  return mi_gather_qmm(y, x, w, scales, biases, nullptr, nullptr, 1, 1, 1, M, N, K, 1, transpose,
                       group_size, bits, mode, false, x_dtype, sb_dtype, stream);
}

int mi_dequantize_rounding(void* out, const uint32_t* w, const void* scales, const void* biases,
                           int64_t rows, int64_t K, mi_optional_int group_size,
                           mi_optional_int bits, const char* mode, int sb_dtype, int out_dtype,
                           int rounding, void* stream) {
  int gs = 0, nb = 0;
  int rc = resolve_common(group_size, bits, mode, true, K, &gs, &nb);
  if (rc) return rc;
  if (sb_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
  if (out_dtype != MI_DTYPE_BFLOAT16 && out_dtype != MI_DTYPE_FLOAT32)
    return fail(MI_ERR_UNSUPPORTED, "output dtype %d not supported", out_dtype);
  if (rounding != 0 && rounding != 1) return fail(MI_ERR_INVALID, "rounding must be 0 or 1");
  if (rows < 0) return fail(MI_ERR_INVALID, "negative rows");
  if (rows == 0) return MI_OK;
  if (!out || !w || !scales || !biases) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_dequantize(out, w, (const uint16_t*)scales, (const uint16_t*)biases,
                                       rows, K, gs, nb, out_dtype == MI_DTYPE_FLOAT32, rounding,
                                       (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "dequantize launch");
}

int mi_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                  int64_t rows, int64_t K, mi_optional_int group_size, mi_optional_int bits,
                  const char* mode, int sb_dtype, int out_dtype, void* stream) {
  return mi_dequantize_rounding(out, w, scales, biases, rows, K, group_size, bits, mode, sb_dtype,
                                out_dtype, 1, stream);
}

int mi_quantize(uint32_t* wq, void* scales, void* biases, const void* w, int64_t rows, int64_t K,
                mi_optional_int group_size, mi_optional_int bits, const char* mode, int w_dtype,
                void* stream) {
  int gs = 0, nb = 0;
  int rc = resolve_common(group_size, bits, mode, true, K, &gs, &nb);
  if (rc) return rc;
  if (w_dtype != MI_DTYPE_BFLOAT16 && w_dtype != MI_DTYPE_FLOAT32)
    return fail(MI_ERR_UNSUPPORTED, "weight dtype %d not supported", w_dtype);
  if (rows < 0) return fail(MI_ERR_INVALID, "negative rows");
  if (rows == 0) return MI_OK;
  if (!wq || !scales || !biases || !w) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_quantize(wq, (uint16_t*)scales, (uint16_t*)biases, w,
                                     w_dtype == MI_DTYPE_FLOAT32, rows, K, gs, nb,
                                     (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "quantize launch");
}

int mi_fill_randn(void* out, int64_t n, uint64_t seed, float mean, float stddev, int dtype,
                  void* stream) {
  if (dtype != MI_DTYPE_BFLOAT16 && dtype != MI_DTYPE_FLOAT32)
    return fail(MI_ERR_UNSUPPORTED, "dtype %d not supported", dtype);
  if (n < 0) return fail(MI_ERR_INVALID, "negative n");
  if (n == 0) return MI_OK;
  if (!out) return fail(MI_ERR_INVALID, "null output");
  hipError_t e = mi::launch_randn(out, n, seed, mean, stddev, dtype == MI_DTYPE_FLOAT32,
                                  (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "randn launch");
}

}  // extern "C"
