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

// Per (device, stream) device workspace, grown on demand. Calls on one stream are
// ordered, so a buffer reused by later calls on the same stream is safe.
struct Workspace {
  void* ptr = nullptr;
  size_t size = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

int workspace(hipStream_t s, size_t bytes, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Workspace& w = g_ws[{dev, s}];
  if (w.size < bytes) {
    if (w.ptr) {
      e = hipStreamSynchronize(s);  // the old buffer may still be read by queued work
      if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
      (void)hipFree(w.ptr);
      w.ptr = nullptr;
      w.size = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    e = hipMalloc(&w.ptr, want);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
    w.size = want;
  }
  *out = w.ptr;
  return MI_OK;
}

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Launch shape for the small-M kernel: enough row tiles per wave to amortise the
// activation fragments, enough waves (split-K) to keep ~16 waves per CU in flight.
mi::QmvConfig qmv_config(int N, int K, int gs, int rows, int64_t n_items, int x_f32) {
  mi::QmvConfig c;
  c.rows = rows;
  const int G = K / gs;
  const int64_t items = n_items < 65535 ? n_items : 65535;
  int rt = 4;
  while (rt > 1 && (int64_t)ceil_div(N, 16 * rt) * items < 1024) rt >>= 1;
  c.rt = rt;
  c.row_groups = ceil_div(N, 16 * rt);
  c.grid_y = (int)items;
  const int64_t blocks = (int64_t)c.row_groups * items;
  int w = 1;
  while (w < 8 && blocks * w < 4096 && G / (2 * w) >= 2) w <<= 1;
  const int mt = rows > 16 ? 2 : 1;
  const int r4 = rows <= 1 ? 1 : rows <= 2 ? 2 : 4;
  const int slots = rt * mt * r4;
  while (w > 1 && (size_t)w * slots * 64 * 4 > 64 * 1024) w >>= 1;
  (void)x_f32;
  c.waves = w;
  return c;
}

bool valid_x_dtype(int d) { return d == MI_DTYPE_BFLOAT16 || d == MI_DTYPE_FLOAT32; }

}  // namespace

extern "C" {

const char* mi_last_error(void) { return g_err.c_str(); }

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
  if (!use_items) {
    const int rows = M <= 32 ? (int)M : 32;
    P.rows_per_item = rows <= 16 ? 16 : 32;
    P.items_per_pair = ceil_div(M, P.rows_per_item);
    const int64_t n_items = n_idx * P.items_per_pair;
    if (n_items > INT32_MAX) return fail(MI_ERR_INVALID, "too many work items");
    P.n_items_fixed = (int)n_items;
    mi::QmvConfig c = qmv_config(P.N, P.K, gs, rows, n_items, P.x_f32);
    hipError_t e = mi::launch_qmv(P, c, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmv launch");
  }

  // Sorted: build (expert run, 32-row chunk) work items on the device.
  P.rows_per_item = 32;
  const int64_t total = n_idx * M;
  const int64_t runs_bound = n_idx < n_experts ? n_idx : n_experts;
  const int64_t max_items = (total + 31) / 32 + n_idx;  // any input order fits
  void* ws = nullptr;
  rc = workspace(s, (size_t)max_items * 16 + 256, &ws);
  if (rc) return rc;
  uint32_t* count = (uint32_t*)ws;
  uint32_t* items = (uint32_t*)((char*)ws + 256);
  hipError_t e = mi::launch_build_items(rhs_indices, n_idx, (int)M, 32, items, count, max_items, s);
  if (e != hipSuccess) return hip_fail(e, "build_items launch");
  P.items = items;
  P.item_count = count;
  P.items_per_pair = 1;
  P.n_items_fixed = 0;
  const int64_t expect_items = (total + 31) / 32 + runs_bound;
  mi::QmvConfig c = qmv_config(P.N, P.K, gs, 32, expect_items, P.x_f32);
  e = mi::launch_qmv(P, c, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "gather qmv launch");
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
