// C ABI (include/mi_qmm.h): argument validation, dispatch to the gfx950 kernels,
// per-stream workspace, error reporting.
#include "mi_qmm.h"

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
// A wave holds at most UG groups of one tile in registers, a block at most 8 waves,
// and the staged activations must fit the LDS budget; K ranges are the fewest that
// satisfy both. Waves per block: enough for ~16 resident waves per CU.
struct QmvPlan {
  mi::QmvConfig cfg;
  int row_blocks, ks, gps;
};

size_t lds_per_block() {
  static size_t cached = 0;
  if (!cached) {
    int v = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        v <= 0)
      v = 64 * 1024;
    cached = (size_t)v;
  }
  return cached;
}

QmvPlan qmv_plan(int N, int K, int gs, int bits, int rows, int64_t n_items, int x_f32) {
  static const int env_w = env_int("MI_QMM_QMV_WAVES", 0);
  static const int env_ks = env_int("MI_QMM_QMV_KS", 0);
  static const int env_units = env_int("MI_QMM_QMV_UNITS", 2048);
  const size_t lds_max = lds_per_block() - 512;  // static row table headroom
  QmvPlan p;
  p.cfg.rows = rows;
  p.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
  const int tiles = ceil_div(N, 32);
  const int G = K / gs;
  const int ug = mi::qmv_groups_per_wave(bits, gs);
  const int mr = mi::qmv_mr_for_rows(rows);
  const int nch = ceil_div(G, ug);  // 256-byte chunks per row
  int w = (env_w >= 1 && env_w <= mi::kQmvMaxWaves) ? env_w : mi::kQmvMaxWaves;
  if (w > tiles) w = tiles;
  // K ranges: enough (wave, tile, range) units to fill the GPU, each >= 1 chunk,
  // and the staged activations of a range within the LDS budget.
  int ks = (int)((env_units + (int64_t)tiles * p.cfg.grid_z - 1) / ((int64_t)tiles * p.cfg.grid_z));
  if (ks > nch) ks = nch;
  if (ks < 1) ks = 1;
  if (env_ks > 0) ks = env_ks < nch ? env_ks : nch;
  for (;;) {
    const int gps = ceil_div(G, ks);
    if (mi::qmv_lds_bytes(gps, gs, mr, x_f32, w) <= lds_max || ks >= G) break;
    ++ks;
  }
  // Whole chunks per range keep every wave's DMA aligned to 256-byte rows.
  p.gps = ceil_div(ceil_div(G, ks), ug) * ug;
  if (p.gps > G) p.gps = G;
  p.ks = ceil_div(G, p.gps);
  p.cfg.waves = w;
  p.row_blocks = ceil_div(tiles, w);
  return p;
}

// Launch shape for the 16-row-tile decode kernel: one block per (tile, item) with
// the waves splitting K; 8 waves per block when the tiles alone give < 512 blocks.
// K splits across blocks only when the staged activations exceed the LDS budget.
QmvPlan qmv16_plan(int N, int K, int gs, int bits, int rows, int64_t n_items, int x_f32) {
  static const int env_w = env_int("MI_QMM_QMV_WAVES", 0);
  const size_t lds_max = lds_per_block() - 512;
  QmvPlan p;
  p.cfg.rows = rows;
  p.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
  const int tiles = ceil_div(N, 16);
  const int G = K / gs;
  const int ug = mi::qmv16_groups_per_chunk(bits, gs);
  const int mp = mi::qmv16_mp_for_rows(rows);
  const int nch = ceil_div(G, ug);
  int w = (int64_t)tiles * p.cfg.grid_z >= 512 ? 4 : 8;
  if (env_w >= 1 && env_w <= 8) w = env_w;
  if (w > nch) w = nch;
  int ks = 1;
  for (;;) {
    const int gps = ceil_div(G, ks);
    if (mi::qmv16_lds_bytes(gps, gs, bits, mp, x_f32, w) <= lds_max) break;
    if (w > 1) {
      w >>= 1;
      continue;
    }
    if (ks >= G) break;
    ++ks;
  }
  // K ranges start on 8-group boundaries (aligned scale runs).
  p.gps = ks == 1 ? G : ceil_div(ceil_div(G, ks), 8) * 8;
  p.ks = ceil_div(G, p.gps);
  p.cfg.waves = w;
  p.row_blocks = tiles;
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
  // Decode widths (<= 16 rows per pair, or sorted runs cut into 16-row items) use the
  // 16-row-tile kernel; 17..32 rows per pair use the 32-row-tile kernel.
  static const int narrow_max = env_int("MI_QMM_NARROW_MAX", 4);
  const bool narrow = (use_items || M <= narrow_max) && mi::qmv16_supported(P.K, gs, nb);
  P.rpi = narrow ? 16 : 32;
  const int rows = (int)(M < P.rpi ? M : P.rpi);
  int64_t n_items, max_items = 0;
  if (!use_items) {
    P.items_per_pair = ceil_div(M, P.rpi);
    n_items = n_idx * P.items_per_pair;
    if (n_items > INT32_MAX) return fail(MI_ERR_INVALID, "too many work items");
    P.n_items_fixed = (int)n_items;
  } else {
    // Runs of equal rhs cut into rpi-row chunks; the bound holds for any input order.
    max_items = (PT + P.rpi - 1) / P.rpi + n_idx;
    const int64_t runs_bound = n_idx < n_experts ? n_idx : n_experts;
    n_items = (PT + P.rpi - 1) / P.rpi + runs_bound;
    P.items_per_pair = 1;
    P.n_items_fixed = 0;
  }
  QmvPlan plan = narrow ? qmv16_plan(P.N, P.K, gs, nb, use_items ? P.rpi : rows, n_items, P.x_f32)
                        : qmv_plan(P.N, P.K, gs, nb, use_items ? P.rpi : rows, n_items, P.x_f32);
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
      hipError_t e = mi::launch_build_items(rhs_indices, n_idx, (int)M, P.rpi, items, count,
                                            max_items, s);
      if (e != hipSuccess) return hip_fail(e, "build_items launch");
      P.items = items;
      P.item_count = count;
    }
  }
  hipError_t e = narrow ? mi::launch_qmv16(P, plan.cfg, s) : mi::launch_qmv(P, plan.cfg, s);
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
