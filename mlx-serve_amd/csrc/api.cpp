// C ABI (include/mi_qmm.h): argument validation, dispatch to the gfx950 kernels,
// per-stream workspace, error reporting.
#include "mi_qmm.h"

#include <algorithm>
#include <cmath>

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
#include "workspace_pool.h"

// Fixed scratch of mi_gather_qmm_noalloc: work items and K-split partials of one call.
// Each device holds its own copy for the life of the process; host code reaches it only
// through the address hipGetSymbolAddress returns for the current device (the name
// itself is a host-side stand-in, never a device address).
static constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

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
  if (*bits != 2 && *bits != 3 && *bits != 4 && *bits != 5 && *bits != 6 && *bits != 8)
    return fail(MI_ERR_UNSUPPORTED, "bits=%d not supported", *bits);
  if (*gs != 32 && *gs != 64 && *gs != 128)
    return fail(MI_ERR_UNSUPPORTED, "group_size=%d not supported", *gs);
  if (K <= 0 || K % *gs != 0)
    return fail(MI_ERR_INVALID, "K=%lld must be a positive multiple of group_size=%d",
                (long long)K, *gs);
  if (K > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "K too large");
  return MI_OK;
}

// Microscaling modes: 0 nvfp4, 1 mxfp4, 2 mxfp8; -1 for affine (or no mode given).
int fp_mode_of(const char* mode) {
  if (!mode || std::strcmp(mode, "affine") == 0) return -1;
  if (std::strcmp(mode, "nvfp4") == 0) return 0;
  if (std::strcmp(mode, "mxfp4") == 0) return 1;
  if (std::strcmp(mode, "mxfp8") == 0) return 2;
  return -2;
}

// Each fp mode defines its (bits, group_size) (src/transformer.zig:16846-16854); given
// values must agree.
int resolve_fp(int fm, mi_optional_int gs_in, mi_optional_int bits_in, bool transpose, int64_t K,
               int sb_dtype, int* gs, int* bits) {
  *bits = fm == 2 ? 8 : 4;
  *gs = fm == 0 ? 16 : 32;
  if (!transpose) return fail(MI_ERR_UNSUPPORTED, "transpose=false not supported");
  if ((gs_in.has_value && gs_in.value != *gs) || (bits_in.has_value && bits_in.value != *bits))
    return fail(MI_ERR_INVALID, "this mode takes group_size=%d bits=%d", *gs, *bits);
  if (K <= 0 || K % *gs) return fail(MI_ERR_INVALID, "K=%lld must be a positive multiple of %d",
                                     (long long)K, *gs);
  if (K > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "K too large");
  if (sb_dtype != MI_DTYPE_UINT8)
    return fail(MI_ERR_UNSUPPORTED, "scales dtype %d not supported (uint8 for this mode)", sb_dtype);
  return MI_OK;
}

// Per-device scratch for sorted work lists and K-split partials. Calls on one
// stream are ordered, so reuse by later calls is safe; calls that overlap on
// different streams of one device must not both use it. It only grows outside
// stream capture (mi_workspace_reserve sizes it up front), and an outgrown generation
// stays allocated until mi_workspace_release: graphs captured earlier keep its address.
std::mutex g_ws_mu;
std::map<int, mi::GrowOnlyBuffer> g_ws;

int workspace(hipStream_t s, size_t bytes, void** data) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  mi::GrowOnlyBuffer& w = g_ws[dev];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
  if (w.size() < bytes || !w.data()) {
    if (capturing)
      return fail(MI_ERR_WORKSPACE, "workspace too small during stream capture "
                  "(call mi_workspace_reserve before capturing)");
    hipError_t ae = hipSuccess;
    const int rc = w.grow(
        bytes,
        [&](void** p, size_t n) {
          ae = hipMalloc(p, n);
          return ae == hipSuccess ? 0 : 1;
        },
        [](void* p) {
          // eager work queued on any stream of the device may still use it
          (void)hipDeviceSynchronize();
          (void)hipFree(p);
        });
    if (rc) return hip_fail(ae, "hipMalloc(workspace)");
  }
  if (capturing) w.mark_captured();  // a graph now holds this generation's address
  *data = w.data();
  return MI_OK;
}

std::mutex g_scratch_mu;
std::map<int, void*> g_scratch;  // device -> device address of `scratch`

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    it = g_scratch.emplace(dev, ptr).first;
  }
  *out = it->second;
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
  bool ok = true;  // false: no (waves, K range) split fits the LDS budget
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
  // Whole chunks per range keep every wave's DMA aligned to 256-byte rows; the LDS check
  // uses that rounded range. When even one-chunk ranges do not fit, fewer waves share
  // the block's LDS.
  const int ks0 = ks;
  for (;;) {
    p.gps = std::min(G, ceil_div(ceil_div(G, ks), ug) * ug);
    if (mi::qmv_lds_bytes(p.gps, gs, mr, x_f32, w) <= lds_max) break;
    if (p.gps > ug) {
      ++ks;
      continue;
    }
    if (w == 1) {
      p.ok = false;
      break;
    }
    w >>= 1;
    ks = ks0;
  }
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
  // K ranges start on 8-group boundaries (aligned scale runs); the LDS check uses that
  // rounded range.
  for (;;) {
    p.gps = ks == 1 ? G : std::min(G, ceil_div(ceil_div(G, ks), 8) * 8);
    if (mi::qmv16_lds_bytes(p.gps, gs, bits, mp, x_f32, w) <= lds_max) break;
    if (w > 1) {
      w >>= 1;
      continue;
    }
    if (p.gps <= 8) {
      p.ok = false;
      break;
    }
    ++ks;
  }
  p.ks = ceil_div(G, p.gps);
  p.cfg.waves = w;
  p.row_blocks = tiles;
  return p;
}

bool valid_x_dtype(int d) { return d == MI_DTYPE_BFLOAT16 || d == MI_DTYPE_FLOAT32; }

// One gather_qmm call: validated arguments, kernel parameters and launch plan, and the
// workspace it needs (work items for sorted runs, then K-split partials).
struct GatherJob {
  mi::QmvParams P{};
  QmvPlan plan{};
  mi::Qmv1Plan plan1{};
  mi::QmvmPlan planm{};
  bool empty = false, narrow = false, use_items = false, one_row = false, multi_row = false;
  bool grouped = false;  // sorted runs on the grouped kernel (gmm.hip)
  int gmm_mt = 0;        // its 32-row tiles per item
  double gmm_items = 0;  // expected work items (distinct experts x items per run)
  int64_t max_items = 0;
  size_t items_bytes = 0, part_bytes = 0;
  size_t items_region() const { return ((items_bytes + 255) / 256) * 256; }
  size_t ws_bytes() const { return items_bytes || part_bytes ? items_region() + part_bytes : 0; }
};

int gather_prepare(GatherJob& J, void* y, const void* x, const uint32_t* w, const void* scales,
                   const void* biases, const uint32_t* lhs_indices,
                   const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div, int64_t x_batch,
                   int64_t M, int64_t N, int64_t K, int64_t n_experts, bool transpose,
                   mi_optional_int group_size, mi_optional_int bits, const char* mode,
                   bool sorted_indices, int x_dtype, int sb_dtype) {
  int gs = 0, nb = 0;
  int rc = resolve_common(group_size, bits, mode, transpose, K, &gs, &nb);
  if (rc) return rc;
  if (nb != 4 && nb != 8)
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm: bits=%d not supported (4 and 8)", nb);
  if (!valid_x_dtype(x_dtype)) return fail(MI_ERR_UNSUPPORTED, "x dtype %d not supported", x_dtype);
  if (sb_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
  if (n_idx < 0 || M < 0 || N < 0 || x_batch < 0 || n_experts < 0 || lhs_div <= 0)
    return fail(MI_ERR_INVALID, "negative size or lhs_div <= 0");
  if (n_idx == 0 || M == 0 || N == 0) {
    J.empty = true;
    return MI_OK;
  }
  if (!y || !x || !w || !scales || !biases) return fail(MI_ERR_INVALID, "null tensor pointer");
  if (x_batch == 0 || n_experts == 0) return fail(MI_ERR_INVALID, "empty x or weight bank");
  if (N > (int64_t)1 << 30 || M > (int64_t)1 << 30) return fail(MI_ERR_INVALID, "N or M too large");
  if (n_idx * M >= ((int64_t)1 << 32)) return fail(MI_ERR_INVALID, "n_idx*M exceeds 2^32");

  mi::QmvParams& P = J.P;
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

  J.use_items = sorted_indices && rhs_indices != nullptr && n_idx > 1;
  const int64_t PT = n_idx * M;
  // Rows per work item. Dense pairs: up to 4 rows per pair ride the 16-row-tile kernel
  // (qmv16), wider pairs the 32-row-tile kernel. Sorted runs are cut into items sized
  // from the average run length (rows / distinct-run bound, known without reading the
  // indices): short runs take qmv16 with 1, 2 or 4 staged rows, longer runs 8..32-row
  // items on the 32-row-tile kernel. A run longer than one item re-reads its expert.
  static const int narrow_max = env_int("MI_QMM_NARROW_MAX", 4);
  static const int item_rows = env_int("MI_QMM_ITEM_ROWS", 0);
  const bool q16 = mi::qmv16_supported(P.K, gs, nb);
  if (J.use_items) {
    const int64_t runs = n_idx < n_experts ? n_idx : n_experts;
    int64_t avg = (PT + runs - 1) / runs;
    if (item_rows <= 0 && nb == 4 && !P.x_f32) {
      // Items for the few-row MFMA kernel: size them for the rows a distinct expert gets
      // under uniform routing, mu = PT / (E (1 - (1 - 1/E)^PT)), plus 3 standard deviations,
      // so a run is rarely cut (each extra item re-reads the expert). configs[4] T=64: mu 2.3
      // -> 8-row items, 2.05 -> 1.67 ms; T=8: mu 1.1 stays at one-row items.
      const double e = (double)n_experts, distinct = e * (1.0 - std::pow(1.0 - 1.0 / e, (double)PT));
      const double mu = distinct > 0 ? (double)PT / distinct : 1.0;
      if (mu > 1.3) avg = std::max<int64_t>(avg, (int64_t)std::ceil(mu + 3.0 * std::sqrt(mu)));
    }
    if (item_rows > 0) avg = item_rows;
    // Runs that average several rows per distinct expert go to the grouped kernel: one
    // block per (item, 128-row weight tile) streams the tile once for all the item's rows
    // (up to 32 * MT), in-register dequantize into 32x32x16 MFMAs. Items are sized for
    // mu + 3 sigma rows as above, so a run is rarely cut.
    static const int use_gmm = env_int("MI_QMM_GMM", 1);
    static const int gmm_min = env_int("MI_QMM_GMM_MIN_ROWS", 4);
    if (use_gmm && item_rows <= 0 &&
        mi::gmm_supported(P.N, P.K, nb, gs, P.x_f32, x_batch * M * K * 2)) {
      const double e = (double)n_experts, distinct = e * (1.0 - std::pow(1.0 - 1.0 / e, (double)PT));
      const double mu = distinct > 0 ? (double)PT / distinct : 1.0;
      if (mu >= gmm_min) {
        const double want = mu + 3.0 * std::sqrt(mu);
        J.grouped = true;
        J.gmm_items = distinct * std::max(1.0, std::ceil(want / 64.0));
        static const int force_mt = env_int("MI_QMM_GMM_MT", 0);
        J.gmm_mt = force_mt == 1 || force_mt == 2 ? force_mt
                   : want <= 32 ? 1 : 2;  // longer runs are cut into 64-row items
      }
    }
    J.narrow = q16 && avg <= 4;
    // (64-row items on the two-pass few-row kernel measured slower than 32-row items
    // that re-read a long run's expert: with a K split at K = 2048, and also at K = 768
    // without one, configs[3] T=512 391 against 293 us per layer)
    P.rpi = avg <= 1 ? 1 : avg <= 2 ? 2 : avg <= 4 ? 4 : avg <= 8 ? 8 : avg <= 16 ? 16 : 32;
    if (!J.narrow && P.rpi < 8) P.rpi = 8;
    if (J.grouped) {
      J.narrow = false;
      P.rpi = 32 * J.gmm_mt;
    }
  } else {
    J.narrow = M <= narrow_max && q16;
    P.rpi = J.narrow ? 16 : 32;
  }
  const int rows = (int)(M < P.rpi ? M : P.rpi);
  int64_t n_items;
  if (!J.use_items) {
    P.items_per_pair = ceil_div(M, P.rpi);
    n_items = n_idx * P.items_per_pair;
    if (n_items > INT32_MAX) return fail(MI_ERR_INVALID, "too many work items");
    P.n_items_fixed = (int)n_items;
  } else {
    // Runs of equal rhs cut into rpi-row chunks; the bound holds for any input order.
    J.max_items = (PT + P.rpi - 1) / P.rpi + n_idx;
    const int64_t runs_bound = n_idx < n_experts ? n_idx : n_experts;
    n_items = (PT + P.rpi - 1) / P.rpi + runs_bound;
    P.items_per_pair = 1;
    P.n_items_fixed = 0;
  }
  // Items of exactly one activation row (dense M == 1, MoE decode pairs, sorted runs cut
  // into single rows) stream through the one-row kernel when it supports the layout.
  static const int use_qmv1 = env_int("MI_QMM_QMV1", 1);
  if (J.grouped) {
    P.ks = 1;
    J.plan.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
    J.items_bytes = (size_t)J.max_items * 16 + 256;
    J.part_bytes = 0;
    return MI_OK;
  }
  J.one_row = use_qmv1 && ((J.use_items && P.rpi == 1) || (!J.use_items && M == 1));
  J.one_row = J.one_row && mi::qmv1_supported(P.N, P.K, gs, nb, P.x_f32);
  if (J.one_row) {
    P.rpi = 1;
    if (!J.use_items) {
      P.items_per_pair = 1;
      P.n_items_fixed = (int)n_idx;
      n_items = n_idx;
    }
    J.plan1 = mi::qmv1_plan(P.N, P.K, gs, n_items);
    P.ks = J.plan1.ks;
    P.gps = J.plan1.gps;
    P.row_blocks = J.plan1.tiles;
    J.plan.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
  } else {
    // Items of 2..32 rows: the MFMA few-row kernel when it supports the layout.
    static const int use_qmvm = env_int("MI_QMM_QMVM_GATHER", 1);
    const int item_rows = J.use_items ? P.rpi : rows;
    J.multi_row = use_qmvm && !P.x_f32 && nb == 4 && item_rows >= 2 &&
                  x_batch * M * K * 2 < ((int64_t)1 << 32) &&
                  mi::qmvm_plan(item_rows, P.N, P.K, gs, nb, n_items, &J.planm);
    J.plan = J.narrow ? qmv16_plan(P.N, P.K, gs, nb, item_rows, n_items, P.x_f32)
                      : qmv_plan(P.N, P.K, gs, nb, item_rows, n_items, P.x_f32);
    if (!J.multi_row && !J.plan.ok)
      return fail(MI_ERR_UNSUPPORTED, "gather_qmm: %d rows per item of K=%d do not fit LDS",
                  item_rows, P.K);
    P.ks = J.multi_row ? J.planm.ks : J.plan.ks;
    P.gps = J.plan.gps;
    P.row_blocks = J.plan.row_blocks;
  }
  // The split reduce indexes outputs with 32-bit math.
  if (P.ks > 1 && PT * N >= ((int64_t)1 << 32))
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm: K-split output of %lld elements exceeds 2^32",
                (long long)(PT * N));
  J.items_bytes = J.use_items ? (size_t)J.max_items * 16 + 256 : 0;
  J.part_bytes = P.ks > 1 ? (size_t)P.ks * PT * N * 4 : 0;
  return MI_OK;
}

// fp-mode gathers (nvfp4 fpm 0, mxfp4 1, mxfp8 2) and affine 2/3/5/6-bit gathers (fpm
// 100 + bits, gs 64) on the few-row MFMA kernel: sorted runs
// cut into work items as for the affine kernels, unsorted pairs one item per pair (and
// 32-row slice). Returns MI_ERR_UNSUPPORTED when the call does not fit the plan: the
// caller then takes the per-pair kernel, which serves up to 8 rows per pair.
int gather_prepare_fp(GatherJob& J, int fpm, int gs, void* y, const void* x, const uint32_t* w,
                      const void* scales, const void* biases, const uint32_t* lhs_indices,
                      const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div,
                      int64_t x_batch, int64_t M, int64_t N, int64_t K, int64_t n_experts,
                      bool sorted_indices) {
  static const int use_fp_mfma = env_int("MI_QMM_FP_MFMA", 1);
  const bool odd = fpm >= 100;
  if (!use_fp_mfma || fpm < 0 || (fpm > 2 && !odd)) return MI_ERR_UNSUPPORTED;
  if (N > (int64_t)1 << 30 || M > (int64_t)1 << 30 || n_idx * M >= ((int64_t)1 << 32) ||
      x_batch * M * K * 2 >= ((int64_t)1 << 32) || x_batch == 0 || n_experts == 0)
    return MI_ERR_UNSUPPORTED;
  mi::QmvParams& P = J.P;
  P.w = w;
  P.scales = (const uint16_t*)scales;  // fp modes: uint8 scales, read as bytes
  P.biases = odd ? (const uint16_t*)biases : nullptr;
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
  P.bits = odd ? fpm - 100 : fpm == 2 ? 8 : 4;
  P.group_size = gs;
  P.x_f32 = 0;
  J.use_items = sorted_indices && rhs_indices != nullptr && n_idx > 1;
  const int64_t PT = n_idx * M;
  int64_t n_items;
  if (J.use_items) {
    // rows a distinct expert gets under uniform routing plus 3 standard deviations (as
    // for the affine items); about one row per run stays on the per-pair kernel
    const double e = (double)n_experts, distinct = e * (1.0 - std::pow(1.0 - 1.0 / e, (double)PT));
    const double mu = distinct > 0 ? (double)PT / distinct : 1.0;
    const int64_t avg = mu <= 1.3 ? 1 : (int64_t)std::ceil(mu + 3.0 * std::sqrt(mu));
    P.rpi = avg <= 1 ? 1 : avg <= 2 ? 2 : avg <= 4 ? 4 : avg <= 8 ? 8 : avg <= 16 ? 16 : 32;
    J.max_items = (PT + P.rpi - 1) / P.rpi + n_idx;
    const int64_t runs_bound = n_idx < n_experts ? n_idx : n_experts;
    n_items = (PT + P.rpi - 1) / P.rpi + runs_bound;
    P.items_per_pair = 1;
    P.n_items_fixed = 0;
  } else {
    P.rpi = 32;
    P.items_per_pair = ceil_div(M, P.rpi);
    n_items = n_idx * P.items_per_pair;
    if (n_items > INT32_MAX) return MI_ERR_UNSUPPORTED;
    P.n_items_fixed = (int)n_items;
  }
  const int item_rows = J.use_items ? P.rpi : (int)(M < P.rpi ? M : P.rpi);
  if (!(odd ? mi::qmvm_plan_odd(item_rows, P.N, P.K, gs, fpm - 100, n_items, &J.planm)
            : mi::qmvm_plan_fp(item_rows, P.N, P.K, fpm, n_items, &J.planm)))
    return MI_ERR_UNSUPPORTED;
  J.multi_row = true;
  P.ks = J.planm.ks;
  J.plan.cfg.grid_z = (int)(n_items < 65535 ? n_items : 65535);
  if (P.ks > 1 && PT * N >= ((int64_t)1 << 32)) return MI_ERR_UNSUPPORTED;
  J.items_bytes = J.use_items ? (size_t)J.max_items * 16 + 256 : 0;
  J.part_bytes = P.ks > 1 ? (size_t)P.ks * PT * N * 4 : 0;
  return MI_OK;
}

// Launch a prepared gather on `s`; `ws` holds at least J.ws_bytes() bytes.
int gather_launch(GatherJob& J, void* ws, hipStream_t s) {
  mi::QmvParams& P = J.P;
  if (J.ws_bytes()) {
    P.part = (float*)((char*)ws + J.items_region());
    if (J.use_items) {
      uint32_t* count = (uint32_t*)ws;
      uint32_t* items = (uint32_t*)((char*)ws + 256);
      hipError_t e = mi::launch_build_items(P.rhs, P.n_pairs, P.M, P.rpi, items, count,
                                            J.max_items, s);
      if (e != hipSuccess) return hip_fail(e, "build_items launch");
      P.items = items;
      P.item_count = count;
    }
  }
  // short K with 64-row items: the x-stationary instance, sized for one round of one block a
  // CU (ns passes of 256 weight rows a block)
  static const int use_xs = env_int("MI_QMM_GMM_XS", 1);
  if (J.grouped && use_xs && J.gmm_mt == 2 && !P.dual && !P.swiglu_gate && mi::gmm_xs_fits(P.K)) {
    const int64_t tiles = (P.N + 255) / 256;
    const int64_t ns = std::min<int64_t>(
        tiles, std::max<int64_t>(1, (int64_t)std::ceil(tiles * J.gmm_items / 256.0)));
    hipError_t e = mi::launch_gmm_xs(P, (int)ns, J.plan.cfg.grid_z, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "grouped (x-stationary) launch");
  }
  hipError_t e = J.grouped     ? mi::launch_gmm(P, J.gmm_mt, J.plan.cfg.grid_z, s)
                 : J.one_row   ? mi::launch_qmv1(P, J.plan1, J.plan.cfg.grid_z, s)
                 : J.multi_row ? mi::launch_qmvm_gather(P, J.planm, J.plan.cfg.grid_z, s)
                 : J.narrow    ? mi::launch_qmv16(P, J.plan.cfg, s)
                               : mi::launch_qmv(P, J.plan.cfg, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "qmv launch");
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Large-M route of the formats the fused kernels do not decode: dequantize the weight into
// the workspace as bf16 (`dequant` launches that), then the prefill kernel's bf16-weight
// instance (prefill.hip, bits = 16). The vendor GEMM (dq_gemm) runs instead only under
// MI_QMM_DQGEMM=1, or for shapes that instance does not take.
template <class Dequant>
int dequant_then_gemm(const void* x, void* y, int64_t M, int64_t N, int64_t K, hipStream_t s,
                      Dequant dequant) {
  static const int use_lib = env_int("MI_QMM_DQGEMM", 0);
  const size_t wbytes = round256((size_t)N * K * 2);
  if (!use_lib && mi::prefill_supported(M, N, K, 16, 64)) {
    mi::PrefillParams Q{nullptr, nullptr, nullptr, (const uint16_t*)x, (uint16_t*)y, (int)M,
                        (int)N, (int)K, 64, nullptr, 1, 0, 16};
    const size_t pbytes = mi::prefill_plan(Q);
    void* data = nullptr;
    int rc = workspace(s, wbytes + pbytes, &data);
    if (rc) return rc;
    hipError_t e = dequant(data);
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    Q.w = (const uint32_t*)data;
    if (pbytes) Q.part = (float*)((char*)data + wbytes);
    e = mi::launch_prefill(Q, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "bf16 prefill launch");
  }
  void* data = nullptr;
  int rc = workspace(s, wbytes + mi::kDqGemmBlasWs, &data);
  if (rc) return rc;
  hipError_t e = dequant(data);
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  const char* err = nullptr;
  if (mi::dq_gemm((const uint16_t*)x, (const uint16_t*)data, (uint16_t*)y, (int)M, (int)N,
                  (int)K, (int)N, (char*)data + wbytes, mi::kDqGemmBlasWs, s, &err) != 0)
    return fail(MI_ERR_HIP, "hipBLASLt GEMM: %s", err ? err : "error");
  return MI_OK;
}

}  // namespace

namespace mi {
// Error reporting for the other translation units of the library (the checkpoint loader).
int report_error(int code, const std::string& msg) { return fail(code, "%s", msg.c_str()); }
}  // namespace mi

extern "C" {

const char* mi_last_error(void) { return g_err.c_str(); }

int mi_workspace_reserve(int64_t bytes, void* stream) {
  if (bytes < 0) return fail(MI_ERR_INVALID, "negative size");
  void* d = nullptr;
  return workspace((hipStream_t)stream, (size_t)bytes, &d);
}

int mi_workspace_release(void* stream) {
  (void)stream;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto it = g_ws.find(dev);
  if (it == g_ws.end() || it->second.retired_count() == 0) return MI_OK;
  e = hipDeviceSynchronize();  // queued work may still use a retired generation
  if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
  it->second.release_retired([](void* p) { (void)hipFree(p); });
  return MI_OK;
}

const char* mi_version(void) { return "mi_qmm 0.1 gfx950"; }

int64_t mi_library_gemm_calls(void) { return mi::g_library_gemms.load(); }

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

}  // extern "C"

namespace {
// The per-pair kernel for fp-mode and affine 2/3/5/6-bit gathers (up to 8 rows per pair):
// one block column per pair, no workspace and no device allocation.
int gather_any(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
               const uint32_t* lhs_indices, const uint32_t* rhs_indices, int64_t n_idx,
               int64_t lhs_div, int64_t x_batch, int64_t M, int64_t N, int64_t K,
               int64_t n_experts, int gs, int nb, int fm, hipStream_t s) {
  hipError_t e = mi::launch_qmv_any_gather(
      (const uint16_t*)x, w, scales, fm < 0 ? (const uint16_t*)biases : nullptr, (uint16_t*)y,
      M, N, K, gs, nb, fm, lhs_indices, rhs_indices, n_idx, lhs_div, x_batch, n_experts, s);
  if (e == hipErrorNotSupported)
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm at this format: up to 8 rows per pair, "
                "65535 pairs and K*rows*2 <= 160 KiB");
  return e == hipSuccess ? MI_OK : hip_fail(e, "qmv_any gather launch");
}
}  // namespace

extern "C" {

int mi_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales,
                  const void* biases, const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                  int64_t n_idx, int64_t lhs_div, int64_t x_batch, int64_t M, int64_t N, int64_t K,
                  int64_t n_experts, bool transpose, mi_optional_int group_size,
                  mi_optional_int bits, const char* mode, bool sorted_indices, int x_dtype,
                  int sb_dtype, void* stream) {
  const int fm = fp_mode_of(mode);
  if (fm >= 0 || (bits.has_value && bits.value != 4 && bits.value != 8 && fm == -1)) {
    // nvfp4 / mxfp4 / mxfp8 and affine 2/3/5/6 bits: one block column per pair of the
    // few-row decode kernel, up to 8 rows per pair
    int gs = 0, nb = 0;
    int rc = fm >= 0 ? resolve_fp(fm, group_size, bits, transpose, K, sb_dtype, &gs, &nb)
                     : resolve_common(group_size, bits, mode, transpose, K, &gs, &nb);
    if (rc) return rc;
    if (fm < 0 && sb_dtype != MI_DTYPE_BFLOAT16)
      return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
    if (x_dtype != MI_DTYPE_BFLOAT16)
      return fail(MI_ERR_UNSUPPORTED, "gather_qmm at this format: bf16 activations only");
    if (n_idx < 0 || M < 0 || N < 0 || x_batch < 0 || n_experts < 0 || lhs_div <= 0)
      return fail(MI_ERR_INVALID, "negative size or lhs_div <= 0");
    if (n_idx == 0 || M == 0 || N == 0) return MI_OK;
    if (!y || !x || !w || !scales || (fm < 0 && !biases))
      return fail(MI_ERR_INVALID, "null tensor pointer");
    {  // items of up to 32 rows on the MFMA kernel
      GatherJob J;
      if (gather_prepare_fp(J, fm >= 0 ? fm : 100 + nb, gs, y, x, w, scales, biases,
                            lhs_indices, rhs_indices, n_idx, lhs_div, x_batch, M, N, K,
                            n_experts, sorted_indices) == MI_OK) {
        hipStream_t s = (hipStream_t)stream;
        void* data = nullptr;
        if (J.ws_bytes()) {
          rc = workspace(s, J.ws_bytes(), &data);
          if (rc) return rc;
        }
        return gather_launch(J, data, s);
      }
    }
    return gather_any(y, x, w, scales, biases, lhs_indices, rhs_indices, n_idx, lhs_div,
                      x_batch, M, N, K, n_experts, gs, nb, fm, (hipStream_t)stream);
  }
  GatherJob J;
  int rc = gather_prepare(J, y, x, w, scales, biases, lhs_indices, rhs_indices, n_idx, lhs_div,
                          x_batch, M, N, K, n_experts, transpose, group_size, bits, mode,
                          sorted_indices, x_dtype, sb_dtype);
  if (rc || J.empty) return rc;
  hipStream_t s = (hipStream_t)stream;
  void* data = nullptr;
  if (J.ws_bytes()) {
    rc = workspace(s, J.ws_bytes(), &data);
    if (rc) return rc;
  }
  return gather_launch(J, data, s);
}

int mi_gather_qmm_swiglu(void* y, const void* gate, const void* x, const uint32_t* w,
                         const void* scales, const void* biases, const uint32_t* lhs_indices,
                         const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div,
                         int64_t x_batch, int64_t M, int64_t N, int64_t K, int64_t n_experts,
                         bool transpose, mi_optional_int group_size, mi_optional_int bits,
                         const char* mode, bool sorted_indices, int x_dtype, int sb_dtype,
                         void* stream) {
  if (fp_mode_of(mode) >= 0 || (bits.has_value && bits.value != 4 && bits.value != 8))
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm_swiglu: affine 4- and 8-bit weights only");
  if (x_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm_swiglu: bf16 activations only");
  GatherJob J;
  int rc = gather_prepare(J, y, x, w, scales, biases, lhs_indices, rhs_indices, n_idx, lhs_div,
                          x_batch, M, N, K, n_experts, transpose, group_size, bits, mode,
                          sorted_indices, x_dtype, sb_dtype);
  if (rc || J.empty) return rc;
  if (!gate) return fail(MI_ERR_INVALID, "null gate pointer");
  if (gate == y) return fail(MI_ERR_INVALID, "gate must not alias y");
  hipStream_t s = (hipStream_t)stream;
  void* data = nullptr;
  if (J.ws_bytes()) {
    rc = workspace(s, J.ws_bytes(), &data);
    if (rc) return rc;
  }
  // The grouped, one-row and few-row kernels (and the K-split reduce behind them) apply
  // SwiGLU as they write; the tile kernels write the product and a SwiGLU pass follows,
  // in place (each element is read and written by one thread).
  if (J.grouped || J.one_row || J.multi_row) {
    J.P.swiglu_gate = (const uint16_t*)gate;
    return gather_launch(J, data, s);
  }
  if ((rc = gather_launch(J, data, s)) != MI_OK) return rc;
  hipError_t e = mi::launch_swiglu((uint16_t*)y, (const uint16_t*)gate, (const uint16_t*)y,
                                   n_idx * M * N, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "swiglu launch");
}

int mi_gather_qmm_gate_up_swiglu(void* y, const void* x, const uint32_t* w_gate,
                                 const void* s_gate, const void* b_gate, const uint32_t* w_up,
                                 const void* s_up, const void* b_up,
                                 const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                                 int64_t n_idx, int64_t lhs_div, int64_t x_batch, int64_t M,
                                 int64_t N, int64_t K, int64_t n_experts, bool transpose,
                                 mi_optional_int group_size, mi_optional_int bits,
                                 const char* mode, bool sorted_indices, int x_dtype,
                                 int sb_dtype, void* stream) {
  if (fp_mode_of(mode) >= 0 || (bits.has_value && bits.value != 4 && bits.value != 8))
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm_gate_up_swiglu: affine 4- and 8-bit weights only");
  if (x_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "gather_qmm_gate_up_swiglu: bf16 activations only");
  GatherJob G;
  int rc = gather_prepare(G, y, x, w_gate, s_gate, b_gate, lhs_indices, rhs_indices, n_idx,
                          lhs_div, x_batch, M, N, K, n_experts, transpose, group_size, bits,
                          mode, sorted_indices, x_dtype, sb_dtype);
  if (rc || G.empty) return rc;
  if (!w_up || !s_up || !b_up) return fail(MI_ERR_INVALID, "null up-bank pointer");
  hipStream_t s = (hipStream_t)stream;
  void* data = nullptr;
  if (G.grouped) {
    // one grouped launch: half the waves of a block on each bank, SwiGLU in the epilogue
    G.P.w2 = w_up;
    G.P.scales2 = (const uint16_t*)s_up;
    G.P.biases2 = (const uint16_t*)b_up;
    G.P.dual = 1;
    if (G.ws_bytes() && (rc = workspace(s, G.ws_bytes(), &data)) != MI_OK) return rc;
    return gather_launch(G, data, s);
  }
  if (G.one_row && G.P.group_size == 64 && G.P.ks == 1 && !G.P.x_f32) {
    // one-row items (a few rows per distinct expert): the one-row kernel's dual mode, both
    // banks' loads of an item in flight together and SwiGLU as it writes, in one launch
    G.P.w2 = w_up;
    G.P.scales2 = (const uint16_t*)s_up;
    G.P.biases2 = (const uint16_t*)b_up;
    G.P.dual = 1;
    if (G.ws_bytes() && (rc = workspace(s, G.ws_bytes(), &data)) != MI_OK) return rc;
    return gather_launch(G, data, s);
  }
  // otherwise the gate product goes to the workspace and the up gather applies SwiGLU as
  // mi_gather_qmm_swiglu does
  GatherJob U;
  rc = gather_prepare(U, y, x, w_up, s_up, b_up, lhs_indices, rhs_indices, n_idx, lhs_div,
                      x_batch, M, N, K, n_experts, transpose, group_size, bits, mode,
                      sorted_indices, x_dtype, sb_dtype);
  if (rc) return rc;
  const size_t half = round256((size_t)n_idx * M * N * 2);
  if ((rc = workspace(s, half + std::max(G.ws_bytes(), U.ws_bytes()), &data)) != MI_OK) return rc;
  uint16_t* g = (uint16_t*)data;
  void* rest = (char*)data + half;
  G.P.y = g;
  if ((rc = gather_launch(G, rest, s)) != MI_OK) return rc;
  if (U.grouped || U.one_row || U.multi_row) {
    U.P.swiglu_gate = g;
    return gather_launch(U, rest, s);
  }
  if ((rc = gather_launch(U, rest, s)) != MI_OK) return rc;
  hipError_t e = mi::launch_swiglu((uint16_t*)y, g, (const uint16_t*)y, n_idx * M * N, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "swiglu launch");
}

int mi_gather_qmm_noalloc(void* y, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const uint32_t* lhs_indices,
                          const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div,
                          int64_t x_batch, int64_t M, int64_t N, int64_t K, int64_t n_experts,
                          bool transpose, mi_optional_int group_size, mi_optional_int bits,
                          const char* mode, bool sorted_indices, int x_dtype, int sb_dtype,
                          void* stream) {
  // The scratch address is resolved (once per device) before anything else, so a first
  // call made under stream capture still finds it.
  void* data = nullptr;
  int rc = scratch_address(&data);
  if (rc) return rc;
  const int fm = fp_mode_of(mode);
  const bool odd_w = fm == -1 && bits.has_value && bits.value != 4 && bits.value != 8;
  if (fm >= 0 || odd_w) {
    // fp-mode and odd-width gathers: the MFMA kernel with items / partials in scratch, else
    // the per-pair kernel, which needs no workspace at all
    int gs = 0, nb = 0;
    rc = fm >= 0 ? resolve_fp(fm, group_size, bits, transpose, K, sb_dtype, &gs, &nb)
                 : resolve_common(group_size, bits, mode, transpose, K, &gs, &nb);
    if (rc) return rc;
    if (fm < 0 && sb_dtype != MI_DTYPE_BFLOAT16)
      return fail(MI_ERR_UNSUPPORTED, "scales/biases dtype %d not supported", sb_dtype);
    if (x_dtype != MI_DTYPE_BFLOAT16)
      return fail(MI_ERR_UNSUPPORTED, "gather_qmm at this format: bf16 activations only");
    if (n_idx < 0 || M < 0 || N < 0 || x_batch < 0 || n_experts < 0 || lhs_div <= 0)
      return fail(MI_ERR_INVALID, "negative size or lhs_div <= 0");
    if (n_idx == 0 || M == 0 || N == 0) return MI_OK;
    if (!y || !x || !w || !scales || (fm < 0 && !biases))
      return fail(MI_ERR_INVALID, "null tensor pointer");
    GatherJob J;
    if (gather_prepare_fp(J, fm >= 0 ? fm : 100 + nb, gs, y, x, w, scales, biases, lhs_indices,
                          rhs_indices, n_idx, lhs_div, x_batch, M, N, K, n_experts,
                          sorted_indices) == MI_OK) {
      if (J.ws_bytes() > kNoAllocScratchBytes)
        return fail(MI_ERR_WORKSPACE, "gather_qmm_noalloc: the call needs %zu bytes of "
                    "scratch, the fixed maximum is %zu", J.ws_bytes(), kNoAllocScratchBytes);
      return gather_launch(J, data, (hipStream_t)stream);
    }
    return gather_any(y, x, w, scales, biases, lhs_indices, rhs_indices, n_idx, lhs_div,
                      x_batch, M, N, K, n_experts, gs, nb, fm, (hipStream_t)stream);
  }
  GatherJob J;
  rc = gather_prepare(J, y, x, w, scales, biases, lhs_indices, rhs_indices, n_idx, lhs_div,
                      x_batch, M, N, K, n_experts, transpose, group_size, bits, mode,
                      sorted_indices, x_dtype, sb_dtype);
  if (rc || J.empty) return rc;
  if (J.ws_bytes() > kNoAllocScratchBytes)
    return fail(MI_ERR_WORKSPACE, "gather_qmm_noalloc: the call needs %zu bytes of scratch, "
                "the fixed maximum is %zu", J.ws_bytes(), kNoAllocScratchBytes);
  return gather_launch(J, data, (hipStream_t)stream);
}

int mi_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, bool transpose,
                        mi_optional_int group_size, mi_optional_int bits, const char* mode,
                        int x_dtype, int sb_dtype, void* stream) {
  int gs = 0, nb = 0;
  const int fm = fp_mode_of(mode);
  if (fm >= 0) {
    // nvfp4 / mxfp4 / mxfp8: the dequantized weight is exact in bf16; dequantize it into the
    // workspace and run the bf16 GEMM (the reference sends these modes to MLX's own
    // quantized_matmul, src/transformer.zig:20905-20921)
    int rc = resolve_fp(fm, group_size, bits, transpose, K, sb_dtype, &gs, &nb);
    if (rc) return rc;
    if (x_dtype != MI_DTYPE_BFLOAT16)
      return fail(MI_ERR_UNSUPPORTED, "mode %s: bf16 activations only", mode);
    if (M < 0 || N < 0) return fail(MI_ERR_INVALID, "negative size");
    if (M == 0 || N == 0) return MI_OK;
    if (!y || !x || !w || !scales) return fail(MI_ERR_INVALID, "null tensor pointer");
    if (N > (int64_t)1 << 30 || M > (int64_t)1 << 30 || N * K * 2 > ((int64_t)1 << 34))
      return fail(MI_ERR_INVALID, "N, M or N*K too large");
    hipStream_t s = (hipStream_t)stream;
    // one row of nvfp4 / mxfp4 / mxfp8: the one-row streaming kernel's fp instances
    static const int fp_qmv1 = env_int("MI_QMM_FP_QMV1", 1);
    if (fp_qmv1 && M == 1 && K % 128 == 0 && N * K * (fm == 2 ? 2 : 1) / 2 < ((int64_t)1 << 31)) {
      mi::Qmv1Plan pl = mi::qmv1_plan((int)N, (int)K, 64, 1);
      // mxfp8 (one byte a code, two loads a chunk): 2 chunks in flight a wave, also in the
      // long-row down plan (Llama MLP M=1 3669 -> 3993 GB/s; 3857 with the down at 4)
      if (fm == 2) pl.depth = 2;
      mi::QmvParams P{};
      P.w = w;
      P.scales = (const uint16_t*)scales;
      P.x = x;
      P.y = y;
      P.n_pairs = 1;
      P.lhs_div = 1;
      P.x_batch = 1;
      P.n_experts = 1;
      P.M = 1;
      P.N = (int)N;
      P.K = (int)K;
      P.bits = fm == 2 ? 8 : 4;
      P.group_size = 64;
      P.rpi = 1;
      P.items_per_pair = 1;
      P.n_items_fixed = 1;
      P.ks = pl.ks;
      P.gps = pl.gps;
      P.row_blocks = pl.tiles;
      if (pl.ks > 1) {
        void* data = nullptr;
        rc = workspace(s, (size_t)pl.ks * N * 4, &data);
        if (rc) return rc;
        P.part = (float*)data;
      }
      hipError_t e = mi::launch_qmv1_fp(P, pl, fm, s);
      return e == hipSuccess ? MI_OK : hip_fail(e, "qmv1 fp launch");
    }
    // 1..32 rows: the few-row MFMA kernel (code x scale exact in bf16)
    static const int fp_mfma = env_int("MI_QMM_FP_MFMA", 1);
    static const int fp_mfma_min = env_int("MI_QMM_FP_MFMA_MIN", 1);
    mi::QmvmPlan fp{};
    if (fp_mfma && M >= fp_mfma_min && M <= 32 &&
        mi::qmvm_plan_fp((int)M, (int)N, (int)K, fm, 1, &fp)) {
      mi::QmvmParams Q{x, w, (const uint16_t*)scales, nullptr, (uint16_t*)y, nullptr, (int)M,
                       (int)N, (int)K, gs, fp.kr, fp.wr};
      if (fp.part_bytes) {
        void* data = nullptr;
        rc = workspace(s, fp.part_bytes, &data);
        if (rc) return rc;
        Q.part = (float*)data;
      }
      hipError_t e = mi::launch_qmvm(Q, fp, s);
      return e == hipSuccess ? MI_OK : hip_fail(e, "qmvm fp launch");
    }
    static const int fp_any_max = env_int("MI_QMM_ANY_MAX", 8);
    if (M <= fp_any_max) {  // decode rows: straight from the packed codes
      hipError_t e = mi::launch_qmv_any((const uint16_t*)x, w, scales, nullptr, (uint16_t*)y, M,
                                        N, K, gs, nb, fm, s);
      if (e != hipErrorNotSupported) return e == hipSuccess ? MI_OK : hip_fail(e, "qmv_any launch");
    }
    return dequant_then_gemm(x, y, M, N, K, s, [&](void* wd) {
      return mi::launch_dequantize_fp(wd, w, (const uint8_t*)scales, N, K, fm, 0, nullptr, s);
    });
  }
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
  // Dispatch, in order:
  //  - 4- and 8-bit weights at M >= MI_QMM_PREFILL_MIN (default 128): the fused prefill kernel
  //    (prefill.hip), which replaces the reference's prefillDqGemm route
  //    (src/transformer.zig:20987-21011) without a bf16 copy of the weight;
  //  - one row of gs-64 2/3/5/6/8-bit weights: the one-row streaming kernel;
  //  - 2/3/5/6 bits: the few-row MFMA kernel (2..32 rows, gs 64), qmv_any (up to
  //    MI_QMM_ANY_MAX rows), else dequantize to bf16 + the prefill kernel's bf16 instance;
  //  - 4/8 bits: the few-row MFMA kernel (up to 64 rows), else the fused qmm kernel.
  //    Dequantize + hipBLASLt is opt-in for every format (MI_QMM_DQGEMM=1; for 4/8 bits from
  //    MI_QMM_DQGEMM_MIN rows).
  static const int dq_min = env_int("MI_QMM_DQGEMM_MIN", 256);
  static const int use_dqgemm = env_int("MI_QMM_DQGEMM", 0);
  static const int prefill_min = env_int("MI_QMM_PREFILL_MIN", 128);
  if (x_dtype == MI_DTYPE_BFLOAT16 && !use_dqgemm && M >= prefill_min &&
      mi::prefill_supported(M, N, K, nb, gs)) {
    mi::PrefillParams Q{w, (const uint16_t*)scales, (const uint16_t*)biases, (const uint16_t*)x,
                        (uint16_t*)y, (int)M, (int)N, (int)K, gs, nullptr, 1, 0, nb};
    const size_t ws = mi::prefill_plan(Q);
    if (ws) {
      void* data = nullptr;
      rc = workspace(s, ws, &data);
      if (rc) return rc;
      Q.part = (float*)data;
    }
    hipError_t e = mi::launch_prefill(Q, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "prefill launch");
  }
  // Dense one row of gs-64 affine weights in a format the one-row streaming kernel has
  // instances for (fpm 100 + bits: 2/3/5/6/8 bits), with its plan and fixed-order K-split
  // reduce.
  auto run_qmv1_fmt = [&](int fpm) -> int {
    mi::Qmv1Plan pl = mi::qmv1_plan((int)N, (int)K, 64, 1);
    // 8-bit (one byte a code): two loads a chunk, so 2 chunks in flight a wave where the
    // 4-bit plan issues 4 ([14336,4096]: 13.77 -> 12.89 us a launch)
    if (fpm == 108 && pl.nc <= 4) pl.depth = 2;
    mi::QmvParams P{};
    P.w = w;
    P.scales = (const uint16_t*)scales;
    P.biases = (const uint16_t*)biases;
    P.x = x;
    P.y = y;
    P.n_pairs = 1;
    P.lhs_div = 1;
    P.x_batch = 1;
    P.n_experts = 1;
    P.M = 1;
    P.N = (int)N;
    P.K = (int)K;
    P.bits = nb;
    P.group_size = 64;
    P.rpi = 1;
    P.items_per_pair = 1;
    P.n_items_fixed = 1;
    P.ks = pl.ks;
    P.gps = pl.gps;
    P.row_blocks = pl.tiles;
    if (pl.ks > 1) {
      void* data = nullptr;
      const int rc2 = workspace(s, (size_t)pl.ks * N * 4, &data);
      if (rc2) return rc2;
      P.part = (float*)data;
    }
    hipError_t e = mi::launch_qmv1_fp(P, pl, fpm, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmv1 format launch");
  };
  const bool odd_width = nb != 4 && nb != 8;
  if (odd_width && (x_dtype != MI_DTYPE_BFLOAT16 || N * K * 2 > ((int64_t)1 << 34)))
    return fail(MI_ERR_UNSUPPORTED, "bits=%d: bf16 activations only", nb);
  // one row at gs 64: the one-row streaming kernel's odd-width instances
  static const int odd_qmv1 = env_int("MI_QMM_ODD_QMV1", 1);
  if (odd_width && odd_qmv1 && M == 1 && gs == 64 && x_dtype == MI_DTYPE_BFLOAT16 &&
      K % 128 == 0 && N * (K / 8 * nb) < ((int64_t)1 << 31))
    return run_qmv1_fmt(100 + nb);
  static const int odd_mfma = env_int("MI_QMM_ODD_MFMA", 1);
  mi::QmvmPlan op{};
  // 2..32 rows, gs 64 (and one row at 2 bits, where the per-code kernel is VALU-bound)
  if (odd_width && odd_mfma && M <= 32 && (M >= 2 || nb == 2) &&
      mi::qmvm_plan_odd((int)M, (int)N, (int)K, gs, nb, 1, &op)) {
    mi::QmvmParams Q{x, w, (const uint16_t*)scales, (const uint16_t*)biases, (uint16_t*)y,
                     nullptr, (int)M, (int)N, (int)K, gs, op.kr, op.wr};
    if (op.part_bytes) {
      void* data = nullptr;
      rc = workspace(s, op.part_bytes, &data);
      if (rc) return rc;
      Q.part = (float*)data;
    }
    hipError_t e = mi::launch_qmvm(Q, op, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmvm odd-width launch");
  }
  static const int any_max = env_int("MI_QMM_ANY_MAX", 8);
  if (odd_width && M <= any_max) {  // decode rows: straight from the packed bitstream
    hipError_t e = mi::launch_qmv_any((const uint16_t*)x, w, scales, (const uint16_t*)biases,
                                      (uint16_t*)y, M, N, K, gs, nb, -1, s);
    if (e != hipErrorNotSupported) return e == hipSuccess ? MI_OK : hip_fail(e, "qmv_any launch");
  }
  if (x_dtype == MI_DTYPE_BFLOAT16 && (odd_width || (use_dqgemm && dq_min > 0 && M >= dq_min)) &&
      K <= INT32_MAX && N * K * 2 <= ((int64_t)1 << 34)) {
    return dequant_then_gemm(x, y, M, N, K, s, [&](void* wd) {
      return mi::launch_dequantize(wd, w, (const uint16_t*)scales, (const uint16_t*)biases, N,
                                   K, gs, nb, 0, 0, s);
    });
  }
  // 2..64 rows: the few-row MFMA kernel (33..64 rows as two 32-row passes per block)
  static const int use_qmvm = env_int("MI_QMM_QMVM", 1);
  static const int qmvm_max = env_int("MI_QMM_QMVM_MAX", 64);
  // 33..64 rows: by default as two launches (32 rows, then the rest) on disjoint output rows.
  // Each re-reads the weights and still beats the 64-row instance's two passes over the
  // staged rows (Llama-3-8B MLP, 4-bit M=64: 36.9 against 48.1 us per call; M=48: 30.6
  // against 44.9).
  static const int qmvm_split = env_int("MI_QMM_QMVM_SPLIT64", 1);
  auto run_qmvm = [&](const void* xc, void* yc, int64_t Mc, const mi::QmvmPlan& pl) -> int {
    mi::QmvmParams Q{xc, w, (const uint16_t*)scales, (const uint16_t*)biases, (uint16_t*)yc,
                     nullptr, (int)Mc, (int)N, (int)K, gs, pl.kr, pl.wr};
    if (pl.part_bytes) {
      void* data = nullptr;
      int rc2 = workspace(s, pl.part_bytes, &data);
      if (rc2) return rc2;
      Q.part = (float*)data;
    }
    hipError_t e = mi::launch_qmvm(Q, pl, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmvm launch");
  };
  mi::QmvmPlan qp{};
  static const int split_max = env_int("MI_QMM_QMVM_SPLIT_MAX", 64);
  // (above 64 rows the chunks measured no better than qmm_kernel / prefill_kernel: 4-bit
  // M=96 54.7 against 57.7 us, 8-bit M=96 69.3 against 65.4, M=128 73-91 against 57-69)
  if (use_qmvm && qmvm_split && x_dtype == MI_DTYPE_BFLOAT16 && M > 32 && M <= split_max) {
    const int64_t mlast = M - 32 * ((M - 1) / 32);  // rows of the last launch
    mi::QmvmPlan q1{}, q2{};
    // only when a 32-row launch fills the GPU by itself at 8 weight tiles a block (on
    // narrow shapes, e.g. the DeepSeek-V3 shared expert, the 32-row plan needs fewer tiles
    // a block to fill the GPU, and two such launches measured slower than one 64-row one)
    if (mi::qmvm_plan(32, (int)N, (int)K, gs, nb, 1, &q1) && q1.wr >= 8 && q1.tiles * q1.ks >= 192 &&
        mi::qmvm_plan((int)mlast, (int)N, (int)K, gs, nb, 1, &q2)) {
      for (int64_t m0 = 0; m0 < M; m0 += 32) {
        const int64_t mc = std::min<int64_t>(32, M - m0);
        rc = run_qmvm((const uint16_t*)x + m0 * K, (uint16_t*)y + m0 * N, mc, mc == 32 ? q1 : q2);
        if (rc != MI_OK) return rc;
      }
      return MI_OK;
    }
  }
  // one row of 8-bit at gs 64: the one-row streaming kernel's 8-bit instances
  static const int q8_qmv1 = env_int("MI_QMM_Q8_QMV1", 1);
  if (q8_qmv1 && nb == 8 && M == 1 && gs == 64 && x_dtype == MI_DTYPE_BFLOAT16 &&
      K % 128 == 0 && N * K < ((int64_t)1 << 31))
    return run_qmv1_fmt(108);
  static const int q8_one = env_int("MI_QMM_Q8_QMVM1", 1);
  if (use_qmvm && x_dtype == MI_DTYPE_BFLOAT16 && M >= (nb == 8 && q8_one ? 1 : 2) &&
      M <= qmvm_max && mi::qmvm_plan((int)M, (int)N, (int)K, gs, nb, 1, &qp))
    return run_qmvm(x, y, M, qp);
  if (x_dtype == MI_DTYPE_BFLOAT16 && M > 32 && mi::qmm_supported((int)M, (int)N, (int)K, nb, gs)) {
    mi::QmmParams Q{w, (const uint16_t*)scales, (const uint16_t*)biases, (const uint16_t*)x,
                    (uint16_t*)y, (int)M, (int)N, (int)K, nb, gs, nullptr, 1, 0, 0};
    const size_t ws = mi::qmm_plan(Q);
    if (ws) {
      void* data = nullptr;
      rc = workspace(s, ws, &data);
      if (rc) return rc;
      Q.part = (float*)data;
    }
    hipError_t e = mi::launch_qmm(Q, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "qmm launch");
  }
  // Dense = gather with a single pair on expert 0; M rows ride in one x batch.
  return mi_gather_qmm(y, x, w, scales, biases, nullptr, nullptr, 1, 1, 1, M, N, K, 1, transpose,
                       group_size, bits, mode, false, x_dtype, sb_dtype, stream);
}

int mi_dequantize_rounding(void* out, const uint32_t* w, const void* scales, const void* biases,
                           int64_t rows, int64_t K, mi_optional_int group_size,
                           mi_optional_int bits, const char* mode, const float* global_scale,
                           int sb_dtype, int out_dtype, int rounding, void* stream) {
  int gs = 0, nb = 0;
  const int fm = fp_mode_of(mode);
  if (global_scale && fm != 0)
    return fail(MI_ERR_INVALID, "global_scale applies to mode nvfp4 only");
  if (fm >= 0) {  // exact in either output dtype without a global scale: rounding does not apply
    int rc = resolve_fp(fm, group_size, bits, true, K, sb_dtype, &gs, &nb);
    if (rc) return rc;
    if (out_dtype != MI_DTYPE_BFLOAT16 && out_dtype != MI_DTYPE_FLOAT32)
      return fail(MI_ERR_UNSUPPORTED, "output dtype %d not supported", out_dtype);
    if (rows < 0) return fail(MI_ERR_INVALID, "negative rows");
    if (rows == 0) return MI_OK;
    if (!out || !w || !scales) return fail(MI_ERR_INVALID, "null tensor pointer");
    hipError_t e = mi::launch_dequantize_fp(out, w, (const uint8_t*)scales, rows, K, fm,
                                            out_dtype == MI_DTYPE_FLOAT32, global_scale,
                                            (hipStream_t)stream);
    return e == hipSuccess ? MI_OK : hip_fail(e, "dequantize launch");
  }
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
                  const char* mode, const float* global_scale, int sb_dtype, int out_dtype,
                  void* stream) {
  return mi_dequantize_rounding(out, w, scales, biases, rows, K, group_size, bits, mode,
                                global_scale, sb_dtype, out_dtype, 1, stream);
}

int mi_quantize(uint32_t* wq, void* scales, void* biases, const void* w, int64_t rows, int64_t K,
                mi_optional_int group_size, mi_optional_int bits, const char* mode,
                const float* global_scale, int w_dtype, void* stream) {
  int gs = 0, nb = 0;
  if (global_scale)
    return fail(MI_ERR_UNSUPPORTED, "global_scale: quantize takes affine only here");
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

// ---------------------------------------------------------------- MoE glue --

int mi_moe_route_topk(uint32_t* inds, void* scores, const float* logits, int64_t T, int64_t E,
                      int k, int scores_dtype, void* stream) {
  if (scores_dtype != MI_DTYPE_FLOAT32 && scores_dtype != MI_DTYPE_BFLOAT16)
    return fail(MI_ERR_UNSUPPORTED, "scores dtype %d not supported", scores_dtype);
  if (T < 0 || E <= 0 || k <= 0) return fail(MI_ERR_INVALID, "bad T/E/k");
  if (E > 1024 || k > 64 || k > E)
    return fail(MI_ERR_UNSUPPORTED, "E=%lld k=%d outside E<=1024, k<=min(64,E)", (long long)E, k);
  if (T == 0) return MI_OK;
  if (!inds || !scores || !logits) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_route_topk(logits, T, (int)E, k, inds, scores,
                                       scores_dtype == MI_DTYPE_BFLOAT16, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "route launch");
}

int mi_moe_route_grouped(uint32_t* inds, float* scores, const float* logits, const float* bias,
                         int64_t T, int64_t E, int k, int n_group, int topk_group, bool route_norm,
                         float route_scale, void* stream) {
  if (T < 0 || E <= 0 || k <= 0) return fail(MI_ERR_INVALID, "bad T/E/k");
  if (n_group <= 0 || topk_group <= 0 || topk_group > n_group || E % n_group != 0 ||
      E / n_group < 2)
    return fail(MI_ERR_INVALID, "bad group geometry (E %% n_group, group size >= 2, "
                "0 < topk_group <= n_group)");
  if (E > 1024 || n_group > 64 || k > 64 || k > E)
    return fail(MI_ERR_UNSUPPORTED, "E <= 1024, n_group <= 64, k <= min(64, E)");
  if (T == 0) return MI_OK;
  if (!inds || !scores || !logits || !bias) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_route_grouped(logits, bias, T, (int)E, k, n_group, topk_group,
                                          route_norm ? 1 : 0, route_scale, inds, scores,
                                          (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "grouped route launch");
}

int mi_moe_sort_dispatch(uint32_t* order, uint32_t* inv, uint32_t* sorted, uint32_t* lhs,
                         uint32_t* seg_offsets, const uint32_t* flat, int64_t n, int k,
                         int64_t n_experts, void* stream) {
  if (n < 0 || k <= 0 || n_experts <= 0) return fail(MI_ERR_INVALID, "bad n/k/n_experts");
  if (n_experts > 8192) return fail(MI_ERR_UNSUPPORTED, "n_experts > 8192");
  if (n >= ((int64_t)1 << 31)) return fail(MI_ERR_INVALID, "n too large");
  if (n == 0 && !seg_offsets) return MI_OK;
  if (n > 0 && (!order || !inv || !sorted || !lhs || !flat))
    return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_sort_dispatch(flat, n, k, (int)n_experts, order, inv, sorted, lhs,
                                          seg_offsets, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "sort_dispatch launch");
}

int mi_take_rows(void* out, const void* in, const uint32_t* indices, int64_t n, int64_t n_src,
                 int64_t row_bytes, void* stream) {
  if (n < 0 || n_src < 0 || row_bytes < 0) return fail(MI_ERR_INVALID, "negative size");
  if (n == 0 || row_bytes == 0) return MI_OK;
  if (!out || !in || !indices) return fail(MI_ERR_INVALID, "null tensor pointer");
  if (n > 65535) return fail(MI_ERR_UNSUPPORTED, "more than 65535 rows per call");
  hipError_t e = mi::launch_take_rows(out, in, indices, n, n_src, row_bytes, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "take_rows launch");
}

int mi_swiglu(void* y, const void* gate, const void* up, int64_t n, int dtype, void* stream) {
  if (dtype != MI_DTYPE_BFLOAT16) return fail(MI_ERR_UNSUPPORTED, "dtype %d not supported", dtype);
  if (n < 0) return fail(MI_ERR_INVALID, "negative n");
  if (n == 0) return MI_OK;
  if (!y || !gate || !up) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_swiglu((uint16_t*)y, (const uint16_t*)gate, (const uint16_t*)up, n,
                                   (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "swiglu launch");
}

int mi_moe_down_reduce(void* y, const void* v, const void* scores, int64_t T, int k, int64_t N,
                       int dtype, void* stream) {
  if (dtype != MI_DTYPE_BFLOAT16) return fail(MI_ERR_UNSUPPORTED, "dtype %d not supported", dtype);
  if (T < 0 || k <= 0 || N < 0) return fail(MI_ERR_INVALID, "bad T/k/N");
  if (T == 0 || N == 0) return MI_OK;
  if (T > 65535) return fail(MI_ERR_UNSUPPORTED, "more than 65535 tokens per call");
  if (!y || !v || !scores) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_down_reduce((uint16_t*)y, (const uint16_t*)v, (const uint16_t*)scores,
                                        T, k, N, (hipStream_t)stream);
  return e == hipSuccess ? MI_OK : hip_fail(e, "down_reduce launch");
}

int mi_moe_down_reduce_rows(void* y, const void* v, const void* scores, const uint32_t* rows,
                            int64_t n_rows, int64_t T, int k, int64_t N, int dtype,
                            void* stream) {
  if (dtype != MI_DTYPE_BFLOAT16) return fail(MI_ERR_UNSUPPORTED, "dtype %d not supported", dtype);
  if (T < 0 || k <= 0 || N < 0 || n_rows < 0) return fail(MI_ERR_INVALID, "bad T/k/N/n_rows");
  if (T == 0 || N == 0) return MI_OK;
  if (T > 65535) return fail(MI_ERR_UNSUPPORTED, "more than 65535 tokens per call");
  if (!y || !v || !scores || !rows) return fail(MI_ERR_INVALID, "null tensor pointer");
  hipError_t e = mi::launch_down_reduce((uint16_t*)y, (const uint16_t*)v, (const uint16_t*)scores,
                                        T, k, N, (hipStream_t)stream, rows, n_rows);
  return e == hipSuccess ? MI_OK : hip_fail(e, "down_reduce launch");
}

int mi_gather_qmv_gate_up_swiglu(void* y, const void* x, const uint32_t* w_gate,
                                 const void* s_gate, const void* b_gate, const uint32_t* w_up,
                                 const void* s_up, const void* b_up, const uint32_t* inds,
                                 int64_t T, int k, int64_t N, int64_t K, int64_t n_experts,
                                 mi_optional_int group_size, mi_optional_int bits,
                                 const char* mode, void* stream) {
  if (T < 0 || k <= 0) return fail(MI_ERR_INVALID, "bad T/k");
  if (!inds && T > 0) return fail(MI_ERR_INVALID, "null indices");
  const int64_t n_idx = T * k;
  if (const int fm = fp_mode_of(mode); fm >= 0) {
    // bias-less modes: gate into the workspace, then up with SwiGLU applied as it writes
    int gs = 0, nb = 0;
    int rc = resolve_fp(fm, group_size, bits, true, K, MI_DTYPE_UINT8, &gs, &nb);
    if (rc) return rc;
    if (T == 0 || N == 0) return MI_OK;
    if (!y || !x || !w_gate || !s_gate || !w_up || !s_up)
      return fail(MI_ERR_INVALID, "null tensor pointer");
    GatherJob G, U;
    if (gather_prepare_fp(G, fm, gs, y, x, w_gate, s_gate, nullptr, nullptr, inds, n_idx, k, T,
                          1, N, K, n_experts, false) != MI_OK ||
        gather_prepare_fp(U, fm, gs, y, x, w_up, s_up, nullptr, nullptr, inds, n_idx, k, T, 1,
                          N, K, n_experts, false) != MI_OK)
      return fail(MI_ERR_UNSUPPORTED, "gate/up at mode %s: shape outside the few-row kernel",
                  mode);
    hipStream_t s = (hipStream_t)stream;
    const size_t half = round256((size_t)n_idx * N * 2);
    void* data = nullptr;
    rc = workspace(s, half + std::max(G.ws_bytes(), U.ws_bytes()), &data);
    if (rc) return rc;
    uint16_t* g = (uint16_t*)data;
    G.P.y = g;
    if ((rc = gather_launch(G, (char*)data + half, s)) != MI_OK) return rc;
    U.P.y = y;
    U.P.swiglu_gate = g;
    return gather_launch(U, (char*)data + half, s);
  }
  GatherJob G, U;
  // Every (token, slot) pair reads its token's row: lhs(i) = i / k.
  int rc = gather_prepare(G, y, x, w_gate, s_gate, b_gate, nullptr, inds, n_idx, k, T, 1, N, K,
                          n_experts, true, group_size, bits, mode, false, MI_DTYPE_BFLOAT16,
                          MI_DTYPE_BFLOAT16);
  if (rc || G.empty) return rc;
  rc = gather_prepare(U, y, x, w_up, s_up, b_up, nullptr, inds, n_idx, k, T, 1, N, K, n_experts,
                      true, group_size, bits, mode, false, MI_DTYPE_BFLOAT16, MI_DTYPE_BFLOAT16);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const size_t half = round256((size_t)n_idx * N * 2);
  const size_t need = 2 * half + std::max(G.ws_bytes(), U.ws_bytes());
  void* data = nullptr;
  rc = workspace(s, need, &data);
  if (rc) return rc;
  uint16_t* g = (uint16_t*)data;
  uint16_t* u = (uint16_t*)((char*)data + half);
  void* rest = (char*)data + 2 * half;
  // One launch for gate, up and SwiGLU when both run on the one-row kernel, gs 64, with a
  // single K range (same shapes, so G's plan is U's plan).
  if (G.one_row && U.one_row && G.P.group_size == 64 && G.P.ks == 1 && !G.P.x_f32) {
    G.P.w2 = w_up;
    G.P.scales2 = (const uint16_t*)s_up;
    G.P.biases2 = (const uint16_t*)b_up;
    G.P.dual = 1;
    G.P.y = y;
    return gather_launch(G, rest, s);
  }
  G.P.y = g;
  if ((rc = gather_launch(G, rest, s)) != MI_OK) return rc;
  // The one-row and few-row kernels (and the K-split reduce) apply SwiGLU as they write the
  // up projection; the other kernels write u and a SwiGLU pass follows.
  if (U.one_row || U.multi_row) {
    U.P.y = y;
    U.P.swiglu_gate = g;
    return gather_launch(U, rest, s);
  }
  U.P.y = u;
  if ((rc = gather_launch(U, rest, s)) != MI_OK) return rc;
  hipError_t e = mi::launch_swiglu((uint16_t*)y, g, u, n_idx * N, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "swiglu launch");
}

int mi_moe_route_gate_up_swiglu(void* y, uint32_t* inds, void* scores, const float* logits,
                                const void* x, const uint32_t* w_gate, const void* s_gate,
                                const void* b_gate, const uint32_t* w_up, const void* s_up,
                                const void* b_up, int64_t T, int64_t E, int k, int64_t N,
                                int64_t K, mi_optional_int group_size, mi_optional_int bits,
                                const char* mode, int scores_dtype, void* stream) {
  if (T < 0 || k <= 0 || E <= 0) return fail(MI_ERR_INVALID, "bad T/E/k");
  if (T == 0) return MI_OK;
  if (!inds || !scores || !logits) return fail(MI_ERR_INVALID, "null routing pointer");
  if (k > E || k > 64) return fail(MI_ERR_INVALID, "k must be <= min(64, E)");
  const int64_t n_idx = T * k;
  if (fp_mode_of(mode) >= 0) {  // bias-less modes: route, then the fused gate + up call
    int rc = mi_moe_route_topk(inds, scores, logits, T, E, k, scores_dtype, stream);
    if (rc) return rc;
    return mi_gather_qmv_gate_up_swiglu(y, x, w_gate, s_gate, b_gate, w_up, s_up, b_up, inds, T,
                                        k, N, K, E, group_size, bits, mode, stream);
  }
  GatherJob G;
  int rc = gather_prepare(G, y, x, w_gate, s_gate, b_gate, nullptr, inds, n_idx, k, T, 1, N, K, E,
                          true, group_size, bits, mode, false, MI_DTYPE_BFLOAT16,
                          MI_DTYPE_BFLOAT16);
  if (rc || G.empty) return rc;
  hipStream_t s = (hipStream_t)stream;
  // Routing inside the gate + up launch: the dual one-row kernel at gs 64 with one K range,
  // up to 256 experts, bf16 scores. Otherwise route, then the fused gate + up call.
  if (scores_dtype == MI_DTYPE_BFLOAT16 && E <= 256 && G.one_row && G.P.group_size == 64 &&
      G.P.ks == 1 && !G.P.x_f32 && !G.ws_bytes()) {
    G.P.w2 = w_up;
    G.P.scales2 = (const uint16_t*)s_up;
    G.P.biases2 = (const uint16_t*)b_up;
    G.P.dual = 1;
    G.P.rhs = nullptr;  // each block finds its pair's expert itself
    G.P.route_logits = logits;
    G.P.route_inds = inds;
    G.P.route_scores = (uint16_t*)scores;
    G.P.route_E = (int)E;
    G.P.route_k = k;
    return gather_launch(G, nullptr, s);
  }
  rc = mi_moe_route_topk(inds, scores, logits, T, E, k, scores_dtype, stream);
  if (rc) return rc;
  return mi_gather_qmv_gate_up_swiglu(y, x, w_gate, s_gate, b_gate, w_up, s_up, b_up, inds, T, k,
                                      N, K, E, group_size, bits, mode, stream);
}

int mi_gather_qmv_down_reduce(void* y, const void* act, const uint32_t* w_down,
                              const void* s_down, const void* b_down, const uint32_t* inds,
                              const void* scores, int64_t T, int k, int64_t N, int64_t K,
                              int64_t n_experts, mi_optional_int group_size, mi_optional_int bits,
                              const char* mode, void* stream) {
  if (T < 0 || k <= 0) return fail(MI_ERR_INVALID, "bad T/k");
  if (T > 65535) return fail(MI_ERR_UNSUPPORTED, "more than 65535 tokens per call");
  if ((!inds || !scores) && T > 0) return fail(MI_ERR_INVALID, "null indices or scores");
  const int64_t n_idx = T * k;
  if (const int fm = fp_mode_of(mode); fm >= 0) {
    // bias-less modes: the k down rows per token into the workspace, then the weighted sum
    int gs = 0, nb = 0;
    int rc = resolve_fp(fm, group_size, bits, true, K, MI_DTYPE_UINT8, &gs, &nb);
    if (rc) return rc;
    if (T == 0 || N == 0) return MI_OK;
    if (!y || !act || !w_down || !s_down) return fail(MI_ERR_INVALID, "null tensor pointer");
    GatherJob D;
    if (gather_prepare_fp(D, fm, gs, y, act, w_down, s_down, nullptr, nullptr, inds, n_idx, 1,
                          n_idx, 1, N, K, n_experts, false) != MI_OK)
      return fail(MI_ERR_UNSUPPORTED, "down at mode %s: shape outside the few-row kernel", mode);
    hipStream_t s = (hipStream_t)stream;
    const size_t vb = round256((size_t)n_idx * N * 2);
    void* data = nullptr;
    rc = workspace(s, vb + D.ws_bytes(), &data);
    if (rc) return rc;
    uint16_t* v = (uint16_t*)data;
    D.P.y = v;
    if ((rc = gather_launch(D, (char*)data + vb, s)) != MI_OK) return rc;
    hipError_t e = mi::launch_down_reduce((uint16_t*)y, v, (const uint16_t*)scores, T, k, N, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "down_reduce launch");
  }
  GatherJob D;
  // act holds one row per (token, slot) pair: lhs(i) = i.
  int rc = gather_prepare(D, y, act, w_down, s_down, b_down, nullptr, inds, n_idx, 1, n_idx, 1, N,
                          K, n_experts, true, group_size, bits, mode, false, MI_DTYPE_BFLOAT16,
                          MI_DTYPE_BFLOAT16);
  if (rc || D.empty) return rc;
  hipStream_t s = (hipStream_t)stream;
  // Few tokens: one launch computes each token's k down rows and their weighted sum (the
  // experts' tiles are read once per token either way at this size).
  static const int fused_max_t = env_int("MI_MOE_DOWN_FUSED_MAXT", 4);
  if (T <= fused_max_t && D.one_row && D.plan1.ks == 1 && !D.P.x_f32 &&
      mi::moe_down_supported(T, k, N, K, D.P.group_size, D.P.bits, D.plan1.waves, D.plan1.nc)) {
    hipError_t e = mi::launch_moe_down((uint16_t*)y, (const uint16_t*)act, w_down,
                                       (const uint16_t*)s_down, (const uint16_t*)b_down, inds,
                                       (const uint16_t*)scores, T, k, N, K, n_experts, D.plan1.waves,
                                       D.plan1.nc, s);
    return e == hipSuccess ? MI_OK : hip_fail(e, "moe_down launch");
  }
  const size_t vb = round256((size_t)n_idx * N * 2);
  void* data = nullptr;
  rc = workspace(s, vb + D.ws_bytes(), &data);
  if (rc) return rc;
  uint16_t* v = (uint16_t*)data;
  D.P.y = v;
  if ((rc = gather_launch(D, (char*)data + vb, s)) != MI_OK) return rc;
  hipError_t e = mi::launch_down_reduce((uint16_t*)y, v, (const uint16_t*)scores, T, k, N, s);
  return e == hipSuccess ? MI_OK : hip_fail(e, "down_reduce launch");
}

}  // extern "C"
