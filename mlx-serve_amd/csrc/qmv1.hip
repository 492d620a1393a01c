// Plan and dispatch of the one-row decode kernel (qmv1_kernel.h; its instances are in
// qmv1_g32.hip, qmv1_g64.hip and qmv1_g128.hip).
#include "qmv1_kernel.h"

#include <algorithm>
#include <cstdlib>

namespace mi {

using qmv1_detail::kChunkVals;

bool qmv1_supported(int N, int K, int gs, int bits, int x_f32) {
  // buffer resources address one expert's matrix with 32-bit byte offsets
  return bits == 4 && !x_f32 && K % kChunkVals == 0 && (gs == 32 || gs == 64 || gs == 128) &&
         (int64_t)N * (K / 2) < ((int64_t)1 << 31);
}

size_t qmv1_lds_bytes(int vals, int waves) {
  return (size_t)vals * 2 + (size_t)(vals / 32) * 4 + (size_t)waves * 16 * 4;
}

namespace {

struct Factor {
  int ks = 0, w = 0, nc = 0;
};

// nch chunks per row = ks (block K splits) x w (waves per block) x nc (chunks per wave),
// exactly, with nc from the instantiated set; cost prefers no K split (it costs a second
// launch), nc near `target`, then more waves. nc == 0 when no exact factorization exists.
Factor exact_factor(int nch, int target, int ks_pen) {
  static const int nc_set[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16};
  Factor f;
  double best = 1e30;
  for (int ks = 1; ks <= nch; ++ks) {
    if (nch % ks) continue;
    const int per_split = nch / ks;
    for (int w = 1; w <= 16; ++w) {
      if (per_split % w) continue;
      const int nc = per_split / w;
      if (w > 8 && nc > 8) continue;  // 16-wave blocks need <= 8 chunks per wave
      bool ok = false;
      for (int v : nc_set) ok |= v == nc;
      if (!ok) continue;
      const double cost = std::abs(nc - target) + ks_pen * (ks - 1) + 0.01 * (16 - w);
      if (cost < best) {
        best = cost;
        f = Factor{ks, w, nc};
      }
    }
  }
  return f;
}

// Rounded-up split when nch has no exact factorization (the last wave repeats a chunk,
// weighted 0).
Factor rounded_factor(int nch, int target) {
  int w = 1;
  while (w < 8 && (nch + w - 1) / w > target) w <<= 1;
  int per = (nch + w - 1) / w;
  int ks = 1;
  if (per > 16) {
    ks = (per + 15) / 16;
    per = 16;
  }
  const int ch_split = (nch + ks - 1) / ks;
  Factor f;
  f.ks = (nch + ch_split - 1) / ch_split;
  f.w = std::max(1, std::min(w, (ch_split + per - 1) / per));
  f.nc = (ch_split + f.w - 1) / f.w;
  if (f.nc > 8 && f.nc < 16 && f.nc % 2) ++f.nc;
  return f;
}

int env_or(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : dflt;
}

}  // namespace

// Two measured regimes on MI355X (256 CUs):
//  - many waves (>= 16 per CU at 4 chunks each): every wave issues its 4 chunk loads up
//    front; the memory system stays full and the dot products hide behind other waves;
//  - fewer waves: ~8 waves per CU, each streaming its chunks with a rolling window of
//    `depth` loads (2 for <= 8 chunks, 4 above), so data arrives in the order it is used
//    and the dot products overlap the stream instead of piling up at the end.
Qmv1Plan qmv1_plan(int N, int K, int gs, int64_t n_items) {
  const int nch = K / kChunkVals;
  const int64_t tiles = (N + 15) / 16;
  const int64_t rows_work = tiles * std::max<int64_t>(1, std::min<int64_t>(n_items, 65535));
  static const int env_target = env_or("MI_QMV1_TARGET", 0);
  static const int env_ks_pen = env_or("MI_QMV1_KSPEN", 20);
  static const int env_depth = env_or("MI_QMV1_DEPTH", 0);
  constexpr int64_t kCUs = 256;
  int target = env_target ? env_target : 4;
  const bool several = rows_work > tiles;  // work items of several pairs / experts
  if (!env_target && several) {
    // ~24 waves per CU over the whole launch: per-item set-up is amortized over more
    // chunks when the launch is large, and small launches keep enough waves
    const int64_t t = (rows_work * nch + 12 * kCUs) / (24 * kCUs);
    target = (int)std::max<int64_t>(4, std::min<int64_t>(16, t));
  }
  Factor f = exact_factor(nch, target, env_ks_pen);
  if (!env_target && !several && f.nc > 4) {
    // 4 chunks per wave does not factor: size waves for ~8 per CU instead
    const int64_t t = rows_work * nch / (8 * kCUs);
    target = (int)std::max<int64_t>(4, std::min<int64_t>(16, t));
    f = exact_factor(nch, target, env_ks_pen);
  }
  if (!f.nc) f = rounded_factor(nch, target);
  Qmv1Plan p;
  const int ch_split = (nch + f.ks - 1) / f.ks;
  p.ks = (nch + ch_split - 1) / ch_split;
  p.gps = ch_split * kChunkVals / gs;
  p.waves = f.w;
  p.nc = f.nc;
  const int64_t waves_total = rows_work * p.ks * p.waves;
  p.depth = env_depth ? env_depth
            : (p.nc <= 4 && waves_total >= 16 * kCUs) ? 4
            : p.nc <= 8 ? 2 : 4;
  p.lds = qmv1_lds_bytes(ch_split * kChunkVals, p.waves);
  p.tiles = (int)tiles;
  return p;
}

hipError_t launch_qmv1(const QmvParams& P, const Qmv1Plan& plan, int grid_z, hipStream_t s) {
  dim3 grid((unsigned)plan.tiles, (unsigned)P.ks, (unsigned)grid_z);
  hipError_t e;
  switch (P.group_size) {
    case 32: e = launch_qmv1_gs<32>(P, grid, plan.waves, plan.nc, plan.depth, plan.lds, s); break;
    case 64: e = launch_qmv1_gs<64>(P, grid, plan.waves, plan.nc, plan.depth, plan.lds, s); break;
    default: e = launch_qmv1_gs<128>(P, grid, plan.waves, plan.nc, plan.depth, plan.lds, s); break;
  }
  if (e != hipSuccess || P.ks == 1) return e;
  return launch_reduce_splits(P, s);
}

}  // namespace mi
