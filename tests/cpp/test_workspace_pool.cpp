// CPU test of the workspace growth rule (mlx-serve_amd/csrc/workspace_pool.h): an outgrown
// generation that was handed out during a capture stays allocated until release_retired;
// one never captured is freed as soon as it is outgrown.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "workspace_pool.h"

static std::set<void*> live;
static int fails = 0;
#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
      ++fails;                                                \
    }                                                         \
  } while (0)

int main() {
  auto alloc = [](void** p, size_t n) {
    *p = std::malloc(n);
    live.insert(*p);
    return 0;
  };
  auto free_fn = [](void* p) {
    live.erase(p);
    std::free(p);
  };
  mi::GrowOnlyBuffer b;
  CHECK(b.grow(100, alloc, free_fn) == 0);
  void* g0 = b.data();
  CHECK(b.size() >= 100 && g0 != nullptr && !b.captured());
  CHECK(b.grow(50, alloc, free_fn) == 0 && b.data() == g0);  // fits: no new generation
  // eager growth: the outgrown generation was never captured, so it is freed at once
  CHECK(b.grow(4 << 20, alloc, free_fn) == 0);
  void* g1 = b.data();
  CHECK(g1 != g0 && live.count(g0) == 0 && b.retired_count() == 0);
  // a capture takes g1: growing past it retires g1 instead of freeing it
  b.mark_captured();
  CHECK(b.captured());
  CHECK(b.grow(8 << 20, alloc, free_fn) == 0);
  void* g2 = b.data();
  CHECK(g2 != g1 && !b.captured());
  CHECK(live.count(g1) == 1 && b.retired_count() == 1);  // a captured graph may still use g1
  b.mark_captured();
  CHECK(b.grow(64 << 20, alloc, free_fn) == 0);
  CHECK(live.count(g2) == 1 && b.retired_count() == 2);
  // a failing allocation leaves the current generation in place
  void* cur = b.data();
  CHECK(b.grow((size_t)1 << 40, [](void**, size_t) { return 7; }, free_fn) == 7);
  CHECK(b.data() == cur && b.retired_count() == 2);
  b.release_retired(free_fn);
  CHECK(b.retired_count() == 0 && live.count(g1) == 0 && live.count(g2) == 0);
  CHECK(live.count(cur) == 1);
  free_fn(cur);
  std::printf(fails ? "workspace_pool: %d failures\n" : "workspace_pool: ok\n", fails);
  return fails ? 1 : 0;
}
