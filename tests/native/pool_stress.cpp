// Stress test of rw::WorkspacePool (rusty_whisper_amd/csrc/rw_pool.hpp) on
// the CPU: threads take the workspaces of a few keys ("streams") with random
// sizes, fill what they asked for with their own pattern, yield, and check
// that nobody else wrote to it or freed it meanwhile.  Built with
// ThreadSanitizer and with AddressSanitizer by tests/test_workspace_pool_cpu.py.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "rw_pool.hpp"

static std::atomic<long> g_allocs{0}, g_frees{0};
static int a_alloc(size_t bytes, void **out) {
  *out = malloc(bytes);
  if (!*out) return -4;
  ++g_allocs;
  return 0;
}
static void a_free(void *p) {
  ++g_frees;
  free(p);
}

int main() {
  constexpr int KEYS = 3, THREADS = 8, ITERS = 3000;
  auto *pool = new rw::WorkspacePool<int>(a_alloc, a_free, 256);
  std::atomic<int> holders[KEYS];
  for (auto &h : holders) h = 0;
  std::atomic<int> bad{0};
  std::vector<std::thread> ts;
  for (int t = 0; t < THREADS; ++t)
    ts.emplace_back([&, t] {
      std::mt19937 rng(1234 + t);
      for (int i = 0; i < ITERS; ++i) {
        const int key = (int)(rng() % KEYS);
        const size_t bytes = 1 + rng() % 20000;
        rw::HoldWs<rw::WorkspacePool<int>> hold;
        rw::WorkspacePool<int>::Slot *s = nullptr;
        if (pool->acquire(key, bytes, &s) != 0) {
          ++bad;
          continue;
        }
        hold.pool = pool;
        hold.slot = s;
        if (++holders[key] != 1) ++bad;  // exclusive per key
        if (s->cap < bytes) ++bad;
        const unsigned char pat = (unsigned char)(t * 31 + i);
        memset(s->p, pat, bytes);
        std::this_thread::yield();
        const unsigned char *p = (const unsigned char *)s->p;
        for (size_t j = 0; j < bytes; ++j)
          if (p[j] != pat) {
            ++bad;
            break;
          }
        --holders[key];
      }
    });
  for (auto &th : ts) th.join();
  delete pool;
  printf("bad=%d allocs=%ld frees=%ld\n", bad.load(), g_allocs.load(), g_frees.load());
  return (bad.load() == 0 && g_allocs.load() == g_frees.load()) ? 0 : 1;
}
