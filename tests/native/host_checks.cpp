// Host-side checks built with sanitizers (AddressSanitizer + UBSan, or
// ThreadSanitizer) by tests/test_device_cache.py: the caching allocator and
// the workspace cache of csrc/device_cache.h over a fake backend (malloc,
// with allocation-failure injection), and the staged-transfer loops of
// csrc/host_copy.cpp at every alignment.  Exit status 0 = all checks passed;
// a sanitizer report makes the process fail.
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "device_cache.h"
#include "host_copy.h"

using namespace tt;

static int g_failures = 0;
#define CHECK(cond)                                                        \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
      ++g_failures;                                                        \
    }                                                                      \
  } while (0)

struct FakeBackend {
  AllocFailureInjector inject;
  std::atomic<long> allocs{0}, releases{0}, syncs{0}, orders{0};
  std::atomic<void*> last_ordered{nullptr};
  int alloc(size_t bytes, void** p) {
    if (inject.next_fails()) return 4;
    *p = std::malloc(bytes);
    ++allocs;
    return *p ? 0 : 4;
  }
  void release(void* p) {
    std::free(p);
    ++releases;
  }
  int sync(void*) {
    ++syncs;
    return 0;
  }
  int order_after_library(void* stream) {
    ++orders;
    last_ordered = stream;
    return 0;
  }
};

static void allocator_checks() {
  FakeBackend be;
  BlockCache<FakeBackend> bc(be);
  void *a = nullptr, *b = nullptr, *c = nullptr;
  CHECK(bc.alloc(1000, &a) == 0 && a);
  std::memset(a, 1, 1000);  // the whole request is usable (ASan would flag an overrun)
  size_t used = 0, cached = 0;
  bc.stats(&used, &cached);
  CHECK(used == 1024 && cached == 0);
  CHECK(bc.release(a));
  CHECK(!bc.release(a));  // double free is refused, not corrupting
  bc.stats(&used, &cached);
  CHECK(used == 0 && cached == 1024);
  CHECK(bc.alloc(600, &b) == 0 && b == a);  // reused: 1024 <= 2 * 1024
  CHECK(bc.alloc(3 << 20, &c) == 0 && c != a);
  std::memset(c, 2, 3 << 20);
  CHECK(bc.release(b) && bc.release(c));
  bc.trim();
  bc.stats(&used, &cached);
  CHECK(used == 0 && cached == 0 && be.allocs == be.releases);

  // out of memory: the cache is trimmed and the allocation retried once
  FakeBackend be2;
  BlockCache<FakeBackend> bc2(be2);
  void* x = nullptr;
  CHECK(bc2.alloc(4096, &x) == 0);
  CHECK(bc2.release(x));
  be2.inject.set_limit(0);
  void* y = nullptr;
  CHECK(bc2.alloc(1 << 22, &y) == 4 && y == nullptr);  // refused twice: reported
  CHECK(be2.releases == 1);                          // the cached block went back
  bc2.stats(&used, &cached);
  CHECK(used == 0 && cached == 0);
}

static void workspace_checks() {
  FakeBackend be;
  BlockCache<FakeBackend> bc(be);
  WorkspaceCache<FakeBackend> ws(be, bc);
  int s1 = 0, s2 = 0;  // two "streams"
  void *p = nullptr, *q = nullptr, *r = nullptr;
  {
    WorkspaceCache<FakeBackend>::Lease l(ws);
    uint64_t uses = 99;
    CHECK(l.get(&s1, 0, 100, &p, &uses) == 0 && uses == 0);  // a new buffer: no earlier use
    // a new buffer: its stream is ordered after the library stream first
    CHECK(be.orders == 1 && be.last_ordered == (void*)&s1);
    CHECK(l.get(&s1, 0, 64, &q, &uses) == 0 && q == p && uses == 1);  // fits: same buffer, no sync, no new ordering
    CHECK(l.get(&s1, 0, 100, &q, &uses) == 0 && q == p && uses == 2);
    CHECK(be.orders == 1);
    CHECK(l.get(&s2, 0, 64, &r) == 0 && r != p);  // another stream: its own buffer
    CHECK(be.orders == 2 && be.last_ordered == (void*)&s2);
  }
  CHECK(be.syncs == 0 && ws.count() == 2);
  // A block freed while library-stream work may still use it (tt_free does
  // not wait) and handed to another stream as its workspace: the ordering
  // step comes before the buffer is returned.
  {
    void* freed = nullptr;
    CHECK(bc.alloc(4096, &freed) == 0);
    CHECK(bc.release(freed));
    int s3 = 0;
    {
      WorkspaceCache<FakeBackend>::Lease l(ws);
      void* w3 = nullptr;
      const long before = be.orders;
      CHECK(l.get(&s3, 0, 4000, &w3) == 0 && w3 == freed);
      CHECK(be.orders == before + 1 && be.last_ordered == (void*)&s3);
    }
    CHECK(ws.release_stream(&s3) == 0);
  }
  {
    WorkspaceCache<FakeBackend>::Lease l(ws);
    void* big = nullptr;
    uint64_t uses = 99;
    CHECK(l.get(&s1, 0, 1 << 21, &big, &uses) == 0 && uses == 0);  // grows: waits for stream 1 first; a new buffer
    std::memset(big, 3, 1 << 21);
  }
  CHECK(be.syncs == 2 && ws.bytes_held() == (size_t(1) << 21) + 64);  // (the first sync: release_stream(&s3))
  // a failed growth leaves no slot behind and reports the error
  be.inject.set_limit(0);
  {
    WorkspaceCache<FakeBackend>::Lease l(ws);
    void* z = nullptr;
    CHECK(l.get(&s2, 1, 10 << 20, &z) == 4 && z == nullptr);
  }
  CHECK(ws.count() == 2);
  be.inject.set_limit(-1);
  const long syncs = be.syncs;
  CHECK(ws.release_stream(&s2) == 0 && ws.count() == 1 && be.syncs == syncs + 1);
  CHECK(ws.release_stream(&s2) == 0 && be.syncs == syncs + 1);  // nothing left: no wait
  CHECK(ws.release_all() == 0 && ws.count() == 0);
  bc.trim();
  CHECK(be.allocs == be.releases);
}

// Leases exclude each other: each thread writes its id over its buffer and
// checks that nobody else wrote there while it held the lease.
static void workspace_thread_checks() {
  FakeBackend be;
  BlockCache<FakeBackend> bc(be);
  WorkspaceCache<FakeBackend> ws(be, bc);
  int stream = 0;
  std::atomic<int> violations{0};
  std::vector<std::thread> th;
  for (int t = 0; t < 8; ++t)
    th.emplace_back([&, t]() {
      for (int it = 0; it < 200; ++it) {
        WorkspaceCache<FakeBackend>::Lease l(ws);
        int* buf = nullptr;
        if (l.get(&stream, 0, 256 * sizeof(int) * (1 + it % 3), (void**)&buf)) {
          ++violations;
          continue;
        }
        for (int i = 0; i < 256; ++i) buf[i] = t;
        std::this_thread::yield();
        for (int i = 0; i < 256; ++i)
          if (buf[i] != t) {
            ++violations;
            break;
          }
      }
    });
  for (auto& x : th) x.join();
  CHECK(violations == 0);
  CHECK(ws.release_all() == 0);
  bc.trim();
  CHECK(be.allocs == be.releases);
}

static uint16_t ref_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

static void host_copy_checks() {
  std::vector<unsigned char> src(5000 + 64), dst(5000 + 64);
  for (size_t i = 0; i < src.size(); ++i) src[i] = (unsigned char)(i * 131 + 7);
  for (size_t n : {0, 1, 15, 16, 17, 63, 64, 65, 127, 128, 1000, 4099})
    for (int doff = 0; doff < 16; ++doff)
      for (int soff : {0, 1, 3, 8}) {
        std::fill(dst.begin(), dst.end(), 0xAA);
        copy_stream(dst.data() + doff, src.data() + soff, n);
        CHECK(std::memcmp(dst.data() + doff, src.data() + soff, n) == 0);
        CHECK(doff == 0 || dst[doff - 1] == 0xAA);
        CHECK(dst[doff + n] == 0xAA);
      }
  std::vector<float> f(3000 + 16), back(3000 + 16);
  std::vector<uint16_t> h(3000 + 16);
  for (size_t i = 0; i < f.size(); ++i) f[i] = std::ldexp((float)((i * 2654435761u) % 10007) - 5003.f, (int)(i % 40) - 20);
  for (size_t n : {0, 1, 7, 8, 9, 31, 32, 33, 1000, 2999})
    for (int off = 0; off < 8; ++off) {
      f32_to_bf16_stream(h.data() + off, f.data() + off, n);
      bool same = true;
      for (size_t i = 0; i < n; ++i) same &= h[off + i] == ref_bf16(f[off + i]);
      CHECK(same);
      bf16_to_f32_stream(back.data() + off, h.data() + off, n);
      for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        std::memcpy(&u, &back[off + i], 4);
        same &= u == (uint32_t(h[off + i]) << 16);
      }
      CHECK(same);
    }
}

int main(int argc, char** argv) {
  const bool threads_only = argc > 1 && std::strcmp(argv[1], "threads") == 0;
#ifdef TT_PLANTED_OVERRUN
  {  // a deliberate one-byte overrun of a cache block: AddressSanitizer must report it
    FakeBackend be;
    BlockCache<FakeBackend> bc(be);
    char* p = nullptr;
    if (bc.alloc(512, (void**)&p) == 0) p[512] = 1;
  }
#endif
  if (!threads_only) {
    allocator_checks();
    workspace_checks();
    host_copy_checks();
  }
  workspace_thread_checks();
  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("host checks passed\n");
  return 0;
}
