// rw_pool.hpp -- the per-(device, stream) workspaces of the device-pointer
// entry points that are called without a caller workspace.
//
// A caller holds its key's buffer exclusively from the moment it asks for it
// until it has queued every launch that uses it (the HoldWs guard's
// lifetime).  That gives two guarantees:
//   - a buffer is never freed or replaced while another caller holds it (a
//     caller that needs more space grows the buffer only while it holds it);
//   - two threads queuing on the same stream cannot interleave their
//     launches over one buffer: the second queues after the first is done,
//     and the stream runs them in that order.
// Callers on different streams use different buffers and never wait for
// each other.  A replaced buffer is freed through the pool's free function
// (hipFree, which waits for the device's queued work first).
//
// Host-only C++ (no HIP types), so the logic is tested on the CPU with a
// plain allocator under ThreadSanitizer.
#pragma once
#include <stddef.h>

#include <map>
#include <memory>
#include <mutex>

namespace rw {

template <class Key>
class WorkspacePool {
 public:
  using AllocFn = int (*)(size_t bytes, void **out);  // 0 on success
  using FreeFn = void (*)(void *p);

  struct Slot {
    std::mutex hold;  // held by the caller using the buffer
    void *p = nullptr;
    size_t cap = 0;
  };

  WorkspacePool(AllocFn a, FreeFn f, size_t min_bytes) : alloc_(a), free_(f), min_(min_bytes) {}
  WorkspacePool(const WorkspacePool &) = delete;
  WorkspacePool &operator=(const WorkspacePool &) = delete;
  ~WorkspacePool() {
    for (auto &kv : slots_)
      if (kv.second->p) free_(kv.second->p);
  }

  // Takes `key`'s slot exclusively and makes its buffer at least `bytes`
  // long (a power of two, at least min_bytes).  On success the slot is held
  // and must be given back with release(); on failure it is not held.
  int acquire(const Key &key, size_t bytes, Slot **out) {
    Slot *s;
    {
      std::lock_guard<std::mutex> lk(map_mu_);
      std::unique_ptr<Slot> &u = slots_[key];
      if (!u) u.reset(new Slot);
      s = u.get();  // slots live as long as the pool
    }
    s->hold.lock();
    if (s->cap < bytes) {
      size_t want = min_;
      while (want < bytes) want *= 2;
      if (s->p) free_(s->p);
      s->p = nullptr;
      s->cap = 0;
      int rc = alloc_(want, &s->p);
      if (rc) {
        s->p = nullptr;
        s->hold.unlock();
        return rc;
      }
      s->cap = want;
    }
    *out = s;
    return 0;
  }

  void release(Slot *s) { s->hold.unlock(); }

 private:
  AllocFn alloc_;
  FreeFn free_;
  size_t min_;
  std::mutex map_mu_;
  std::map<Key, std::unique_ptr<Slot>> slots_;
};

// RAII hold of one slot: the entry point keeps it until its launches are queued
template <class Pool>
struct HoldWs {
  Pool *pool = nullptr;
  typename Pool::Slot *slot = nullptr;
  HoldWs() = default;
  HoldWs(const HoldWs &) = delete;
  HoldWs &operator=(const HoldWs &) = delete;
  ~HoldWs() {
    if (slot) pool->release(slot);
  }
};

}  // namespace rw
