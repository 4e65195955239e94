// page_arena.hpp — fixed-size page slots carved from device slabs that never move.
//
// A sealed page must keep its device address for as long as any page table points at it, so the arena never
// reallocates: it adds slabs (8, 16, 32, ... slots, each slab one hipMalloc) and hands out slots from a free list.
// A slot released after a failed or cleared seal goes back to the free list; slabs are freed only when the arena
// is destroyed. Host-side bookkeeping only; callers order device work on their stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace cfnib {

class PageArena {
 public:
  explicit PageArena(uint64_t slot_bytes = 0) : slot_bytes_((slot_bytes + 255u) & ~uint64_t(255)) {}
  PageArena(const PageArena &) = delete;
  PageArena &operator=(const PageArena &) = delete;
  ~PageArena() {
    for (void *s : slabs_) (void)hipFree(s);
  }

  void set_slot_bytes(uint64_t b) { slot_bytes_ = (b + 255u) & ~uint64_t(255); }
  uint64_t slot_bytes() const { return slot_bytes_; }

  // A free slot, adding a slab when none is left.
  hipError_t acquire(char **slot) {
    if (free_.empty()) {
      const uint64_t n = slabs_.empty() ? 8u : next_slab_slots_;
      void *p = nullptr;
      hipError_t e = hipMalloc(&p, n * slot_bytes_);
      if (e != hipSuccess) return e;
      slabs_.push_back(p);
      reserved_ += n * slot_bytes_;
      next_slab_slots_ = n * 2u;
      for (uint64_t i = n; i-- > 0;) free_.push_back(static_cast<char *>(p) + i * slot_bytes_);
    }
    *slot = free_.back();
    free_.pop_back();
    return hipSuccess;
  }

  void release(char *slot) {
    if (slot) free_.push_back(slot);
  }

  uint64_t reserved_bytes() const { return reserved_; }

 private:
  uint64_t slot_bytes_;
  uint64_t reserved_ = 0;
  uint64_t next_slab_slots_ = 8;
  std::vector<void *> slabs_;
  std::vector<char *> free_;
};

// Owning device buffer (hipMalloc / hipFree).
struct DeviceBuffer {
  void *ptr = nullptr;
  uint64_t bytes = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&o) noexcept : ptr(o.ptr), bytes(o.bytes) {
    o.ptr = nullptr;
    o.bytes = 0;
  }
  DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
    if (this != &o) {
      reset();
      ptr = o.ptr;
      bytes = o.bytes;
      o.ptr = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DeviceBuffer() { reset(); }
  hipError_t allocate(uint64_t n) {
    if (ptr && bytes == n) return hipSuccess;
    reset();
    if (n == 0) return hipSuccess;
    hipError_t e = hipMalloc(&ptr, n);
    if (e != hipSuccess) {
      ptr = nullptr;
      return e;
    }
    bytes = n;
    return hipSuccess;
  }
  void reset() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  template <typename T>
  T *as() const {
    return static_cast<T *>(ptr);
  }
};

}  // namespace cfnib
