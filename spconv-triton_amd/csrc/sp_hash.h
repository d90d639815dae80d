// Open-addressing hash tables on device memory, shared by pair generation,
// voxelisation and the HashTable API.
//
//  * Table32: 32-bit keys packed with their 32-bit value into one 64-bit slot
//    (inserted with one 64-bit CAS);
//  * Table64: 64-bit keys in one array, 32-bit values in a side array.
// Linear probing from a mixed home slot; an empty slot is all ones.  A table
// is full when a probe sequence wraps around: insert() then raises the
// overflow flag.  Values of repeated keys are combined with atomicMin.
#pragma once
#include "sp_common.h"

namespace sp {

constexpr uint64_t kEmpty64 = ~uint64_t(0);

__device__ __forceinline__ uint32_t mix32(uint32_t k) {
  // lowbias32 integer finaliser (Chris Wellons, public domain)
  k ^= k >> 16;
  k *= 0x7feb352du;
  k ^= k >> 15;
  k *= 0x846ca68bu;
  k ^= k >> 16;
  return k;
}

__device__ __forceinline__ uint64_t mix64(uint64_t k) {
  // splitmix64 finaliser (Steele, Lea, Flood 2014)
  k ^= k >> 30;
  k *= 0xbf58476d1ce4e5b9ull;
  k ^= k >> 27;
  k *= 0x94d049bb133111ebull;
  k ^= k >> 31;
  return k;
}

// 32-bit keys: slot = (row << 32) | key; all-ones is the empty slot (keys are
// < 2^31, so no key is 0xFFFFFFFF).
struct Table32 {
  uint64_t* slots;
  uint64_t mask;
  int* overflow;

  __device__ __forceinline__ uint64_t home(uint64_t key) const { return mix32(uint32_t(key)) & mask; }

  // Returns true when this call inserted the key.  An existing key keeps the
  // smaller row value.
  __device__ bool insert(uint64_t key64, int32_t val) const {
    const uint32_t key = uint32_t(key64);
    const uint64_t desired = (uint64_t(uint32_t(val)) << 32) | key;
    uint64_t s = home(key64);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t prev = atomicCAS((unsigned long long*)&slots[s], (unsigned long long)kEmpty64,
                                      (unsigned long long)desired);
      if (prev == kEmpty64) return true;
      if (uint32_t(prev) == key) {
        atomicMin(reinterpret_cast<int32_t*>(&slots[s]) + 1, val);
        return false;
      }
      s = (s + 1) & mask;
    }
    atomicExch(overflow, 1);
    return false;
  }

  // The slot holding `key64`, inserting it (with value 0) when absent; -1
  // (and the overflow flag) when the table is full.
  __device__ int64_t insert_slot(uint64_t key64) const {
    const uint32_t key = uint32_t(key64);
    uint64_t s = home(key64);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t prev = atomicCAS((unsigned long long*)&slots[s], (unsigned long long)kEmpty64,
                                      (unsigned long long)key);
      if (prev == kEmpty64 || uint32_t(prev) == key) return int64_t(s);
      s = (s + 1) & mask;
    }
    atomicExch(overflow, 1);
    return -1;
  }

  __device__ __forceinline__ int64_t find_slot(uint64_t key64) const {
    const uint32_t key = uint32_t(key64);
    uint64_t s = home(key64);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t v = slots[s];
      if (uint32_t(v) == key) return int64_t(s);
      if (v == kEmpty64) return -1;
      s = (s + 1) & mask;
    }
    return -1;
  }

  // Split lookups: load the home slot's word (several lookups can have theirs
  // in flight at once), then finish from it.
  __device__ __forceinline__ uint64_t word(uint64_t s) const { return slots[s]; }
  __device__ __forceinline__ int64_t find_from(uint64_t s, uint64_t w, uint64_t key64) const {
    const uint32_t key = uint32_t(key64);
    for (uint64_t i = 0; i <= mask; ++i) {
      if (uint32_t(w) == key) return int64_t(s);
      if (w == kEmpty64) return -1;
      s = (s + 1) & mask;
      w = slots[s];
    }
    return -1;
  }

  __device__ __forceinline__ int32_t find(uint64_t key64) const {
    const uint32_t key = uint32_t(key64);
    uint64_t s = home(key64);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t v = slots[s];
      if (uint32_t(v) == key) return int32_t(uint32_t(v >> 32));
      if (v == kEmpty64) return -1;
      s = (s + 1) & mask;
    }
    return -1;
  }

  __device__ __forceinline__ void set_value(int64_t slot, int32_t val) const {
    reinterpret_cast<int32_t*>(&slots[slot])[1] = val;
  }
};

// 64-bit keys (key volume >= 2^31): key array + row array.
struct Table64 {
  uint64_t* keys;
  int32_t* vals;
  uint64_t mask;
  int* overflow;

  __device__ __forceinline__ uint64_t home(uint64_t key) const { return mix64(key) & mask; }

  __device__ bool insert(uint64_t key, int32_t val) const {
    uint64_t s = home(key);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t prev = atomicCAS((unsigned long long*)&keys[s], (unsigned long long)kEmpty64,
                                      (unsigned long long)key);
      if (prev == kEmpty64 || prev == key) {
        atomicMin(&vals[s], val);
        return prev == kEmpty64;
      }
      s = (s + 1) & mask;
    }
    atomicExch(overflow, 1);
    return false;
  }

  // The slot holding `key`, inserting it when absent (its value is left as
  // is); -1 (and the overflow flag) when the table is full.
  __device__ int64_t insert_slot(uint64_t key) const {
    uint64_t s = home(key);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t prev = atomicCAS((unsigned long long*)&keys[s], (unsigned long long)kEmpty64,
                                      (unsigned long long)key);
      if (prev == kEmpty64 || prev == key) return int64_t(s);
      s = (s + 1) & mask;
    }
    atomicExch(overflow, 1);
    return -1;
  }

  __device__ __forceinline__ int64_t find_slot(uint64_t key) const {
    uint64_t s = home(key);
    for (uint64_t i = 0; i <= mask; ++i) {
      const uint64_t v = keys[s];
      if (v == key) return int64_t(s);
      if (v == kEmpty64) return -1;
      s = (s + 1) & mask;
    }
    return -1;
  }

  __device__ __forceinline__ int32_t find(uint64_t key) const {
    const int64_t s = find_slot(key);
    return s >= 0 ? vals[s] : -1;
  }

  // Split lookups, as Table32's.
  __device__ __forceinline__ uint64_t word(uint64_t s) const { return keys[s]; }
  __device__ __forceinline__ int64_t find_from(uint64_t s, uint64_t w, uint64_t key) const {
    for (uint64_t i = 0; i <= mask; ++i) {
      if (w == key) return int64_t(s);
      if (w == kEmpty64) return -1;
      s = (s + 1) & mask;
      w = keys[s];
    }
    return -1;
  }

  __device__ __forceinline__ void set_value(int64_t slot, int32_t val) const { vals[slot] = val; }
};

template <typename T>
__global__ void fill_value(T* __restrict__ p, int64_t n, T v) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

template <typename T>
static inline int launch_fill(T* p, int64_t n, T v, hipStream_t s) {
  if (n <= 0) return SP_OK;
  const int64_t blocks = cdiv(n, 256);
  SP_CHECK_ARG(blocks <= kMaxGridX, "fill: too many elements");
  fill_value<T><<<dim3(unsigned(blocks)), dim3(256), 0, s>>>(p, n, v);
  SP_LAUNCHED();
  return SP_OK;
}

static inline int launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s) {
  return launch_fill<int32_t>(p, n, v, s);
}

static inline int launch_fill_u64(uint64_t* p, int64_t n, uint64_t v, hipStream_t s) {
  return launch_fill<uint64_t>(p, n, v, s);
}

}  // namespace sp
