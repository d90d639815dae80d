// Shared helpers for the gfx950 sparse-convolution library: error plumbing,
// launch checks, wave64 primitives and the device-wide scan used by the pair
// generator, the radix sort and the compaction kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "spconv_hip.h"

namespace sp {

// ---- host-side error reporting ------------------------------------------
int set_error(int code, const char* fmt, ...);  // defined in sp_capi.hip

#define SP_CHECK_ARG(cond, ...)                                 \
  do {                                                          \
    if (!(cond)) return ::sp::set_error(SP_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

#define SP_HIP(call)                                                          \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess)                                                     \
      return ::sp::set_error(SP_ERR_HIP, "%s failed: %s (%s:%d)", #call,      \
                             hipGetErrorString(e_), __FILE__, __LINE__);      \
  } while (0)

#define SP_LAUNCHED()                                                         \
  do {                                                                        \
    hipError_t e_ = hipGetLastError();                                        \
    if (e_ != hipSuccess)                                                     \
      return ::sp::set_error(SP_ERR_HIP, "kernel launch failed: %s (%s:%d)",  \
                             hipGetErrorString(e_), __FILE__, __LINE__);      \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Grid sizes are checked on the host before every launch: the x dimension
// of a HIP grid holds at most 2^31-1 workgroups.
constexpr int64_t kMaxGridX = 0x7fffffffLL;

// Bump allocator over a caller-provided workspace (256-byte aligned slices).
struct WsCursor {
  char* base;
  size_t size;
  size_t off = 0;
  WsCursor(void* b, size_t s) : base(static_cast<char*>(b)), size(s) {}
  template <typename T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = reinterpret_cast<T*>(base + off);
    off += count * sizeof(T);
    return p;
  }
  bool ok() const { return off <= size; }
};

// Size-only twin of WsCursor: the *_workspace_size queries run the same
// sequence of take() calls without a base pointer.
struct WsSizer {
  size_t off = 0;
  template <typename T>
  void take(size_t count) {
    off = align_up(off, 256);
    off += count * sizeof(T);
  }
};

// ---- wave64 primitives ----------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  return (uint64_t(1) << lane_id()) - 1;  // lane 0 -> 0
}

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v |= __shfl_xor(v, off, 64);
  return v;
}

// Exclusive scan of NT per-thread values within one workgroup.
// lds holds NT/64 + 1 words.  Returns this thread's exclusive prefix and the
// workgroup total in *total.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* lds,
                                                         uint32_t* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  if (wave == 0) {
    uint32_t s = lane < NW ? lds[lane] : 0u;
    uint32_t t = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      uint32_t y = __shfl_up(t, off, 64);
      if (lane >= off) t += y;
    }
    if (lane < NW) lds[lane] = t - s;
    if (lane == NW - 1) lds[NW] = t;
  }
  __syncthreads();
  uint32_t res = lds[wave] + x - v;
  *total = lds[NW];
  __syncthreads();
  return res;
}

// ---- device-wide exclusive scan of uint32 counts ---------------------------
// Three phases: per-chunk sums, a single-workgroup scan of the chunk sums,
// then a per-chunk scan that adds the chunk base.  Scan size <= 2^31.
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;                       // per thread
constexpr int kScanChunk = kScanThreads * kScanItems;  // 4096 counts per chunk

size_t scan_workspace_bytes(int64_t len);
// in and out may alias.  total (nullable, device) receives the grand total.
int exclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t len, uint32_t* total,
                       void* ws, hipStream_t stream);
// The same over the population counts of `words` (out[i] = set bits of
// words[0..i-1]; *total = all set bits); out must not alias words.
int exclusive_scan_popc(const uint32_t* words, uint32_t* out, int64_t len, uint32_t* total,
                        void* ws, hipStream_t stream);

}  // namespace sp
