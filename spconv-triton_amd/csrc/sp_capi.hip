// Library-wide C ABI pieces: version/arch queries, the thread-local error
// message, and the device-wide exclusive scan shared by the other sources.
#include <stdarg.h>
#include <stdio.h>

#include "sp_common.h"

namespace sp {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// POPC: the values scanned are the population counts of the input words (the
// ranks of set bits in a bitmap) rather than the words themselves.
template <bool POPC>
__device__ __forceinline__ uint32_t scan_value(uint32_t w) {
  return POPC ? uint32_t(__popc(w)) : w;
}

template <bool POPC>
__global__ __launch_bounds__(kScanThreads) void scan_chunk_sums(const uint32_t* __restrict__ in,
                                                                int64_t len,
                                                                uint32_t* __restrict__ sums) {
  __shared__ uint32_t lds[kScanThreads / 64 + 1];
  const int64_t base = int64_t(blockIdx.x) * kScanChunk;
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + int64_t(i) * kScanThreads + threadIdx.x;
    if (idx < len) s += scan_value<POPC>(in[idx]);
  }
  uint32_t tot;
  block_exclusive_scan<kScanThreads>(s, lds, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// One workgroup of 1024 threads scans all chunk sums in place.
__global__ __launch_bounds__(1024) void scan_sums_single(uint32_t* __restrict__ sums, int64_t n,
                                                         uint32_t* __restrict__ total) {
  __shared__ uint32_t lds[1024 / 64 + 1];
  const int64_t per = (n + 1023) / 1024;
  const int64_t lo = int64_t(threadIdx.x) * per;
  const int64_t hi = lo + per < n ? lo + per : n;
  uint32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += sums[i];
  uint32_t tot;
  uint32_t run = block_exclusive_scan<1024>(s, lds, &tot);
  for (int64_t i = lo; i < hi; ++i) {
    uint32_t v = sums[i];
    sums[i] = run;
    run += v;
  }
  if (threadIdx.x == 0 && total) *total = tot;
}

// Each thread owns kScanItems consecutive counts of the chunk; with VEC4
// (16-byte aligned arrays) a thread's whole counts move as 16-byte loads and
// stores (one count per load had each instruction touch 64 lines).
template <bool VEC4, bool POPC>
__global__ __launch_bounds__(kScanThreads) void scan_chunk_apply(const uint32_t* __restrict__ in,
                                                                 uint32_t* __restrict__ out,
                                                                 int64_t len,
                                                                 const uint32_t* __restrict__ sums) {
  static_assert(kScanItems % 4 == 0, "whole 16-byte pieces");
  __shared__ uint32_t lds[kScanThreads / 64 + 1];
  const int64_t base = int64_t(blockIdx.x) * kScanChunk + int64_t(threadIdx.x) * kScanItems;
  const bool whole = VEC4 && base + kScanItems <= len;
  uint32_t v[kScanItems];
  uint32_t s = 0;
  if (whole) {
#pragma unroll
    for (int q = 0; q < kScanItems / 4; ++q) {
      const uint4 x = reinterpret_cast<const uint4*>(in + base)[q];
      v[4 * q] = x.x;
      v[4 * q + 1] = x.y;
      v[4 * q + 2] = x.z;
      v[4 * q + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      int64_t idx = base + i;
      v[i] = idx < len ? in[idx] : 0u;
    }
  }
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    v[i] = scan_value<POPC>(v[i]);
    s += v[i];
  }
  uint32_t tot;
  uint32_t run = block_exclusive_scan<kScanThreads>(s, lds, &tot) + sums[blockIdx.x];
  uint32_t o[kScanItems];
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    o[i] = run;
    run += v[i];
  }
  if (whole) {
#pragma unroll
    for (int q = 0; q < kScanItems / 4; ++q)
      reinterpret_cast<uint4*>(out + base)[q] =
          uint4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
  } else {
#pragma unroll
    for (int i = 0; i < kScanItems; ++i)
      if (base + i < len) out[base + i] = o[i];
  }
}

size_t scan_workspace_bytes(int64_t len) {
  int64_t chunks = cdiv(len > 0 ? len : 1, kScanChunk);
  return align_up(size_t(chunks) * sizeof(uint32_t), 256);
}

template <bool POPC>
static int exclusive_scan(const uint32_t* in, uint32_t* out, int64_t len, uint32_t* total,
                          void* ws, hipStream_t stream) {
  if (len <= 0) return SP_OK;
  const int64_t chunks = cdiv(len, kScanChunk);
  uint32_t* sums = static_cast<uint32_t*>(ws);
  scan_chunk_sums<POPC><<<dim3(unsigned(chunks)), dim3(kScanThreads), 0, stream>>>(in, len, sums);
  SP_LAUNCHED();
  scan_sums_single<<<dim3(1), dim3(1024), 0, stream>>>(sums, chunks, total);
  SP_LAUNCHED();
  if (((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0)
    scan_chunk_apply<true, POPC>
        <<<dim3(unsigned(chunks)), dim3(kScanThreads), 0, stream>>>(in, out, len, sums);
  else
    scan_chunk_apply<false, POPC>
        <<<dim3(unsigned(chunks)), dim3(kScanThreads), 0, stream>>>(in, out, len, sums);
  SP_LAUNCHED();
  return SP_OK;
}

int exclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t len, uint32_t* total,
                       void* ws, hipStream_t stream) {
  return exclusive_scan<false>(in, out, len, total, ws, stream);
}

int exclusive_scan_popc(const uint32_t* words, uint32_t* out, int64_t len, uint32_t* total,
                        void* ws, hipStream_t stream) {
  return exclusive_scan<true>(words, out, len, total, ws, stream);
}

}  // namespace sp

extern "C" {

int sp_abi_version(void) { return SP_ABI_VERSION; }

int sp_version(void) { return (0 << 16) | (1 << 8) | 0; }

const char* sp_arch(void) { return "gfx950"; }

const char* sp_last_error(void) { return sp::g_err; }

}  // extern "C"
