// Gather-plan builder (layout and purpose in sp_plan.h).
//
// One workgroup per tile of kTileRows output rows: the tile's kTileRows * kv
// entries are sorted in LDS with a bitonic network (no pair = INT32_MAX sorts
// last), the distinct values are compacted in place, the tile's items are
// numbered, and every entry's slot is found by binary search in the compacted
// list and stored as its staged LDS address.  A second, single-workgroup
// kernel lists the tiles whose rows do not fit in LDS; their number is copied
// back to the host (the build's one synchronisation), so that a GEMM launches
// the direct-gather kernel for them only when there are any.  The plan depends
// only on the table, so the caller builds it once per table and reuses it for
// every GEMM on that table.
#include "sp_plan.h"

namespace sp {

constexpr int kPlanThreads = 512;

template <int NP>
__global__ __launch_bounds__(kPlanThreads) void plan_build_kernel(
    const int32_t* __restrict__ pairs, int64_t M, int kv, int64_t n_src,
    int32_t* __restrict__ count, int32_t* __restrict__ rows_out, int32_t* __restrict__ nact_out,
    int32_t* __restrict__ koff_out, uint16_t* __restrict__ addr_out, int E) {
  __shared__ int32_t keys[NP];
  __shared__ uint32_t scan_lds[kPlanThreads / 64 + 1];
  __shared__ int32_t s_item[kPlanMaxKv];  // item number of offset k in the tile, or -1
  __shared__ int32_t s_nact;
  constexpr int PER = NP / kPlanThreads;
  static_assert(PER <= 32, "first-occurrence flags are kept in one 32-bit mask");
  constexpr int32_t kNone = 0x7fffffff;
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * kTileRows;
  const int n_ent = kTileRows * kv;
  for (int e = threadIdx.x; e < NP; e += kPlanThreads) {
    int32_t key = kNone;
    if (e < n_ent) {
      const int k = e / kTileRows;
      const int64_t r = r0 + (e - k * kTileRows);
      if (r < M) {
        const int32_t v = pairs[int64_t(k) * M + r];
        if (v >= 0 && v < n_src) key = v;
      }
    }
    keys[e] = key;
  }
  __syncthreads();
  for (int size = 2; size <= NP; size <<= 1) {
    for (int half = size >> 1; half > 0; half >>= 1) {
      for (int i = threadIdx.x; i < NP / 2; i += kPlanThreads) {
        const int lo = 2 * i - (i & (half - 1));
        const int hi = lo + half;
        const bool up = (lo & size) == 0;
        const int32_t a = keys[lo], b = keys[hi];
        if ((a > b) == up) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  // first occurrences of valid values; thread t owns entries [t*PER, (t+1)*PER)
  const int base = threadIdx.x * PER;
  int32_t v[PER];
  int32_t prev = base > 0 ? keys[base - 1] : kNone;
  uint32_t firsts = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] = keys[base + i];
    if (v[i] != kNone && v[i] != prev) firsts |= 1u << i;
    prev = v[i];
  }
  uint32_t total = 0;
  uint32_t pos = block_exclusive_scan<kPlanThreads>(uint32_t(__builtin_popcount(firsts)),
                                                    scan_lds, &total);
  __syncthreads();  // all entries read: compact in place (pos <= entry index)
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (firsts & (1u << i)) keys[pos++] = v[i];
  __syncthreads();
  const int U = int(total);
  if (threadIdx.x == 0) count[tile] = U;
  if (U >= kLdsRows) return;  // the GEMM gathers this tile straight from memory
  // the list is padded with -1 to kLdsRows entries, so that the GEMM can load
  // it without waiting for the count
  for (int i = threadIdx.x; i < kLdsRows; i += kPlanThreads)
    rows_out[tile * kLdsRows + i] = i < U ? keys[i] : -1;

  // items of the tile: the offsets with a pair among its rows
  for (int i = threadIdx.x; i < kPlanMaxKv; i += kPlanThreads) s_item[i] = -1;
  __syncthreads();
  for (int e = threadIdx.x; e < n_ent; e += kPlanThreads) {
    const int k = e / kTileRows, lr = e - k * kTileRows;
    const int64_t r = r0 + lr;
    if (r >= M) continue;
    const int32_t x = pairs[int64_t(k) * M + r];
    if (x >= 0 && x < n_src) s_item[k] = 0;  // every writer stores the same value
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* ko = koff_out + tile * E;
    int n = 0;
    for (int k = 0; k < kv; ++k)
      if (s_item[k] == 0) {
        s_item[k] = n;
        ko[n++] = k;
      }
    for (int q = 0; q < kPad; ++q) ko[n + q] = -1;
    s_nact = n;
    nact_out[tile] = n;
  }
  __syncthreads();
  // LDS address of every (item, row): the row's slot, found by binary search
  // in the distinct list, or the zero row
  const uint16_t zero = uint16_t(chunk_base(uint32_t(U)));
  uint16_t* at = addr_out + tile * E * kTileRows;
  for (int e = threadIdx.x; e < n_ent; e += kPlanThreads) {
    const int k = e / kTileRows, lr = e - k * kTileRows;
    const int item = s_item[k];
    if (item < 0) continue;
    const int64_t r = r0 + lr;
    uint16_t a = zero;
    const int32_t x = r < M ? pairs[int64_t(k) * M + r] : -1;
    if (x >= 0 && x < n_src) {
      int lo = 0, hi = U;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (keys[mid] < x) lo = mid + 1;
        else hi = mid;
      }
      a = uint16_t(chunk_base(uint32_t(lo)));
    }
    const int w = lr / 64, ml = lr % 64;
    at[((item * 4 + w) * 32 + (ml % 32)) * 2 + ml / 32] = a;
  }
  // padding items: every row reads the zero row
  for (int i = threadIdx.x; i < kPad * kTileRows; i += kPlanThreads) {
    const int q = i / kTileRows, lr = i % kTileRows, w = lr / 64, ml = lr % 64;
    at[(((s_nact + q) * 4 + w) * 32 + (ml % 32)) * 2 + ml / 32] = zero;
  }
}

// Single workgroup: ascending list of the overflow tiles and their number.
__global__ __launch_bounds__(256) void plan_overflow_kernel(const int32_t* __restrict__ count,
                                                            int64_t ntiles,
                                                            int32_t* __restrict__ n_overflow,
                                                            int32_t* __restrict__ overflow) {
  __shared__ uint32_t scan_lds[256 / 64 + 1];
  uint32_t base = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += 256) {
    const int64_t t = t0 + threadIdx.x;
    const bool over = t < ntiles && count[t] >= kLdsRows;
    uint32_t total;
    const uint32_t pos = block_exclusive_scan<256>(over ? 1u : 0u, scan_lds, &total);
    if (over) overflow[base + pos] = int32_t(t);
    base += total;
  }
  if (threadIdx.x == 0) *n_overflow = int32_t(base);
}

template <int NP>
static void launch_plan(unsigned nt, hipStream_t s, const int32_t* pairs, int64_t M, int kv,
                        int64_t n_src, const PlanLayout& p, char* b) {
  plan_build_kernel<NP><<<nt, kPlanThreads, 0, s>>>(
      pairs, M, kv, n_src, reinterpret_cast<int32_t*>(b + p.count_off),
      reinterpret_cast<int32_t*>(b + p.rows_off), reinterpret_cast<int32_t*>(b + p.nact_off),
      reinterpret_cast<int32_t*>(b + p.koff_off), reinterpret_cast<uint16_t*>(b + p.addr_off),
      p.E);
}

}  // namespace sp

using namespace sp;

extern "C" {

size_t sp_gather_plan_bytes(int64_t M, int64_t kv) {
  if (kv < 1 || kv > kPlanMaxKv || M < 0) return 0;
  return plan_layout(M, kv).total;
}

int sp_gather_plan_build(const int32_t* pairs, int64_t kv, int64_t M, int64_t n_src, void* plan,
                         size_t plan_bytes, int64_t* n_overflow, void* stream) {
  SP_CHECK_ARG(kv >= 1 && kv <= kPlanMaxKv, "gather plan: kv=%lld outside 1..%d", (long long)kv,
               kPlanMaxKv);
  SP_CHECK_ARG(M >= 0 && M < (int64_t(1) << 31) && n_src >= 0 && n_src < (int64_t(1) << 31),
               "gather plan: bad sizes M=%lld n_src=%lld", (long long)M, (long long)n_src);
  SP_CHECK_ARG(n_overflow != nullptr, "gather plan: null n_overflow");
  *n_overflow = 0;
  if (M == 0) return SP_OK;
  SP_CHECK_ARG(pairs && plan, "gather plan: null pointer");
  const PlanLayout p = plan_layout(M, kv);
  if (plan_bytes < p.total)
    return set_error(SP_ERR_WORKSPACE, "gather plan: buffer %zu < %zu", plan_bytes, p.total);
  SP_CHECK_ARG(p.ntiles <= kMaxGridX, "gather plan: too many rows");
  char* b = static_cast<char*>(plan);
  int32_t* n_ovf = reinterpret_cast<int32_t*>(b);
  int32_t* count = reinterpret_cast<int32_t*>(b + p.count_off);
  int32_t* ovf = reinterpret_cast<int32_t*>(b + p.overflow_off);
  hipStream_t s = as_stream(stream);
  const unsigned nt = unsigned(p.ntiles);
  const int n_ent = kTileRows * int(kv);
  const int k = int(kv);
  if (n_ent <= 1024) launch_plan<1024>(nt, s, pairs, M, k, n_src, p, b);
  else if (n_ent <= 2048) launch_plan<2048>(nt, s, pairs, M, k, n_src, p, b);
  else if (n_ent <= 4096) launch_plan<4096>(nt, s, pairs, M, k, n_src, p, b);
  else if (n_ent <= 8192) launch_plan<8192>(nt, s, pairs, M, k, n_src, p, b);
  else launch_plan<16384>(nt, s, pairs, M, k, n_src, p, b);
  SP_LAUNCHED();
  plan_overflow_kernel<<<1, 256, 0, s>>>(count, p.ntiles, n_ovf, ovf);
  SP_LAUNCHED();
  int32_t h = 0;
  SP_HIP(hipMemcpyAsync(&h, n_ovf, sizeof(h), hipMemcpyDeviceToHost, s));
  SP_HIP(hipStreamSynchronize(s));
  *n_overflow = h;
  return SP_OK;
}

}  // extern "C"
