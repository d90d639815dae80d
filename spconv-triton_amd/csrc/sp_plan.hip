// Gather-plan builder (layout and purpose in sp_plan.h).
//
// One workgroup per tile of kTileRows output rows.  The tile's kTileRows * kv
// entries are read once into registers (thread t holds entries i * 512 + t,
// so the loads are coalesced along the rows).  The distinct valid entries are
// then found in one of two ways:
//   * bitmap (the usual case): the entries of a tile of a locality-ordered
//     table fall in a narrow window [lo, hi] of source rows.  When the window
//     fits in a bitmap in LDS, every entry sets its bit, a block scan of the
//     words' popcounts gives every word's rank offset, and the rank of a row
//     is that offset plus the popcount of the lower bits of its word: O(n)
//     work with no sort;
//   * sort (any table): the entries are sorted in LDS with a bitonic network
//     (no pair = INT32_MAX sorts last), the distinct values are compacted in
//     place, and every entry's rank is found by binary search.
// Both give U and the ascending distinct list; the tile's items are numbered
// and every (item, row) gets the staged LDS address of its rank.
// With kv above kPlanDenseKv (COMPACT) the tile's live offsets are found
// first (from the rows' mask words, or by a scan of the tile's entries that
// keeps only one bit per offset), numbered as items, and only their entries
// are read: at most kPlanMaxItems of them, in one group of kPlanGroupOffsets,
// a tile with more or spanning two groups being an overflow tile.  The GEMM
// finds a plan's overflow tiles from their counts; on request only (the host's
// row-order decisions), a second, single-workgroup kernel lists them and their
// number is copied back (one synchronisation).  The plan depends only on the
// table, so the caller builds it once per table and reuses it for every GEMM
// on that table.
#include "sp_plan.h"

namespace sp {

constexpr int kPlanThreads = 512;

template <int NP, bool COMPACT>
__global__ __launch_bounds__(kPlanThreads) void plan_build_kernel(
    const int32_t* __restrict__ pairs, int64_t M, int kv, int64_t n_src,
    int32_t* __restrict__ count, int32_t* __restrict__ rows_out, int32_t* __restrict__ nact_out,
    int32_t* __restrict__ koff_out, uint16_t* __restrict__ addr_out, int E,
    const uint32_t* __restrict__ words, int mic) {
  // sort path: the entries; bitmap path: NP / 2 bitmap words, then NP / 2
  // word rank offsets
  __shared__ int32_t keys[NP];
  __shared__ uint32_t scan_lds[kPlanThreads / 64 + 1];
  // dense: item number of offset k in the tile, or -1; COMPACT: offset of item i
  __shared__ int32_t s_item[kPlanMaxItems];
  __shared__ int32_t s_red[2][kPlanThreads / 64];
  __shared__ int32_t s_nact;
  constexpr int PER = NP / kPlanThreads;
  static_assert(PER <= 32, "first-occurrence flags are kept in one 32-bit mask");
  static_assert(kPlanDenseKv <= kPlanMaxItems && kPlanMaxItems <= 64,
                "one wave numbers the items");
  static_assert(!COMPACT || NP >= kTileRows * kPlanMaxItems, "a tile's entries fit in NP");
  constexpr int32_t kNone = 0x7fffffff;
  constexpr int kBmWords = NP / 2;
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * kTileRows;

  // live offsets: with the rows' mask words, the offsets no row of the tile
  // has are not read (dense: 2 words; COMPACT: up to kPlanMaxKv / 32)
  constexpr int kLiveWords = COMPACT ? kPlanMaxKv / 32 : 2;
  __shared__ uint32_t s_live[kLiveWords];
  const int nlw = COMPACT ? (kv + 31) / 32 : 2;
  if (tid < kPlanMaxItems) s_item[tid] = -1;
  if (tid < nlw) s_live[tid] = (words || COMPACT) ? 0u : 0xffffffffu;
  __syncthreads();
  if (words) {  // (uniform)
    const int64_t r = r0 + tid;
    if (tid < kTileRows && r < M) {
      const uint32_t* wr = words + r * int64_t(mic);
      if (COMPACT) {
        for (int j = 0; j < nlw; ++j) {
          const uint32_t w = wr[j];
          if (w) atomicOr(&s_live[j], w);
        }
      } else {
        const uint32_t w0 = wr[0], w1 = mic > 1 ? wr[1] : 0u;
        if (w0) atomicOr(&s_live[0], w0);
        if (w1) atomicOr(&s_live[1], w1);
      }
    }
    __syncthreads();
  } else if (COMPACT) {
    // scan: wave w reads offsets w / 4, w / 4 + 2, ... of its 64 rows, and
    // one lane per offset sets its bit if any of them has a pair
    const int lr = tid & (kTileRows - 1), k0 = tid / kTileRows;
    const int64_t r = r0 + lr;
    constexpr int kScanStep = kPlanThreads / kTileRows;
    constexpr int kBatch = 8;
    for (int kb = k0; kb < kv; kb += kScanStep * kBatch) {
      int32_t x[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int k = kb + j * kScanStep;
        x[j] = (k < kv && r < M) ? pairs[int64_t(k) * M + r] : -1;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int k = kb + j * kScanStep;
        const bool any = __builtin_amdgcn_ballot_w64(x[j] >= 0 && x[j] < n_src) != 0;
        if (any && (tid & 63) == 0) atomicOr(&s_live[k >> 5], 1u << (k & 31));
      }
    }
    __syncthreads();
  }
  if (COMPACT) {
    // items: the live offsets ascending, numbered by one wave (a scan of the
    // words' popcounts); more than kPlanMaxItems, or items in two groups of
    // kPlanGroupOffsets, make an overflow tile
    if (tid < 64) {
      uint32_t w = tid < nlw ? s_live[tid] : 0u;
      if (tid == nlw - 1 && (kv & 31)) w &= (1u << (kv & 31)) - 1u;
      const int c = __builtin_popcount(w);
      int incl = c;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (tid >= off) incl += o;
      }
      int pos = incl - c;
      while (w) {
        const int b = __builtin_ctz(w);
        w &= w - 1u;
        if (pos < kPlanMaxItems) s_item[pos] = tid * 32 + b;
        ++pos;
      }
      if (tid == 63) s_nact = incl;
    }
    __syncthreads();
    static_assert(kPlanMaxItems <= kPlanGroupOffsets, "items of one group");
    const int na = s_nact;
    if (na > kPlanMaxItems ||
        (na > 0 && s_item[0] / kPlanGroupOffsets != s_item[na - 1] / kPlanGroupOffsets)) {
      // (uniform) the GEMM gathers this tile directly
      if (tid == 0) count[tile] = kLdsRows;
      return;
    }
  }
  const int n_ent = kTileRows * (COMPACT ? s_nact : kv);
  // ---- entries into registers; window and items
  int32_t v[PER];
  int32_t lo = kNone, hi = -1;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = i * kPlanThreads + tid;
    int32_t key = kNone;
    if (e < n_ent) {
      const int q = e / kTileRows;  // dense: the offset; COMPACT: the item
      const int k = COMPACT ? s_item[q] : q;
      const int64_t r = r0 + (e - q * kTileRows);
      if (r < M && (COMPACT || ((s_live[k >> 5] >> (k & 31)) & 1u))) {
        const int32_t x = pairs[int64_t(k) * M + r];
        if (x >= 0 && x < n_src) {
          key = x;
          if (!COMPACT) s_item[k] = 0;  // every writer stores the same value
        }
      }
    }
    v[i] = key;
    if (key != kNone) {
      lo = key < lo ? key : lo;
      hi = key > hi ? key : hi;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int32_t ol = __shfl_xor(lo, off, 64), oh = __shfl_xor(hi, off, 64);
    lo = ol < lo ? ol : lo;
    hi = oh > hi ? oh : hi;
  }
  if ((tid & 63) == 0) {
    s_red[0][tid >> 6] = lo;
    s_red[1][tid >> 6] = hi;
  }
  __syncthreads();
  lo = kNone;
  hi = -1;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    lo = s_red[0][w] < lo ? s_red[0][w] : lo;
    hi = s_red[1][w] > hi ? s_red[1][w] : hi;
  }
  const int64_t window = hi >= 0 ? int64_t(hi) - lo + 1 : 0;
  const bool use_bitmap = window <= int64_t(kBmWords) * 32;
  uint32_t* bm = reinterpret_cast<uint32_t*>(keys);
  uint32_t* pre = bm + kBmWords;
  int32_t* rows_t = rows_out + tile * kLdsRows;
  int U;
  if (use_bitmap) {
    const int nw = int((window + 31) / 32);
    for (int w = tid; w < nw; w += kPlanThreads) bm[w] = 0u;
    __syncthreads();
    // a thread's entries are one row's neighbours, often in the same word:
    // bits of consecutive entries in one word go out as one atomic
    uint32_t pw = 0xffffffffu, pbits = 0u;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (v[i] != kNone) {
        const uint32_t d = uint32_t(v[i] - lo);
        if ((d >> 5) != pw) {
          if (pbits) atomicOr(&bm[pw], pbits);
          pw = d >> 5;
          pbits = 0u;
        }
        pbits |= 1u << (d & 31);
      }
    if (pbits) atomicOr(&bm[pw], pbits);
    __syncthreads();
    // thread t ranks words [t * wpt, (t + 1) * wpt)
    const int wpt = (nw + kPlanThreads - 1) / kPlanThreads;
    const int w0 = tid * wpt, w1 = w0 + wpt < nw ? w0 + wpt : nw;
    uint32_t cnt = 0;
    for (int w = w0; w < w1; ++w) cnt += uint32_t(__builtin_popcount(bm[w]));
    uint32_t total = 0;
    uint32_t pos = block_exclusive_scan<kPlanThreads>(cnt, scan_lds, &total);
    U = int(total);
    for (int w = w0; w < w1; ++w) {
      pre[w] = pos;
      uint32_t bits = bm[w];
      if (U < kLdsRows)
        while (bits) {
          const int b = __builtin_ctz(bits);
          bits &= bits - 1;
          rows_t[pos++] = lo + w * 32 + b;
        }
      else
        pos += uint32_t(__builtin_popcount(bits));
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) keys[i * kPlanThreads + tid] = v[i];
    __syncthreads();
    // the entries past n_ent are kNone, already in place: sort the first np2
    int np2 = 2 * kPlanThreads;
    while (np2 < n_ent) np2 <<= 1;
    for (int size = 2; size <= np2; size <<= 1) {
      for (int half = size >> 1; half > 0; half >>= 1) {
        for (int i = tid; i < np2 / 2; i += kPlanThreads) {
          const int a = 2 * i - (i & (half - 1));
          const int c = a + half;
          const bool up = (a & size) == 0;
          const int32_t x = keys[a], y = keys[c];
          if ((x > y) == up) {
            keys[a] = y;
            keys[c] = x;
          }
        }
        __syncthreads();
      }
    }
    // first occurrences of valid values; thread t owns entries [t*PER, (t+1)*PER)
    const int base = tid * PER;
    int32_t sv[PER];
    int32_t prev = base > 0 ? keys[base - 1] : kNone;
    uint32_t firsts = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      sv[i] = keys[base + i];
      if (sv[i] != kNone && sv[i] != prev) firsts |= 1u << i;
      prev = sv[i];
    }
    uint32_t total = 0;
    uint32_t pos = block_exclusive_scan<kPlanThreads>(uint32_t(__builtin_popcount(firsts)),
                                                      scan_lds, &total);
    __syncthreads();  // all entries read: compact in place (pos <= entry index)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (firsts & (1u << i)) keys[pos++] = sv[i];
    __syncthreads();
    U = int(total);
    if (U < kLdsRows)
      for (int i = tid; i < U; i += kPlanThreads) rows_t[i] = keys[i];
  }
  if (tid == 0) count[tile] = U;
  if (U >= kLdsRows) return;  // the GEMM gathers this tile straight from memory
  // the list is padded with -1 to kLdsRows entries, so that the GEMM can load
  // it without waiting for the count
  for (int i = U + tid; i < kLdsRows; i += kPlanThreads) rows_t[i] = -1;

  // items of the tile: the offsets with a pair among its rows, numbered in
  // ascending order by one wave (dense: kv <= kPlanDenseKv <= 64 lanes)
  if (COMPACT) {
    if (tid < E) koff_out[tile * E + tid] = tid < s_nact ? s_item[tid] : -1;
    if (tid == 0) nact_out[tile] = s_nact;
  } else if (tid < 64) {
    int32_t* ko = koff_out + tile * E;
    const bool live = tid < kv && s_item[tid] == 0;
    const uint64_t m = __builtin_amdgcn_ballot_w64(live);
    const int n = __popcll(m);
    if (live) {
      const int item = __popcll(m & ((uint64_t(1) << tid) - 1));
      s_item[tid] = item;
      ko[item] = tid;
    }
    if (tid >= n && tid < E) ko[tid] = -1;
    if (tid == 0) {
      s_nact = n;
      nact_out[tile] = n;
    }
  }
  __syncthreads();
  // LDS address of every (item, row): the staged slot of the row's rank, or
  // the zero row
  const uint16_t zero = uint16_t(chunk_base(uint32_t(U)));
  uint16_t* at = addr_out + tile * E * kTileRows;
  auto rec = [&](int item, int lr) -> uint16_t& {  // [item][wave][l32][mt]
    const int w = lr / 64, ml = lr % 64;
    return at[((item * 4 + w) * 32 + (ml % 32)) * 2 + ml / 32];
  };
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = i * kPlanThreads + tid;
    if (e >= n_ent) continue;
    const int q = e / kTileRows, lr = e - q * kTileRows;
    const int item = COMPACT ? q : s_item[q];
    if (item < 0) continue;
    uint16_t a = zero;
    const int32_t x = v[i];
    if (x != kNone) {
      int rank;
      if (use_bitmap) {
        const uint32_t d = uint32_t(x - lo);
        rank = int(pre[d >> 5]) + __builtin_popcount(bm[d >> 5] & ((1u << (d & 31)) - 1u));
      } else {
        int l = 0, h = U;
        while (l < h) {
          const int mid = (l + h) >> 1;
          if (keys[mid] < x) l = mid + 1;
          else h = mid;
        }
        rank = l;
      }
      a = uint16_t(chunk_base(uint32_t(rank)));
    }
    rec(item, lr) = a;
  }
  // the items that fill up the last group read the zero row
  const int n_fill = (kItemGroup - s_nact % kItemGroup) % kItemGroup;
  for (int i = tid; i < n_fill * kTileRows; i += kPlanThreads)
    rec(s_nact + i / kTileRows, i % kTileRows) = zero;
}

// Single workgroup: ascending list of the overflow tiles and their number.
// One workgroup; in each round thread i reads the counts of kOvPer consecutive
// tiles at once (16 loads in flight), so one memory round trip covers 16384
// tiles; a block scan of the threads' overflow counts places their tiles in
// ascending order.
constexpr int kOvThreads = 1024;
constexpr int kOvPer = 16;
__global__ __launch_bounds__(kOvThreads) void plan_overflow_kernel(
    const int32_t* __restrict__ count, int64_t ntiles, int32_t* __restrict__ n_overflow,
    int32_t* __restrict__ overflow) {
  __shared__ uint32_t scan_lds[kOvThreads / 64 + 1];
  static_assert(kOvPer <= 32, "a thread's overflow flags are one 32-bit mask");
  uint32_t base = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += int64_t(kOvThreads) * kOvPer) {
    const int64_t my0 = t0 + int64_t(threadIdx.x) * kOvPer;
    int32_t c[kOvPer];
#pragma unroll
    for (int j = 0; j < kOvPer; ++j) c[j] = my0 + j < ntiles ? count[my0 + j] : 0;
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < kOvPer; ++j) bits |= (c[j] >= kLdsRows ? 1u : 0u) << j;
    uint32_t total;
    uint32_t pos = block_exclusive_scan<kOvThreads>(uint32_t(__popc(bits)), scan_lds, &total);
    while (bits) {
      const int j = __builtin_ctz(bits);
      overflow[base + pos++] = int32_t(my0 + j);
      bits &= bits - 1u;
    }
    base += total;
  }
  if (threadIdx.x == 0) *n_overflow = int32_t(base);
}

// Per 256-row tile of a gather table: its pairs (valid entries), the offsets
// with a pair in the tile and the (64-row wave block, offset) pairs with a
// pair, summed into stats[0..2] (zeroed by the caller).  Measured in a given
// row order, they give the share of a GEMM's MFMA work spent on pairs: the
// staged kernel runs 256 rows per live tile offset, the direct one 64 rows
// per live wave offset.
// A workgroup takes tiles blockIdx.x, blockIdx.x + gridDim.x, ... and adds
// its totals with one atomic per counter (a few hundred atomics in all: one
// per wave and tile serialised on the three addresses for ~175 us).
__global__ __launch_bounds__(256) void table_stats_kernel(const int32_t* __restrict__ pairs,
                                                          int64_t M, int kv, int64_t n_src,
                                                          int64_t ntiles,
                                                          unsigned long long* __restrict__ stats) {
  constexpr int kMaxWords = 16;  // offsets counted per launch: kv <= 512
  __shared__ uint32_t s_or[kMaxWords];
  __shared__ uint32_t s_sum[2][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = (kv + 31) / 32;
  uint32_t npair = 0, wave_live = 0, tile_live = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r = tile * 256 + tid;
    if (tid < kMaxWords) s_or[tid] = 0u;
    __syncthreads();
    for (int w = 0; w < nw; ++w) {
      // the row's validity bits for offsets 32 w .. 32 w + 31, loads 8 at a time
      uint32_t bits = 0;
      for (int j0 = 0; j0 < 32; j0 += 8) {
        int32_t x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = 32 * w + j0 + j;
          x[j] = (r < M && k < kv) ? pairs[int64_t(k) * M + r] : -1;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (x[j] >= 0 && x[j] < n_src) bits |= 1u << (j0 + j);
      }
      npair += uint32_t(__builtin_popcount(bits));
      uint32_t any = bits;  // offsets live in the wave
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) any |= __shfl_xor(any, off, 64);
      wave_live += uint32_t(__builtin_popcount(any));
      if (lane == 0) atomicOr(&s_or[w], any);
    }
    __syncthreads();
    if (tid == 0)
      for (int w = 0; w < nw; ++w) tile_live += uint32_t(__builtin_popcount(s_or[w]));
    __syncthreads();  // s_or is cleared for the next tile
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) npair += __shfl_xor(npair, off, 64);
  if (lane == 0) {
    s_sum[0][wave] = npair;
    s_sum[1][wave] = wave_live;
  }
  __syncthreads();
  if (tid == 0) {
    unsigned long long a = 0, b = 0;
    for (int w = 0; w < 4; ++w) {
      a += s_sum[0][w];
      b += s_sum[1][w];
    }
    atomicAdd(&stats[0], a);
    atomicAdd(&stats[1], (unsigned long long)tile_live);
    atomicAdd(&stats[2], b);
  }
}

// out[k, i] = pairs[k, order[i]]: the table in a given row order (-1 where
// order[i] is not a row).
// With the rows' mask words (kv <= 32), entries whose bit is clear are -1
// without a read: the reads are random (one cache line per entry), and a
// table with few pairs per row has mostly clear bits.
__global__ __launch_bounds__(256) void permute_table_kernel(const int32_t* __restrict__ pairs,
                                                            int64_t M, int kv,
                                                            const int32_t* __restrict__ order,
                                                            const uint32_t* __restrict__ words,
                                                            int32_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= M) return;
  const int32_t src = order[i];
  const bool ok = src >= 0 && src < M;
  const uint32_t w = words ? words[i] : 0xFFFFFFFFu;
  for (int k = 0; k < kv; ++k) {
    int32_t v = -1;
    if (ok && ((w >> (k & 31)) & 1u)) v = pairs[int64_t(k) * M + src];
    out[int64_t(k) * M + i] = v;
  }
}

template <int NP, bool COMPACT = false>
static void launch_plan(unsigned nt, hipStream_t s, const int32_t* pairs, int64_t M, int kv,
                        int64_t n_src, const PlanLayout& p, char* b, const uint32_t* words,
                        int mic) {
  plan_build_kernel<NP, COMPACT><<<nt, kPlanThreads, 0, s>>>(
      pairs, M, kv, n_src, reinterpret_cast<int32_t*>(b + p.count_off),
      reinterpret_cast<int32_t*>(b + p.rows_off), reinterpret_cast<int32_t*>(b + p.nact_off),
      reinterpret_cast<int32_t*>(b + p.koff_off), reinterpret_cast<uint16_t*>(b + p.addr_off),
      p.E, words, mic);
}

// The overflow list and its count of a built plan (the build leaves them out
// unless asked: no GEMM reads them), copied back to the host (one sync).
static int list_overflow(const PlanLayout& p, const int32_t* count, int32_t* n_ovf,
                         int32_t* ovf, int64_t* n_overflow, hipStream_t s) {
  plan_overflow_kernel<<<1, kOvThreads, 0, s>>>(count, p.ntiles, n_ovf, ovf);
  SP_LAUNCHED();
  int32_t h = 0;
  SP_HIP(hipMemcpyAsync(&h, n_ovf, sizeof(h), hipMemcpyDeviceToHost, s));
  SP_HIP(hipStreamSynchronize(s));
  *n_overflow = h;
  return SP_OK;
}

}  // namespace sp

using namespace sp;

extern "C" {

size_t sp_gather_plan_bytes(int64_t M, int64_t kv) {
  if (kv < 1 || kv > kPlanMaxKv || M < 0) return 0;
  return plan_layout(M, kv).total;
}

int sp_gather_plan_build(const int32_t* pairs, int64_t kv, int64_t M, int64_t n_src,
                         const uint32_t* row_words, int32_t words_per_row, void* plan,
                         size_t plan_bytes, int64_t* n_overflow, void* stream) {
  SP_CHECK_ARG(kv >= 1 && kv <= kPlanMaxKv, "gather plan: kv=%lld outside 1..%d", (long long)kv,
               kPlanMaxKv);
  SP_CHECK_ARG(!row_words || (words_per_row >= (kv + 31) / 32 && words_per_row <= 1024),
               "gather plan: %d mask words per row for kv=%lld", words_per_row, (long long)kv);
  SP_CHECK_ARG(M >= 0 && M < (int64_t(1) << 31) && n_src >= 0 && n_src < (int64_t(1) << 31),
               "gather plan: bad sizes M=%lld n_src=%lld", (long long)M, (long long)n_src);
  if (n_overflow) *n_overflow = 0;
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
  if (kv > kPlanDenseKv)
    launch_plan<kTileRows * kPlanMaxItems, true>(nt, s, pairs, M, k, n_src, p, b, row_words,
                                                 words_per_row);
  else if (n_ent <= 1024) launch_plan<1024>(nt, s, pairs, M, k, n_src, p, b, row_words, words_per_row);
  else if (n_ent <= 2048) launch_plan<2048>(nt, s, pairs, M, k, n_src, p, b, row_words, words_per_row);
  else if (n_ent <= 4096) launch_plan<4096>(nt, s, pairs, M, k, n_src, p, b, row_words, words_per_row);
  else if (n_ent <= 8192) launch_plan<8192>(nt, s, pairs, M, k, n_src, p, b, row_words, words_per_row);
  else launch_plan<16384>(nt, s, pairs, M, k, n_src, p, b, row_words, words_per_row);
  SP_LAUNCHED();
  if (n_overflow) return list_overflow(p, count, n_ovf, ovf, n_overflow, s);
  return SP_OK;
}

int sp_gather_plan_overflow(void* plan, size_t plan_bytes, int64_t kv, int64_t M,
                            int64_t* n_overflow, void* stream) {
  SP_CHECK_ARG(n_overflow, "gather plan overflow: null count");
  *n_overflow = 0;
  SP_CHECK_ARG(kv >= 1 && kv <= kPlanMaxKv && M >= 0 && M < (int64_t(1) << 31),
               "gather plan overflow: bad sizes kv=%lld M=%lld", (long long)kv, (long long)M);
  if (M == 0) return SP_OK;
  SP_CHECK_ARG(plan, "gather plan overflow: null plan");
  const PlanLayout p = plan_layout(M, kv);
  if (plan_bytes < p.total)
    return set_error(SP_ERR_WORKSPACE, "gather plan overflow: buffer %zu < %zu", plan_bytes,
                     p.total);
  char* b = static_cast<char*>(plan);
  return list_overflow(p, reinterpret_cast<const int32_t*>(b + p.count_off),
                       reinterpret_cast<int32_t*>(b), reinterpret_cast<int32_t*>(b + p.overflow_off),
                       n_overflow, as_stream(stream));
}

int sp_table_stats(const int32_t* pairs, int64_t kv, int64_t M, int64_t n_src, int64_t* stats,
                   void* stream) {
  SP_CHECK_ARG(kv >= 1 && M >= 0 && n_src >= 0, "table stats: bad sizes");
  if (M == 0) return SP_OK;
  SP_CHECK_ARG(pairs && stats, "table stats: null pointer");
  const int64_t nt = cdiv(M, int64_t(256));
  SP_CHECK_ARG(nt <= kMaxGridX, "table stats: too many rows");
  SP_CHECK_ARG(kv <= 512, "table stats: kv=%lld above 512", (long long)kv);
  const unsigned grid = unsigned(nt < 512 ? nt : 512);
  table_stats_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      pairs, M, int(kv), n_src, nt, reinterpret_cast<unsigned long long*>(stats));
  SP_LAUNCHED();
  return SP_OK;
}

int sp_permute_table(const int32_t* pairs, int64_t kv, int64_t M, const int32_t* order,
                     const uint32_t* order_words, int32_t* out, void* stream) {
  SP_CHECK_ARG(kv >= 1 && M >= 0, "permute table: bad sizes");
  if (M == 0) return SP_OK;
  SP_CHECK_ARG(pairs && order && out, "permute table: null pointer");
  SP_CHECK_ARG(!order_words || kv <= 32, "permute table: mask words need kv <= 32, not %lld",
               (long long)kv);
  const int64_t nb = cdiv(M, int64_t(256));
  SP_CHECK_ARG(nb <= kMaxGridX && kv < 65536, "permute table: too many rows");
  permute_table_kernel<<<unsigned(nb), 256, 0, as_stream(stream)>>>(pairs, M, int(kv), order,
                                                                     order_words, out);
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
