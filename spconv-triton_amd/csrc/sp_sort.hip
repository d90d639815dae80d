// Stable LSD radix sort and the mask-word split/sort entry point.
//
// Digits are up to kRsMaxBits = 9 bits wide: a sort over B key bits takes
// ceil(B / 9) passes with the bits spread evenly over them (27-bit mask words:
// 3 passes of 9 bits; 32-bit keys: 4 of 8).  A pass costs about the same at
// 8 or 9 bits, and for these sizes (10^5 - 10^6 items) its cost is mostly
// latency, so fewer passes is what pays.
//
// Tile layout: a workgroup of 512 threads (8 waves) owns a tile of 2048
// consecutive items, visited in 4 rounds; in round r wave w holds items
// [r*512 + w*64, +64).  The 32 (round, wave) segments are in item order, so a
// per-digit exclusive scan over them plus the in-wave peer rank gives a stable
// local rank.  Global placement of digit d of tile b: all items with a smaller
// digit plus the items of digit d in tiles before b.  Up to kRsFusedTiles
// tiles, the histograms are stored tile-major and every scatter workgroup
// sums them itself (coalesced rows, 32 tiles per memory round trip, then a
// block scan), so a pass is two launches; above that they are stored
// digit-major, one workgroup per digit scans its row over the tiles in place
// and writes the digit's total, and every scatter workgroup scans the 512
// totals itself: three launches.  The
// first pass of a row sort generates the row indices itself.
#include "sp_sort.h"

namespace sp {

constexpr int kRsThreads = 512;
constexpr int kRsRounds = 4;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsTile = kRsThreads * kRsRounds;  // 2048
constexpr int kRsMaxBits = 9;
constexpr int kRsMaxRadix = 1 << kRsMaxBits;             // 512
constexpr int kRsSegs = kRsRounds * kRsWaves;  // 32: segment r * kRsWaves + wave
constexpr int64_t kRsFusedTiles = 128;
static_assert(kRsTile < 65536, "segment counts are stored as uint16");

// The scatters drop a position outside 0..n-1 instead of writing it (which
// needs inconsistent histograms, i.e. a bug), and count it here, so a sort
// that lost items is reported (sp_sort_dropped_positions) rather than leaving
// holes unnoticed.  One counter per device.
__device__ unsigned long long g_sort_drops = 0;

struct RowWordDigit {
  const uint32_t* words;
  int mic;
  int w;
  uint32_t andmask;
  int shift;
  uint32_t dmask;
  __device__ __forceinline__ uint32_t operator()(uint32_t row) const {
    return ((words[int64_t(row) * mic + w] & andmask) >> shift) & dmask;
  }
};

struct KeyDigit32 {
  int shift;
  uint32_t dmask;
  __device__ __forceinline__ uint32_t operator()(uint32_t k) const { return (k >> shift) & dmask; }
};

struct KeyDigit64 {
  int shift;
  uint32_t dmask;
  __device__ __forceinline__ uint32_t operator()(uint64_t k) const {
    return uint32_t(k >> shift) & dmask;
  }
};

// Lanes of the wave holding the same digit of `db` bits (restricted to `active`).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t active, int db) {
  uint64_t peers = active;
#pragma unroll
  for (int b = 0; b < kRsMaxBits; ++b) {
    if (b < db) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
  }
  return peers;
}

// Item idx of a pass: in[idx], or idx itself when in is null (the first pass
// of a row sort).
template <class Item>
__device__ __forceinline__ Item rs_item(const Item* __restrict__ in, int64_t idx) {
  return in ? in[idx] : Item(idx);
}

template <class Item, class Digit>
__global__ __launch_bounds__(kRsThreads) void rs_hist(const Item* __restrict__ in, int64_t n,
                                                     Digit dig, int db,
                                                     uint32_t* __restrict__ hist, int64_t ntiles) {
  __shared__ uint32_t cnt[kRsMaxRadix];
  const int R = 1 << db;
  for (int i = threadIdx.x; i < R; i += kRsThreads) cnt[i] = 0;
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = int64_t(blockIdx.x) * kRsTile;
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    const bool valid = idx < n;
    const uint32_t d = valid ? dig(rs_item(in, idx)) : 0u;
    const uint64_t peers = match_digit(d, __ballot(valid), db);
    if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&cnt[d], uint32_t(__popcll(peers)));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < R; i += kRsThreads) {
    if (ntiles <= kRsFusedTiles)
      hist[int64_t(blockIdx.x) * R + i] = cnt[i];  // [tile][digit]
    else
      hist[int64_t(i) * ntiles + blockIdx.x] = cnt[i];  // [digit][tile]
  }
}

// Placement of this tile's digits from tile-major histograms, into
// tile_base[0..R).  Thread t owns digit t (R <= kRsMaxRadix == kRsThreads), so
// a wave reads 256 consecutive bytes of a histogram row; 64 tiles per memory
// round trip.
static_assert(kRsMaxRadix <= kRsThreads, "one digit per thread in fused_tile_base");
__device__ __forceinline__ void fused_tile_base(const uint32_t* __restrict__ hist, int64_t ntiles,
                                                int R, uint32_t* tile_base, uint32_t* scan_lds) {
  constexpr int kBatch = 64;
  const int64_t me = blockIdx.x;
  uint32_t tot = 0, pre = 0;
  const int d = int(threadIdx.x);
  for (int64_t b = 0; b < ntiles; b += kBatch) {
    uint32_t h[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) h[u] = (b + u < ntiles && d < R) ? hist[(b + u) * R + d] : 0u;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      tot += h[u];
      pre += b + u < me ? h[u] : 0u;
    }
  }
  uint32_t all = 0;
  const uint32_t run = block_exclusive_scan<kRsThreads>(tot, scan_lds, &all);
  if (d < R) tile_base[d] = run + pre;
}

// Digit-major histograms [R][ntiles]: exclusive scan of digit blockIdx.x's
// row over the tiles, in place, and the digit's total.
constexpr int kDsThreads = 256;
constexpr int kDsPer = 8;  // consecutive tiles per thread and round
__global__ __launch_bounds__(kDsThreads) void rs_digit_prefix(uint32_t* __restrict__ hist,
                                                             int64_t ntiles,
                                                             uint32_t* __restrict__ totals) {
  __shared__ uint32_t scan_lds[kDsThreads / 64 + 1];
  uint32_t* row = hist + int64_t(blockIdx.x) * ntiles;
  uint32_t base = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += int64_t(kDsThreads) * kDsPer) {
    const int64_t my0 = t0 + int64_t(threadIdx.x) * kDsPer;
    uint32_t v[kDsPer];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kDsPer; ++j) {
      v[j] = my0 + j < ntiles ? row[my0 + j] : 0u;
      sum += v[j];
    }
    uint32_t tot;
    uint32_t run = base + block_exclusive_scan<kDsThreads>(sum, scan_lds, &tot);
#pragma unroll
    for (int j = 0; j < kDsPer; ++j) {
      if (my0 + j < ntiles) row[my0 + j] = run;
      run += v[j];
    }
    base += tot;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = base;
}

template <class Item, class Digit>
__global__ __launch_bounds__(kRsThreads) void rs_scatter(const Item* __restrict__ in,
                                                        Item* __restrict__ out, int64_t n,
                                                        Digit dig, int db,
                                                        const uint32_t* __restrict__ offsets,
                                                        const uint32_t* __restrict__ totals,
                                                        int64_t ntiles) {
  __shared__ __align__(16) uint16_t seg[kRsSegs][kRsMaxRadix];
  __shared__ uint32_t tile_base[kRsMaxRadix];
  __shared__ uint32_t scan_lds[kRsThreads / 64 + 1];
  const int R = 1 << db;
  for (int i = threadIdx.x; i < kRsSegs * kRsMaxRadix / 8; i += kRsThreads)
    reinterpret_cast<uint4*>(&seg[0][0])[i] = make_uint4(0u, 0u, 0u, 0u);
  // the tile's items and digits first: their loads overlap the histogram
  // loads of the placement below
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = int64_t(blockIdx.x) * kRsTile;
  Item items[kRsRounds];
  uint32_t digits[kRsRounds];
  uint32_t ranks[kRsRounds];
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    items[r] = idx < n ? rs_item(in, idx) : Item(0);
  }
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    digits[r] = idx < n ? dig(items[r]) : 0u;
  }
  if (ntiles <= kRsFusedTiles) {
    // (the barriers of its block scan also order the zeroing of seg before
    // the segment counts below)
    fused_tile_base(offsets, ntiles, R, tile_base, scan_lds);
  } else {
    // digit d's items start after all items of smaller digits (a block scan of
    // the totals; thread d owns digit d) and after its items in earlier tiles
    const int d = int(threadIdx.x);
    const uint32_t t = d < R ? totals[d] : 0u;
    const uint32_t pre = d < R ? offsets[int64_t(d) * ntiles + blockIdx.x] : 0u;
    uint32_t all = 0;
    const uint32_t below = block_exclusive_scan<kRsThreads>(t, scan_lds, &all);
    if (d < R) tile_base[d] = below + pre;
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    const bool valid = idx < n;
    const uint32_t d = digits[r];
    const uint64_t peers = match_digit(d, __ballot(valid), db);
    const uint64_t below = peers & lanemask_lt();
    ranks[r] = uint32_t(__popcll(below));
    if (valid && below == 0) seg[r * kRsWaves + wave][d] = uint16_t(__popcll(peers));
  }
  __syncthreads();
  // per digit, exclusive scan over the 32 segments (all 32 reads in flight)
  for (int d = threadIdx.x; d < R; d += kRsThreads) {
    uint32_t c[kRsSegs];
#pragma unroll
    for (int sgi = 0; sgi < kRsSegs; ++sgi) c[sgi] = seg[sgi][d];
    uint32_t run = 0;
#pragma unroll
    for (int sgi = 0; sgi < kRsSegs; ++sgi) {
      seg[sgi][d] = uint16_t(run);
      run += c[sgi];
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    if (idx < n) {
      const uint32_t d = digits[r];
      const uint32_t pos = tile_base[d] + seg[r * kRsWaves + wave][d] + ranks[r];
      if (pos < uint64_t(n))
        out[pos] = items[r];
      else
        atomicAdd(&g_sort_drops, 1ull);  // never for consistent counts
    }
  }
}

struct RsBuffers {
  uint32_t* hist;
  uint32_t* totals;  // kRsMaxRadix digit totals (digit-major histograms)
};

static size_t rs_hist_words(int64_t n) {
  return size_t(kRsMaxRadix) * size_t(cdiv(n, kRsTile));
}

// One pass over the digit dig (db bits).  in == nullptr: the items are the
// indices 0..n-1.
template <class Item, class Digit>
static int radix_pass(const Item* in, Item* out, int64_t n, Digit dig, int db, const RsBuffers& b,
                      hipStream_t s) {
  const int64_t ntiles = cdiv(n, kRsTile);
  SP_CHECK_ARG(ntiles <= kMaxGridX, "radix sort: %lld items exceed the grid limit", (long long)n);
  rs_hist<Item, Digit><<<dim3(unsigned(ntiles)), dim3(kRsThreads), 0, s>>>(in, n, dig, db,
                                                                          b.hist, ntiles);
  SP_LAUNCHED();
  if (ntiles > kRsFusedTiles) {
    rs_digit_prefix<<<dim3(1u << db), dim3(kDsThreads), 0, s>>>(b.hist, ntiles, b.totals);
    SP_LAUNCHED();
  }
  rs_scatter<Item, Digit><<<dim3(unsigned(ntiles)), dim3(kRsThreads), 0, s>>>(
      in, out, n, dig, db, b.hist, b.totals, ntiles);
  SP_LAUNCHED();
  return SP_OK;
}

// Digit widths of a sort over `bits` key bits: ceil(bits / 9) passes with the
// bits spread evenly (widths differ by at most one, wider first).
static int digit_plan(int bits, int* widths) {
  if (bits <= 0) return 0;
  const int passes = (bits + kRsMaxBits - 1) / kRsMaxBits;
  for (int i = 0; i < passes; ++i) widths[i] = bits / passes + (i < bits % passes ? 1 : 0);
  return passes;
}

template <class W>
static void rows_layout(W& w, int64_t n) {
  w.template take<uint32_t>(size_t(n));                  // perm A
  w.template take<uint32_t>(size_t(n));                  // perm B
  w.template take<uint32_t>(rs_hist_words(n));           // histograms
  w.template take<uint32_t>(size_t(kRsMaxRadix));         // digit totals
}

size_t sort_rows_ws_bytes(int64_t n) {
  WsSizer z;
  rows_layout(z, n);
  return z.off;
}

__global__ void iota_u32(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = uint32_t(i);
}

int sort_rows_by_words(const uint32_t* words, int64_t n, int mic, int kv, uint32_t split,
                       uint32_t** perm_out, void* ws, hipStream_t stream) {
  WsCursor c(ws, ~size_t(0));
  uint32_t* a = c.take<uint32_t>(size_t(n));
  uint32_t* b = c.take<uint32_t>(size_t(n));
  RsBuffers bufs;
  bufs.hist = c.take<uint32_t>(rs_hist_words(n));
  bufs.totals = c.take<uint32_t>(size_t(kRsMaxRadix));
  bool first = true;  // the first pass reads the identity permutation implicitly
  for (int w = 0; w < mic; ++w) {
    int bits = (w < mic - 1) ? 32 : kv - 32 * (mic - 1);
    uint32_t andmask = 0xFFFFFFFFu;
    if (w == 0) {
      andmask = split;
      const int top = split ? 32 - __builtin_clz(split) : 0;
      bits = bits < top ? bits : top;
    }
    int widths[8];
    const int passes = digit_plan(bits, widths);
    int shift = 0;
    for (int i = 0; i < passes; ++i) {
      RowWordDigit d{words, mic, w, andmask, shift, (1u << widths[i]) - 1u};
      int rc = radix_pass(first ? static_cast<const uint32_t*>(nullptr) : a, b, n, d, widths[i],
                          bufs, stream);
      if (rc) return rc;
      first = false;
      shift += widths[i];
      uint32_t* t = a;
      a = b;
      b = t;
    }
  }
  if (first) {  // nothing to sort by: the identity permutation
    iota_u32<<<dim3(unsigned(cdiv(n, 256))), dim3(256), 0, stream>>>(a, n);
    SP_LAUNCHED();
  }
  *perm_out = a;
  return SP_OK;
}

template <class W>
static void keys_layout(W& w, int64_t n) {
  w.template take<uint32_t>(rs_hist_words(n));
  w.template take<uint32_t>(size_t(kRsMaxRadix));  // digit totals
}

size_t sort_keys_ws_bytes(int64_t n) {
  WsSizer z;
  keys_layout(z, n);
  return z.off;
}

template <class Item, class Digit>
static int sort_keys_impl(Item* keys, Item* tmp, int64_t n, int bits, Item** result, void* ws,
                          hipStream_t stream) {
  WsCursor c(ws, ~size_t(0));
  RsBuffers bufs;
  bufs.hist = c.take<uint32_t>(rs_hist_words(n));
  bufs.totals = c.take<uint32_t>(size_t(kRsMaxRadix));
  Item* a = keys;
  Item* b = tmp;
  int widths[8];
  const int passes = digit_plan(bits, widths);
  int shift = 0;
  for (int i = 0; i < passes; ++i) {
    int rc = radix_pass(a, b, n, Digit{shift, (1u << widths[i]) - 1u}, widths[i], bufs, stream);
    if (rc) return rc;
    shift += widths[i];
    Item* t = a;
    a = b;
    b = t;
  }
  *result = a;
  return SP_OK;
}

int sort_keys_u32(uint32_t* keys, uint32_t* tmp, int64_t n, int bits, uint32_t** result,
                  void* ws, hipStream_t stream) {
  return sort_keys_impl<uint32_t, KeyDigit32>(keys, tmp, n, bits, result, ws, stream);
}

int sort_keys_u64(uint64_t* keys, uint64_t* tmp, int64_t n, int bits, uint64_t** result,
                  void* ws, hipStream_t stream) {
  return sort_keys_impl<uint64_t, KeyDigit64>(keys, tmp, n, bits, result, ws, stream);
}

// pair_mask[i, w] = words[perm[i], w] (word 0 ANDed with split), argsort[i] = perm[i].
__global__ void mask_gather(const uint32_t* __restrict__ words, const uint32_t* __restrict__ perm,
                            int64_t n, int mic, uint32_t split, int32_t* __restrict__ pm,
                            int32_t* __restrict__ args) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t row = perm ? perm[i] : uint32_t(i);
  args[i] = int32_t(row);
  for (int w = 0; w < mic; ++w) {
    uint32_t v = words[int64_t(row) * mic + w];
    if (w == 0) v &= split;
    pm[i * mic + w] = int32_t(v);
  }
}

// ---- sort of single-word masks ------------------------------------------------
// The mask sort of tables with kv <= 32 (one word per row): the items are
// (key, row) pairs carried from pass to pass, so no pass gathers the words
// through a permutation, and the last pass writes pair_mask and argsort itself
// (no separate gather).  A pass is three launches: the tiles' histograms,
// stored digit-major; rs_digit_prefix (one workgroup per digit: the digit's
// exclusive prefix over the tiles, in place, and its total); the scatter, whose
// workgroups read their own 512 prefixes and the 512 totals.  (Measured on the
// 200k-row metric table, 3 passes: with tile-major histograms summed by every
// scatter workgroup itself, two launches a pass, each scatter took 15 us
// instead of 7.4 and the sort 63 us instead of 55: 98 workgroups each reading
// all 98 tiles' histograms cost more than a launch.  Adding the next pass's
// histogram into global memory from each scatter with atomics, to save the
// histogram launches, measured slower still: 27 us per scatter, the cross-XCD
// atomics costing more than the launches they save.)
constexpr int kMsMaxPasses = 4;

template <bool kFirst>
__global__ __launch_bounds__(kRsThreads) void ms_hist(const uint32_t* __restrict__ words,
                                                     uint32_t split,
                                                     const uint32_t* __restrict__ keys_in,
                                                     int64_t n, int shift, int db,
                                                     uint32_t* __restrict__ hist, int64_t ntiles) {
  __shared__ uint32_t cnt[kRsMaxRadix];
  for (int i = threadIdx.x; i < kRsMaxRadix; i += kRsThreads) cnt[i] = 0;
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = int64_t(blockIdx.x) * kRsTile;
  const uint32_t dmask = (1u << db) - 1u;
  uint32_t keys[kRsRounds];
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    keys[r] = idx < n ? (kFirst ? words[idx] & split : keys_in[idx]) : 0u;
  }
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    const bool valid = idx < n;
    const uint32_t d = (keys[r] >> shift) & dmask;
    const uint64_t peers = match_digit(d, __ballot(valid), db);
    if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&cnt[d], uint32_t(__popcll(peers)));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kRsMaxRadix; i += kRsThreads)
    hist[int64_t(i) * ntiles + blockIdx.x] = cnt[i];  // [digit][tile]
}

template <bool kFirst, bool kLast>
__global__ __launch_bounds__(kRsThreads) void ms_scatter(
    const uint32_t* __restrict__ words, uint32_t split, const uint32_t* __restrict__ keys_in,
    const uint32_t* __restrict__ rows_in, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ rows_out, int32_t* __restrict__ pm_out, int32_t* __restrict__ ar_out,
    int64_t n, int shift, int db, const uint32_t* __restrict__ hist,
    const uint32_t* __restrict__ totals, int64_t ntiles) {
  __shared__ __align__(16) uint16_t seg[kRsSegs][kRsMaxRadix];
  __shared__ uint32_t tile_base[kRsMaxRadix];
  __shared__ uint32_t scan_lds[kRsThreads / 64 + 1];
  const uint32_t dmask = (1u << db) - 1u;
  for (int i = threadIdx.x; i < kRsSegs * kRsMaxRadix / 8; i += kRsThreads)
    reinterpret_cast<uint4*>(&seg[0][0])[i] = make_uint4(0u, 0u, 0u, 0u);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = int64_t(blockIdx.x) * kRsTile;
  uint32_t keys[kRsRounds], rows[kRsRounds], digits[kRsRounds], ranks[kRsRounds];
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    const bool valid = idx < n;
    if (kFirst) {
      keys[r] = valid ? words[idx] & split : 0u;
      rows[r] = uint32_t(idx);
    } else {
      keys[r] = valid ? keys_in[idx] : 0u;
      rows[r] = valid ? rows_in[idx] : 0u;
    }
  }
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) digits[r] = (keys[r] >> shift) & dmask;
  // (the barriers of its block scan also order the zeroing of seg before
  // the segment counts below)
  {
    const int d = int(threadIdx.x);
    const uint32_t t = totals[d];
    const uint32_t pre = hist[int64_t(d) * ntiles + blockIdx.x];
    uint32_t all = 0;
    const uint32_t below = block_exclusive_scan<kRsThreads>(t, scan_lds, &all);
    tile_base[d] = below + pre;
  }
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    const bool valid = idx < n;
    const uint64_t peers = match_digit(digits[r], __ballot(valid), db);
    const uint64_t below = peers & lanemask_lt();
    ranks[r] = uint32_t(__popcll(below));
    if (valid && below == 0) seg[r * kRsWaves + wave][digits[r]] = uint16_t(__popcll(peers));
  }
  __syncthreads();
  for (int d = threadIdx.x; d < (1 << db); d += kRsThreads) {
    uint32_t c[kRsSegs];
#pragma unroll
    for (int sgi = 0; sgi < kRsSegs; ++sgi) c[sgi] = seg[sgi][d];
    uint32_t run = 0;
#pragma unroll
    for (int sgi = 0; sgi < kRsSegs; ++sgi) {
      seg[sgi][d] = uint16_t(run);
      run += c[sgi];
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRsRounds; ++r) {
    const int64_t idx = base + r * kRsThreads + wave * 64 + lane;
    if (idx < n) {
      const uint32_t d = digits[r];
      const uint32_t pos = tile_base[d] + seg[r * kRsWaves + wave][d] + ranks[r];
      if (pos >= uint64_t(n)) {  // never for consistent counts
        atomicAdd(&g_sort_drops, 1ull);
        continue;
      }
      if (kLast) {
        pm_out[pos] = int32_t(keys[r]);
        ar_out[pos] = int32_t(rows[r]);
      } else {
        keys_out[pos] = keys[r];
        rows_out[pos] = rows[r];
      }
    }
  }
}

template <class W>
static void mask_fused_layout(W& w, int64_t n) {
  for (int i = 0; i < 4; ++i) w.template take<uint32_t>(size_t(n));  // keys/rows ping-pong
  w.template take<uint32_t>(size_t(kRsMaxRadix) * size_t(cdiv(n, kRsTile)));  // tile histograms
  w.template take<uint32_t>(size_t(kRsMaxRadix));  // digit totals
}

static size_t mask_fused_ws_bytes(int64_t n) {
  WsSizer z;
  mask_fused_layout(z, n);
  return z.off;
}

// Whether sp_mask_sort takes this path (single words).
static bool mask_fused_ok(int64_t n, int mic) { return mic == 1 && cdiv(n, kRsTile) <= kMaxGridX; }

static int sort_masks_fused(const uint32_t* words, int64_t n, int kv, uint32_t split,
                            int32_t* pm, int32_t* ar, void* ws, hipStream_t s) {
  WsCursor c(ws, ~size_t(0));
  uint32_t* ka = c.take<uint32_t>(size_t(n));
  uint32_t* ra = c.take<uint32_t>(size_t(n));
  uint32_t* kb = c.take<uint32_t>(size_t(n));
  uint32_t* rb = c.take<uint32_t>(size_t(n));
  const int64_t ntiles = cdiv(n, kRsTile);
  uint32_t* hist = c.take<uint32_t>(size_t(kRsMaxRadix) * size_t(ntiles));
  uint32_t* totals = c.take<uint32_t>(size_t(kRsMaxRadix));
  int bits = kv;
  const int top = split ? 32 - __builtin_clz(split) : 0;
  bits = bits < top ? bits : top;
  int widths[8];
  const int passes = digit_plan(bits, widths);
  if (passes == 0) {  // nothing to sort by: the identity permutation
    mask_gather<<<dim3(unsigned(cdiv(n, 256))), dim3(256), 0, s>>>(words, nullptr, n, 1, split,
                                                                   pm, ar);
    SP_LAUNCHED();
    return SP_OK;
  }
  SP_CHECK_ARG(passes <= kMsMaxPasses, "mask sort: %d passes", passes);
  const dim3 grid{unsigned(ntiles), 1u, 1u}, block{unsigned(kRsThreads), 1u, 1u};
  int shift = 0;
  const uint32_t *kin = nullptr, *rin = nullptr;
  uint32_t *kout = ka, *rout = ra;
  for (int p = 0; p < passes; ++p) {
    const bool first = p == 0, last = p + 1 == passes;
    if (first)
      ms_hist<true><<<grid, block, 0, s>>>(words, split, nullptr, n, shift, widths[p], hist,
                                           ntiles);
    else
      ms_hist<false><<<grid, block, 0, s>>>(nullptr, 0u, kin, n, shift, widths[p], hist, ntiles);
    SP_LAUNCHED();
    rs_digit_prefix<<<dim3(unsigned(kRsMaxRadix)), dim3(kDsThreads), 0, s>>>(hist, ntiles, totals);
    SP_LAUNCHED();
    auto kern = first ? (last ? ms_scatter<true, true> : ms_scatter<true, false>)
                      : (last ? ms_scatter<false, true> : ms_scatter<false, false>);
    kern<<<grid, block, 0, s>>>(words, split, kin, rin, kout, rout, pm, ar, n, shift, widths[p],
                                hist, totals, ntiles);
    SP_LAUNCHED();
    shift += widths[p];
    kin = kout;
    rin = rout;
    kout = kout == ka ? kb : ka;
    rout = rout == ra ? rb : ra;
  }
  return SP_OK;
}

}  // namespace sp

using namespace sp;

extern "C" {

int sp_sort_dropped_positions(uint64_t* count, int32_t reset) {
  SP_CHECK_ARG(count, "sort drops: null pointer");
  // sorts may still run on any stream of the current device (torch's side
  // streams do not synchronise with the null stream): wait for all of them
  SP_HIP(hipDeviceSynchronize());
  unsigned long long v = 0;
  SP_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_sort_drops), sizeof(v)));
  *count = uint64_t(v);
  if (reset) {
    const unsigned long long zero = 0;
    SP_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_sort_drops), &zero, sizeof(zero)));
  }
  return SP_OK;
}

size_t sp_mask_sort_workspace_size(int64_t n, int32_t mic) {
  const int64_t m = n > 0 ? n : 1;
  const size_t a = sort_rows_ws_bytes(m);
  const size_t b = mask_fused_ok(m, mic) ? mask_fused_ws_bytes(m) : 0;
  return a > b ? a : b;
}

int sp_mask_sort(const uint32_t* words, int64_t n, int32_t mic, int32_t kv, uint32_t split_mask,
                 int32_t do_sort, int32_t* pair_mask, int32_t* argsort, void* ws, size_t ws_bytes,
                 void* stream) {
  hipStream_t s = as_stream(stream);
  SP_CHECK_ARG(n >= 0 && mic >= 1 && kv >= 1 && kv <= 32 * mic, "mask_sort: bad sizes n=%lld mic=%d kv=%d",
               (long long)n, mic, kv);
  if (n == 0) return SP_OK;
  SP_CHECK_ARG(words && pair_mask && argsort, "mask_sort: null pointer");
  SP_CHECK_ARG(n < (int64_t(1) << 31), "mask_sort: n too large");
  uint32_t* perm = nullptr;
  if (do_sort && mask_fused_ok(n, mic)) {
    const size_t need = mask_fused_ws_bytes(n);
    if (ws_bytes < need || !ws)
      return set_error(SP_ERR_WORKSPACE, "mask_sort: workspace %zu < %zu", ws_bytes, need);
    return sort_masks_fused(words, n, kv, split_mask, pair_mask, argsort, ws, s);
  }
  if (do_sort) {
    if (ws_bytes < sort_rows_ws_bytes(n) || !ws)
      return set_error(SP_ERR_WORKSPACE, "mask_sort: workspace %zu < %zu", ws_bytes,
                       sort_rows_ws_bytes(n));
    int rc = sort_rows_by_words(words, n, mic, kv, split_mask, &perm, ws, s);
    if (rc) return rc;
  }
  mask_gather<<<dim3(unsigned(cdiv(n, 256))), dim3(256), 0, s>>>(words, perm, n, mic, split_mask,
                                                                 pair_mask, argsort);
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
