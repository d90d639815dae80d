// Rulebook (pair) generation for submanifold, regular and transposed sparse
// convolution on gfx950.
//
// The reference finds neighbours by sorting the input keys and binary
// searching every (offset, point) candidate (spconv_triton/pytorch/_impl/
// pairs.py:196-220, pair_kernels.py:298-482).  Here the coordinates go into a
// lookup structure instead -- for subm a dense cell -> row grid (small key
// volumes) or a brick index (4-cell bricks in an open-addressing hash, each
// with an occupancy mask and a popcount-ranked row list); for regular and
// transposed convs an occupancy bitmap or an open-addressing hash of the
// output keys (32-bit keys packed with their row into one 64-bit slot, or
// 64-bit keys with a side array of rows) -- and every output row probes its kv
// neighbours directly ("output stationary"): each thread owns one row and
// writes column r of every offset row of the table, so the stores of a wave
// are contiguous, and the per-row offset bitmask comes out of the same loop in
// registers.
//
// Output order is the reference's, bit for bit:
//  * subm: output rows are the input rows (pairs.py:400-401);
//  * regular/transpose: output rows are the unique candidate keys in ascending
//    batch-major order (torch.unique, pairs.py:206-219) -- a radix sort of the
//    deduplicated keys restores that order, and the sorted position of each key
//    is written back into its hash slot as its output row.
#include <type_traits>

#include "sp_common.h"
#include "sp_hash.h"
#include "sp_sort.h"

namespace sp {

// ---------------------------------------------------------------------------
// geometry
// ---------------------------------------------------------------------------
// Division of n < 2^31 by a fixed divisor 1 <= d < 2^31 as a multiply-high
// and a shift (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994): with l = ceil(log2 d) and m = ceil(2^(31+l) / d),
// floor(n * m / 2^(31+l)) = floor(n / d) for every n < 2^31, because
// m * d - 2^(31+l) < d <= 2^l keeps the error term n * (m * d - 2^(31+l)) /
// 2^(31+l) below 1 - (n mod d) / d.  For d >= 2, d > 2^(l-1) gives m < 2^32,
// so the quotient is umulhi(n, m) >> (l - 1); d = 1 is the identity (m = 0
// marks it).  The int32-key paths divide only such values (strides, output
// extents): two instructions instead of a 32-bit division routine.
struct Div31 {
  uint32_t m;  // 0: d = 1
  int sh;
};

static Div31 make_div31(uint32_t d) {
  if (d <= 1) return Div31{0u, 0};
  int l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  return Div31{uint32_t(((uint64_t(1) << (31 + l)) + d - 1) / d), l - 1};
}

__device__ __forceinline__ uint32_t div31(uint32_t n, const Div31& q) {
  return q.m ? (__umulhi(n, q.m) >> q.sh) : n;
}

struct GeomDev {
  int ndim;
  int mode;
  int kv;
  int64_t batch;
  int64_t in_shape[4];
  int64_t out_shape[4];
  int32_t ks[4], st[4], pad[4], dil[4];
  Div31 st_div[4], out_div[4];  // for values below 2^31 (int32-key paths)
};

static int64_t prod_shape(const int64_t* s, int ndim) {
  int64_t p = 1;
  for (int d = 0; d < ndim; ++d) p *= s[d];
  return p;
}

static int make_geom(const sp_geom* g, GeomDev* out) {
  SP_CHECK_ARG(g != nullptr, "geometry is null");
  SP_CHECK_ARG(g->ndim >= 1 && g->ndim <= 4, "ndim %d not in 1..4", g->ndim);
  SP_CHECK_ARG(g->mode >= SP_PAIR_SUBM && g->mode <= SP_PAIR_TRANSPOSE, "bad mode %d", g->mode);
  SP_CHECK_ARG(g->batch_size >= 1, "batch_size %lld < 1", (long long)g->batch_size);
  GeomDev d{};
  d.ndim = g->ndim;
  d.mode = g->mode;
  d.batch = g->batch_size;
  int64_t kv = 1;
  for (int i = 0; i < g->ndim; ++i) {
    SP_CHECK_ARG(g->ksize[i] >= 1, "ksize[%d]=%d < 1", i, g->ksize[i]);
    SP_CHECK_ARG(g->dilation[i] >= 1, "dilation[%d] < 1", i);
    SP_CHECK_ARG(g->in_shape[i] >= 1 && g->out_shape[i] >= 1, "shape[%d] must be >= 1", i);
    d.in_shape[i] = g->in_shape[i];
    d.out_shape[i] = g->out_shape[i];
    d.ks[i] = g->ksize[i];
    d.dil[i] = g->dilation[i];
    if (g->mode == SP_PAIR_SUBM) {
      SP_CHECK_ARG(g->ksize[i] % 2 == 1, "subm needs odd kernel sizes");
      SP_CHECK_ARG(g->out_shape[i] == g->in_shape[i], "subm out_shape must equal in_shape");
      d.pad[i] = (g->ksize[i] / 2) * g->dilation[i];
      d.st[i] = 1;
    } else {
      SP_CHECK_ARG(g->stride[i] >= 1, "stride[%d] < 1", i);
      d.pad[i] = g->padding[i];
      d.st[i] = g->stride[i];
    }
    kv *= g->ksize[i];
    d.st_div[i] = make_div31(uint32_t(d.st[i]));
    d.out_div[i] = make_div31(uint32_t(d.out_shape[i] < (int64_t(1) << 31) ? d.out_shape[i] : 1));
  }
  SP_CHECK_ARG(kv <= 4096, "kernel volume %lld too large", (long long)kv);
  d.kv = int(kv);
  *out = d;
  return SP_OK;
}

static bool need_key64(const GeomDev& g) {
  // pairs.py:166-171 -- int32 keys iff batch * volume < 2^31
  const double lim = 2147483648.0;
  double vo = double(g.batch);
  double vi = double(g.batch);
  for (int d = 0; d < g.ndim; ++d) {
    vo *= double(g.out_shape[d]);
    vi *= double(g.in_shape[d]);
  }
  if (g.mode == SP_PAIR_SUBM) vo = vo > vi ? vo : vi;
  return vo >= lim;
}

static int bit_length_u64(uint64_t v) { return v ? 64 - __builtin_clzll(v) : 0; }

// ---------------------------------------------------------------------------
// coordinate helpers
// ---------------------------------------------------------------------------
struct Coord {
  int64_t b;
  int64_t x[4];
  bool ok;  // batch and coordinates inside [0, batch) x [0, shape)
};

__device__ __forceinline__ Coord load_coord(const int32_t* __restrict__ idx, int64_t row,
                                            const GeomDev& g) {
  Coord c;
  const int32_t* p = idx + row * (g.ndim + 1);
  c.b = p[0];
  c.ok = c.b >= 0 && c.b < g.batch;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < g.ndim) {
      c.x[d] = p[d + 1];
      c.ok = c.ok && c.x[d] >= 0 && c.x[d] < g.in_shape[d];
    }
  }
  return c;
}

// Candidate output key for (offset odometer `off`, input coordinate c)
// following pair_kernels.py:76-91; returns false when geometrically invalid.
// I = int32_t when every key and coordinate fits in 31 bits (int32 keys):
// the stride division is then a 32-bit one, several times cheaper than the
// 64-bit routine.
template <typename I = int64_t>
__device__ __forceinline__ bool candidate_key(const GeomDev& g, const Coord& c, const int* off,
                                              uint64_t* key) {
  using U = std::make_unsigned_t<I>;
  U acc = U(c.b);  // unsigned: wraps (defined) for invalid candidates
  bool ok = c.ok;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < g.ndim) {
      const I koff = I(off[d]) * I(g.dil[d]);
      const I x = I(c.x[d]);
      I o;
      if (g.mode == SP_PAIR_TRANSPOSE) {
        o = x * I(g.st[d]) - I(g.pad[d]) + koff;
      } else {
        const I num = x + I(g.pad[d]) - koff;
        if (g.st[d] == 1) {
          o = num;
        } else {
          const U st = U(g.st[d]);
          U q;
          if constexpr (sizeof(I) == 4)  // num < 2^31: the multiply-shift division
            q = U(div31(uint32_t(num >= 0 ? num : 0), g.st_div[d]));
          else
            q = U(num >= 0 ? num : 0) / st;
          ok = ok && num >= 0 && U(num) == q * st;
          o = num >= 0 ? I(q) : I(-1);
        }
      }
      ok = ok && o >= 0 && o < I(g.out_shape[d]);
      acc = acc * U(g.out_shape[d]) + U(o);
    }
  }
  *key = uint64_t(acc);
  return ok;
}

// Input key of the k-th neighbour feeding output coordinate c (subm):
// x_in = x_out - pad + off*dil (the inverse of the subm candidate formula).
__device__ __forceinline__ bool subm_source_key(const GeomDev& g, const Coord& c, const int* off,
                                                uint64_t* key) {
  int64_t acc = c.b;
  bool ok = c.ok;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < g.ndim) {
      const int64_t q = c.x[d] - g.pad[d] + int64_t(off[d]) * g.dil[d];
      ok = ok && q >= 0 && q < g.in_shape[d];
      acc = acc * g.in_shape[d] + q;
    }
  }
  *key = uint64_t(acc);
  return ok;
}

// Integer type of a table's keys: Table32 holds keys below 2^31.
template <class Table>
using KeyInt = std::conditional_t<std::is_same_v<Table, Table32>, int32_t, int64_t>;

// (unrolled to 4 with a guard, so that `off` stays in registers)
__device__ __forceinline__ void odometer_next(const GeomDev& g, int (&off)[4]) {
  bool carry = true;
#pragma unroll
  for (int d = 3; d >= 0; --d) {
    if (d < g.ndim && carry) {
      if (++off[d] < g.ks[d]) carry = false;
      else off[d] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// subm
// ---------------------------------------------------------------------------
// ---- subm on a dense grid ---------------------------------------------------
// When the key volume is small next to the number of rows, a dense cell -> row
// array replaces the hash: filling it is cheaper than hashing, every probe is
// one load, and the neighbours of consecutive rows share cache lines.  The
// probe issues its loads in batches with no dependence between them (the
// hash's probe chains serialise each thread's kv lookups).  Same results as
// the hash: an empty cell holds kNoRow, and a cell held by several rows keeps
// the smallest (atomicMin, like Table32/Table64::insert).
constexpr int64_t kDenseMaxCells = int64_t(1) << 26;  // 256 MiB of int32
constexpr int64_t kDenseCellsPerRow = 256;            // beyond this the fill costs more
constexpr int32_t kNoRow = 0x7fffffff;
constexpr int kDenseBatch = 9;                        // probe loads in flight per thread

static bool subm_dense(const GeomDev& g, int64_t n) {
  const double vol = double(g.batch) * double(prod_shape(g.in_shape, g.ndim));
  return vol <= double(kDenseMaxCells) && vol <= double(kDenseCellsPerRow) * double(n);
}

static int64_t subm_cells(const GeomDev& g) { return g.batch * prod_shape(g.in_shape, g.ndim); }

// 16-byte stores: the grid is the only large fill of a dense build.
__global__ __launch_bounds__(256) void fill_i32x4(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t n4 = n / 4;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  int4* q = reinterpret_cast<int4*>(p);
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride)
    q[i] = make_int4(v, v, v, v);
  const int64_t t = n4 * 4 + int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < n) p[t] = v;
}

__global__ __launch_bounds__(256) void subm_insert_dense(const int32_t* __restrict__ idx,
                                                         int64_t n, GeomDev g,
                                                         int32_t* __restrict__ grid) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  Coord c = load_coord(idx, r, g);
  if (!c.ok) return;
  int64_t acc = c.b;
#pragma unroll
  for (int d = 0; d < 4; ++d)  // (unrolled: c.x stays in registers)
    if (d < g.ndim) acc = acc * g.in_shape[d] + c.x[d];
  atomicMin(&grid[acc], int32_t(r));
}

// subm_probe with the dense grid: the same outputs.
__global__ __launch_bounds__(256) void subm_probe_dense(const int32_t* __restrict__ idx,
                                                        int64_t n, GeomDev g,
                                                        const int32_t* __restrict__ grid,
                                                        int32_t* __restrict__ pf,
                                                        int32_t* __restrict__ pb,
                                                        uint32_t* __restrict__ words, int mic) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const Coord c = load_coord(idx, r, g);
  int off[4] = {0, 0, 0, 0};
  uint32_t word = 0;
  for (int k0 = 0; k0 < g.kv; k0 += kDenseBatch) {
    int32_t v[kDenseBatch];
#pragma unroll
    for (int u = 0; u < kDenseBatch; ++u) {
      uint64_t key;
      v[u] = kNoRow;
      if (k0 + u < g.kv) {
        if (subm_source_key(g, c, off, &key)) v[u] = grid[key];
        odometer_next(g, off);
      }
    }
#pragma unroll
    for (int u = 0; u < kDenseBatch; ++u) {
      const int k = k0 + u;
      if (k < g.kv) {
        const int32_t j = v[u] == kNoRow ? -1 : v[u];
        if (pf) pf[int64_t(k) * n + r] = j;
        if (pb) pb[int64_t(g.kv - 1 - k) * n + r] = j;
        if (j >= 0) word |= 1u << (k & 31);
        if ((k & 31) == 31 || k == g.kv - 1) {
          if (words) words[r * mic + (k >> 5)] = word;
          word = 0;
        }
      }
    }
  }
}

// ---- dense-grid probe with per-offset tables ---------------------------------
// The same outputs as subm_probe_dense, in 32-bit arithmetic (a dense grid has
// at most kDenseMaxCells < 2^31 cells): the kernel window's per-dimension
// displacements and linear key displacements are tabulated once per workgroup
// in LDS, so a lookup is a bounds test per dimension and one load, and all of a
// row's lookups (up to kProbeBatch) are in flight together.
//
// EPOCH grids hold stamped cells, (epoch << 24) | (0xFFFFFF - row): a cell is
// occupied in this build iff its stamp is the build's epoch (the caller keeps
// the grid between builds and moves to a new epoch for each, so cells of
// earlier builds read as empty with no fill), and atomicMax on the stamp keeps
// the smallest row of a cell, as atomicMin does on a filled grid.
constexpr int kProbeMaxKv = 512;  // a multiple of kProbeBatch
constexpr int64_t kGridPad = 4;  // cells before a grid's first and after its last one
constexpr int kProbeBatch = 32;
constexpr int32_t kStampRowBits = 24;
constexpr int32_t kStampRowMask = (1 << kStampRowBits) - 1;

__device__ __forceinline__ bool grid_base(const int32_t* __restrict__ idx, int32_t r,
                                          const GeomDev& g, int32_t (&x)[4], int32_t* base) {
  // every load first, then the checks (short-circuit tests between the loads
  // would wait for each one in turn); bitwise &, not &&, for the same reason
  const int32_t* p = idx + int64_t(r) * (g.ndim + 1);
  int32_t c[5];
  c[0] = p[0];
#pragma unroll
  for (int d = 0; d < 4; ++d) c[d + 1] = d < g.ndim ? p[d + 1] : 0;
  bool ok = (c[0] >= 0) & (c[0] < int32_t(g.batch));
  int32_t acc = c[0];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    x[d] = c[d + 1];
    if (d < g.ndim) {
      ok = ok & (uint32_t(x[d]) < uint32_t(g.in_shape[d]));
      acc = acc * int32_t(g.in_shape[d]) + x[d];
    }
  }
  *base = acc;
  return ok;
}

template <bool EPOCH>
__global__ __launch_bounds__(256) void subm_insert_grid(const int32_t* __restrict__ idx,
                                                        int32_t n, GeomDev g,
                                                        int32_t* __restrict__ grid,
                                                        uint32_t epoch) {
  const int32_t r = int32_t(blockIdx.x) * int32_t(blockDim.x) + int32_t(threadIdx.x);
  if (r >= n) return;
  int32_t x[4], key;
  if (!grid_base(idx, r, g, x, &key)) return;
  if (EPOCH)
    atomicMax(reinterpret_cast<uint32_t*>(grid) + key,
              (epoch << kStampRowBits) | uint32_t(kStampRowMask - r));
  else
    atomicMin(grid + key, r);
}

// RUN = 3 (last kernel dimension 3 wide, dilation 1): the three cells of a
// run of offsets along the last dimension are adjacent in the grid and come
// in one 12-byte load, which touches one or two cache lines where three 4-byte
// loads touch up to three: with the rows of a wave spread over many grid lines,
// the number of lines a load instruction touches is what the lookups cost.
// RUN = 1: one cell per load, any window.  A grid buffer holds kGridPad cells
// before cell 0 and after the last cell (`grid` points at cell 0), so a run's
// load starts and ends inside the buffer: a buffer load starting out of range
// reads zeros in all three lanes, in range or not.
template <bool EPOCH, int RUN>
__global__ __launch_bounds__(256) void subm_probe_grid(
    const int32_t* __restrict__ idx, int32_t n, GeomDev g, const int32_t* __restrict__ grid,
    uint32_t grid_bytes, uint32_t epoch, int32_t* __restrict__ pf, int32_t* __restrict__ pb,
    uint32_t* __restrict__ words, int mic, int32_t* __restrict__ npl) {
  static_assert(RUN == 1 || RUN == 3, "runs of 1 or 3 cells");
  constexpr int kRunBatch = kProbeBatch / RUN;  // runs per batch of lookups
  // per run: displacement of its first cell per dimension and linear
  // displacement; the runs past the last one, up to a whole batch, fail every
  // bounds test, so the lookup loop runs whole batches without a branch
  __shared__ int32_t s_lin[kProbeMaxKv];
  __shared__ int32_t s_disp[kProbeMaxKv][4];
  const int kv = g.kv;
  const int nruns = kv / RUN;
  const int nrb = (nruns + kRunBatch - 1) / kRunBatch * kRunBatch;
  for (int j = threadIdx.x; j < nrb; j += blockDim.x) {
    int rem = j * RUN, lin = 0, stride = 1;
    int disp[4] = {0, 0, 0, 0};
    for (int d = g.ndim - 1; d >= 0; --d) {
      const int o = rem % g.ks[d];
      rem /= g.ks[d];
      disp[d] = j < nruns ? o * g.dil[d] - g.pad[d] : int(g.in_shape[d]);  // padding: out of range
      lin += disp[d] * stride;
      stride *= int(g.in_shape[d]);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) s_disp[j][d] = disp[d];
    s_lin[j] = lin;
  }
  if (npl && blockIdx.x == 0)
    for (int k = threadIdx.x; k < kv; k += blockDim.x) npl[k] = 0;
  __syncthreads();
  const int32_t r = int32_t(blockIdx.x) * int32_t(blockDim.x) + int32_t(threadIdx.x);
  if (r >= n) return;
  int32_t x[4], base;
  const bool ok = grid_base(idx, r, g, x, &base);
  uint32_t shape[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) shape[d] = d < g.ndim ? uint32_t(g.in_shape[d]) : 1u;
  const int last = g.ndim - 1;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(grid - kGridPad), (short)0, int(grid_bytes), 0x00020000);
  uint32_t word = 0;
  for (int j0 = 0; j0 < nruns; j0 += kRunBatch) {
    int32_t v[kRunBatch][RUN];
    bool in[kRunBatch][RUN];
#pragma unroll
    for (int u = 0; u < kRunBatch; ++u) {
      const int j = j0 + u;
      // all dimensions but the run's own (the last one, when RUN > 1)
      bool b = ok;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        if (RUN == 1 || d != last) b = b & (uint32_t(x[d] + s_disp[j][d]) < shape[d]);
      const uint32_t off =
          b ? uint32_t(base + s_lin[j] + int32_t(kGridPad)) * 4u : 0xFFFFFFF0u;  // else 0s
      if constexpr (RUN == 3) {
        const auto t3 = __builtin_amdgcn_raw_buffer_load_b96(rg, off, 0, 0);
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          v[u][t] = int32_t(t3[t]);
          in[u][t] = b & (uint32_t(x[last] + s_disp[j][last] + t) < shape[last]);
        }
      } else {
        v[u][0] = int32_t(__builtin_amdgcn_raw_buffer_load_b32(rg, off, 0, 0));
        in[u][0] = b;
      }
    }
#pragma unroll
    for (int u = 0; u < kRunBatch; ++u) {
#pragma unroll
      for (int t = 0; t < RUN; ++t) {
        const int k = (j0 + u) * RUN + t;
        if (k < kv) {
          int32_t jr;
          if (EPOCH)
            jr = in[u][t] && (uint32_t(v[u][t]) >> kStampRowBits) == epoch
                     ? kStampRowMask - (v[u][t] & kStampRowMask)
                     : -1;
          else
            jr = in[u][t] && v[u][t] != kNoRow ? v[u][t] : -1;
          if (pf) pf[int64_t(k) * n + r] = jr;
          if (pb) pb[int64_t(kv - 1 - k) * n + r] = jr;
          if (jr >= 0) word |= 1u << (k & 31);
          if ((k & 31) == 31 || k == kv - 1) {
            if (words) words[int64_t(r) * mic + (k >> 5)] = word;
            word = 0;
          }
        }
      }
    }
  }
}

// Whether the probe takes runs of 3 cells along the last dimension.
static bool probe_runs3(const GeomDev& g) {
  return g.ks[g.ndim - 1] == 3 && g.dil[g.ndim - 1] == 1;
}

template <bool EPOCH>
static int launch_probe_grid(const int32_t* idx, int64_t n, const GeomDev& d,
                             const int32_t* grid, int64_t cells, uint32_t epoch, int32_t* pf,
                             int32_t* pb, uint32_t* words, int mic, int32_t* npl, hipStream_t s) {
  const unsigned blocks = unsigned(cdiv(n, 256));
  const uint32_t bytes = uint32_t((cells + 2 * kGridPad) * 4);  // the whole buffer
  if (probe_runs3(d))
    subm_probe_grid<EPOCH, 3><<<blocks, 256, 0, s>>>(idx, int32_t(n), d, grid, bytes, epoch, pf,
                                                     pb, words, mic, npl);
  else
    subm_probe_grid<EPOCH, 1><<<blocks, 256, 0, s>>>(idx, int32_t(n), d, grid, bytes, epoch, pf,
                                                     pb, words, mic, npl);
  SP_LAUNCHED();
  return SP_OK;
}

// ---------------------------------------------------------------------------
// regular / transpose
// ---------------------------------------------------------------------------
struct ConvWs {
  int* flags;          // [0] overflow
  uint32_t* counter;   // number of unique keys
  void* table_a;       // Table32 slots or Table64 keys
  int32_t* table_vals; // Table64 rows
  void* list;          // unique keys (u32 or u64)
  void* tmp;           // radix-sort ping-pong buffer
  void* sort_ws;
  uint64_t cap;
  int64_t bound;
};

static int64_t conv_bound(const GeomDev& g, int64_t n) {
  // unique outputs <= min(kv * n, batch * prod(out_shape))
  double a = double(g.kv) * double(n);
  double b = double(g.batch) * double(prod_shape(g.out_shape, g.ndim));
  double m = a < b ? a : b;
  return int64_t(m < 1.0 ? 1.0 : m);
}

static uint64_t table_capacity(int64_t items) {
  uint64_t want = uint64_t(items) * 2;
  uint64_t cap = 1024;
  while (cap < want) cap <<= 1;
  return cap;
}

template <class W>
static void conv_layout(W& w, const GeomDev& g, int64_t n, bool key64, ConvWs* out) {
  const int64_t bound = conv_bound(g, n);
  const uint64_t cap = table_capacity(bound);
  auto* flags = w.template take<int>(64);
  auto* counter = w.template take<uint32_t>(64);
  void* ta = w.template take<uint64_t>(cap);
  int32_t* tv = key64 ? w.template take<int32_t>(cap) : nullptr;
  void* list = key64 ? (void*)w.template take<uint64_t>(size_t(bound))
                     : (void*)w.template take<uint32_t>(size_t(bound));
  void* tmp = key64 ? (void*)w.template take<uint64_t>(size_t(bound))
                    : (void*)w.template take<uint32_t>(size_t(bound));
  void* sws = w.template take<char>(sort_keys_ws_bytes(bound));
  if (out) {
    out->flags = flags;
    out->counter = counter;
    out->table_a = ta;
    out->table_vals = tv;
    out->list = list;
    out->tmp = tmp;
    out->sort_ws = sws;
    out->cap = cap;
    out->bound = bound;
  }
}

// ---- subm on a brick index (key volumes a dense grid does not fit) ----------
// Above the dense grid's limits, every row's kv neighbours were separate
// lookups in a coordinate hash, each a random probe chain: config 5 case 1
// (4-D, ~500k rows, kv = 81) took 689 us for its rulebook probe.  Here the
// coordinates are grouped into bricks of 4 cells along each of the last
// min(ndim, 3) dimensions (at most 64 cells, one 64-bit occupancy mask), and
// only bricks are hashed:
//   * insert: every row sets its cell's bit in its brick's mask (the brick is
//     inserted into the hash on first sight; its slot holds the mask);
//   * bases: each slot's first entry in a compact row array, from a block scan
//     of the masks' popcounts (one atomic per workgroup places the blocks:
//     the positions depend on the order they run in, the lookups do not);
//   * scatter: every row writes itself at base + popcount(mask below its
//     cell), keeping the smallest row of a repeated coordinate (atomicMin, the
//     rule of the other lookup structures);
//   * probe: a row's window, 3 cells wide per dimension for a 3^D kernel,
//     touches 1-2 bricks per bricked dimension; they are looked up once per
//     slice of the leading (unbricked) dimensions into a per-thread LDS cache
//     (at most kBrickWindow bricks; wider windows look each brick up as the
//     offsets reach it, keeping the last one), and each offset is a bit test
//     and a popcount rank.
// Same results as the hash and the grid, bit for bit.
constexpr int kBrickWindow = 8;  // bricks cached per row and leading slice

struct BrickDev {
  int nb;              // trailing dimensions cut into bricks of 4 cells
  int64_t bshape[4];   // bricks per dimension (ceil(shape / 4) bricked, else shape)
  uint64_t* masks;     // [cap] occupancy of the brick in hash slot s (bit = cell)
  uint32_t* base;      // [cap] first entry of the slot's cells in rows
  int32_t* rows;       // [n] row of each occupied cell
  uint32_t* total;     // occupied cells (the base scan's running total)
};

static BrickDev brick_geom(const GeomDev& g) {
  BrickDev b{};
  b.nb = g.ndim < 3 ? g.ndim : 3;
  for (int d = 0; d < g.ndim; ++d)
    b.bshape[d] = d >= g.ndim - b.nb ? (g.in_shape[d] + 3) / 4 : g.in_shape[d];
  return b;
}

// Brick volume (keys of the brick hash are below it).
static double brick_volume(const GeomDev& g) {
  const BrickDev b = brick_geom(g);
  double v = double(g.batch);
  for (int d = 0; d < g.ndim; ++d) v *= double(b.bshape[d]);
  return v;
}

// Brick key and cell of an in-range coordinate.
__device__ __forceinline__ void brick_of(const GeomDev& g, const BrickDev& bd, const Coord& c,
                                         uint64_t* bkey, uint32_t* cell) {
  int64_t acc = c.b;
  uint32_t cl = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < g.ndim) {
      const bool bricked = d >= g.ndim - bd.nb;
      acc = acc * bd.bshape[d] + (bricked ? (c.x[d] >> 2) : c.x[d]);
      if (bricked) cl = cl * 4u + uint32_t(c.x[d] & 3);
    }
  }
  *bkey = uint64_t(acc);
  *cell = cl;
}

__global__ __launch_bounds__(256) void brick_fill(uint64_t* __restrict__ table, uint64_t cap,
                                                  uint64_t* __restrict__ masks,
                                                  int32_t* __restrict__ rows, int64_t n,
                                                  uint32_t* __restrict__ total,
                                                  uint32_t* __restrict__ words, int64_t n_words) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (uint64_t(i) < cap) {
    table[i] = kEmpty64;
    masks[i] = 0;
  }
  if (i < n) rows[i] = kNoRow;
  if (i < n_words) words[i] = 0;  // (the slice-parallel probe ORs into them)
  if (i == 0) *total = 0;
}

template <class Table>
__global__ __launch_bounds__(256) void brick_insert(const int32_t* __restrict__ idx, int64_t n,
                                                    GeomDev g, Table t, BrickDev bd) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const Coord c = load_coord(idx, r, g);
  if (!c.ok) return;
  uint64_t bkey;
  uint32_t cell;
  brick_of(g, bd, c, &bkey, &cell);
  const int64_t s = t.insert_slot(bkey);
  if (s >= 0) atomicOr(reinterpret_cast<unsigned long long*>(&bd.masks[s]), 1ull << cell);
}

constexpr int kBasePer = 8;  // slots per thread of brick_bases
__global__ __launch_bounds__(256) void brick_bases(BrickDev bd, uint64_t cap) {
  __shared__ uint32_t scan_lds[256 / 64 + 1];
  __shared__ uint32_t s_first;
  const uint64_t s0 = (uint64_t(blockIdx.x) * 256 + threadIdx.x) * kBasePer;
  uint32_t cnt[kBasePer];
  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < kBasePer; ++j) {
    cnt[j] = s0 + j < cap ? uint32_t(__popcll(bd.masks[s0 + j])) : 0u;
    sum += cnt[j];
  }
  uint32_t tot;
  uint32_t run = block_exclusive_scan<256>(sum, scan_lds, &tot);
  if (threadIdx.x == 0) s_first = atomicAdd(bd.total, tot);
  __syncthreads();
  run += s_first;
#pragma unroll
  for (int j = 0; j < kBasePer; ++j) {
    if (s0 + j < cap) bd.base[s0 + j] = run;
    run += cnt[j];
  }
}

template <class Table>
__global__ __launch_bounds__(256) void brick_scatter(const int32_t* __restrict__ idx, int64_t n,
                                                     GeomDev g, Table t, BrickDev bd) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const Coord c = load_coord(idx, r, g);
  if (!c.ok) return;
  uint64_t bkey;
  uint32_t cell;
  brick_of(g, bd, c, &bkey, &cell);
  const int64_t s = t.find_slot(bkey);
  if (s < 0) return;  // (never: every row's brick was inserted)
  const uint32_t pos =
      bd.base[s] + uint32_t(__popcll(bd.masks[s] & ((uint64_t(1) << cell) - 1u)));
  atomicMin(&bd.rows[pos], int32_t(r));
}

// One thread per output row, as subm_probe; the same outputs.  Latency is
// what bounds a probe (its loads are random), so no load waits for another:
// the hash lookups of a slice's window bricks have their home slots in
// flight together, and the offsets go in batches of kBrickBatch whose rows'
// positions come from the LDS cache first, then all their row loads, then
// their stores.
constexpr int kBrickBatch = 9;

template <class Table>
__global__ __launch_bounds__(256) void brick_probe(const int32_t* __restrict__ idx, int64_t n,
                                                   GeomDev g, Table t, BrickDev bd,
                                                   int32_t* __restrict__ pf,
                                                   int32_t* __restrict__ pb,
                                                   uint32_t* __restrict__ words, int mic) {
  __shared__ uint64_t s_mask[kBrickWindow][256];
  __shared__ uint32_t s_base[kBrickWindow][256];
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;  // (no barrier below: every LDS slot belongs to one thread)
  const int tid = threadIdx.x;
  const Coord c = load_coord(idx, r, g);
  const int lead = g.ndim - bd.nb;
  // the window's bricks along each bricked dimension: lo[d] .. lo[d] + nw[d] - 1
  // (every loop over dimensions is unrolled to 4 with a guard, so the small
  // arrays stay in registers)
  int64_t lo[4] = {0, 0, 0, 0};
  int nw[4] = {1, 1, 1, 1};
  int W = 1;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < g.ndim && d >= lead) {
      const int64_t c0 = c.x[d] - g.pad[d];
      const int64_t c1 = c0 + int64_t(g.ks[d] - 1) * g.dil[d];
      lo[d] = c0 >> 2;  // floor (arithmetic shift)
      nw[d] = int((c1 >> 2) - lo[d] + 1);
      W *= nw[d];
    }
  }
  const bool cached = W <= kBrickWindow;
  // brick key of brick coordinates bc (cell coordinates in the leading
  // dimensions), or false when out of range
  auto brick_key = [&](const int64_t (&bc)[4], uint64_t* key) -> bool {
    int64_t acc = c.b;
    bool ok = c.ok;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      if (d < g.ndim) {
        ok = ok && bc[d] >= 0 && bc[d] < bd.bshape[d];
        acc = acc * bd.bshape[d] + bc[d];
      }
    }
    *key = uint64_t(acc);
    return ok;
  };
  // the window's bricks of the leading slice holding cell coordinates q into
  // the LDS cache; their lookups overlap
  auto fill_window = [&](const int64_t (&q)[4]) {
    uint64_t key[kBrickWindow], w[kBrickWindow];
    bool ok[kBrickWindow];
#pragma unroll
    for (int e = 0; e < kBrickWindow; ++e) {
      int64_t bc[4] = {0, 0, 0, 0};
      int rem = e;
#pragma unroll
      for (int dd = 3; dd >= 0; --dd) {
        if (dd < g.ndim) {
          if (dd >= lead) {
            bc[dd] = lo[dd] + rem % nw[dd];
            rem /= nw[dd];
          } else {
            bc[dd] = q[dd];
          }
        }
      }
      ok[e] = e < W && brick_key(bc, &key[e]);
      w[e] = ok[e] ? t.word(t.home(key[e])) : kEmpty64;
    }
    int64_t slot[kBrickWindow];
#pragma unroll
    for (int e = 0; e < kBrickWindow; ++e)
      slot[e] = ok[e] ? t.find_from(t.home(key[e]), w[e], key[e]) : -1;
#pragma unroll
    for (int e = 0; e < kBrickWindow; ++e) {
      if (e < W) {
        s_mask[e][tid] = slot[e] >= 0 ? bd.masks[slot[e]] : 0ull;
        s_base[e][tid] = slot[e] >= 0 ? bd.base[slot[e]] : 0u;
      }
    }
  };
  // offsets per leading slice (the bricked dimensions' kernel volume)
  int kvb = 1;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    if (d < g.ndim && d >= lead) kvb *= g.ks[d];
  int off[4] = {0, 0, 0, 0};
  uint64_t last_key = ~uint64_t(0), last_mask = 0;  // the uncached path's one-brick cache
  uint32_t last_base = 0;
  uint32_t word = 0;
  int k = 0;
  for (int sl = 0; sl < g.kv / kvb; ++sl) {
    if (cached) {  // the slice's window bricks (off holds its leading offsets, the rest 0)
      int64_t q[4] = {0, 0, 0, 0};
#pragma unroll
      for (int d = 0; d < 4; ++d)
        if (d < g.ndim) q[d] = c.x[d] - g.pad[d] + int64_t(off[d]) * g.dil[d];
      fill_window(q);
    }
    for (int b0 = 0; b0 < kvb; b0 += kBrickBatch) {
      int32_t pos[kBrickBatch];  // entry of the batch's offsets in bd.rows, or -1
#pragma unroll
      for (int i = 0; i < kBrickBatch; ++i) {
        pos[i] = -1;
        if (b0 + i < kvb) {
          int64_t q[4] = {0, 0, 0, 0};
          bool ok = c.ok;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            if (d < g.ndim) {
              q[d] = c.x[d] - g.pad[d] + int64_t(off[d]) * g.dil[d];
              ok = ok && q[d] >= 0 && q[d] < g.in_shape[d];
            }
          }
          if (ok) {
            uint32_t cell = 0;
            int e = 0;
            int64_t bc[4] = {0, 0, 0, 0};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              if (d < g.ndim) {
                if (d >= lead) {
                  cell = cell * 4u + uint32_t(q[d] & 3);
                  e = e * nw[d] + int((q[d] >> 2) - lo[d]);
                  bc[d] = q[d] >> 2;
                } else {
                  bc[d] = q[d];
                }
              }
            }
            uint64_t m;
            uint32_t bs;
            if (cached) {
              m = s_mask[e][tid];
              bs = s_base[e][tid];
            } else {
              uint64_t key;
              brick_key(bc, &key);
              if (key != last_key) {
                const int64_t sk = t.find_slot(key);
                last_mask = sk >= 0 ? bd.masks[sk] : 0ull;
                last_base = sk >= 0 ? bd.base[sk] : 0u;
                last_key = key;
              }
              m = last_mask;
              bs = last_base;
            }
            if ((m >> cell) & 1u)
              pos[i] = int32_t(bs + uint32_t(__popcll(m & ((uint64_t(1) << cell) - 1u))));
          }
          odometer_next(g, off);
        }
      }
      int32_t j[kBrickBatch];
#pragma unroll
      for (int i = 0; i < kBrickBatch; ++i) j[i] = pos[i] >= 0 ? bd.rows[pos[i]] : -1;
#pragma unroll
      for (int i = 0; i < kBrickBatch; ++i) {
        if (b0 + i < kvb) {
          if (pf) pf[int64_t(k) * n + r] = j[i];
          if (pb) pb[int64_t(g.kv - 1 - k) * n + r] = j[i];
          if (j[i] >= 0) word |= 1u << (k & 31);
          if ((k & 31) == 31 || k == g.kv - 1) {
            if (words) words[r * mic + (k >> 5)] = word;
            word = 0;
          }
          ++k;
        }
      }
    }
  }
}

// brick_probe for the usual window: 3 cells (dilation 1) along each of the
// three bricked dimensions, NDIM = 3, or 4 with any leading kernel size and
// dilation.  The window's per-dimension cells (valid, cell in brick, which of
// its 1-2 bricks) are computed once per row, so each of a slice's 27 offsets
// is a handful of register operations; the same outputs.  NDIM = 4: one
// thread per (leading slice, row), slice-major, so that the kernel keeps the
// 3-D instance's registers (a loop over the slices in one thread needed 232
// VGPRs); the threads of a row OR their bits into its mask words, which
// brick_fill zeroed.
template <class Table, int NDIM>
__global__ __launch_bounds__(256) void brick_probe3(const int32_t* __restrict__ idx, int64_t n,
                                                    GeomDev g, Table t, BrickDev bd,
                                                    int32_t* __restrict__ pf,
                                                    int32_t* __restrict__ pb,
                                                    uint32_t* __restrict__ words, int mic) {
  static_assert(NDIM == 3 || NDIM == 4, "three bricked dimensions, at most one leading");
  constexpr int LEAD = NDIM - 3;
  __shared__ uint64_t s_mask[kBrickWindow][256];
  __shared__ uint32_t s_base[kBrickWindow][256];
  const int ns = LEAD ? g.ks[0] : 1;  // leading slices
  const int64_t tg = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tg >= n * ns) return;  // (no barrier below: every LDS slot belongs to one thread)
  const int64_t r = LEAD ? tg % n : tg;
  const int sl = LEAD ? int(tg / n) : 0;
  const int tid = threadIdx.x;
  const Coord c = load_coord(idx, r, g);
  // per bricked dimension d and window position o (cell x - 1 + o): in range,
  // cell index in its brick, and whether it lies in the window's second brick
  int64_t lo[3];
  int nw[3];
  bool vin[3][3];
  uint32_t cc[3][3], eb[3][3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const int64_t x = c.x[LEAD + d];
    lo[d] = (x - 1) >> 2;
    nw[d] = int(((x + 1) >> 2) - lo[d] + 1);
#pragma unroll
    for (int o = 0; o < 3; ++o) {
      const int64_t v = x - 1 + o;
      vin[d][o] = v >= 0 && v < g.in_shape[LEAD + d];
      cc[d][o] = uint32_t(v & 3);
      eb[d][o] = uint32_t((v >> 2) - lo[d]);
    }
  }
  uint32_t word = 0;
  {
    int64_t q0 = 0;
    bool slice_ok = c.ok;
    if (LEAD) {
      q0 = c.x[0] - g.pad[0] + int64_t(sl) * g.dil[0];
      slice_ok = slice_ok && q0 >= 0 && q0 < g.in_shape[0];
    }
    // the slice's window bricks (i, j, l) in {0, 1}^3 into the LDS cache
    {
      uint64_t key[kBrickWindow], w[kBrickWindow];
      bool ok[kBrickWindow];
#pragma unroll
      for (int e = 0; e < kBrickWindow; ++e) {
        const int i = e >> 2, j = (e >> 1) & 1, l = e & 1;
        const int64_t b0 = lo[0] + i, b1 = lo[1] + j, b2 = lo[2] + l;
        ok[e] = slice_ok && i < nw[0] && j < nw[1] && l < nw[2] && b0 >= 0 &&
                b0 < bd.bshape[LEAD] && b1 >= 0 && b1 < bd.bshape[LEAD + 1] && b2 >= 0 &&
                b2 < bd.bshape[LEAD + 2];
        int64_t acc = c.b;
        if (LEAD) acc = acc * bd.bshape[0] + q0;
        acc = ((acc * bd.bshape[LEAD] + b0) * bd.bshape[LEAD + 1] + b1) * bd.bshape[LEAD + 2] +
              b2;
        key[e] = uint64_t(acc);
        w[e] = ok[e] ? t.word(t.home(key[e])) : kEmpty64;
      }
      int64_t slot[kBrickWindow];
#pragma unroll
      for (int e = 0; e < kBrickWindow; ++e)
        slot[e] = ok[e] ? t.find_from(t.home(key[e]), w[e], key[e]) : -1;
#pragma unroll
      for (int e = 0; e < kBrickWindow; ++e) {
        s_mask[e][tid] = slot[e] >= 0 ? bd.masks[slot[e]] : 0ull;
        s_base[e][tid] = slot[e] >= 0 ? bd.base[slot[e]] : 0u;
      }
    }
    // the 27 offsets, 9 at a time (one plane of the first bricked dimension)
#pragma unroll
    for (int oz = 0; oz < 3; ++oz) {
      int32_t pos[9];
#pragma unroll
      for (int oy = 0; oy < 3; ++oy) {
#pragma unroll
        for (int ox = 0; ox < 3; ++ox) {
          const bool ok = slice_ok && vin[0][oz] && vin[1][oy] && vin[2][ox];
          const uint32_t cell = cc[0][oz] * 16u + cc[1][oy] * 4u + cc[2][ox];
          const uint32_t e = eb[0][oz] * 4u + eb[1][oy] * 2u + eb[2][ox];
          int32_t p = -1;
          if (ok) {
            const uint64_t m = s_mask[e][tid];
            if ((m >> cell) & 1u)
              p = int32_t(s_base[e][tid] + uint32_t(__popcll(m & ((uint64_t(1) << cell) - 1u))));
          }
          pos[oy * 3 + ox] = p;
        }
      }
      int32_t jr[9];
#pragma unroll
      for (int i = 0; i < 9; ++i) jr[i] = pos[i] >= 0 ? bd.rows[pos[i]] : -1;
      // offset k = sl * 27 + oz * 9 + i: pf row k, pb row kv - 1 - k
      const int k0 = sl * 27 + oz * 9;
      int32_t* pfk = pf ? pf + int64_t(k0) * n + r : nullptr;
      int32_t* pbk = pb ? pb + int64_t(g.kv - 1 - k0) * n + r : nullptr;
#pragma unroll
      for (int i = 0; i < 9; ++i) {
        const int k = k0 + i;
        if (pf) pfk[int64_t(i) * n] = jr[i];
        if (pb) pbk[-int64_t(i) * n] = jr[i];
        if (jr[i] >= 0) word |= 1u << (k & 31);
        // a slice's last offset ends its bits too (NDIM = 4: other slices'
        // threads fill the rest of the word)
        if ((k & 31) == 31 || k == g.kv - 1 || (LEAD && k == sl * 27 + 26)) {
          if (words) {
            if (LEAD) {
              if (word) atomicOr(&words[r * mic + (k >> 5)], word);
            } else {
              words[r * mic + (k >> 5)] = word;
            }
          }
          word = 0;
        }
      }
    }
  }
}

// Whether brick_probe3 serves this geometry.
static bool brick_probe3_ok(const GeomDev& g) {
  if (g.ndim != 3 && g.ndim != 4) return false;
  for (int d = g.ndim - 3; d < g.ndim; ++d)
    if (g.ks[d] != 3 || g.dil[d] != 1) return false;
  return true;
}

template <class W>
static void brick_layout(W& w, int64_t n, bool key64, BrickDev* bd, uint64_t** table, int** flags,
                         uint64_t* cap_out) {
  const uint64_t cap = table_capacity(n);
  *flags = w.template take<int>(64);
  uint32_t* total = w.template take<uint32_t>(64);
  *table = w.template take<uint64_t>(cap);  // Table32 slots or Table64 keys
  uint64_t* masks = w.template take<uint64_t>(cap);
  uint32_t* base = w.template take<uint32_t>(cap);
  int32_t* rows = w.template take<int32_t>(size_t(n));
  (void)key64;
  if (bd) {
    bd->masks = masks;
    bd->base = base;
    bd->rows = rows;
    bd->total = total;
  }
  *cap_out = cap;
}

template <class Table>
static int run_brick_subm(const int32_t* indices, int64_t n, const GeomDev& d, Table t,
                          const BrickDev& bd, uint64_t cap, uint64_t* table, int32_t* pair_fwd,
                          int32_t* pair_bwd, uint32_t* mask_words, int mic, hipStream_t s) {
  const bool slices = brick_probe3_ok(d) && d.ndim == 4;  // the slice-parallel probe
  const int64_t n_words = slices && mask_words ? n * mic : 0;
  int64_t fill = int64_t(cap) > n ? int64_t(cap) : n;
  fill = fill > n_words ? fill : n_words;
  SP_CHECK_ARG(cdiv(fill, 256) <= kMaxGridX, "pairgen_subm: too many rows");
  brick_fill<<<unsigned(cdiv(fill, 256)), 256, 0, s>>>(table, cap, bd.masks, bd.rows, n, bd.total,
                                                       mask_words, n_words);
  SP_LAUNCHED();
  const unsigned blocks = unsigned(cdiv(n, 256));
  brick_insert<Table><<<blocks, 256, 0, s>>>(indices, n, d, t, bd);
  SP_LAUNCHED();
  brick_bases<<<unsigned(cdiv(int64_t(cap), 256 * kBasePer)), 256, 0, s>>>(bd, cap);
  SP_LAUNCHED();
  brick_scatter<Table><<<blocks, 256, 0, s>>>(indices, n, d, t, bd);
  SP_LAUNCHED();
  if (brick_probe3_ok(d) && d.ndim == 3)
    brick_probe3<Table, 3><<<blocks, 256, 0, s>>>(indices, n, d, t, bd, pair_fwd, pair_bwd,
                                                   mask_words, mic);
  else if (slices) {
    SP_CHECK_ARG(cdiv(n * d.ks[0], 256) <= kMaxGridX, "pairgen_subm: too many rows");
    brick_probe3<Table, 4><<<unsigned(cdiv(n * d.ks[0], 256)), 256, 0, s>>>(
        indices, n, d, t, bd, pair_fwd, pair_bwd, mask_words, mic);
  }
  else
    brick_probe<Table><<<blocks, 256, 0, s>>>(indices, n, d, t, bd, pair_fwd, pair_bwd,
                                              mask_words, mic);
  SP_LAUNCHED();
  return SP_OK;
}

// ---- regular / transposed convs on an occupancy bitmap ------------------------
// With int32 keys and an output key volume of at most kBitmapCellsPerRow cells
// per input row, one bit per output cell replaces the hash, the key sort and
// the ranking.  Candidates set their cell's bit; an exclusive scan of the
// 32-bit words' popcounts gives each word's first rank; a key's output row is
// that prefix plus the popcount of its word's lower bits, i.e. its rank in
// ascending key order (torch.unique's order, as the hash path's sort gives).
// The set bits, read in word order, are the sorted unique keys themselves.
// The bitmap's passes cost in proportion to the output volume, the hash
// path's in proportion to the candidates (n * kv, each an insert with probing,
// then a radix sort and a ranking pass): the bitmap is taken up to 4096 cells
// per input row, or 1024 per candidate while the bitmap and its prefix stay
// within kBitmapMaxCandidateCells cells (256 MiB of workspace; the hash
// path's is O(n * kv)).  (Measured on a transposed k3 s2 conv of 50k uniform
// voxels in 41 x 1600 x 1408: 749M output cells, 15k per row but 555 per
// candidate; the hash path's insert alone took 270 us.)
constexpr int64_t kBitmapCellsPerRow = 4096;
constexpr int64_t kBitmapCellsPerCandidate = 1024;
constexpr double kBitmapMaxCandidateCells = double(int64_t(1) << 30);

static bool conv_bitmap(const GeomDev& g, int64_t n, bool key64) {
  if (key64) return false;
  const double vol = double(g.batch) * double(prod_shape(g.out_shape, g.ndim));
  return vol <= double(kBitmapCellsPerRow) * double(n) ||
         (vol <= kBitmapMaxCandidateCells &&
          vol <= double(kBitmapCellsPerCandidate) * double(n) * double(g.kv));
}

struct BitmapWs {
  uint32_t* bits;    // [words] occupancy, bit key % 32 of word key / 32
  uint32_t* prefix;  // [words] set bits in the words before
  uint32_t* total;   // number of set bits
  void* scan_ws;
  int64_t words;
};

template <class W>
static void bitmap_layout(W& w, const GeomDev& g, BitmapWs* out) {
  const int64_t words = cdiv(g.batch * prod_shape(g.out_shape, g.ndim), 32);
  auto* bits = w.template take<uint32_t>(size_t(words));
  auto* prefix = w.template take<uint32_t>(size_t(words));
  auto* total = w.template take<uint32_t>(64);
  void* sws = w.template take<char>(scan_workspace_bytes(words));
  if (out) *out = BitmapWs{bits, prefix, total, sws, words};
}

// Pair counts go to kCountSpread 64-bit counters, one atomic per workgroup on
// counter blockIdx.x % kCountSpread; the reader sums them (count_sum).  Atomics
// on one address serialise: one per wave onto a single counter took ~25 us of
// conv_mark's 31 us on the LiDAR encoder's first k3 s2 layer (1 250 waves).
// Every thread of the workgroup must call it (it has barriers).
constexpr int kCountSpread = 16;
__device__ __forceinline__ void block_count(uint32_t cnt, unsigned long long* counters) {
  __shared__ uint32_t s_cnt;
  for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  if (threadIdx.x == 0) s_cnt = 0;
  __syncthreads();
  if (lane_id() == 0 && cnt != 0) atomicAdd(&s_cnt, cnt);
  __syncthreads();
  if (threadIdx.x == 0 && s_cnt != 0)
    atomicAdd(&counters[blockIdx.x % kCountSpread], (unsigned long long)s_cnt);
}

// The total of the counters block_count adds to, from their host copy
// (2 * kCountSpread 32-bit words, little-endian halves).
static int64_t count_sum(const uint32_t* h) {
  uint64_t t = 0;
  for (int i = 0; i < kCountSpread; ++i) t += uint64_t(h[2 * i]) | (uint64_t(h[2 * i + 1]) << 32);
  return int64_t(t);
}

// One thread per input row j: set the bits of its candidate outputs.  The kv
// candidates of a row come in key order along the fastest dimension, so runs
// in one word are ORed together before the atomic.
// The candidates (the table's pairs) are counted into *npairs.
// (Measured with each row's offsets split over four threads, as conv_fill_bitmap
// does: 31.5 -> 54.3 us on the LiDAR encoder's first k3 s2 layer, the rows'
// atomics meeting on the same bitmap words at the same time.)
__global__ __launch_bounds__(256) void conv_mark(const int32_t* __restrict__ idx, int64_t n,
                                                 GeomDev g, uint32_t* __restrict__ bits,
                                                 unsigned long long* __restrict__ npairs) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t cnt = 0;
  if (j < n) {
    const Coord c = load_coord(idx, j, g);
    int off[4] = {0, 0, 0, 0};
    uint32_t cw = 0, cb = 0;  // pending word and its bits (cb == 0: none)
    for (int k = 0; k < g.kv; ++k) {
      uint64_t key;
      if (candidate_key<int32_t>(g, c, off, &key)) {
        const uint32_t w = uint32_t(key >> 5), b = 1u << uint32_t(key & 31u);
        if (cb != 0 && w != cw) {
          atomicOr(&bits[cw], cb);
          cb = 0;
        }
        cw = w;
        cb |= b;
        ++cnt;
      }
      odometer_next(g, off);
    }
    if (cb != 0) atomicOr(&bits[cw], cb);
  }
  block_count(cnt, npairs);
}

// conv_fill_bitmap splits each input row's kv offsets over the four waves of
// a workgroup: wave w of workgroup b takes rows 64 b .. 64 b + 63 (one per
// lane) and the contiguous offsets [w * per, (w + 1) * per), per =
// ceil(kv / 4).  With one thread walking all kv offsets of its row the launch
// held too few waves to hide the loop's latency (50k rows: 782 waves on 1 024
// SIMDs): 26.4 -> 15.2 us on the LiDAR encoder's first k3 s2 layer.
constexpr int kBitmapRowsPerBlock = 64;
constexpr int kBitmapParts = 4;  // waves per workgroup, each a part of the offsets

// First offset of this wave's part, its end, and its per-dimension offsets.
__device__ __forceinline__ void offset_part(const GeomDev& g, int part, int* k0, int* k1,
                                            int (&off)[4]) {
  const int per = (g.kv + kBitmapParts - 1) / kBitmapParts;
  *k0 = part * per < g.kv ? part * per : g.kv;
  *k1 = *k0 + per < g.kv ? *k0 + per : g.kv;
  int rem = *k0;
#pragma unroll
  for (int d = 3; d >= 0; --d) {  // the odometer order: the last dimension fastest
    off[d] = 0;
    if (d < g.ndim) {
      off[d] = rem % g.ks[d];
      rem /= g.ks[d];
    }
  }
}

// Output row of a marked key.
__device__ __forceinline__ int64_t bitmap_rank(const uint32_t* __restrict__ bits,
                                               const uint32_t* __restrict__ prefix, uint64_t key) {
  const uint64_t w = key >> 5;
  const uint32_t below = bits[w] & ((1u << uint32_t(key & 31u)) - 1u);
  return int64_t(prefix[w]) + __popc(below);
}

// conv_fill with the bitmap's ranks.  The rows' mask words (bit k of word
// k / 32: offset k has a pair) are gathered from the four parts in the
// dynamic LDS, mic * 64 words (launched with none when words is null).
__global__ __launch_bounds__(256) void conv_fill_bitmap(
    const int32_t* __restrict__ idx, int64_t n, GeomDev g, const uint32_t* __restrict__ bits,
    const uint32_t* __restrict__ prefix, int64_t n_keep, int32_t* __restrict__ pf,
    int32_t* __restrict__ pb, uint32_t* __restrict__ words, int mic) {
  extern __shared__ uint32_t s_words[];  // [mic][64]
  const int lane = int(threadIdx.x & 63);
  const int64_t j = int64_t(blockIdx.x) * kBitmapRowsPerBlock + lane;
  if (words) {
    for (int i = int(threadIdx.x); i < mic * kBitmapRowsPerBlock; i += blockDim.x)
      s_words[i] = 0u;
    __syncthreads();
  }
  if (j < n) {
    const Coord c = load_coord(idx, j, g);
    int off[4], k0, k1;
    offset_part(g, int(threadIdx.x >> 6), &k0, &k1, off);
    uint32_t word = 0;
    for (int k = k0; k < k1; ++k) {
      uint64_t key;
      int32_t r = -1;
      if (candidate_key<int32_t>(g, c, off, &key)) {
        const int64_t rank = bitmap_rank(bits, prefix, key);
        r = rank < n_keep ? int32_t(rank) : -1;
      }
      if (r >= 0) {
        if (pf) pf[int64_t(k) * n_keep + r] = int32_t(j);
        word |= 1u << (k & 31);
      }
      if (pb) pb[int64_t(k) * n + j] = r;
      if (((k & 31) == 31 || k == k1 - 1) && word) {
        if (words) atomicOr(&s_words[(k >> 5) * kBitmapRowsPerBlock + lane], word);
        word = 0;
      }
      odometer_next(g, off);
    }
  }
  if (words) {
    __syncthreads();
    for (int i = int(threadIdx.x); i < mic * kBitmapRowsPerBlock; i += blockDim.x) {
      const int r = i / mic, w = i % mic;  // row-major: consecutive threads, consecutive words
      const int64_t jr = int64_t(blockIdx.x) * kBitmapRowsPerBlock + r;
      if (jr < n) words[jr * mic + w] = s_words[w * kBitmapRowsPerBlock + r];
    }
  }
}

// Output coordinates of the kept rows: one thread per bitmap word, its set
// bits in order (rows prefix[w], prefix[w] + 1, ...).
// Each thread scans 4 words (one 16-byte load; the bitmap sits at the start of
// a 256-byte aligned workspace part) and reads the prefix of the non-empty
// ones only: in a sparse volume almost every word is empty, and one thread
// per word spent the kernel on workgroup dispatch.
__global__ __launch_bounds__(256) void emit_bitmap_keys(const uint32_t* __restrict__ bits,
                                                        const uint32_t* __restrict__ prefix,
                                                        int64_t nwords, GeomDev g, int64_t n_keep,
                                                        int32_t* __restrict__ out) {
  const int64_t w0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (w0 >= nwords) return;
  uint32_t m4[4];
  if (w0 + 4 <= nwords) {
    const uint4 v = *reinterpret_cast<const uint4*>(bits + w0);
    m4[0] = v.x;
    m4[1] = v.y;
    m4[2] = v.z;
    m4[3] = v.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) m4[i] = w0 + i < nwords ? bits[w0 + i] : 0u;
  }
  if ((m4[0] | m4[1] | m4[2] | m4[3]) == 0) return;
  for (int i = 0; i < 4; ++i) {
    uint32_t m = m4[i];
    if (m == 0) continue;
    const int64_t w = w0 + i;
    int64_t r = prefix[w];
    while (m != 0 && r < n_keep) {
      const int b = __ffs(m) - 1;
      m &= m - 1u;
      uint32_t rem = uint32_t(w) * 32u + uint32_t(b);  // bitmap keys are below 2^31
      int32_t co[5] = {0, 0, 0, 0, 0};  // (batch, x0, .., x3); the loop is unrolled, so the
#pragma unroll                          // divisors stay in registers across rows
      for (int d = 3; d >= 0; --d) {
        if (d < g.ndim) {
          const uint32_t q = div31(rem, g.out_div[d]);  // rem < 2^31
          co[d + 1] = int32_t(rem - q * uint32_t(g.out_shape[d]));
          rem = q;
        }
      }
      co[0] = int32_t(rem);
      int32_t* o = out + r * (g.ndim + 1);
      if (g.ndim == 3 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {  // one 16-byte store
        *reinterpret_cast<int4*>(o) = make_int4(co[0], co[1], co[2], co[3]);
      } else {
#pragma unroll
        for (int d = 0; d < 5; ++d)
          if (d <= g.ndim) o[d] = co[d];
      }
      ++r;
    }
  }
}

// Sizer variant returning nulls (the WsSizer::take returns void).
struct WsSizerP {
  size_t off = 0;
  template <typename T>
  T* take(size_t count) {
    off = align_up(off, 256);
    off += count * sizeof(T);
    return nullptr;
  }
};


// counter[0]: unique keys; the candidates (the table's pairs) are counted
// into *npairs.
template <class Table, typename KeyT>
__global__ __launch_bounds__(256) void conv_insert(const int32_t* __restrict__ idx, int64_t n,
                                                   GeomDev g, Table t, KeyT* __restrict__ list,
                                                   uint32_t* __restrict__ counter, int64_t bound,
                                                   unsigned long long* __restrict__ npairs) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool live = j < n;
  Coord c;
  if (live) c = load_coord(idx, j, g);
  else c.ok = false;
  int off[4] = {0, 0, 0, 0};
  uint32_t cnt = 0;
  for (int k = 0; k < g.kv; ++k) {
    uint64_t key = 0;
    bool fresh = false;
    if (live && candidate_key<KeyInt<Table>>(g, c, off, &key)) {
      fresh = t.insert(key, 0);
      ++cnt;
    }
    // wave-aggregated append of newly inserted keys
    const uint64_t b = __ballot(fresh);
    if (b) {
      const int leader = __ffsll((unsigned long long)b) - 1;
      uint32_t base = 0;
      if (lane_id() == leader) base = atomicAdd(counter, uint32_t(__popcll(b)));
      base = __shfl(base, leader, 64);
      if (fresh) {
        const int64_t pos = int64_t(base) + __popcll(b & lanemask_lt());
        if (pos < bound) list[pos] = KeyT(key);
      }
    }
    odometer_next(g, off);
  }
  block_count(cnt, npairs);
}

template <class Table, typename KeyT>
__global__ void conv_rank(const KeyT* __restrict__ sorted, int64_t n_out, Table t) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n_out) return;
  const int64_t s = t.find_slot(uint64_t(sorted[r]));
  if (s >= 0) t.set_value(s, int32_t(r));
}

template <typename KeyT>
__global__ void copy_keys(const KeyT* __restrict__ src, KeyT* __restrict__ dst, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

template <typename KeyT>
__global__ void delinearize(const KeyT* __restrict__ keys, int64_t n, GeomDev g,
                            int32_t* __restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  int32_t* o = out + r * (g.ndim + 1);
  if constexpr (sizeof(KeyT) == 4) {  // int32 keys: below 2^31, the multiply-shift division
    uint32_t rem = uint32_t(keys[r]);
#pragma unroll
    for (int d = 3; d >= 0; --d) {  // (unrolled: the divisors are loaded once)
      if (d < g.ndim) {
        const uint32_t q = div31(rem, g.out_div[d]);
        o[d + 1] = int32_t(rem - q * uint32_t(g.out_shape[d]));
        rem = q;
      }
    }
    o[0] = int32_t(rem);
  } else {
    uint64_t rem = uint64_t(keys[r]);
    for (int d = g.ndim - 1; d >= 0; --d) {
      const uint64_t s = uint64_t(g.out_shape[d]);
      o[d + 1] = int32_t(rem % s);
      rem /= s;
    }
    o[0] = int32_t(rem);
  }
}

// One thread per input row j: pb[k, j] = output row of candidate (k, j) or -1,
// pf[k, pb[k, j]] = j; the backward bitmask of row j is built in registers.
template <class Table>
__global__ __launch_bounds__(256) void conv_fill(const int32_t* __restrict__ idx, int64_t n,
                                                 GeomDev g, Table t, int64_t n_keep,
                                                 int32_t* __restrict__ pf, int32_t* __restrict__ pb,
                                                 uint32_t* __restrict__ words, int mic) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const Coord c = load_coord(idx, j, g);
  int off[4] = {0, 0, 0, 0};
  uint32_t word = 0;
  for (int k = 0; k < g.kv; ++k) {
    uint64_t key;
    int32_t r = -1;
    if (candidate_key<KeyInt<Table>>(g, c, off, &key)) {
      r = t.find(key);
      if (r >= n_keep) r = -1;
    }
    if (r >= 0) {
      if (pf) pf[int64_t(k) * n_keep + r] = int32_t(j);
      word |= 1u << (k & 31);
    }
    if (pb) pb[int64_t(k) * n + j] = r;
    if ((k & 31) == 31 || k == g.kv - 1) {
      if (words) words[j * mic + (k >> 5)] = word;
      word = 0;
    }
    odometer_next(g, off);
  }
}

// ---------------------------------------------------------------------------
// mask words, compaction, native -> tables
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mask_words_kernel(const int32_t* __restrict__ table,
                                                         int64_t kv, int64_t n,
                                                         uint32_t* __restrict__ words, int mic) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n) return;
  uint32_t word = 0;
  for (int64_t k = 0; k < kv; ++k) {
    if (table[k * n + r] >= 0) word |= 1u << (k & 31);
    if ((k & 31) == 31 || k == kv - 1) {
      words[r * mic + (k >> 5)] = word;
      word = 0;
    }
  }
}

constexpr int kCompactThreads = 256;
constexpr int kCompactRounds = 8;
constexpr int kCompactTile = kCompactThreads * kCompactRounds;

// grid (tiles, kv): number of valid entries per (row k, tile)
__global__ __launch_bounds__(kCompactThreads) void compact_count(const int32_t* __restrict__ table,
                                                                 int64_t n, int64_t ntiles,
                                                                 uint32_t* __restrict__ cnt) {
  __shared__ uint32_t lds[kCompactThreads / 64 + 1];
  const int64_t k = blockIdx.y;
  const int64_t base = int64_t(blockIdx.x) * kCompactTile;
  uint32_t s = 0;
#pragma unroll
  for (int r = 0; r < kCompactRounds; ++r) {
    const int64_t i = base + r * kCompactThreads + threadIdx.x;
    if (i < n && table[k * n + i] >= 0) ++s;
  }
  uint32_t tot;
  block_exclusive_scan<kCompactThreads>(s, lds, &tot);
  if (threadIdx.x == 0) cnt[k * ntiles + blockIdx.x] = tot;
}

__global__ __launch_bounds__(kCompactThreads) void compact_scatter(
    const int32_t* __restrict__ table, int64_t n, int64_t ntiles, const uint32_t* __restrict__ off,
    int32_t* __restrict__ pos_out, int32_t* __restrict__ val_out) {
  __shared__ uint32_t lds[kCompactThreads / 64 + 1];
  const int64_t k = blockIdx.y;
  const int64_t base = int64_t(blockIdx.x) * kCompactTile;
  // segmented: subtract the start of row k in the flat scan
  uint32_t run = off[k * ntiles + blockIdx.x] - off[k * ntiles];
  for (int r = 0; r < kCompactRounds; ++r) {
    const int64_t i = base + r * kCompactThreads + threadIdx.x;
    int32_t v = -1;
    if (i < n) v = table[k * n + i];
    const uint32_t flag = v >= 0 ? 1u : 0u;
    uint32_t tot;
    const uint32_t pre = block_exclusive_scan<kCompactThreads>(flag, lds, &tot);
    if (flag) {
      const int64_t p = k * n + run + pre;
      pos_out[p] = int32_t(i);
      val_out[p] = v;
    }
    run += tot;
  }
}

__global__ void compact_counts(const uint32_t* __restrict__ off, const uint32_t* __restrict__ total,
                               int64_t kv, int64_t ntiles, int32_t* __restrict__ counts,
                               int32_t* __restrict__ npl, int npl_limit) {
  const int64_t k = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k >= kv) return;
  const uint32_t end = (k + 1 < kv) ? off[(k + 1) * ntiles] : *total;
  const int32_t c = int32_t(end - off[k * ntiles]);
  if (counts) counts[k] = c;
  if (npl) npl[k] = k < npl_limit ? c : 0;
}

__global__ void native_scatter(const int32_t* __restrict__ pin, const int32_t* __restrict__ pout,
                               int64_t kv, int64_t np, int64_t n_in, int64_t n_out,
                               int32_t* __restrict__ pf, int32_t* __restrict__ pb) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= kv * np) return;
  const int64_t k = i / np;
  const int32_t a = pin[i], b = pout[i];
  if (a >= 0 && b >= 0 && a < n_in && b < n_out) {
    pf[k * n_out + b] = a;
    if (pb) pb[k * n_in + a] = b;
  }
}

}  // namespace sp

using namespace sp;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int sp_geom_key64(const sp_geom* g) {
  GeomDev d;
  if (make_geom(g, &d)) return -1;
  return need_key64(d) ? 1 : 0;
}

size_t sp_pairgen_workspace_size(const sp_geom* g, int64_t n) {
  GeomDev d;
  if (make_geom(g, &d)) return 0;
  if (n < 1) n = 1;
  const bool key64 = need_key64(d);
  if (d.mode == SP_PAIR_SUBM) {
    WsSizerP z;
    if (subm_dense(d, n)) {
      z.take<int32_t>(size_t(subm_cells(d) + 2 * kGridPad));
      return z.off;
    }
    uint64_t* ta;
    int* fl;
    uint64_t cap;
    brick_layout(z, n, key64, nullptr, &ta, &fl, &cap);
    return z.off;
  }
  WsSizerP z;
  if (conv_bitmap(d, n, key64)) {
    bitmap_layout(z, d, nullptr);
    return z.off;
  }
  conv_layout(z, d, n, key64, nullptr);
  return z.off;
}

int sp_pairgen_subm(const sp_geom* g, const int32_t* indices, int64_t n, int32_t* pair_fwd,
                    int32_t* pair_bwd, uint32_t* mask_words, void* ws, size_t ws_bytes,
                    void* stream) {
  GeomDev d;
  int rc = make_geom(g, &d);
  if (rc) return rc;
  SP_CHECK_ARG(d.mode == SP_PAIR_SUBM, "sp_pairgen_subm needs SP_PAIR_SUBM");
  SP_CHECK_ARG(n >= 1 && n < (int64_t(1) << 31), "n=%lld out of range", (long long)n);
  SP_CHECK_ARG(indices && (pair_fwd || pair_bwd), "null pointer");
  const size_t need = sp_pairgen_workspace_size(g, n);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "pairgen_subm: workspace %zu < %zu", ws_bytes, need);
  SP_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 15) == 0,
               "pairgen_subm: workspace must be 16-byte aligned (its parts take 16-byte accesses)");
  hipStream_t s = as_stream(stream);
  const bool key64 = need_key64(d);
  WsCursor c(ws, ws_bytes);
  const int mic = (d.kv + 31) / 32;
  const unsigned blocks = unsigned(cdiv(n, 256));
  if (subm_dense(d, n)) {
    const int64_t cells = subm_cells(d);
    int32_t* buf = c.take<int32_t>(size_t(cells + 2 * kGridPad));
    int32_t* grid = buf + kGridPad;  // cell 0
    const int64_t fb = cdiv(cdiv(cells + 2 * kGridPad, 4), 256);
    fill_i32x4<<<unsigned(fb < 4096 ? fb : 4096), 256, 0, s>>>(buf, cells + 2 * kGridPad, kNoRow);
    SP_LAUNCHED();
    if (d.kv <= kProbeMaxKv) {
      subm_insert_grid<false><<<blocks, 256, 0, s>>>(indices, int32_t(n), d, grid, 0u);
      SP_LAUNCHED();
      return launch_probe_grid<false>(indices, n, d, grid, cells, 0u, pair_fwd, pair_bwd,
                                      mask_words, mic, nullptr, s);
    }
    subm_insert_dense<<<blocks, 256, 0, s>>>(indices, n, d, grid);
    SP_LAUNCHED();
    subm_probe_dense<<<blocks, 256, 0, s>>>(indices, n, d, grid, pair_fwd, pair_bwd, mask_words,
                                            mic);
    SP_LAUNCHED();
    return SP_OK;
  }
  // the brick index (bricks hashed with 32-bit keys while the brick volume
  // allows, whatever the key width of the cells)
  BrickDev bd = brick_geom(d);
  uint64_t* table;
  int* flags;
  uint64_t cap;
  brick_layout(c, n, key64, &bd, &table, &flags, &cap);
  (void)blocks;
  if (brick_volume(d) < 2147483648.0)
    return run_brick_subm(indices, n, d, Table32{table, cap - 1, flags}, bd, cap, table, pair_fwd,
                          pair_bwd, mask_words, mic, s);
  return run_brick_subm(indices, n, d, Table64{table, nullptr, cap - 1, flags}, bd, cap, table,
                        pair_fwd, pair_bwd, mask_words, mic, s);
}

int64_t sp_pairgen_subm_grid_cells(const sp_geom* g, int64_t n) {
  GeomDev d;
  if (make_geom(g, &d) != SP_OK) return 0;
  if (d.mode != SP_PAIR_SUBM || n < 1 || n > kStampRowMask || d.kv > kProbeMaxKv) return 0;
  return subm_dense(d, n) ? subm_cells(d) + 2 * kGridPad : 0;
}

int sp_pairgen_subm_grid(const sp_geom* g, const int32_t* indices, int64_t n, int32_t* pair_fwd,
                         int32_t* pair_bwd, uint32_t* mask_words, int32_t* npl, int32_t* grid,
                         int64_t grid_cells, uint32_t epoch, void* stream) {
  GeomDev d;
  int rc = make_geom(g, &d);
  if (rc) return rc;
  SP_CHECK_ARG(d.mode == SP_PAIR_SUBM, "sp_pairgen_subm_grid needs SP_PAIR_SUBM");
  SP_CHECK_ARG(indices && grid && (pair_fwd || pair_bwd), "null pointer");
  const int64_t cells = sp_pairgen_subm_grid_cells(g, n);
  SP_CHECK_ARG(cells > 0, "pairgen_subm_grid: no dense grid for this geometry (n=%lld)",
               (long long)n);
  SP_CHECK_ARG(grid_cells >= cells, "pairgen_subm_grid: grid of %lld cells < %lld",
               (long long)grid_cells, (long long)cells);
  SP_CHECK_ARG(epoch >= 1 && epoch <= 255, "pairgen_subm_grid: epoch %u not in 1..255", epoch);
  hipStream_t s = as_stream(stream);
  const int mic = (d.kv + 31) / 32;
  const unsigned blocks = unsigned(cdiv(n, 256));
  int32_t* cell0 = grid + kGridPad;
  subm_insert_grid<true><<<blocks, 256, 0, s>>>(indices, int32_t(n), d, cell0, epoch);
  SP_LAUNCHED();
  return launch_probe_grid<true>(indices, n, d, cell0, cells - 2 * kGridPad, epoch, pair_fwd,
                                 pair_bwd, mask_words, mic, npl, s);
}

int sp_pairgen_conv_build(const sp_geom* g, const int32_t* indices, int64_t n, void* ws,
                          size_t ws_bytes, int64_t* n_out, int64_t* n_pairs, void* stream) {
  GeomDev d;
  int rc = make_geom(g, &d);
  if (rc) return rc;
  SP_CHECK_ARG(d.mode != SP_PAIR_SUBM, "sp_pairgen_conv_build is for regular/transpose convs");
  SP_CHECK_ARG(n >= 1 && n < (int64_t(1) << 31), "n=%lld out of range", (long long)n);
  SP_CHECK_ARG(indices && n_out, "null pointer");
  const size_t need = sp_pairgen_workspace_size(g, n);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "pairgen_conv_build: workspace %zu < %zu", ws_bytes, need);
  SP_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 15) == 0,
               "pairgen_conv_build: workspace must be 16-byte aligned (its parts take 16-byte accesses)");
  hipStream_t s = as_stream(stream);
  const bool key64 = need_key64(d);
  WsCursor c(ws, ws_bytes);
  if (conv_bitmap(d, n, key64)) {
    BitmapWs b;
    bitmap_layout(c, d, &b);
    const int64_t fb = cdiv(cdiv(b.words, 4), 256);
    fill_i32x4<<<unsigned(fb < 4096 ? fb : 4096), 256, 0, s>>>(
        reinterpret_cast<int32_t*>(b.bits), b.words, 0);
    SP_LAUNCHED();
    // total[0]: set bits (from the scan); total[32..63]: the pair counters
    auto* npairs = reinterpret_cast<unsigned long long*>(b.total + 32);
    SP_HIP(hipMemsetAsync(npairs, 0, kCountSpread * sizeof(unsigned long long), s));
    conv_mark<<<unsigned(cdiv(n, 256)), 256, 0, s>>>(indices, n, d, b.bits, npairs);
    SP_LAUNCHED();
    SP_CHECK_ARG(cdiv(b.words, 256) <= kMaxGridX, "pairgen: output volume too large");
    rc = exclusive_scan_popc(b.bits, b.prefix, b.words, b.total, b.scan_ws, s);
    if (rc) return rc;
    uint32_t h[32 + 2 * kCountSpread] = {};
    SP_HIP(hipMemcpyAsync(h, b.total, sizeof(h), hipMemcpyDeviceToHost, s));
    SP_HIP(hipStreamSynchronize(s));
    *n_out = int64_t(h[0]);
    if (n_pairs) *n_pairs = count_sum(h + 32);
    return SP_OK;
  }
  ConvWs w;
  conv_layout(c, d, n, key64, &w);
  SP_HIP(hipMemsetAsync(w.flags, 0, 256, s));
  SP_HIP(hipMemsetAsync(w.counter, 0, 256, s));
  auto* npairs = reinterpret_cast<unsigned long long*>(w.counter + 32);
  rc = launch_fill_u64(static_cast<uint64_t*>(w.table_a), int64_t(w.cap), kEmpty64, s);
  if (rc) return rc;
  const unsigned blocks = unsigned(cdiv(n, 256));
  if (key64) {
    rc = launch_fill_i32(w.table_vals, int64_t(w.cap), 0x7fffffff, s);
    if (rc) return rc;
    Table64 t{static_cast<uint64_t*>(w.table_a), w.table_vals, w.cap - 1, w.flags};
    conv_insert<Table64, uint64_t><<<blocks, 256, 0, s>>>(
        indices, n, d, t, static_cast<uint64_t*>(w.list), w.counter, w.bound, npairs);
  } else {
    Table32 t{static_cast<uint64_t*>(w.table_a), w.cap - 1, w.flags};
    conv_insert<Table32, uint32_t><<<blocks, 256, 0, s>>>(
        indices, n, d, t, static_cast<uint32_t*>(w.list), w.counter, w.bound, npairs);
  }
  SP_LAUNCHED();
  uint32_t host[32 + 2 * kCountSpread] = {};  // counter[0]: unique keys, [32..63]: pairs
  uint32_t overflow = 0;
  SP_HIP(hipMemcpyAsync(host, w.counter, sizeof(host), hipMemcpyDeviceToHost, s));
  SP_HIP(hipMemcpyAsync(&overflow, w.flags, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  SP_HIP(hipStreamSynchronize(s));
  if (overflow) return set_error(SP_ERR_HASH_FULL, "pairgen: coordinate hash overflow");
  if (n_pairs) *n_pairs = count_sum(host + 32);
  const int64_t cnt = int64_t(host[0]);
  if (cnt > w.bound) return set_error(SP_ERR_HASH_FULL, "pairgen: %lld keys > bound %lld",
                                      (long long)cnt, (long long)w.bound);
  *n_out = cnt;
  if (cnt == 0) return SP_OK;
  // sort the unique keys (bits of the largest possible key) and rank them
  const double vol = double(d.batch) * double(prod_shape(d.out_shape, d.ndim));
  const int bits = bit_length_u64(uint64_t(vol) - 1);
  const unsigned rb = unsigned(cdiv(cnt, 256));
  if (key64) {
    uint64_t* res = nullptr;
    rc = sort_keys_u64(static_cast<uint64_t*>(w.list), static_cast<uint64_t*>(w.tmp), cnt, bits,
                       &res, w.sort_ws, s);
    if (rc) return rc;
    if (res != w.list) {
      copy_keys<<<rb, 256, 0, s>>>(res, static_cast<uint64_t*>(w.list), cnt);
      SP_LAUNCHED();
    }
    Table64 t{static_cast<uint64_t*>(w.table_a), w.table_vals, w.cap - 1, w.flags};
    conv_rank<<<rb, 256, 0, s>>>(static_cast<const uint64_t*>(w.list), cnt, t);
  } else {
    uint32_t* res = nullptr;
    rc = sort_keys_u32(static_cast<uint32_t*>(w.list), static_cast<uint32_t*>(w.tmp), cnt, bits,
                       &res, w.sort_ws, s);
    if (rc) return rc;
    if (res != w.list) {
      copy_keys<<<rb, 256, 0, s>>>(res, static_cast<uint32_t*>(w.list), cnt);
      SP_LAUNCHED();
    }
    Table32 t{static_cast<uint64_t*>(w.table_a), w.cap - 1, w.flags};
    conv_rank<<<rb, 256, 0, s>>>(static_cast<const uint32_t*>(w.list), cnt, t);
  }
  SP_LAUNCHED();
  return SP_OK;
}

int sp_pairgen_conv_fill(const sp_geom* g, const int32_t* indices, int64_t n, const void* ws,
                         size_t ws_bytes, int64_t n_keep, int32_t* out_indices, int32_t* pair_fwd,
                         int32_t* pair_bwd, uint32_t* mask_words_bwd, void* stream) {
  GeomDev d;
  int rc = make_geom(g, &d);
  if (rc) return rc;
  SP_CHECK_ARG(d.mode != SP_PAIR_SUBM, "sp_pairgen_conv_fill is for regular/transpose convs");
  SP_CHECK_ARG(n >= 1 && n < (int64_t(1) << 31), "n=%lld out of range", (long long)n);
  SP_CHECK_ARG(indices && out_indices && (pair_fwd || pair_bwd), "null pointer");
  SP_CHECK_ARG(n_keep >= 1 && n_keep < (int64_t(1) << 31), "n_keep=%lld out of range",
               (long long)n_keep);
  const size_t need = sp_pairgen_workspace_size(g, n);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "pairgen_conv_fill: workspace %zu < %zu", ws_bytes, need);
  SP_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 15) == 0,
               "pairgen_conv_fill: workspace must be 16-byte aligned (its parts take 16-byte accesses)");
  SP_CHECK_ARG(n_keep <= conv_bound(d, n), "n_keep exceeds the number of candidate outputs");
  hipStream_t s = as_stream(stream);
  const bool key64 = need_key64(d);
  WsCursor c(const_cast<void*>(ws), ws_bytes);
  const int mic = (d.kv + 31) / 32;
  if (pair_fwd) {
    rc = launch_fill_i32(pair_fwd, int64_t(d.kv) * n_keep, -1, s);
    if (rc) return rc;
  }
  if (conv_bitmap(d, n, key64)) {
    BitmapWs b;
    bitmap_layout(c, d, &b);
    const size_t lds = mask_words_bwd ? size_t(mic) * kBitmapRowsPerBlock * 4 : 0;  // <= 32 KiB
    conv_fill_bitmap<<<unsigned(cdiv(n, kBitmapRowsPerBlock)), 256, lds, s>>>(
        indices, n, d, b.bits, b.prefix, n_keep, pair_fwd, pair_bwd, mask_words_bwd, mic);
    SP_LAUNCHED();
    emit_bitmap_keys<<<unsigned(cdiv(b.words, 1024)), 256, 0, s>>>(b.bits, b.prefix, b.words, d,
                                                                   n_keep, out_indices);
    SP_LAUNCHED();
    return SP_OK;
  }
  ConvWs w;
  conv_layout(c, d, n, key64, &w);
  const unsigned blocks = unsigned(cdiv(n, 256));
  const unsigned rb = unsigned(cdiv(n_keep, 256));
  if (key64) {
    Table64 t{static_cast<uint64_t*>(w.table_a), w.table_vals, w.cap - 1, w.flags};
    conv_fill<<<blocks, 256, 0, s>>>(indices, n, d, t, n_keep, pair_fwd, pair_bwd, mask_words_bwd,
                                     mic);
    SP_LAUNCHED();
    delinearize<<<rb, 256, 0, s>>>(static_cast<const uint64_t*>(w.list), n_keep, d, out_indices);
  } else {
    Table32 t{static_cast<uint64_t*>(w.table_a), w.cap - 1, w.flags};
    conv_fill<<<blocks, 256, 0, s>>>(indices, n, d, t, n_keep, pair_fwd, pair_bwd, mask_words_bwd,
                                     mic);
    SP_LAUNCHED();
    delinearize<<<rb, 256, 0, s>>>(static_cast<const uint32_t*>(w.list), n_keep, d, out_indices);
  }
  SP_LAUNCHED();
  return SP_OK;
}

int sp_mask_words(const int32_t* table, int64_t kv, int64_t n, uint32_t* words, void* stream) {
  SP_CHECK_ARG(kv >= 1 && n >= 0, "mask_words: bad sizes");
  if (n == 0) return SP_OK;
  SP_CHECK_ARG(table && words, "mask_words: null pointer");
  const int mic = int((kv + 31) / 32);
  const int64_t blocks = cdiv(n, 256);
  SP_CHECK_ARG(blocks <= kMaxGridX, "mask_words: n too large");
  mask_words_kernel<<<unsigned(blocks), 256, 0, as_stream(stream)>>>(table, kv, n, words, mic);
  SP_LAUNCHED();
  return SP_OK;
}

static void compact_layout_sizes(int64_t kv, int64_t n, size_t* cnt_words, size_t* total) {
  const int64_t ntiles = cdiv(n > 0 ? n : 1, kCompactTile);
  *cnt_words = size_t(kv * ntiles);
  WsSizer z;
  z.take<uint32_t>(*cnt_words);
  z.take<uint32_t>(64);
  z.take<char>(scan_workspace_bytes(int64_t(*cnt_words)));
  *total = z.off;
}

size_t sp_compact_workspace_size(int64_t kv, int64_t n) {
  size_t cw, tot;
  compact_layout_sizes(kv, n, &cw, &tot);
  return tot;
}

int sp_compact_table(const int32_t* table, int64_t kv, int64_t n, int32_t* pos_out,
                     int32_t* val_out, int32_t* counts, int32_t* npl, int32_t npl_limit, void* ws,
                     size_t ws_bytes, void* stream) {
  SP_CHECK_ARG(kv >= 1 && kv <= 65535 && n >= 0 && n < (int64_t(1) << 31),
               "compact: bad sizes kv=%lld n=%lld", (long long)kv, (long long)n);
  SP_CHECK_ARG(table && pos_out && val_out, "compact: null pointer");
  hipStream_t s = as_stream(stream);
  size_t cw, need;
  compact_layout_sizes(kv, n, &cw, &need);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "compact: workspace %zu < %zu", ws_bytes, need);
  int rc = launch_fill_i32(pos_out, kv * n, -1, s);
  if (rc) return rc;
  rc = launch_fill_i32(val_out, kv * n, -1, s);
  if (rc) return rc;
  if (n == 0) {
    if (counts) { rc = launch_fill_i32(counts, kv, 0, s); if (rc) return rc; }
    if (npl) { rc = launch_fill_i32(npl, kv, 0, s); if (rc) return rc; }
    return SP_OK;
  }
  WsCursor c(ws, ws_bytes);
  uint32_t* cnt = c.take<uint32_t>(cw);
  uint32_t* total = c.take<uint32_t>(64);
  void* scan_ws = c.take<char>(scan_workspace_bytes(int64_t(cw)));
  const int64_t ntiles = cdiv(n, kCompactTile);
  SP_CHECK_ARG(ntiles <= kMaxGridX, "compact: n too large");
  const dim3 grid{unsigned(ntiles), unsigned(kv), 1u};
  compact_count<<<grid, kCompactThreads, 0, s>>>(table, n, ntiles, cnt);
  SP_LAUNCHED();
  rc = exclusive_scan_u32(cnt, cnt, int64_t(cw), total, scan_ws, s);
  if (rc) return rc;
  compact_scatter<<<grid, kCompactThreads, 0, s>>>(table, n, ntiles, cnt, pos_out, val_out);
  SP_LAUNCHED();
  if (counts || npl) {
    compact_counts<<<unsigned(cdiv(kv, 256)), 256, 0, s>>>(cnt, total, kv, ntiles, counts, npl,
                                                          npl_limit);
    SP_LAUNCHED();
  }
  return SP_OK;
}

int sp_native_to_tables(const int32_t* pair, int64_t kv, int64_t n_pairs, int32_t inverse,
                        int64_t n_in, int64_t n_out, int32_t* pf, int32_t* pb, void* stream) {
  SP_CHECK_ARG(kv >= 1 && n_pairs >= 0 && n_in >= 0 && n_out >= 0, "native_to_tables: bad sizes");
  SP_CHECK_ARG(pair && pf, "native_to_tables: null pointer");
  hipStream_t s = as_stream(stream);
  int rc = launch_fill_i32(pf, kv * n_out, -1, s);
  if (rc) return rc;
  if (pb) {
    rc = launch_fill_i32(pb, kv * n_in, -1, s);
    if (rc) return rc;
  }
  if (kv * n_pairs == 0) return SP_OK;
  const int32_t* pin = pair + (inverse ? kv * n_pairs : 0);
  const int32_t* pout = pair + (inverse ? 0 : kv * n_pairs);
  const int64_t blocks = cdiv(kv * n_pairs, 256);
  SP_CHECK_ARG(blocks <= kMaxGridX, "native_to_tables: too large");
  native_scatter<<<unsigned(blocks), 256, 0, s>>>(pin, pout, kv, n_pairs, n_in, n_out, pf, pb);
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
