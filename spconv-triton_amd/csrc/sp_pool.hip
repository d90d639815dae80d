// Sparse max/avg pooling through gather tables (spconv_triton/pytorch/_impl/
// pool.py).
//
// Vector kernels (rows of a whole number of 16-byte pieces, up to 256 pieces,
// 16-byte aligned): one thread per 16-byte piece of a row; a 256-thread
// workgroup covers 256 / P2 rows, P2 the piece count rounded up to a power of
// two.  A thread loads 8 table entries, then the 8 rows they name, before it
// reduces any of them, so a wave keeps 8 gathers per lane in flight.  Row
// loads are raw buffer loads: an absent entry (-1) reads zeros, which leave a
// max that starts at 0 and every sum unchanged, so no load waits behind a
// branch.  Workgroups are spread over the XCDs in contiguous ranges, so a
// table line is read by one XCD's L2 (with round-robin placement the 8 XCDs
// each fetched the lines their neighbours also read: max-pool forward read
// twice its algorithmic bytes).
//
// Scalar kernels (other widths): one thread per (row, channel); a workgroup
// covers 4 rows x 64 channels.
//
// Numerics follow the reference exactly: fp32 accumulator (fp64 for double
// inputs), max starts at 0 (all-negative windows give 0, pool.py:75-76),
// max-pool backward routes the gradient to every input equal to the output
// (pool.py:134-149), sums run over k in ascending order, and avg-pool backward
// multiplies by the window count (pool.py:251-252).  Terms the reference adds
// as +0.0 are skipped (or added as +0.0) here, which leaves every fp32/fp64
// sum unchanged (the accumulator starts at +0.0 and can never become -0.0 by
// addition).
#include <initializer_list>

#include "sp_common.h"

namespace sp {

template <typename T>
struct Acc {
  using type = float;
};
template <>
struct Acc<double> {
  using type = double;
};

template <typename T>
__device__ __forceinline__ typename Acc<T>::type widen(T v) {
  return typename Acc<T>::type(v);
}

template <typename T>
__global__ __launch_bounds__(256) void maxpool_fwd_kernel(const T* __restrict__ x, int64_t n_in,
                                                          int64_t C, const int32_t* __restrict__ pf,
                                                          int64_t kv, int64_t n_out,
                                                          T* __restrict__ out) {
  using A = typename Acc<T>::type;
  const int64_t m = int64_t(blockIdx.x) * 4 + threadIdx.y;
  const int64_t c = int64_t(blockIdx.y) * 64 + threadIdx.x;
  if (m >= n_out || c >= C) return;
  A acc = A(0);
  for (int64_t k = 0; k < kv; ++k) {
    const int32_t j = pf[k * n_out + m];
    if (j < 0 || j >= n_in) continue;
    const A v = widen(x[int64_t(j) * C + c]);
    acc = v > acc ? v : acc;
  }
  out[m * C + c] = T(acc);
}

template <typename T>
__global__ __launch_bounds__(256) void maxpool_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ out, const T* __restrict__ g, int64_t n_in,
    int64_t C, const int32_t* __restrict__ pb, int64_t kv, int64_t n_out, T* __restrict__ dx) {
  using A = typename Acc<T>::type;
  const int64_t j = int64_t(blockIdx.x) * 4 + threadIdx.y;
  const int64_t c = int64_t(blockIdx.y) * 64 + threadIdx.x;
  if (j >= n_in || c >= C) return;
  const T f = x[j * C + c];
  A acc = A(0);
  for (int64_t k = 0; k < kv; ++k) {
    const int32_t m = pb[k * n_in + j];
    if (m < 0 || m >= n_out) continue;
    if (out[int64_t(m) * C + c] == f) acc += widen(g[int64_t(m) * C + c]);
  }
  dx[j * C + c] = T(acc);
}

template <typename T>
__global__ __launch_bounds__(256) void avgpool_fwd_kernel(const T* __restrict__ x, int64_t n_in,
                                                          int64_t C, const int32_t* __restrict__ pf,
                                                          int64_t kv, int64_t n_out,
                                                          T* __restrict__ out,
                                                          int32_t* __restrict__ count) {
  using A = typename Acc<T>::type;
  const int64_t m = int64_t(blockIdx.x) * 4 + threadIdx.y;
  const int64_t c = int64_t(blockIdx.y) * 64 + threadIdx.x;
  if (m >= n_out || c >= C) return;
  A acc = A(0);
  int32_t cnt = 0;
  for (int64_t k = 0; k < kv; ++k) {
    const int32_t j = pf[k * n_out + m];
    if (j < 0 || j >= n_in) continue;
    acc += widen(x[int64_t(j) * C + c]);
    ++cnt;
  }
  acc = acc / A(cnt > 1 ? cnt : 1);
  out[m * C + c] = T(acc);
  if (count && c == 0) count[m] = cnt;
}

template <typename T>
__global__ __launch_bounds__(256) void avgpool_bwd_kernel(
    const T* __restrict__ g, const int32_t* __restrict__ count, int64_t n_out, int64_t C,
    const int32_t* __restrict__ pb, int64_t kv, int64_t n_in, T* __restrict__ dx) {
  // product and sum rounded separately, like the reference's
  // acc += where(ok, g * cnt, 0): no fused multiply-add here
#pragma clang fp contract(off)
  using A = typename Acc<T>::type;
  const int64_t j = int64_t(blockIdx.x) * 4 + threadIdx.y;
  const int64_t c = int64_t(blockIdx.y) * 64 + threadIdx.x;
  if (j >= n_in || c >= C) return;
  A acc = A(0);
  for (int64_t k = 0; k < kv; ++k) {
    const int32_t m = pb[k * n_in + j];
    if (m < 0 || m >= n_out) continue;
    acc += widen(g[int64_t(m) * C + c]) * A(count[m]);
  }
  dx[j * C + c] = T(acc);
}

// ---------------------------------------------------------------------------
// Vector kernels

constexpr uint32_t kPoolOob = 0xFFFFFFF0u;  // buffer offset that reads zeros
constexpr int64_t kPoolMaxBytes = 0xFFFFFF00LL;  // buffer size limit (host check)
constexpr int kPoolBatch = 8;                // table entries loaded before use

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pool_rsrc(const void* p, int64_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, int(uint32_t(bytes)),
                                           0x00020000);
}

// Contiguous block ranges per XCD (workgroup b runs on XCD b % 8).
__device__ __forceinline__ int64_t pool_block(int64_t b, int64_t nb) {
  const int64_t q = nb / 8, r = nb % 8;
  const int64_t x = b % 8, local = b / 8;
  return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

using Raw16 = __attribute__((ext_vector_type(4))) uint32_t;

template <typename T>
struct Piece {
  static constexpr int V = 16 / int(sizeof(T));
  using A = typename Acc<T>::type;
  A v[V];
  __device__ __forceinline__ void load(Raw16 raw) {
    T e[V];
    __builtin_memcpy(e, &raw, 16);
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = widen(e[i]);
  }
  __device__ __forceinline__ Raw16 pack() const {
    T e[V];
#pragma unroll
    for (int i = 0; i < V; ++i) e[i] = T(v[i]);
    Raw16 raw;
    __builtin_memcpy(&raw, e, 16);
    return raw;
  }
};

// Row and piece of this thread; false for threads past the last row or piece.
__device__ __forceinline__ bool pool_slot(int64_t rows, int32_t P, int32_t pshift, int64_t* row,
                                          int32_t* piece) {
  const int64_t b = pool_block(blockIdx.x, gridDim.x);
  const int t = int(threadIdx.x);
  *piece = t & ((1 << pshift) - 1);
  *row = b * (256 >> pshift) + (t >> pshift);
  return *row < rows && *piece < P;
}

// Table entries k0..k0+7 of row r (an [kv, rows] table); -1 past kv.
__device__ __forceinline__ void load_entries(__amdgpu_buffer_rsrc_t rt, int32_t k0, int32_t kv,
                                             int64_t rows, int64_t r, int32_t (&e)[kPoolBatch]) {
#pragma unroll
  for (int u = 0; u < kPoolBatch; ++u) {
    const bool in = k0 + u < kv;
    const uint32_t off = in ? uint32_t(((k0 + u) * rows + r) * 4) : kPoolOob;
    const int32_t v = int32_t(__builtin_amdgcn_raw_buffer_load_b32(rt, off, 0, 0));
    e[u] = in ? v : -1;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void maxpool_fwd_vec(const T* __restrict__ x, int64_t n_in,
                                                       int32_t P, int32_t pshift,
                                                       const int32_t* __restrict__ pf, int32_t kv,
                                                       int64_t n_out, T* __restrict__ out) {
  using A = typename Acc<T>::type;
  constexpr int V = Piece<T>::V;
  int64_t m;
  int32_t piece;
  if (!pool_slot(n_out, P, pshift, &m, &piece)) return;
  const uint32_t row_bytes = uint32_t(P) * 16;
  const __amdgpu_buffer_rsrc_t rx = pool_rsrc(x, n_in * row_bytes);
  const __amdgpu_buffer_rsrc_t rt = pool_rsrc(pf, int64_t(kv) * n_out * 4);
  Piece<T> acc;
#pragma unroll
  for (int i = 0; i < V; ++i) acc.v[i] = A(0);
  for (int32_t k0 = 0; k0 < kv; k0 += kPoolBatch) {
    int32_t j[kPoolBatch];
    load_entries(rt, k0, kv, n_out, m, j);
    Raw16 raw[kPoolBatch];
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      const bool ok = j[u] >= 0 && j[u] < n_in;
      raw[u] = __builtin_amdgcn_raw_buffer_load_b128(
          rx, ok ? uint32_t(j[u]) * row_bytes + uint32_t(piece) * 16 : kPoolOob, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      Piece<T> p;
      p.load(raw[u]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc.v[i] = p.v[i] > acc.v[i] ? p.v[i] : acc.v[i];
    }
  }
  *reinterpret_cast<Raw16*>(reinterpret_cast<char*>(out) + m * row_bytes + piece * 16) =
      acc.pack();
}

template <typename T>
__global__ __launch_bounds__(256) void maxpool_bwd_vec(
    const T* __restrict__ x, const T* __restrict__ out, const T* __restrict__ g, int64_t n_in,
    int32_t P, int32_t pshift, const int32_t* __restrict__ pb, int32_t kv, int64_t n_out,
    T* __restrict__ dx) {
  using A = typename Acc<T>::type;
  constexpr int V = Piece<T>::V;
  int64_t j;
  int32_t piece;
  if (!pool_slot(n_in, P, pshift, &j, &piece)) return;
  const uint32_t row_bytes = uint32_t(P) * 16;
  const __amdgpu_buffer_rsrc_t ro = pool_rsrc(out, n_out * row_bytes);
  const __amdgpu_buffer_rsrc_t rg = pool_rsrc(g, n_out * row_bytes);
  const __amdgpu_buffer_rsrc_t rt = pool_rsrc(pb, int64_t(kv) * n_in * 4);
  Piece<T> f;
  f.load(*reinterpret_cast<const Raw16*>(reinterpret_cast<const char*>(x) + j * row_bytes +
                                         piece * 16));
  Piece<T> acc;
#pragma unroll
  for (int i = 0; i < V; ++i) acc.v[i] = A(0);
  for (int32_t k0 = 0; k0 < kv; k0 += kPoolBatch) {
    int32_t m[kPoolBatch];
    load_entries(rt, k0, kv, n_in, j, m);
    Raw16 ro_raw[kPoolBatch], rg_raw[kPoolBatch];
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      const bool ok = m[u] >= 0 && m[u] < n_out;
      const uint32_t off = ok ? uint32_t(m[u]) * row_bytes + uint32_t(piece) * 16 : kPoolOob;
      ro_raw[u] = __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0);
      rg_raw[u] = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      Piece<T> o, gg;
      o.load(ro_raw[u]);
      gg.load(rg_raw[u]);
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (o.v[i] == f.v[i]) acc.v[i] += gg.v[i];
    }
  }
  *reinterpret_cast<Raw16*>(reinterpret_cast<char*>(dx) + j * row_bytes + piece * 16) =
      acc.pack();
}

template <typename T>
__global__ __launch_bounds__(256) void avgpool_fwd_vec(const T* __restrict__ x, int64_t n_in,
                                                       int32_t P, int32_t pshift,
                                                       const int32_t* __restrict__ pf, int32_t kv,
                                                       int64_t n_out, T* __restrict__ out,
                                                       int32_t* __restrict__ count) {
  using A = typename Acc<T>::type;
  constexpr int V = Piece<T>::V;
  int64_t m;
  int32_t piece;
  if (!pool_slot(n_out, P, pshift, &m, &piece)) return;
  const uint32_t row_bytes = uint32_t(P) * 16;
  const __amdgpu_buffer_rsrc_t rx = pool_rsrc(x, n_in * row_bytes);
  const __amdgpu_buffer_rsrc_t rt = pool_rsrc(pf, int64_t(kv) * n_out * 4);
  Piece<T> acc;
#pragma unroll
  for (int i = 0; i < V; ++i) acc.v[i] = A(0);
  int32_t cnt = 0;
  for (int32_t k0 = 0; k0 < kv; k0 += kPoolBatch) {
    int32_t j[kPoolBatch];
    load_entries(rt, k0, kv, n_out, m, j);
    Raw16 raw[kPoolBatch];
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      const bool ok = j[u] >= 0 && j[u] < n_in;
      cnt += ok ? 1 : 0;
      raw[u] = __builtin_amdgcn_raw_buffer_load_b128(
          rx, ok ? uint32_t(j[u]) * row_bytes + uint32_t(piece) * 16 : kPoolOob, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      Piece<T> p;
      p.load(raw[u]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc.v[i] += p.v[i];
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i) acc.v[i] = acc.v[i] / A(cnt > 1 ? cnt : 1);
  *reinterpret_cast<Raw16*>(reinterpret_cast<char*>(out) + m * row_bytes + piece * 16) =
      acc.pack();
  if (count && piece == 0) count[m] = cnt;
}

template <typename T>
__global__ __launch_bounds__(256) void avgpool_bwd_vec(
    const T* __restrict__ g, const int32_t* __restrict__ count, int64_t n_out, int32_t P,
    int32_t pshift, const int32_t* __restrict__ pb, int32_t kv, int64_t n_in,
    T* __restrict__ dx) {
  // product and sum rounded separately, like the reference's
  // acc += where(ok, g * cnt, 0): no fused multiply-add here
#pragma clang fp contract(off)
  using A = typename Acc<T>::type;
  constexpr int V = Piece<T>::V;
  int64_t j;
  int32_t piece;
  if (!pool_slot(n_in, P, pshift, &j, &piece)) return;
  const uint32_t row_bytes = uint32_t(P) * 16;
  const __amdgpu_buffer_rsrc_t rg = pool_rsrc(g, n_out * row_bytes);
  const __amdgpu_buffer_rsrc_t rc = pool_rsrc(count, n_out * 4);
  const __amdgpu_buffer_rsrc_t rt = pool_rsrc(pb, int64_t(kv) * n_in * 4);
  Piece<T> acc;
#pragma unroll
  for (int i = 0; i < V; ++i) acc.v[i] = A(0);
  for (int32_t k0 = 0; k0 < kv; k0 += kPoolBatch) {
    int32_t m[kPoolBatch];
    load_entries(rt, k0, kv, n_in, j, m);
    Raw16 raw[kPoolBatch];
    int32_t c[kPoolBatch];
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      const bool ok = m[u] >= 0 && m[u] < n_out;
      raw[u] = __builtin_amdgcn_raw_buffer_load_b128(
          rg, ok ? uint32_t(m[u]) * row_bytes + uint32_t(piece) * 16 : kPoolOob, 0, 0);
      c[u] = int32_t(__builtin_amdgcn_raw_buffer_load_b32(rc, ok ? uint32_t(m[u]) * 4 : kPoolOob,
                                                          0, 0));
    }
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      Piece<T> p;
      p.load(raw[u]);
      const A cu = A(c[u]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc.v[i] += p.v[i] * cu;
    }
  }
  *reinterpret_cast<Raw16*>(reinterpret_cast<char*>(dx) + j * row_bytes + piece * 16) =
      acc.pack();
}

// Vector-kernel geometry of rows of C elements of e bytes: false when the
// scalar kernels must run (width not a whole number of 16-byte pieces, over
// 256 pieces, an unaligned pointer, or a buffer beyond 32-bit offsets).
static bool vec_geometry(int64_t C, int64_t e, int64_t max_rows, int64_t table_entries,
                         std::initializer_list<const void*> ptrs, int32_t* P, int32_t* pshift) {
  if (e == 0 || (C * e) % 16 != 0 || C * e / 16 > 256) return false;
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15) != 0) return false;
  if (max_rows * C * e > kPoolMaxBytes || table_entries * 4 > kPoolMaxBytes) return false;
  *P = int32_t(C * e / 16);
  int32_t s = 0;
  while ((1 << s) < *P) ++s;
  *pshift = s;
  return true;
}

static int64_t pool_elem_bytes(int32_t dtype) {
  switch (dtype) {
    case SP_F16: case SP_BF16: return 2;
    case SP_F32: return 4;
    case SP_F64: return 8;
    default: return 0;  // the dispatch rejects it
  }
}

static int vec_grid(int64_t rows, int32_t pshift, dim3* grid) {
  const int64_t nb = cdiv(rows, int64_t(256 >> pshift));
  SP_CHECK_ARG(nb <= kMaxGridX, "pool: too many rows");
  *grid = dim3(unsigned(nb));
  return SP_OK;
}

static int grid_for(int64_t rows, int64_t C, dim3* grid) {
  const int64_t gx = cdiv(rows, 4);
  const int64_t gy = cdiv(C, 64);
  SP_CHECK_ARG(gx <= kMaxGridX && gy <= 65535, "pool: too many rows/channels");
  *grid = dim3(unsigned(gx), unsigned(gy));
  return SP_OK;
}

#define SP_POOL_DISPATCH(dtype, CALL)                                           \
  switch (dtype) {                                                              \
    case SP_F16: { using T = _Float16; CALL; break; }                           \
    case SP_BF16: { using T = __bf16; CALL; break; }                            \
    case SP_F32: { using T = float; CALL; break; }                              \
    case SP_F64: { using T = double; CALL; break; }                             \
    default: return set_error(SP_ERR_UNSUPPORTED, "pool: dtype %d", int(dtype)); \
  }

}  // namespace sp

using namespace sp;

extern "C" {

int sp_maxpool_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C, const int32_t* pf,
                   int64_t kv, int64_t n_out, void* out, void* stream) {
  SP_CHECK_ARG(n_in >= 0 && C >= 0 && kv >= 1 && n_out >= 0, "maxpool_fwd: bad sizes");
  if (n_out == 0 || C == 0) return SP_OK;
  SP_CHECK_ARG(x && pf && out, "maxpool_fwd: null pointer");
  hipStream_t s = as_stream(stream);
  int32_t P, pshift;
  dim3 grid;
  int rc;
  if (kv <= INT32_MAX &&
      vec_geometry(C, pool_elem_bytes(dtype), n_in > n_out ? n_in : n_out, kv * n_out,
                   {x, out}, &P, &pshift)) {
    if ((rc = vec_grid(n_out, pshift, &grid))) return rc;
    SP_POOL_DISPATCH(dtype, (maxpool_fwd_vec<T><<<grid, 256, 0, s>>>(
                                static_cast<const T*>(x), n_in, P, pshift, pf, int32_t(kv), n_out,
                                static_cast<T*>(out))));
    SP_LAUNCHED();
    return SP_OK;
  }
  if ((rc = grid_for(n_out, C, &grid))) return rc;
  SP_POOL_DISPATCH(dtype, (maxpool_fwd_kernel<T><<<grid, dim3(64, 4), 0, s>>>(
                              static_cast<const T*>(x), n_in, C, pf, kv, n_out, static_cast<T*>(out))));
  SP_LAUNCHED();
  return SP_OK;
}

int sp_maxpool_bwd(const void* x, const void* out, const void* gout, int32_t dtype, int64_t n_in,
                   int64_t C, const int32_t* pb, int64_t kv, int64_t n_out, void* dx,
                   void* stream) {
  SP_CHECK_ARG(n_in >= 0 && C >= 0 && kv >= 1 && n_out >= 0, "maxpool_bwd: bad sizes");
  if (n_in == 0 || C == 0) return SP_OK;
  SP_CHECK_ARG(x && out && gout && pb && dx, "maxpool_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  int32_t P, pshift;
  dim3 grid;
  int rc;
  if (kv <= INT32_MAX &&
      vec_geometry(C, pool_elem_bytes(dtype), n_in > n_out ? n_in : n_out, kv * n_in,
                   {x, out, gout, dx}, &P, &pshift)) {
    if ((rc = vec_grid(n_in, pshift, &grid))) return rc;
    SP_POOL_DISPATCH(dtype, (maxpool_bwd_vec<T><<<grid, 256, 0, s>>>(
                                static_cast<const T*>(x), static_cast<const T*>(out),
                                static_cast<const T*>(gout), n_in, P, pshift, pb, int32_t(kv),
                                n_out, static_cast<T*>(dx))));
    SP_LAUNCHED();
    return SP_OK;
  }
  if ((rc = grid_for(n_in, C, &grid))) return rc;
  SP_POOL_DISPATCH(dtype, (maxpool_bwd_kernel<T><<<grid, dim3(64, 4), 0, s>>>(
                              static_cast<const T*>(x), static_cast<const T*>(out),
                              static_cast<const T*>(gout), n_in, C, pb, kv, n_out,
                              static_cast<T*>(dx))));
  SP_LAUNCHED();
  return SP_OK;
}

int sp_avgpool_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C, const int32_t* pf,
                   int64_t kv, int64_t n_out, void* out, int32_t* count, void* stream) {
  SP_CHECK_ARG(n_in >= 0 && C >= 0 && kv >= 1 && n_out >= 0, "avgpool_fwd: bad sizes");
  if (n_out == 0 || C == 0) return SP_OK;
  SP_CHECK_ARG(x && pf && out, "avgpool_fwd: null pointer");
  hipStream_t s = as_stream(stream);
  int32_t P, pshift;
  dim3 grid;
  int rc;
  if (kv <= INT32_MAX &&
      vec_geometry(C, pool_elem_bytes(dtype), n_in > n_out ? n_in : n_out, kv * n_out,
                   {x, out}, &P, &pshift)) {
    if ((rc = vec_grid(n_out, pshift, &grid))) return rc;
    SP_POOL_DISPATCH(dtype, (avgpool_fwd_vec<T><<<grid, 256, 0, s>>>(
                                static_cast<const T*>(x), n_in, P, pshift, pf, int32_t(kv), n_out,
                                static_cast<T*>(out), count)));
    SP_LAUNCHED();
    return SP_OK;
  }
  if ((rc = grid_for(n_out, C, &grid))) return rc;
  SP_POOL_DISPATCH(dtype, (avgpool_fwd_kernel<T><<<grid, dim3(64, 4), 0, s>>>(
                              static_cast<const T*>(x), n_in, C, pf, kv, n_out,
                              static_cast<T*>(out), count)));
  SP_LAUNCHED();
  return SP_OK;
}

int sp_avgpool_bwd(const void* gout, const int32_t* count, int32_t dtype, int64_t n_out,
                   int64_t C, const int32_t* pb, int64_t kv, int64_t n_in, void* dx,
                   void* stream) {
  SP_CHECK_ARG(n_in >= 0 && C >= 0 && kv >= 1 && n_out >= 0, "avgpool_bwd: bad sizes");
  if (n_in == 0 || C == 0) return SP_OK;
  SP_CHECK_ARG(gout && count && pb && dx, "avgpool_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  int32_t P, pshift;
  dim3 grid;
  int rc;
  if (kv <= INT32_MAX && n_out * 4 <= kPoolMaxBytes &&
      vec_geometry(C, pool_elem_bytes(dtype), n_in > n_out ? n_in : n_out, kv * n_in,
                   {gout, dx}, &P, &pshift)) {
    if ((rc = vec_grid(n_in, pshift, &grid))) return rc;
    SP_POOL_DISPATCH(dtype, (avgpool_bwd_vec<T><<<grid, 256, 0, s>>>(
                                static_cast<const T*>(gout), count, n_out, P, pshift, pb,
                                int32_t(kv), n_in, static_cast<T*>(dx))));
    SP_LAUNCHED();
    return SP_OK;
  }
  if ((rc = grid_for(n_in, C, &grid))) return rc;
  SP_POOL_DISPATCH(dtype, (avgpool_bwd_kernel<T><<<grid, dim3(64, 4), 0, s>>>(
                              static_cast<const T*>(gout), count, n_out, C, pb, kv, n_in,
                              static_cast<T*>(dx))));
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
