// Sparse max/avg pooling through gather tables (spconv_triton/pytorch/_impl/
// pool.py).  One thread per (row, channel); a workgroup covers 4 rows x 64
// channels, so the 64 lanes of a wave read one row's channels contiguously and
// the table entry of the row is a broadcast load.
//
// Numerics follow the reference exactly: fp32 accumulator (fp64 for double
// inputs), max starts at 0 (all-negative windows give 0, pool.py:75-76),
// max-pool backward routes the gradient to every input equal to the output
// (pool.py:134-149), sums run over k in ascending order, and avg-pool backward
// multiplies by the window count (pool.py:251-252).  Terms the reference adds
// as +0.0 are skipped here, which leaves every fp32/fp64 sum unchanged (the
// accumulator starts at +0.0 and can never become -0.0 by addition).
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
  dim3 grid;
  int rc = grid_for(n_out, C, &grid);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
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
  dim3 grid;
  int rc = grid_for(n_in, C, &grid);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
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
  dim3 grid;
  int rc = grid_for(n_out, C, &grid);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
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
  dim3 grid;
  int rc = grid_for(n_in, C, &grid);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  SP_POOL_DISPATCH(dtype, (avgpool_bwd_kernel<T><<<grid, dim3(64, 4), 0, s>>>(
                              static_cast<const T*>(gout), count, n_out, C, pb, kv, n_in,
                              static_cast<T*>(dx))));
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
