// Implicit gather-GEMM for sparse convolution on gfx950 (CDNA4 MFMA).
//
// Forward and input-gradient share one output-stationary kernel
// (the reference does the same, spconv_triton/pytorch/_impl/gemm.py:206-321):
//
//   out[m, n] = bias[n] + sum_k sum_r A[pairs[k, m], r] * B[k][n][r]
//
// The kernels themselves (sp_gather_gemm.h): a workgroup owns 256 output rows
// x 64 output columns, a wave 64 x 64 as 2 x 2 tiles of 32x32 MFMAs.  Gathered
// A rows come from LDS, where the tile's distinct source rows are staged once
// per 64-byte reduction chunk using a gather plan (sp_plan.h), or straight
// from global memory when there is no plan (or the tile's rows do not fit).  B (the weights) is relaid once into [k][r / V][n][V]
// (V elements = 16 bytes), which makes every B operand load a coalesced 1 KiB
// read.  Any assignment of reduction indices to (MFMA step, lane group,
// element) is valid as long as A and B use the same one.
//
// Masked mode (MaskImplicitGemm, gemm.py:282-296): the reference visits rows in
// mask_argsort order to skip offsets that are empty for a whole tile.  Here the
// kernels skip such offsets per tile (staged) or 64-row wave tile (direct) by
// themselves and by default keep the rows' natural order, whose tiles share
// most of their source rows.  For sparse tables, whose natural tiles have a
// pair for most offsets but in few rows, the ordered entry point takes the
// rows in a given order (the stable mask argsort): the table is permuted once
// (sp_permute_table), tile row i is output row order[i], and rows with equal
// masks share tiles, so far fewer offsets are live per tile.  Skipped terms
// are exactly zero and every row sums its offsets in ascending order, so all
// orders give the same result bit for bit.
//
// Weight gradient (gemm.py:324-426): per offset k, dW[k] = X_k^T G_k over the
// compacted pairs of that offset.  The pair dimension is the MFMA reduction
// dimension, so gathered rows are staged in LDS transposed ([channel][pair])
// and read back as 16-byte MFMA operands.  The pair list of each offset is cut
// into `splits` contiguous ranges whose fp32 partials are summed in a fixed
// order by a second kernel (deterministic, no atomics).
#include <mutex>
#include <type_traits>

#include "sp_common.h"
#include "sp_plan.h"

namespace sp {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
  using frag = half8;
  static constexpr int V = 8;       // elements per 16-byte lane load
  static constexpr int KSTEP = 16;  // reduction indices per step (2 halves x V)
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, floatx16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<__bf16> {
  using frag = bf16x8;
  static constexpr int V = 8;
  static constexpr int KSTEP = 16;
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, floatx16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  using frag = float4v;
  static constexpr int V = 4;
  static constexpr int KSTEP = 8;
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, floatx16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c, 0, 0, 0);
  }
};

__device__ __forceinline__ float to_f32(_Float16 v) { return float(v); }
__device__ __forceinline__ float to_f32(__bf16 v) { return float(v); }
__device__ __forceinline__ float to_f32(float v) { return v; }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return _Float16(v); }
template <>
__device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return __bf16(v); }
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }

__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case SP_F16: return float(static_cast<const _Float16*>(p)[i]);
    case SP_BF16: return float(static_cast<const __bf16*>(p)[i]);
    case SP_F32: return static_cast<const float*>(p)[i];
    default: return float(static_cast<const double*>(p)[i]);
  }
}

// bf16 parts of an fp32 value v: hi = bf16(v) and lo = bf16(v - hi) (v - hi
// is exact in fp32).  hi*hi' + hi*lo' + lo*hi' on the bf16 matrix cores, with
// fp32 accumulation, recovers the fp32 product to about 2^-16 relative: the
// split-bf16 method of Henry, Tang & Heinecke, "Leveraging the bfloat16
// artificial intelligence datatype for higher-precision computations", ARITH
// 2019.  It serves SPCONV_ALLOW_TF32 (the reference's tl.dot in TF32,
// gemm.py:46-71, :456-463), at a precision above TF32's (2^-11).
__device__ __forceinline__ float split_part(float v, bool lo) {
  const float hi = float(__bf16(v));
  return lo ? v - hi : hi;
}

// ---------------------------------------------------------------------------
// weight relayout: KRSC [K][kv][C] -> Bt[k][r/V][n][V] (zero padded in r)
//   forward: n = output channel (K), r = input channel (C)
//   dgrad:   n = input channel (C),  r = output channel (K)
// ---------------------------------------------------------------------------
// One launch writes both parts of a packed weight: the relaid B, one 16-byte
// piece (V elements) per thread, and, from its first N threads, the fp32 bias
// (zeros without one).  The packed buffer stays below 1 GiB, so indices fit
// in 32 bits.
template <typename T>
__global__ void relayout_weight(const void* __restrict__ w, int w_dtype, int K, int kv, int C,
                                int transpose, int N, int R, int Rp, int split_r,
                                T* __restrict__ bt, const void* __restrict__ bias,
                                float* __restrict__ bias_out) {
  constexpr int V = Mfma<T>::V;
  const int pieces = kv * (Rp / V) * N;
  const int i = int(blockIdx.x) * int(blockDim.x) + int(threadIdx.x);
  if (i < N) bias_out[i] = bias ? load_any(bias, w_dtype, i) : 0.f;
  if (i >= pieces) return;
  const int n = i % N;
  const int t = i / N;
  const int rv = t % (Rp / V);
  const int k = t / (Rp / V);
  T vals[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    int r = rv * V + e;
    float v = 0.f;
    if (r < R) {
      // split_r > 0: the reduction axis holds [hi | lo | hi] of the weight's
      // own split_r-long axis (bf16 parts of an fp32 weight, see split_part)
      const int part = split_r ? r / split_r : 0;
      if (split_r) r -= part * split_r;
      const int64_t src =
          transpose ? (int64_t(r) * kv + k) * C + n : (int64_t(n) * kv + k) * C + r;
      v = load_any(w, w_dtype, src);
      if (split_r) v = split_part(v, part == 1);
    }
    vals[e] = from_f32<T>(v);
  }
  *reinterpret_cast<uint4*>(bt + int64_t(i) * V) = __builtin_bit_cast(uint4, vals);
}

// ---------------------------------------------------------------------------
// forward / dgrad gather-GEMM
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag load_frag_vec(const T* p) {
  return *reinterpret_cast<const typename Mfma<T>::frag*>(p);
}

#include "sp_gather_gemm.h"

// ---------------------------------------------------------------------------
// weight gradient
// ---------------------------------------------------------------------------
// dW[n, k, c] = sum over the pairs (i, o) of offset k of X[i, c] * G[o, n]:
// per offset a GEMM whose reduction runs over that offset's compacted pair
// list.  A workgroup owns (offset k, a contiguous share of its pairs, a
// BW x BW block of (c, n)); each wave a BW/2 x BW/2 block of 32x32 MFMA tiles.
// The MFMA operands need the pair index as the reduction index, i.e. X and G
// transposed, so the rows gathered for a stage of pairs are written to LDS as
// [channel][pair] (two pairs per write) and read back as 16-byte fragments.
// Gathers are 16-byte vector loads; the next stage's rows and the pair indices
// two stages ahead are in flight while the stage's MFMAs run.  Every (c, n)
// block gathers the rows of all its pairs again, so wide layers take
// BW = 128: half the gathered bytes of BW = 64 at C, K >= 128.
// fp32 partials per share are summed in a fixed order by wgrad_reduce
// (deterministic, no atomics).
template <typename T, int BW>
struct WgShape {
  static constexpr int kStage = BW == 64 || sizeof(T) == 2 ? 128 : 64;  // pairs per LDS stage
  static constexpr int kPitch = kStage + Mfma<T>::V;   // LDS row pitch (rows stay 16-B aligned)
  static constexpr int kPairRows = kStage / 2;         // staging threads per channel group
  static constexpr int kGroups = 256 / kPairRows;      // channel groups of the staging threads
  static constexpr int kCh = BW / kGroups;             // channels per staging thread
  static constexpr int kNv = kCh / Mfma<T>::V;         // vectors per thread, tensor and pair
  static constexpr int kMt = BW / 64;                  // 32x32 tiles per wave and dimension
  static_assert(kCh % Mfma<T>::V == 0 && kStage % Mfma<T>::KSTEP == 0, "wgrad staging shape");
  static_assert(2 * BW * kPitch * sizeof(T) <= 72 * 1024, "wgrad LDS");
};

// VEC bit 0: X rows are whole 16-byte vectors (C % V == 0, aligned base),
// bit 1: the same for the G rows; otherwise that tensor is read element-wise.
template <typename T, int VEC, int BW>
__global__ __launch_bounds__(256) void wgrad_partial(
    const T* __restrict__ X, int64_t n_in, const T* __restrict__ G, int64_t n_out, int C, int K,
    int kv, const int32_t* __restrict__ in_rows, const int32_t* __restrict__ out_rows,
    const int32_t* __restrict__ counts, int64_t stride, int splits, float* __restrict__ part,
    uint32_t x_bytes, uint32_t g_bytes, int cblocks, int nblocks) {
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using S = WgShape<T, BW>;
  constexpr int V = MF::V;
  constexpr int KSTEP = MF::KSTEP;
  constexpr uint32_t ES = sizeof(T);
  constexpr int STAGE = S::kStage, NV = S::kNv, MT = S::kMt;
  // 16-bit rows are gathered coalesced: the four lanes of a pair read 64
  // contiguous bytes of its row per load (16 rows per load instruction,
  // against 64 rows of one 16-byte piece each otherwise).
  // The 8-pair columns of their channel-major LDS rows are XOR-swizzled by
  // channel bit 4, so that both the staging writes and the MFMA fragment
  // reads are free of bank conflicts; the swizzle is constant over a thread's
  // 8 channels of a vector, so the write addresses stay base + immediate.
  constexpr bool COAL = sizeof(T) == 2 && STAGE == 128;
  constexpr int PITCH = S::kPitch;
  __shared__ __align__(16) T Xs[BW][PITCH];
  __shared__ __align__(16) T Gs[BW][PITCH];
  // element offset of pair p within channel row c
  auto elem = [](int c, int p) -> int {
    return COAL ? ((((p >> 3) ^ (((c >> 4) & 1) << 2)) << 3) | (p & 7)) : p;
  };

  // (offset, split) pair ks and (c, n) block of this workgroup: the
  // cblocks * nblocks blocks of one pair gather the same pairs' rows (each
  // input row for every n block, each gradient row for every c block), so
  // they run back to back on one XCD (workgroup b runs on XCD b % 8) and the
  // second reader of a row finds it in that XCD's L2
  const int bpk = cblocks * nblocks;
  const int64_t t = blockIdx.x / 8;
  const int64_t ks = (t / bpk) * 8 + blockIdx.x % 8;
  if (ks >= int64_t(kv) * splits) return;  // padding of the last group of 8 pairs
  const int blk = int(t % bpk);
  const int k = int(ks / splits);
  const int split = int(ks % splits);
  const int c0 = (blk / nblocks) * BW, n0 = (blk % nblocks) * BW;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, l32 = lane & 31;
  const int ctile = (wave >> 1) * (BW / 2), ntile = (wave & 1) * (BW / 2);
  // staging role: pairs 2 pp and 2 pp + 1 of a stage and NV vectors of V
  // channels each, vector j at channel ch_of(j): kCh contiguous channels from
  // kCh q, or (COAL) channels 4 V j + V ql of a 4-lane group per pair pair
  const int pp = COAL ? 16 * wave + (lane >> 2) : tid % S::kPairRows;
  const int q = COAL ? (lane & 3) : tid / S::kPairRows;
  auto ch_of = [&](int j) -> int { return COAL ? j * 4 * V + q * V : q * S::kCh + j * V; };

  const int64_t cnt = counts[k];
  const int64_t chunk = (cnt + splits - 1) / splits;
  const int64_t p_lo = split * chunk;
  const int64_t p_hi = p_lo + chunk < cnt ? p_lo + chunk : cnt;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(X, x_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(G, g_bytes);
  const int32_t* ir = in_rows + int64_t(k) * stride;
  const int32_t* orow = out_rows + int64_t(k) * stride;

  // pair indices of stage s0 (-1 past the share's end)
  auto load_idx = [&](int64_t s0, int32_t (&iv)[2], int32_t (&ov)[2]) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t p = s0 + 2 * pp + e;
      const bool ok = p < p_hi;
      const int32_t i = ok ? ir[ok ? p : 0] : -1;
      const int32_t o = ok ? orow[ok ? p : 0] : -1;
      iv[e] = (i >= 0 && i < n_in) ? i : -1;
      ov[e] = (o >= 0 && o < n_out) ? o : -1;
    }
  };
  auto row_off = [&](int32_t r, int ch, int width, int dim) -> uint32_t {
    return (r >= 0 && ch < dim) ? uint32_t((int64_t(r) * width + ch) * ES) : kOob;
  };
  auto load_rows = [&](const int32_t (&iv)[2], const int32_t (&ov)[2], frag (&xv)[2][NV],
                       frag (&gv)[2][NV]) {
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int cx = c0 + ch_of(j), nx = n0 + ch_of(j);
        if (VEC & 1)
          xv[e][j] = buf_frag<T>(rx, row_off(iv[e], cx, C, C));
        else
          xv[e][j] = buf_frag_elems<T>(rx, iv[e] >= 0 ? uint32_t(int64_t(iv[e]) * C * ES) : kOob,
                                       cx, C);
        if (VEC & 2)
          gv[e][j] = buf_frag<T>(rg, row_off(ov[e], nx, K, K));
        else
          gv[e][j] = buf_frag_elems<T>(rg, ov[e] >= 0 ? uint32_t(int64_t(ov[e]) * K * ES) : kOob,
                                       nx, K);
      }
  };
  // channel-major LDS rows: both pairs' values of a channel in one write
  using T2 = __attribute__((ext_vector_type(2))) T;
  auto put_rows = [&](const frag (&xv)[2][NV], const frag (&gv)[2][NV]) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int t = 0; t < V; ++t) {
        const int c = ch_of(j) + t;
        const int e = elem(c, 2 * pp);
        const T2 xp = {xv[0][j][t], xv[1][j][t]};
        const T2 gp = {gv[0][j][t], gv[1][j][t]};
        *reinterpret_cast<T2*>(&Xs[c][e]) = xp;
        *reinterpret_cast<T2*>(&Gs[c][e]) = gp;
      }
  };

  floatx16 acc[MT][MT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < MT; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;

  int32_t iv[2], ov[2], iv2[2], ov2[2];
  frag xv[2][NV], gv[2][NV];
  load_idx(p_lo, iv, ov);
  load_rows(iv, ov, xv, gv);
  load_idx(p_lo + STAGE, iv2, ov2);
  for (int64_t s0 = p_lo; s0 < p_hi; s0 += STAGE) {
    __syncthreads();  // the previous stage's fragments are read
    put_rows(xv, gv);
    __syncthreads();
    // next stage's rows and the indices after it, in flight during the MFMAs
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      iv[e] = iv2[e];
      ov[e] = ov2[e];
    }
    load_rows(iv, ov, xv, gv);
    load_idx(s0 + 2 * STAGE, iv2, ov2);
#pragma unroll
    for (int st = 0; st < STAGE; st += KSTEP) {
      frag a[MT], b[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const int ca = ctile + 32 * m + l32, cb = ntile + 32 * m + l32;
        a[m] = *reinterpret_cast<const frag*>(&Xs[ca][elem(ca, st + h * V)]);
        b[m] = *reinterpret_cast<const frag*>(&Gs[cb][elem(cb, st + h * V)]);
      }
#pragma unroll
      for (int mc = 0; mc < MT; ++mc)
#pragma unroll
        for (int mn = 0; mn < MT; ++mn) MF::mma(a[mc], b[mn], acc[mc][mn]);
    }
  }
  // D[c][n]: lane holds column n = l32 of rows c = 8*(i/4) + 4*h + (i%4)
#pragma unroll
  for (int mc = 0; mc < MT; ++mc)
#pragma unroll
    for (int mn = 0; mn < MT; ++mn) {
      const int n = n0 + ntile + 32 * mn + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int c = c0 + ctile + 32 * mc + (i >> 2) * 8 + h * 4 + (i & 3);
        if (c < C && n < K) part[((int64_t(split) * K + n) * kv + k) * C + c] = acc[mc][mn][i];
      }
    }
}

template <typename T>
__global__ void wgrad_reduce(const float* __restrict__ part, int splits, int64_t total,
                             T* __restrict__ dw) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  float s = 0.f;
  for (int p = 0; p < splits; ++p) s += part[int64_t(p) * total + i];
  dw[i] = from_f32<T>(s);
}

// The weight gradient of split-bf16 operands (SP_BF16X3): the partials hold
// [2K][kv][2C] = the four products of X's and G's [hi | lo] halves, which are
// summed in a fixed order into the fp32 dW [K][kv][C].
__global__ void wgrad_reduce_split(const float* __restrict__ part, int splits, int64_t K,
                                   int64_t kv, int64_t C, float* __restrict__ dw) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = K * kv * C;
  if (i >= total) return;
  const int64_t c = i % C, nk = i / C, k = nk % kv, n = nk / kv;
  const int64_t part_total = 4 * total;
  float s = 0.f;
  for (int p = 0; p < splits; ++p)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        s += part[int64_t(p) * part_total + ((a * K + n) * kv + k) * 2 * C + b * C + c];
  dw[i] = s;
}

// out [rows][parts * cols] bf16 from x [rows][cols] fp32: pattern 0 = [hi |
// hi | lo], 1 = [hi | lo | hi], 2 = [hi | lo] (split_part).  Four columns per
// thread with vec4 (cols % 4 == 0, x 16-byte and out 8-byte aligned).
__global__ void split_bf16_rows(const float* __restrict__ x, int64_t rows, int64_t cols,
                                int pattern, bool vec4, __bf16* __restrict__ out) {
  const int parts = pattern == 2 ? 2 : 3;
  const int64_t per_row = vec4 ? cols / 4 : cols;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t row = i / per_row, q = i % per_row;
  const int width = vec4 ? 4 : 1;
  const int64_t c0 = q * width;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (vec4) {
    const float4 f = *reinterpret_cast<const float4*>(x + row * cols + c0);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    v[0] = x[row * cols + c0];
  }
  __bf16* o = out + row * parts * cols + c0;
  for (int pi = 0; pi < parts; ++pi) {
    const bool lo = pattern == 0 ? pi == 2 : pi == 1;
    __bf16 h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = __bf16(split_part(v[e], lo));
    if (vec4) {
      *reinterpret_cast<uint2*>(o + pi * cols) = __builtin_bit_cast(uint2, h);
    } else {
      o[pi * cols] = h[0];
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int elem_size(int dtype) {
  switch (dtype) {
    case SP_F16: case SP_BF16: case SP_BF16X3: return 2;
    case SP_F32: return 4;
    case SP_F64: return 8;
    default: return 0;
  }
}

static int vec_of(int dtype) { return dtype == SP_F32 ? 4 : 8; }

static int64_t padded(int64_t r, int v) { return (r + v - 1) / v * v; }

// Packed weight buffer: Bt [kv][Rp/V][N][V] of the compute dtype, then the
// bias as N floats at a 256-byte aligned offset.
struct Packed {
  int N, R, Rp;
  size_t bt_bytes, bias_off, total;
};

// SP_BF16X3 (the split-bf16 form of an fp32 weight) is the SP_BF16 layout of a
// reduction three times as long: [hi | lo | hi] along C (forward) or K (dgrad).
static Packed packed_layout(int64_t K, int64_t kv, int64_t C, int dtype, int transpose) {
  Packed p;
  p.N = int(transpose ? C : K);
  p.R = int(transpose ? K : C) * (dtype == SP_BF16X3 ? 3 : 1);
  // the reduction runs in MFMA steps of 4 * V (four lane groups of V each)
  p.Rp = int(padded(p.R, 4 * vec_of(dtype)));
  p.bt_bytes = size_t(kv) * size_t(p.Rp) * size_t(p.N) * size_t(elem_size(dtype));
  p.bias_off = align_up(p.bt_bytes, 256);
  p.total = p.bias_off + align_up(size_t(p.N) * sizeof(float), 256);
  return p;
}

static bool gemm_dtype_ok(int dtype) { return dtype == SP_F16 || dtype == SP_BF16 || dtype == SP_F32; }

static int pack_weight(const void* w, int w_dtype, const void* bias, int64_t K, int64_t kv,
                       int64_t C, int dtype, int transpose, void* packed, hipStream_t s) {
  SP_CHECK_ARG(gemm_dtype_ok(dtype) || dtype == SP_BF16X3,
               "pack: compute dtype %d not supported (f16/bf16/f32/bf16x3)", dtype);
  SP_CHECK_ARG(elem_size(w_dtype) > 0, "pack: weight dtype %d not supported", w_dtype);
  SP_CHECK_ARG(K >= 1 && C >= 1 && kv >= 1 && K < 65536 && C < 65536 && kv < 65536,
               "pack: bad sizes K=%lld kv=%lld C=%lld", (long long)K, (long long)kv, (long long)C);
  SP_CHECK_ARG(w && packed, "pack: null pointer");
  const Packed p = packed_layout(K, kv, C, dtype, transpose);
  SP_CHECK_ARG(p.bt_bytes < kMaxBtBytes, "pack: packed weights of %zu B exceed 1 GiB", p.bt_bytes);
  const int64_t tot = kv * int64_t(p.Rp / vec_of(dtype)) * p.N;  // 16-byte pieces
  const unsigned rb = unsigned(cdiv(tot > p.N ? tot : p.N, 256));
  char* base = static_cast<char*>(packed);
  float* bias_out = reinterpret_cast<float*>(base + p.bias_off);
  switch (dtype) {
    case SP_F16:
      relayout_weight<_Float16><<<rb, 256, 0, s>>>(w, w_dtype, int(K), int(kv), int(C), transpose,
                                                   p.N, p.R, p.Rp, 0, reinterpret_cast<_Float16*>(base),
                                                   bias, bias_out);
      break;
    case SP_BF16:
      relayout_weight<__bf16><<<rb, 256, 0, s>>>(w, w_dtype, int(K), int(kv), int(C), transpose,
                                                 p.N, p.R, p.Rp,
                                                 0, reinterpret_cast<__bf16*>(base), bias,
                                                 bias_out);
      break;
    case SP_BF16X3:
      relayout_weight<__bf16><<<rb, 256, 0, s>>>(w, w_dtype, int(K), int(kv), int(C), transpose,
                                                 p.N, p.R, p.Rp,
                                                 p.R / 3, reinterpret_cast<__bf16*>(base), bias,
                                                 bias_out);
      break;
    default:
      relayout_weight<float><<<rb, 256, 0, s>>>(w, w_dtype, int(K), int(kv), int(C), transpose,
                                                p.N, p.R, p.Rp,
                                                0, reinterpret_cast<float*>(base), bias,
                                                bias_out);
  }
  SP_LAUNCHED();
  return SP_OK;
}

// Launch description shared by the typed launchers.
struct GemmCall {
  int64_t n_src, M;
  int N, R, Rp, kv;
  bool planned;
  PlanDev plan;
  const float* bias;
  const int32_t* order;  // tile row -> output row, or null (natural order)
  const uint32_t* words;  // ordered direct kernel: the rows' mask words (nullable), mic per row
  int mic;
  bool vec;
  int thin;              // planned: 1 the thin kernel (tiles of at most kThinItems items),
                         // 2 its quarter instance with every heavy tile split
};

// Raises a kernel's dynamic LDS limit to `bytes` (once per kernel and process).
static int allow_lds(const void* kern, uint32_t bytes, bool& done) {
  if (!done) {
    SP_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)));
    done = true;
  }
  return SP_OK;
}

template <typename T, typename OutT, bool VEC>
static int launch_direct(dim3 grid, hipStream_t s, const T* A, const T* bt, const int32_t* pairs,
                         OutT* o, GemmBufs nb, const GemmCall& c) {
  const int G = c.kv < kGroupOffsets ? c.kv : kGroupOffsets;
  const uint32_t lds = direct_lds(G + kPad, uint32_t(sizeof(OutT))).total;
  auto kern = c.order ? gather_gemm_direct<T, OutT, VEC, true>
                      : gather_gemm_direct<T, OutT, VEC, false>;
  static bool attr_set[2] = {false, false};  // per kernel instance
  int rc = allow_lds(reinterpret_cast<const void*>(kern),
                     direct_lds(kGroupOffsets + kPad, uint32_t(sizeof(OutT))).total,
                     attr_set[c.order ? 1 : 0]);
  if (rc) return rc;
  kern<<<grid, 256, lds, s>>>(A, bt, pairs, c.order, c.bias, o, nb, c.n_src, c.M, c.N, c.R, c.Rp,
                              c.kv, c.words, c.mic);
  SP_LAUNCHED();
  return SP_OK;
}

// LDS of the staged kernel: its own layout, or the direct path's for an
// overflow tile (smaller for every kv the plans cover; the max keeps it safe).
static uint32_t staged_kernel_lds(int E, int kv, uint32_t out_size) {
  const uint32_t a = staged_lds(E, out_size).total;
  const int G = kv < kGroupOffsets ? kv : kGroupOffsets;
  const uint32_t b = direct_lds(G + kPad, out_size).total;
  return a > b ? a : b;
}

// Compute units of the current device (cached per process: the one-GPU boxes
// this targets hold one kind of device).
static int device_cus() {
  static int n = 0;
  if (n <= 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

// A staged grid of one column block whose tile count exceeds a multiple of the
// CU count by at most kStagedSplitMax tiles splits those last tiles into
// quarters (gather_gemm_staged's SPLIT instances): run whole, they make a
// last round on as many CUs that the rest of the chip waits for.  Measured on
// the 64 -> 64 surface-cloud layer (256 CUs, tiles past 2 or 3 rounds of 256):
// 14 past 768 (the 200k-voxel metric) 49.6 -> 47.9 us, 32 past 768 50.4 ->
// 48.2, 40 past 512 38.8 -> 37.5, 64 past 512 38.9 -> 38.6, 96 past 512
// 39.3 -> 44.8 (the quarters' direct gathers then cost more than the round).
constexpr int kStagedSplitMax = 48;

template <typename T, typename OutT, bool VEC>
static int launch_staged(dim3 grid, hipStream_t s, const T* A, const T* bt, const int32_t* pairs,
                         OutT* o, GemmBufs nb, const GemmCall& c) {
  const uint32_t lds = staged_kernel_lds(c.plan.E, c.kv, uint32_t(sizeof(OutT)));
  int n_split = 0;
  if (!c.order && c.N <= 64) {
    const int64_t nt = cdiv(c.M, kTileRows), ncu = device_cus();
    const int64_t rem = nt % ncu;
    if (nt > ncu && rem > 0 && rem <= kStagedSplitMax) n_split = int(rem);
  }
  auto kern = n_split ? gather_gemm_staged<T, OutT, VEC, false, true>
                      : (c.order ? gather_gemm_staged<T, OutT, VEC, true>
                                 : gather_gemm_staged<T, OutT, VEC, false>);
  static bool attr_set[3] = {false, false, false};  // per kernel instance
  int rc = allow_lds(reinterpret_cast<const void*>(kern),
                     staged_kernel_lds(plan_layout(1, kPlanMaxKv).E, kPlanMaxKv, uint32_t(sizeof(OutT))),
                     attr_set[n_split ? 2 : (c.order ? 1 : 0)]);
  if (rc) return rc;
  if (n_split) {  // the split tiles' quarters in front, the other tiles after them
    const int64_t n_extra = staged_split_extra(n_split);
    SP_CHECK_ARG(n_extra + grid.x - n_split <= kMaxGridX, "gemm: too many tiles");
    grid.x = unsigned(n_extra + grid.x - n_split);
  }
  kern<<<grid, 256, lds, s>>>(A, bt, pairs, c.order, c.plan, c.bias, o, nb, c.n_src, c.M, c.N,
                              c.R, c.Rp, c.kv, n_split);
  SP_LAUNCHED();
  return SP_OK;
}

// LDS of the thin kernel: its own layout, or the direct path's for the tiles
// it hands over.
static uint32_t thin_kernel_lds(int kv, uint32_t out_size) {
  const uint32_t a = thin_lds(out_size).total;
  const int G = kv < kGroupOffsets ? kv : kGroupOffsets;
  const uint32_t b = direct_lds(G + kPad, out_size).total;
  return a > b ? a : b;
}

template <typename T, typename OutT, bool VEC>
static int launch_thin(dim3 grid, hipStream_t s, const T* A, const T* bt, const int32_t* pairs,
                       OutT* o, GemmBufs nb, const GemmCall& c) {
  const uint32_t lds = thin_kernel_lds(c.kv, uint32_t(sizeof(OutT)));
  const bool quarter = sizeof(T) == 4 || grid.x <= kThinQuarterGrid || c.thin == 2;
  auto kern = quarter ? (c.order ? gather_gemm_thin<T, OutT, VEC, true, true>
                                 : gather_gemm_thin<T, OutT, VEC, false, true>)
                      : (c.order ? gather_gemm_thin<T, OutT, VEC, true, false>
                                 : gather_gemm_thin<T, OutT, VEC, false, false>);
  static bool attr_set[4] = {false, false, false, false};  // per kernel instance
  int rc = allow_lds(reinterpret_cast<const void*>(kern),
                     thin_kernel_lds(kPlanMaxKv, uint32_t(sizeof(OutT))),
                     attr_set[(c.order ? 1 : 0) + (quarter ? 2 : 0)]);
  if (rc) return rc;
  const int64_t nt = cdiv(c.M, kTileRows);
  // thin == 2: every tile the direct path takes is spread over four
  // workgroups (tables whose tiles mostly hold more items than the thin
  // layout, with fp32 operands: their waves' MFMAs set the kernel's end)
  const int n_split = !quarter ? 0
                      : c.thin == 2 ? int(nt)
                                    : int(nt < kThinSplitTiles ? nt : kThinSplitTiles);
  const int64_t n_extra = thin_split_extra(n_split, int(cdiv(c.N, 64)));
  SP_CHECK_ARG(n_extra + grid.x <= kMaxGridX, "gemm: too many tiles");
  grid.x = unsigned(n_extra + grid.x);
  kern<<<grid, 256, lds, s>>>(A, bt, pairs, c.order, c.plan, c.bias, o, nb, c.n_src, c.M, c.N,
                              c.R, c.Rp, c.kv, n_split);
  SP_LAUNCHED();
  return SP_OK;
}

// Planned call: the staged kernel (or the thin one) over all tiles (overflow
// tiles take its direct path).  Unplanned call: the direct kernel over all
// tiles.
template <typename T, typename OutT, bool VEC>
static int launch_modes(unsigned gx, unsigned gy, hipStream_t s, const T* A, const T* bt,
                        const int32_t* pairs, OutT* o, GemmBufs nb, const GemmCall& c) {
  // grid order: block_tile (direct) or staged_tile (staged), both 1-D
  const uint64_t nwg = gy == 1 ? uint64_t(gx) : 8ull * gy * ((uint64_t(gx) + 7) / 8);
  SP_CHECK_ARG(nwg <= uint64_t(kMaxGridX), "gemm: too many tiles");
  if (!c.planned)
    return launch_direct<T, OutT, VEC>(dim3{unsigned(nwg), 1u, 1u}, s, A, bt, pairs, o, nb, c);
  if constexpr (VEC) {  // (rows of whole 16-byte pieces; others take the staged kernel)
    if (c.thin)
      return launch_thin<T, OutT, VEC>(dim3{unsigned(nwg), 1u, 1u}, s, A, bt, pairs, o, nb, c);
  }
  return launch_staged<T, OutT, VEC>(dim3{unsigned(nwg), 1u, 1u}, s, A, bt, pairs, o, nb, c);
}

// The mask tables (pair_mask / mask_argsort) of the reference's masked path
// are accepted but not needed: the kernel skips offsets that are empty for a
// whole wave tile by itself and keeps rows in their natural order (better
// locality for the gathers, the table reads and the output writes).
template <typename T, typename OutT>
static int launch_gemm_typed(const T* A, const T* bt, const int32_t* pairs, void* out,
                             const GemmCall& c, hipStream_t s) {
  const int64_t gx = cdiv(c.M, kTileRows);
  SP_CHECK_ARG(gx <= kMaxGridX, "gemm: too many rows");
  // buffer instructions take 32-bit byte offsets
  const int64_t lim = int64_t(kOob);
  const int64_t a_bytes = c.n_src * c.R * int64_t(sizeof(T));
  const int64_t bt_bytes = int64_t(c.kv) * c.Rp * c.N * int64_t(sizeof(T));
  const int64_t p_bytes = int64_t(c.kv) * c.M * 4;
  const int64_t o_bytes = c.M * c.N * int64_t(sizeof(OutT));
  if (a_bytes >= lim || bt_bytes >= lim || p_bytes >= lim || o_bytes >= lim)
    return set_error(SP_ERR_UNSUPPORTED,
                     "gemm: a tensor exceeds 4 GiB (features %lld B, pairs %lld B, out %lld B)",
                     (long long)a_bytes, (long long)p_bytes, (long long)o_bytes);
  if (bt_bytes >= int64_t(kMaxBtBytes))
    return set_error(SP_ERR_UNSUPPORTED, "gemm: packed weights of %lld B exceed 1 GiB",
                     (long long)bt_bytes);
  GemmBufs nb{uint32_t(a_bytes), uint32_t(bt_bytes), uint32_t(p_bytes), uint32_t(o_bytes)};
  const unsigned gy = unsigned(cdiv(c.N, 64));
  OutT* o = static_cast<OutT*>(out);
  if (c.vec) return launch_modes<T, OutT, true>(unsigned(gx), gy, s, A, bt, pairs, o, nb, c);
  return launch_modes<T, OutT, false>(unsigned(gx), gy, s, A, bt, pairs, o, nb, c);
}

template <typename T>
static int launch_gemm_out(int out_dtype, const T* A, const T* bt, const int32_t* pairs,
                           void* out, const GemmCall& c, hipStream_t s) {
  switch (out_dtype) {
    case SP_F16:
      return launch_gemm_typed<T, _Float16>(A, bt, pairs, out, c, s);
    case SP_BF16:
      return launch_gemm_typed<T, __bf16>(A, bt, pairs, out, c, s);
    case SP_F32:
      return launch_gemm_typed<T, float>(A, bt, pairs, out, c, s);
    default:
      return set_error(SP_ERR_UNSUPPORTED, "gemm: output dtype %d not supported", out_dtype);
  }
}

// plan (nullable) is a gather plan of `pairs` built by sp_gather_plan_build;
// order (nullable) maps tile rows to output rows (`pairs` is then the table
// permuted by it).
static int gemm_packed(const void* A, int dtype, int64_t n_src, const void* packed, int64_t K,
                       int64_t kv, int64_t C, int transpose, int has_bias, const int32_t* pairs,
                       int64_t M, const int32_t* pm, const int32_t* ar, const void* plan,
                       size_t plan_bytes, void* out, int out_dtype, hipStream_t s,
                       const int32_t* order = nullptr, int thin = 0,
                       const uint32_t* words = nullptr, int mic = 0) {
  SP_CHECK_ARG(gemm_dtype_ok(dtype), "gemm: feature dtype %d not supported (f16/bf16/f32)", dtype);
  SP_CHECK_ARG(K >= 1 && C >= 1 && kv >= 1 && M >= 0 && n_src >= 0, "gemm: bad sizes");
  SP_CHECK_ARG(K < 65536 && C < 65536 && kv < 65536, "gemm: channel/kernel size too large");
  SP_CHECK_ARG(!((pm == nullptr) ^ (ar == nullptr)), "gemm: pair_mask and argsort go together");
  SP_CHECK_ARG(!(pm && kv > 32), "gemm: masked path needs kv <= 32");
  SP_CHECK_ARG(!words || (order && mic >= (kv + 31) / 32 && mic <= 1024),
               "gemm: row mask words need a row order and >= ceil(kv/32) words per row (%d)", mic);
  SP_CHECK_ARG(thin >= 0 && thin <= 2, "gemm: thin_tiles must be 0, 1 or 2, not %d", thin);
  if (M == 0) return SP_OK;
  SP_CHECK_ARG(A && packed && pairs && out, "gemm: null pointer");
  const Packed p = packed_layout(K, kv, C, dtype, transpose);
  const char* base = static_cast<const char*>(packed);
  GemmCall c;
  c.n_src = n_src;
  c.M = M;
  c.N = p.N;
  c.R = p.R;
  c.Rp = p.Rp;
  c.kv = int(kv);
  c.bias = has_bias ? reinterpret_cast<const float*>(base + p.bias_off) : nullptr;
  c.order = order;
  c.words = words;
  c.mic = words ? mic : 0;
  c.vec = (p.R % vec_of(dtype) == 0) && (reinterpret_cast<uintptr_t>(A) % 16 == 0);
  c.planned = plan != nullptr;
  c.thin = plan != nullptr ? thin : 0;
  c.plan = PlanDev{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0};
  if (plan) {
    SP_CHECK_ARG(kv <= kPlanMaxKv, "gemm: gather plans need kv <= %d", kPlanMaxKv);
    const PlanLayout pl = plan_layout(M, kv);
    SP_CHECK_ARG(plan_bytes >= pl.total, "gemm: plan buffer %zu < %zu bytes", plan_bytes,
                 pl.total);
    c.plan = plan_view(plan, M, kv);
  }
  switch (dtype) {
    case SP_F16:
      return launch_gemm_out<_Float16>(out_dtype, static_cast<const _Float16*>(A),
                                       reinterpret_cast<const _Float16*>(base), pairs, out, c, s);
    case SP_BF16:
      return launch_gemm_out<__bf16>(out_dtype, static_cast<const __bf16*>(A),
                                     reinterpret_cast<const __bf16*>(base), pairs, out, c, s);
    default:
      return launch_gemm_out<float>(out_dtype, static_cast<const float*>(A),
                                    reinterpret_cast<const float*>(base), pairs, out, c, s);
  }
}

// Shared body of forward (transpose = 0) and dgrad (transpose = 1): pack the
// weight into the workspace, then run the packed GEMM.
static int gemm_common(const void* A, int dtype, int64_t n_src, const void* w, int w_dtype,
                       int64_t K, int64_t kv, int64_t C, int transpose, const int32_t* pairs,
                       int64_t M, const void* bias, const int32_t* pm, const int32_t* ar,
                       void* out, int out_dtype, void* ws, size_t ws_bytes, hipStream_t s) {
  SP_CHECK_ARG(gemm_dtype_ok(dtype), "gemm: feature dtype %d not supported (f16/bf16/f32)", dtype);
  if (M == 0) return SP_OK;
  const Packed p = packed_layout(K, kv, C, dtype, transpose);
  if (!ws || ws_bytes < p.total)
    return set_error(SP_ERR_WORKSPACE, "gemm: workspace %zu < %zu", ws_bytes, p.total);
  int rc = pack_weight(w, w_dtype, bias, K, kv, C, dtype, transpose, ws, s);
  if (rc) return rc;
  return gemm_packed(A, dtype, n_src, ws, K, kv, C, transpose, bias != nullptr, pairs, M, pm, ar,
                     nullptr, 0, out, out_dtype, s);
}

// (c, n) block width of the weight-gradient workgroups
static int wgrad_block(int64_t C, int64_t K) { return C >= 128 && K >= 128 ? 128 : 64; }

// Splits per (offset, block): 64 workgroups per offset (at least 512 in all), so that the
// per-split fp32 partials (splits x kv x C x K x 4 bytes, written and read back) stay in
// proportion to the gathered bytes.  Measured over the 12 calls of the ResUNet training step
// (forced split counts 4..64 per call): the best count per call is close to 64 / blocks in
// every call (the 256 -> 256 call at 16, the 64 -> 32 calls at 64), 1.14 -> 0.94 ms in all
// against a target of 1 024 workgroups per call.
static int wgrad_splits(int64_t kv, int64_t C, int64_t K, int64_t n_rows) {
  const int bw = wgrad_block(C, K);
  const int64_t tiles = kv * cdiv(C, bw) * cdiv(K, bw);
  const int64_t target = 64 * kv > 512 ? 64 * kv : 512;
  int64_t splits = cdiv(target, tiles);
  const int64_t by_len = cdiv(n_rows, 1024);    // keep >= ~1k rows of work per split
  if (splits > by_len) splits = by_len;
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  return int(splits);
}

// ---- the forward without a caller workspace (sp_conv_fwd_noalloc) ---------
// The relaid weights and fp32 bias, which sp_conv_fwd writes into its
// workspace, go into this file-scope array instead: one copy per GPU, held
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): the device
// address comes from hipGetSymbolAddress, taken once per device with that
// device current, and kernels receive that pointer.
static_assert(SP_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size is a multiple of 256");
static __device__ __align__(256) unsigned char scratch[SP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Device address of this device's `scratch` (nullptr and an error on failure).
static void* scratch_address(int* rc) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = set_error(SP_ERR_HIP, "fwd_noalloc: no current device (%d)", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = set_error(SP_ERR_HIP, "fwd_noalloc: hipGetSymbolAddress(scratch) failed on device "
                      "%d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = p;
  }
  *rc = SP_OK;
  return addr[dev];
}

}  // namespace sp

using namespace sp;

extern "C" {

size_t sp_conv_workspace_size(int64_t K, int64_t kv, int64_t C, int32_t dtype) {
  const Packed a = packed_layout(K, kv, C, dtype, 0);
  const Packed b = packed_layout(K, kv, C, dtype, 1);
  return a.total > b.total ? a.total : b.total;
}

size_t sp_conv_packed_bytes(int64_t K, int64_t kv, int64_t C, int32_t dtype, int32_t transpose) {
  return packed_layout(K, kv, C, dtype, transpose).total;
}

int sp_conv_pack_weight(const void* w, int32_t w_dtype, const void* bias, int64_t K, int64_t kv,
                        int64_t C, int32_t dtype, int32_t transpose, void* packed,
                        void* stream) {
  return pack_weight(w, w_dtype, bias, K, kv, C, dtype, transpose, packed, as_stream(stream));
}

int sp_conv_gemm_packed(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                        int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                        const int32_t* pairs, int64_t M, const int32_t* pair_mask,
                        const int32_t* mask_argsort, void* out, int32_t out_dtype, void* stream) {
  return gemm_packed(a, dtype, n_src, packed, K, kv, C, transpose, has_bias, pairs, M, pair_mask,
                     mask_argsort, nullptr, 0, out, out_dtype, as_stream(stream));
}

int sp_conv_gemm_planned(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                         int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                         const int32_t* pairs, int64_t M, const void* plan, size_t plan_bytes,
                         void* out, int32_t out_dtype, void* stream) {
  SP_CHECK_ARG(plan != nullptr, "gemm: null gather plan");
  return gemm_packed(a, dtype, n_src, packed, K, kv, C, transpose, has_bias, pairs, M, nullptr,
                     nullptr, plan, plan_bytes, out, out_dtype, as_stream(stream));
}

int sp_conv_gemm_ordered(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                         int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                         const int32_t* pairs_perm, int64_t M, const int32_t* row_order,
                         const void* plan, size_t plan_bytes, int32_t thin_tiles,
                         const uint32_t* row_words, int32_t words_per_row, void* out,
                         int32_t out_dtype, void* stream) {
  SP_CHECK_ARG(row_order != nullptr, "gemm: null row order");
  return gemm_packed(a, dtype, n_src, packed, K, kv, C, transpose, has_bias, pairs_perm, M,
                     nullptr, nullptr, plan, plan_bytes, out, out_dtype, as_stream(stream),
                     row_order, int(thin_tiles), row_words, int(words_per_row));
}

int sp_conv_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C, const void* w,
                int32_t w_dtype, int64_t K, int64_t kv, const int32_t* pf, int64_t n_out,
                const void* bias, const int32_t* pair_mask, const int32_t* mask_argsort, void* out,
                int32_t out_dtype, void* ws, size_t ws_bytes, void* stream) {
  return gemm_common(x, dtype, n_in, w, w_dtype, K, kv, C, 0, pf, n_out, bias, pair_mask,
                     mask_argsort, out, out_dtype, ws, ws_bytes, as_stream(stream));
}

int sp_conv_fwd_noalloc(const void* x, int32_t dtype, int64_t n_in, int64_t C, const void* w,
                        int32_t w_dtype, int64_t K, int64_t kv, const int32_t* pf, int64_t n_out,
                        const void* bias, const int32_t* pair_mask, const int32_t* mask_argsort,
                        void* out, int32_t out_dtype, void* stream) {
  SP_CHECK_ARG(gemm_dtype_ok(dtype), "fwd_noalloc: feature dtype %d not supported (f16/bf16/f32)",
               dtype);
  SP_CHECK_ARG(K >= 1 && C >= 1 && kv >= 1 && K < 65536 && C < 65536 && kv < 65536,
               "fwd_noalloc: bad sizes K=%lld C=%lld kv=%lld", (long long)K, (long long)C,
               (long long)kv);
  const size_t need = packed_layout(K, kv, C, dtype, 0).total;
  if (need > SP_NOALLOC_SCRATCH_BYTES)
    return set_error(SP_ERR_UNSUPPORTED,
                     "fwd_noalloc: relaid weights of K=%lld kv=%lld C=%lld need %zu bytes, more "
                     "than the %d-byte scratch (use sp_conv_fwd with a workspace)",
                     (long long)K, (long long)kv, (long long)C, need, SP_NOALLOC_SCRATCH_BYTES);
  if (n_out == 0) return SP_OK;
  int rc = SP_OK;
  void* ws = scratch_address(&rc);
  if (!ws) return rc;
  return gemm_common(x, dtype, n_in, w, w_dtype, K, kv, C, 0, pf, n_out, bias, pair_mask,
                     mask_argsort, out, out_dtype, ws, SP_NOALLOC_SCRATCH_BYTES,
                     as_stream(stream));
}

int sp_conv_dgrad(const void* g, int32_t dtype, int64_t n_out, int64_t K, const void* w,
                  int32_t w_dtype, int64_t kv, int64_t C, const int32_t* pb, int64_t n_in,
                  const int32_t* pair_mask, const int32_t* mask_argsort, void* dx, void* ws,
                  size_t ws_bytes, void* stream) {
  return gemm_common(g, dtype, n_out, w, w_dtype, K, kv, C, 1, pb, n_in, nullptr, pair_mask,
                     mask_argsort, dx, dtype, ws, ws_bytes, as_stream(stream));
}

size_t sp_wgrad_workspace_size(int64_t K, int64_t kv, int64_t C, int64_t n_rows) {
  const int splits = wgrad_splits(kv, C, K, n_rows);
  return align_up(size_t(splits) * size_t(K * kv * C) * sizeof(float), 256);
}

int sp_conv_wgrad(const void* x, int64_t n_in, const void* g, int64_t n_out, int32_t dtype,
                  int64_t C, int64_t K, int64_t kv, const int32_t* in_rows,
                  const int32_t* out_rows, const int32_t* counts, int64_t row_stride, void* dw,
                  void* ws, size_t ws_bytes, void* stream) {
  SP_CHECK_ARG(dtype == SP_F16 || dtype == SP_BF16 || dtype == SP_F32 || dtype == SP_BF16X3,
               "wgrad: dtype %d not supported (f16/bf16/f32/bf16x3)", dtype);
  SP_CHECK_ARG(K >= 1 && C >= 1 && kv >= 1 && row_stride >= 0, "wgrad: bad sizes");
  SP_CHECK_ARG(x && g && in_rows && out_rows && counts && dw, "wgrad: null pointer");
  hipStream_t s = as_stream(stream);
  // split-bf16 operands: X [n_in, 2C] and G [n_out, 2K] bf16 halves [hi | lo]
  const bool split = dtype == SP_BF16X3;
  const int64_t Cg = split ? 2 * C : C, Kg = split ? 2 * K : K;
  SP_CHECK_ARG(Kg < 65536 && Cg < 65536 && kv < 65536, "wgrad: channel/kernel size too large");
  const int elem = split ? SP_BF16 : dtype;
  const int splits = wgrad_splits(kv, Cg, Kg, row_stride);
  const size_t need = sp_wgrad_workspace_size(Kg, kv, Cg, row_stride);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "wgrad: workspace %zu < %zu", ws_bytes, need);
  float* part = static_cast<float*>(ws);
  const int64_t gx = kv * splits;
  SP_CHECK_ARG(gx <= kMaxGridX, "wgrad: grid too large");
  const int64_t es = elem == SP_F32 ? 4 : 2;
  const int64_t xb = n_in * Cg * es, gb = n_out * Kg * es;
  if (xb >= int64_t(kOob) || gb >= int64_t(kOob))
    return set_error(SP_ERR_UNSUPPORTED, "wgrad: features exceed 4 GiB");
  // 16-byte row gathers need whole vectors per row and aligned bases
  const int v = vec_of(elem);
  const int vec = (Cg % v == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 ? 1 : 0) |
                  (Kg % v == 0 && reinterpret_cast<uintptr_t>(g) % 16 == 0 ? 2 : 0);
  const int bw = wgrad_block(Cg, Kg);
  const int cblocks = int(cdiv(Cg, bw)), nblocks = int(cdiv(Kg, bw));
  const int64_t nwg = 8 * cdiv(gx, 8) * cblocks * nblocks;
  SP_CHECK_ARG(nwg <= kMaxGridX, "wgrad: grid too large");
  const dim3 grid{unsigned(nwg), 1u, 1u};
  const int64_t tot = K * kv * C;
  const unsigned rb = unsigned(cdiv(tot, 256));
  auto run = [&](auto tag) {
    using T = decltype(tag);
    using Kern = decltype(&wgrad_partial<T, 3, 64>);
    const Kern k64[4] = {wgrad_partial<T, 0, 64>, wgrad_partial<T, 1, 64>,
                         wgrad_partial<T, 2, 64>, wgrad_partial<T, 3, 64>};
    const Kern k128[4] = {wgrad_partial<T, 0, 128>, wgrad_partial<T, 1, 128>,
                          wgrad_partial<T, 2, 128>, wgrad_partial<T, 3, 128>};
    const Kern kern = bw == 128 ? k128[vec] : k64[vec];
    kern<<<grid, 256, 0, s>>>(static_cast<const T*>(x), n_in, static_cast<const T*>(g), n_out,
                              int(Cg), int(Kg), int(kv), in_rows, out_rows, counts, row_stride,
                              splits, part, uint32_t(xb), uint32_t(gb), cblocks, nblocks);
    if (split)
      wgrad_reduce_split<<<rb, 256, 0, s>>>(part, splits, K, kv, C, static_cast<float*>(dw));
    else
      wgrad_reduce<T><<<rb, 256, 0, s>>>(part, splits, tot, static_cast<T*>(dw));
  };
  switch (elem) {
    case SP_F16: run(_Float16{}); break;
    case SP_BF16: run(__bf16{}); break;
    default: run(float{});
  }
  SP_LAUNCHED();
  return SP_OK;
}

int sp_split_bf16x3(const float* x, int64_t rows, int64_t cols, int32_t pattern, void* out,
                    void* stream) {
  SP_CHECK_ARG(rows >= 0 && cols >= 1 && pattern >= 0 && pattern <= 2,
               "split_bf16x3: bad sizes or pattern (rows=%lld cols=%lld pattern=%d)",
               (long long)rows, (long long)cols, pattern);
  if (rows == 0) return SP_OK;
  SP_CHECK_ARG(x && out, "split_bf16x3: null pointer");
  const bool vec4 = cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(out) % 8 == 0;
  const int64_t work = rows * (vec4 ? cols / 4 : cols);
  SP_CHECK_ARG(cdiv(work, 256) <= kMaxGridX, "split_bf16x3: too many elements");
  split_bf16_rows<<<unsigned(cdiv(work, 256)), 256, 0, as_stream(stream)>>>(
      x, rows, cols, pattern, vec4, static_cast<__bf16*>(out));
  SP_LAUNCHED();
  return SP_OK;
}

}  // extern "C"
