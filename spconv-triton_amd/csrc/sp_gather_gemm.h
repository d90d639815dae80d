// Forward / input-gradient gather-GEMM kernel (included by sp_gemm.hip).
//
//   out[m, n] = bias[n] + sum_k sum_r A[pairs[k, m], r] * Bt[k][n][r]
//
// One wave computes 64 consecutive output rows x 64 output columns as 4 x 4
// tiles of v_mfma_f32_16x16x32_{f16,bf16} (v_mfma_f32_16x16x4f32 for fp32);
// the 16-row shape lets four lanes read one feature row's 64 contiguous bytes,
// which halves the cache lines a gather instruction touches compared with the
// 32-row shape.
//
// Memory access is built on raw buffer instructions: a load whose offset lies
// past the buffer's size returns zeros and a store there is dropped, so a
// missing neighbour (pair index -1) is just an out-of-range offset -- no
// branch per load.  Branch-free loads also let the compiler count outstanding
// loads exactly, which the software pipeline below depends on.
//
// Per chunk of up to 32 kernel offsets the wave stages the source row of each
// (offset, row) in LDS, with all pair-table loads in flight at once, and keeps
// only the offsets that have a valid source somewhere in its 64 rows (ballot).
// It then pipelines over (offset, reduction chunk) items: the A (gathered
// feature rows) and B (packed weights) fragments of item i+1 are loaded while
// the MFMAs of item i run.  Rows keep their natural order: the [kv, M] pair
// table is read with coalesced 256-byte accesses and output rows are
// contiguous.  Every row's sum runs over its offsets in ascending order for any
// tiling, so skipped offsets and tile composition never change a result bit.
// Included inside namespace sp, after the Mfma<> traits and from_f32<>.
#pragma once

constexpr int kStageOffsets = 32;  // kernel offsets staged in LDS at once
constexpr uint32_t kOob = 0xFFFFFFF0u;  // byte offset past every buffer (loads give 0)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, int(bytes),
                                           0x00020000);
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag buf_frag(__amdgpu_buffer_rsrc_t r,
                                                           uint32_t off) {
  return __builtin_bit_cast(typename Mfma<T>::frag,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <typename T>
__device__ __forceinline__ T buf_elem(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <>
__device__ __forceinline__ _Float16 buf_elem<_Float16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <>
__device__ __forceinline__ __bf16 buf_elem<__bf16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(__bf16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <>
__device__ __forceinline__ float buf_elem<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

template <typename T>
__device__ __forceinline__ void buf_store(T v, __amdgpu_buffer_rsrc_t r, uint32_t off);
template <>
__device__ __forceinline__ void buf_store<_Float16>(_Float16 v, __amdgpu_buffer_rsrc_t r,
                                                    uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, off, 0, 0);
}
template <>
__device__ __forceinline__ void buf_store<__bf16>(__bf16 v, __amdgpu_buffer_rsrc_t r,
                                                  uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, off, 0, 0);
}
template <>
__device__ __forceinline__ void buf_store<float>(float v, __amdgpu_buffer_rsrc_t r,
                                                 uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8).  Give every XCD a contiguous range of row tiles, so tiles whose
// neighbourhoods overlap share that XCD's L2.  Bijective for any count nb.
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t nb) {
  constexpr int64_t kXcd = 8;
  const int64_t q = nb / kXcd, r = nb % kXcd;
  const int64_t x = b % kXcd, local = b / kXcd;
  return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

// Byte sizes of the buffers a launch touches; the host checks they fit in 32 bits.
struct GemmBufs {
  uint32_t a_bytes, bt_bytes, pairs_bytes, out_bytes;
};

// 16x16 MFMA shapes.  Lane l holds row (or column) l % 16 of the tile and the
// 4 lane groups g = l / 16 hold consecutive slices of V reduction elements, so
// one A-fragment load instruction reads 16 feature rows x 64 contiguous bytes.
template <typename T>
struct M16;

template <>
struct M16<_Float16> {
  using frag = half8;
  static constexpr int V = 8;
  static constexpr int KSTEP = 32;
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, float4v& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct M16<__bf16> {
  using frag = bf16x8;
  static constexpr int V = 8;
  static constexpr int KSTEP = 32;
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, float4v& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct M16<float> {
  using frag = float4v;
  static constexpr int V = 4;
  static constexpr int KSTEP = 16;
  __device__ static __forceinline__ void mma(const frag& a, const frag& b, float4v& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename M16<T>::frag buf_frag16(__amdgpu_buffer_rsrc_t r,
                                                            uint32_t off) {
  return __builtin_bit_cast(typename M16<T>::frag,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// One wave computes 64 rows x 64 columns as 4 x 4 tiles of 16 x 16.  RS = MFMA
// K-steps per pipeline item (RS * KSTEP reduction indices).  The reduction
// index of (step s, lane group g, element e) is s * KSTEP + g * V + e, for A
// and B alike.
template <typename T, typename OutT, bool VEC, int RS>
__global__ __launch_bounds__(256) void gather_gemm(
    const T* __restrict__ A, const T* __restrict__ Bt, const int32_t* __restrict__ pairs,
    const float* __restrict__ bias, OutT* __restrict__ out, GemmBufs nb, int64_t n_src,
    int64_t M, int N, int R, int Rp, int kv) {
  using MF = M16<T>;
  using frag = typename MF::frag;
  constexpr int V = MF::V;
  constexpr int KSTEP = MF::KSTEP;
  constexpr int RCH = RS * KSTEP;
  constexpr uint32_t ES = sizeof(T);
  __shared__ int32_t s_src[4][kStageOffsets][64];
  __shared__ int32_t s_k[4][kStageOffsets];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, l16 = lane & 15;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t slot0 = (tile * 4 + wave) * 64;
  const int n0 = blockIdx.y * 64;
  const int64_t my_row = slot0 + lane;
  const bool row_ok = my_row < M;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, nb.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bt, nb.bt_bytes);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(pairs, nb.pairs_bytes);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, nb.out_bytes);

  float4v acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.f;

  const uint32_t bk_bytes = uint32_t(Rp / V) * uint32_t(N) * V * ES;  // one offset of Bt
  const uint32_t row_bytes = uint32_t(R) * ES;
  const int nrc = Rp / RCH;  // reduction chunks per offset
  int32_t* src_tab = &s_src[wave][0][0];
  uint32_t bcol[4];  // byte offset of this lane's B column inside an (offset, r/V) slab
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int col = n0 + nt * 16 + l16;
    bcol[nt] = col < N ? uint32_t(col) * V * ES : kOob;
  }

  for (int kc = 0; kc < kv; kc += kStageOffsets) {
    const int kn = kv - kc < kStageOffsets ? kv - kc : kStageOffsets;
    // ---- stage the source rows of the offsets that are live in this tile
    int nact = 0;
    for (int u0 = 0; u0 < kn; u0 += 8) {
      int32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t off = row_ok && u0 + u < kn
                                 ? uint32_t((int64_t(kc + u0 + u) * M + my_row) * 4)
                                 : kOob;
        v[u] = int32_t(__builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const bool ok = row_ok && u0 + u < kn && v[u] >= 0 && v[u] < n_src;
        if (__ballot(ok)) {  // wave-uniform
          src_tab[nact * 64 + lane] = ok ? v[u] : -1;
          if (lane == 0) s_k[wave][nact] = kc + u0 + u;
          ++nact;
        }
      }
    }
    __syncthreads();

    // ---- pipelined gather + MFMA over (offset, reduction chunk) items
    const int nitems = nact * nrc;
    auto load_item = [&](int it, frag (&a)[4][RS], frag (&b)[4][RS]) {
      const int si = it / nrc;
      const int rc = it - si * nrc;
      const uint32_t kb = uint32_t(s_k[wave][si]) * bk_bytes;
      uint32_t abase[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int32_t s = src_tab[si * 64 + mt * 16 + l16];
        abase[mt] = s >= 0 ? uint32_t(s) * row_bytes : kOob;
      }
#pragma unroll
      for (int st = 0; st < RS; ++st) {
        const int rr = rc * RCH + st * KSTEP + g * V;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          if (VEC) {
            const uint32_t off = (abase[mt] != kOob && rr < R) ? abase[mt] + uint32_t(rr) * ES
                                                               : kOob;
            a[mt][st] = buf_frag16<T>(ra, off);
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) {
              const uint32_t off = (abase[mt] != kOob && rr + e < R)
                                       ? abase[mt] + uint32_t(rr + e) * ES
                                       : kOob;
              a[mt][st][e] = buf_elem<T>(ra, off);
            }
          }
        }
        const uint32_t slab = kb + uint32_t(rr / V) * uint32_t(N) * V * ES;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          b[nt][st] = buf_frag16<T>(rb, bcol[nt] != kOob ? slab + bcol[nt] : kOob);
      }
    };
    auto mma_item = [&](const frag (&a)[4][RS], const frag (&b)[4][RS]) {
#pragma unroll
      for (int st = 0; st < RS; ++st)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) MF::mma(a[mt][st], b[nt][st], acc[mt][nt]);
    };
    frag a0[4][RS], b0[4][RS], a1[4][RS], b1[4][RS];
    if (nitems > 0) load_item(0, a0, b0);
    for (int it = 0; it < nitems; it += 2) {
      if (it + 1 < nitems) load_item(it + 1, a1, b1);
      mma_item(a0, b0);
      if (it + 1 < nitems) {
        if (it + 2 < nitems) load_item(it + 2, a0, b0);
        mma_item(a1, b1);
      }
    }
    __syncthreads();  // the next chunk overwrites the staged sources
  }

  // ---- epilogue: lane l holds column l%16 of rows 4*(l/16) + i of each tile;
  // rows past M fall outside the output buffer and their stores are dropped
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int col = n0 + nt * 16 + l16;
    const float bv = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = slot0 + mt * 16 + g * 4 + i;
        const uint32_t off = (row < M && col < N)
                                 ? uint32_t((row * N + col) * int64_t(sizeof(OutT)))
                                 : kOob;
        buf_store<OutT>(from_f32<OutT>(acc[mt][nt][i] + bv), ro, off);
      }
    }
  }
}
