// Forward / input-gradient gather-GEMM kernels (included by sp_gemm.hip).
//
//   out[m, n] = bias[n] + sum_k sum_r A[pairs[k, m], r] * Bt[k][n][r]
//
// A workgroup owns kTileRows = 256 consecutive output rows x 64 output columns;
// each of its 4 waves computes 64 rows x 64 columns as 2 x 2 tiles of
// v_mfma_f32_32x32x16_{f16,bf16} (4 x v_mfma_f32_32x32x2f32 for fp32, the
// Mfma<> traits).  Measured on MI355X, one 32x32x16 issues every ~38.5 clocks
// per SIMD whether one or two waves share the SIMD (2.1 PFLOP/s), while
// 16x16x32 needs two interleaved waves to get near that (31 clocks per half
// the work for a lone wave).  One "item" is one kernel offset for one chunk
// of 64 bytes of the reduction dimension (32 f16/bf16 or 16 f32): 8 MFMAs per
// wave fed by 4 A fragments (gathered rows) and 4 B fragments (weights).
//
// Two kernels:
//  * gather_gemm_staged (with a gather plan, sp_plan.h).  Measured on MI355X,
//    LDS delivers ~228 B/clk per CU against ~60 B/clk for L1 hits, so both
//    operands come from LDS:
//      - A: for each chunk the workgroup copies the tile's distinct source
//        rows (~765 for 256 rows of a surface cloud, against ~2600 pairs)
//        into LDS with coalesced 16-byte loads, four lanes per row; the next
//        chunk's rows are loaded into registers while the current one is
//        multiplied.  Fragments are read at the LDS addresses the plan holds
//        for every (item, row).
//      - B: the four waves share the tile's item list, and each item's 4 KiB
//        weight slab is loaded once per workgroup (16 bytes per thread) into a
//        4-slot LDS ring, one barrier per two items.
//    Tiles whose distinct rows do not fit in LDS (the plan's overflow tiles)
//    take the direct path inside the same kernel.
//  * gather_gemm_direct: fragments are gathered straight from global memory
//    (A) and B is read through L1 by every wave.  It runs every tile of an
//    unplanned call (its body, direct_tile, also serves the overflow tiles of
//    a planned one), and builds its per-wave item tables from the pair table
//    itself.
//
// Both pipelines keep per-item work to loads and MFMAs: B offsets and A
// addresses are precomputed per item, and the item lists end with padding
// items (zero row, out-of-range B), so the loops run in whole groups (3 items
// direct, 4 staged) and read ahead without per-item conditions.  Padding items
// multiply zeros, which leaves every sum unchanged.  Raw buffer instructions make global
// loads branch-free (an offset past the buffer's size reads zeros, a store
// there is dropped), and sched_barrier keeps loads issued ahead of the MFMAs
// that consume them, so the compiler's load counters stay exact.
//
// Fragment layouts (32 x 32 MFMA, lane l, h = l / 32): A and B fragments hold
// row (column) l % 32 of the tile and 16-byte piece 2 * ks + h of the 64-byte
// chunk, ks = 0, 1 being the MFMA K-step within the item; the accumulator
// element i of lane l is row 8 * (i / 4) + 4 * h + i % 4, column l % 32.
//
// Summation order.  Offsets are taken in groups of up to 64 (one group when
// kv <= 64); within a group the chunks are the outer loop and the offsets,
// ascending, the inner one.  Offsets without any pair in the wave's (direct)
// or the tile's (staged) rows are skipped; their terms are exactly zero, so a
// row's result does not depend on the tile it falls in or on the kernel.
// Included inside namespace sp, after sp_plan.h, the Mfma<> traits and
// from_f32<>.
#pragma once

constexpr uint32_t kOob = 0xFFFFFFF0u;     // byte offset past every buffer (loads give 0)
constexpr uint32_t kBOob = 0x80000000u;    // B offset of padding items
constexpr uint32_t kColOob = 0x40000000u;  // B column offset of columns >= N
constexpr uint32_t kMaxBtBytes = 0x40000000u;  // packed weights must stay below (host check)
constexpr int kGroupOffsets = 64;          // kernel offsets per group (direct kernel)
static_assert(kGroupOffsets == kPlanGroupOffsets,
              "planned tiles keep their items in one group of the direct kernel");
constexpr uint32_t kSlabBytes = 4096;      // B of one item: 4 pieces x 64 columns x 16 B
constexpr int kPad = 5;                    // padding items after a direct-kernel item list

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, int(bytes),
                                           0x00020000);
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

// Tile and first output column of a direct-kernel workgroup.  One column
// block (N <= 64): a grid of one workgroup per tile, mapped by xcd_tile.
// Several: a 1-D grid of 8 * gy * ceil(ntiles / 8) workgroups in which XCD
// x's queue holds its contiguous range of ceil(ntiles / 8) tiles, each
// tile's gy column blocks back to back, so they run together on that XCD and
// gather the same source rows through its L2.  Returns false for the padding
// workgroups past the last tile, which must exit at once.  (Measured: the
// 4-D 3^4 128 -> 128 layer 351 -> 334 us; the staged kernel, which reads
// its rows once per tile and chunk into LDS, is slower with it.)
__device__ __forceinline__ bool block_tile(int64_t M, int N, int64_t* tile, int* n0) {
  const int64_t nt = (M + kTileRows - 1) / kTileRows;
  const int gy = (N + 63) / 64;
  if (gy == 1) {
    *tile = xcd_tile(blockIdx.x, gridDim.x);
    *n0 = 0;
    return true;
  }
  const int64_t per = (nt + 7) / 8;
  const int64_t b = blockIdx.x, x = b % 8, k = b / 8;
  *tile = x * per + k / gy;
  *n0 = int(k % gy) * 64;
  return *tile < nt;
}

// Tile and first output column of a staged-kernel workgroup.  One column
// block (N <= 64): as block_tile.  Several: a 1-D grid of
// 8 * gy * ceil(ntiles / 8) workgroups in which tile t runs on XCD t % 8 and
// its gy column blocks are back to back in that XCD's queue, so they stage
// the same rows through its L2 at about the same time, while consecutive
// tiles are spread over the XCDs (in mask order the tiles' costs vary along
// the table, so contiguous ranges per XCD leave some XCDs far more work).
// Measured, fp16 forward: LiDAR 50k 256 -> 256 in mask order 183 -> 149 us,
// 1024^3 surface 256 -> 256 in mask order 675 -> 572 us, LiDAR natural
// 168 -> 153 us (the 2-D grid, whose column blocks of a tile land on
// different XCDs, against this one).  Returns false for the padding
// workgroups past the last tile, which must exit at once.
__device__ __forceinline__ bool staged_tile_of(int64_t b, int64_t nwg, int64_t M, int N,
                                               int64_t* tile, int* n0) {
  const int gy = (N + 63) / 64;
  if (gy == 1) {
    *tile = xcd_tile(b, nwg);
    *n0 = 0;
    return true;
  }
  const int64_t nt = (M + kTileRows - 1) / kTileRows;
  const int64_t x = b % 8, k = b / 8;
  *tile = (k / gy) * 8 + x;
  *n0 = int(k % gy) * 64;
  return *tile < nt;
}
__device__ __forceinline__ bool staged_tile(int64_t M, int N, int64_t* tile, int* n0) {
  return staged_tile_of(blockIdx.x, gridDim.x, M, N, tile, n0);
}

// LDS writes of this wave are complete, then the workgroup barrier.  Written
// as one asm statement with a memory clobber: the compiler neither moves LDS
// accesses across it nor adds waits for outstanding global loads (which the
// B and A pipelines keep in flight across barriers).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The same with the wave's last `kPending` LDS operations still in flight
// (LDS operations complete in order, so every earlier one is complete).
template <int kPending>
__device__ __forceinline__ void lds_barrier_pending() {
  static_assert(kPending >= 0 && kPending < 16, "lgkmcnt holds 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" ::"n"(kPending) : "memory");
}

// Byte sizes of the buffers a launch touches; the host checks they fit in 32 bits.
struct GemmBufs {
  uint32_t a_bytes, bt_bytes, pairs_bytes, out_bytes;
};

template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag buf_frag(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(typename Mfma<T>::frag,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// V elements of one row starting at element e0 (zeros past R), one load per
// element: the path for rows whose length is not a multiple of V.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag buf_frag_elems(__amdgpu_buffer_rsrc_t r,
                                                                 uint32_t row_off, int e0, int R) {
  typename Mfma<T>::frag f;
#pragma unroll
  for (int e = 0; e < Mfma<T>::V; ++e) {
    const uint32_t off =
        (row_off != kOob && e0 + e < R) ? row_off + uint32_t(e0 + e) * uint32_t(sizeof(T)) : kOob;
    f[e] = buf_elem<T>(r, off);
  }
  return f;
}

// One item: fragments [ks][mt] (A) and [ks][nt] (B), K-steps ascending.
template <typename T>
__device__ __forceinline__ void mma_item(const typename Mfma<T>::frag (&a)[2][2],
                                         const typename Mfma<T>::frag (&b)[2][2],
                                         floatx16 (&acc)[2][2]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Mfma<T>::mma(a[ks][mt], b[ks][nt], acc[mt][nt]);
}

__device__ __forceinline__ void zero_acc(floatx16 (&acc)[2][2]) {
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.f;
}

// Epilogue staging: each wave's 64 x 64 output tile, rows padded by 16 bytes.
__host__ __device__ constexpr uint32_t epi_pitch(uint32_t out_size) { return 64u * out_size + 16u; }
__host__ __device__ constexpr uint32_t epi_bytes(uint32_t out_size) {
  return 4u * 64u * epi_pitch(out_size);
}

// Writes the wave's 64 x 64 tile (plus bias).  When a row's 64 columns split
// into whole 16-byte pieces, the tile goes through LDS (`stage`, this wave's
// 64 * epi_pitch bytes, free once the caller has passed a barrier) and is
// stored as whole rows, otherwise element by element.  Rows past M fall
// outside the output buffer and their stores are dropped.  With a row order
// (nullable), tile row `slot` is output row order[slot]; an entry outside
// 0..M-1 is treated as a row past M (its stores are dropped).
template <typename OutT>
__device__ __forceinline__ void store_tile(const floatx16 (&acc)[2][2], const float* bias,
                                           __amdgpu_buffer_rsrc_t ro, unsigned char* stage,
                                           int64_t slot0, int n0, int64_t M, int N, int lane,
                                           const int32_t* __restrict__ order) {
  auto out_row = [&](int64_t slot) -> int64_t {
    if (!order || slot >= M) return slot;
    const int64_t r = order[slot];
    return (r >= 0 && r < M) ? r : M;
  };
  constexpr uint32_t OS = sizeof(OutT);
  constexpr int kPer16 = int(16 / OS);  // output elements per 16-byte piece
  const int h = lane >> 5, l32 = lane & 31;
  if (N % kPer16 == 0) {
    constexpr uint32_t pitch = epi_pitch(OS);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + nt * 32 + l32;
      const float bv = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          *reinterpret_cast<OutT*>(stage +
                                   uint32_t(mt * 32 + 8 * (i / 4) + 4 * h + (i % 4)) * pitch +
                                   uint32_t(nt * 32 + l32) * OS) =
              from_f32<OutT>(acc[mt][nt][i] + bv);
    }
    // (each wave reads back only its own rows: no barrier needed)
    constexpr int kPieces = 64 / kPer16;        // 16-byte pieces per row of 64 columns
    constexpr int kRowsPerPass = 64 / kPieces;  // rows one instruction covers
    const int pc = lane % kPieces, pr = lane / kPieces;
    const int col = n0 + pc * kPer16;
#pragma unroll
    for (int j = 0; j < 64 / kRowsPerPass; ++j) {
      const int r = pr + j * kRowsPerPass;
      const uint4 v =
          *reinterpret_cast<const uint4*>(stage + uint32_t(r) * pitch + uint32_t(pc) * 16u);
      const int64_t row = out_row(slot0 + r);
      const uint32_t off = (row < M && col < N) ? uint32_t((row * N + col) * int64_t(OS)) : kOob;
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, v), ro, off, 0, 0);
    }
    return;
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = n0 + nt * 32 + l32;
    const float bv = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t row = out_row(slot0 + mt * 32 + 8 * (i / 4) + 4 * h + (i % 4));
        const uint32_t off =
            (row < M && col < N) ? uint32_t((row * N + col) * int64_t(OS)) : kOob;
        buf_store<OutT>(from_f32<OutT>(acc[mt][nt][i] + bv), ro, off);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// direct kernel
// ---------------------------------------------------------------------------

// Dynamic LDS of the direct kernel: per wave E item entries; the epilogue
// tiles overlap the tables (used after the last item).
struct DirectLds {
  uint32_t kb_off, src_off, a_off, total;
};

__host__ __device__ inline DirectLds direct_lds(int E, uint32_t out_size) {
  DirectLds l;
  l.kb_off = 0;                                          // uint32 B offsets [4][E]
  l.src_off = (16u * uint32_t(E) + 255u) / 256u * 256u;  // int32 source rows [4][E][32][2]
  l.a_off = l.src_off + uint32_t(E) * 1024u;             // direct_tile's A slots [4][32][64 B]
  l.total = l.a_off + 4u * 2048u;
  if (l.total < l.src_off + epi_bytes(out_size)) l.total = l.src_off + epi_bytes(out_size);
  return l;
}

// One (tile, 64-column block) of the direct kernel, the whole workgroup:
// every tile of an unplanned call, and the tiles of a planned call whose
// distinct rows do not fit in LDS.  Uses direct_lds(min(kv, 64) + kPad) bytes
// of `smem`.  words (nullable): the mask words of the table's rows, `mic` per
// row (bit k of row r set iff pairs[k, r] >= 0); with them a wave reads the
// table entries of only the offsets set in its rows' masks, instead of all kv
// (the items found, and so the result, are the same).
template <typename T, typename OutT, bool VEC, bool SLOT = true>
__device__ __forceinline__ void direct_tile(const T* __restrict__ A, const T* __restrict__ Bt,
                                            const int32_t* __restrict__ pairs,
                                            const float* __restrict__ bias,
                                            OutT* __restrict__ out, const GemmBufs& nb,
                                            int64_t n_src, int64_t M, int N, int R, int Rp,
                                            int kv, int64_t tile, int n0, unsigned char* smem,
                                            const int32_t* __restrict__ order,
                                            const uint32_t* __restrict__ words = nullptr,
                                            int mic = 0) {
  using frag = typename Mfma<T>::frag;
  constexpr int V = Mfma<T>::V;
  constexpr uint32_t ES = sizeof(T);
  constexpr int kChunk = kChunkBytes / int(ES);  // reduction elements per item

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t slot0 = tile * kTileRows + wave * 64;
  const int64_t my_row = slot0 + lane;
  const bool row_ok = my_row < M;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, nb.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bt, nb.bt_bytes);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, nb.out_bytes);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(pairs, nb.pairs_bytes);

  const int G = kv < kGroupOffsets ? kv : kGroupOffsets;
  const int E = G + kPad;
  const DirectLds L = direct_lds(E, uint32_t(sizeof(OutT)));
  uint32_t* s_kb = reinterpret_cast<uint32_t*>(smem + L.kb_off) + wave * E;
  // byte offset in A of each (item, row) source row, kOob for none
  uint32_t* s_src = reinterpret_cast<uint32_t*>(smem + L.src_off) + wave * E * 64;

  const uint32_t row_bytes = uint32_t(R) * ES;
  const uint32_t slab_bytes = uint32_t(N) * V * ES;        // one (offset, r / V) slab of Bt
  const uint32_t k_bytes = uint32_t(Rp / V) * slab_bytes;  // one offset of Bt
  const int nrc = Rp / kChunk;                             // chunks per offset
  uint32_t bcol[2];  // byte offset of this lane's B column inside a slab
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = n0 + nt * 32 + l32;
    bcol[nt] = col < N ? uint32_t(col) * V * ES : kColOob;
  }

  floatx16 acc[2][2];
  zero_acc(acc);
  for (int kc = 0; kc < kv; kc += G) {
    const int kn = kv - kc < G ? kv - kc : G;
    __syncthreads();  // the previous group's tables are no longer read
    // ---- per-wave tables of the offsets with a pair in this wave's 64 rows
    int nact = 0;
    constexpr int kTabBatch = 16;  // table loads in flight per lane
    if (words) {
      // the offsets kc .. kc + kn - 1 set in any of the wave's rows' masks
      // (kc is a multiple of 64, so they are bits of words kc / 32 and the next)
      uint32_t m_lo = 0u, m_hi = 0u;
      if (row_ok) {
        const int w0 = kc >> 5;
        const uint32_t* wr = words + my_row * int64_t(mic);
        m_lo = w0 < mic ? wr[w0] : 0u;
        m_hi = w0 + 1 < mic ? wr[w0 + 1] : 0u;
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        m_lo |= __shfl_xor(m_lo, off, 64);
        m_hi |= __shfl_xor(m_hi, off, 64);
      }
      // wave-uniform after the reduction; readfirstlane puts it (and the batch
      // loop below, and so nact) in scalar registers
      m_lo = __builtin_amdgcn_readfirstlane(m_lo);
      m_hi = __builtin_amdgcn_readfirstlane(m_hi);
      uint64_t live = (uint64_t(m_hi) << 32) | m_lo;
      if (kn < 64) live &= (uint64_t(1) << kn) - 1u;
      while (live) {  // a batch of the lowest set offsets, ascending
        int us[kTabBatch];
#pragma unroll
        for (int b = 0; b < kTabBatch; ++b) {
          us[b] = live ? int(__builtin_ctzll(live)) : -1;
          live &= live ? live - 1u : uint64_t(0);
        }
        int32_t v[kTabBatch];
#pragma unroll
        for (int b = 0; b < kTabBatch; ++b) {
          const bool in = row_ok && us[b] >= 0;
          const int64_t e = int64_t(kc + (us[b] >= 0 ? us[b] : 0)) * M + my_row;
          v[b] = int32_t(
              __builtin_amdgcn_raw_buffer_load_b32(rp, in ? uint32_t(e * 4) : kOob, 0, 0));
        }
#pragma unroll
        for (int b = 0; b < kTabBatch; ++b) {
          const bool ok = row_ok && us[b] >= 0 && v[b] >= 0 && v[b] < n_src;
          if (us[b] >= 0 && __ballot(ok)) {  // wave-uniform
            s_src[(nact * 32 + l32) * 2 + h] = ok ? uint32_t(v[b]) * row_bytes : kOob;
            if (lane == 0) s_kb[nact] = uint32_t(kc + us[b]) * k_bytes;
            ++nact;
          }
        }
      }
    } else {
      for (int u0 = 0; u0 < kn; u0 += kTabBatch) {
        int32_t v[kTabBatch];
#pragma unroll
        for (int u = 0; u < kTabBatch; ++u) {
          const bool in = row_ok && u0 + u < kn;
          const int64_t e = int64_t(kc + u0 + u) * M + my_row;
          v[u] = int32_t(
              __builtin_amdgcn_raw_buffer_load_b32(rp, in ? uint32_t(e * 4) : kOob, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < kTabBatch; ++u) {
          const bool ok = row_ok && u0 + u < kn && v[u] >= 0 && v[u] < n_src;
          if (u0 + u < kn && __ballot(ok)) {  // wave-uniform
            // [item][l32][mt], mt = lane / 32
            s_src[(nact * 32 + l32) * 2 + h] = ok ? uint32_t(v[u]) * row_bytes : kOob;
            if (lane == 0) s_kb[nact] = uint32_t(kc + u0 + u) * k_bytes;
            ++nact;
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kPad; ++q) {  // padding items: no source row, out-of-range B
      s_src[((nact + q) * 32 + l32) * 2 + h] = kOob;
      if (lane == 0) s_kb[nact + q] = kBOob;
    }

    nact = __builtin_amdgcn_readfirstlane(nact);  // wave-uniform: the cursors below are scalar
    if (nact == 0) continue;                      // no pair in this wave's rows
    // The group's (chunk, item) steps as one software pipeline, chunk by chunk
    // and items ascending inside a chunk (the summation order of every
    // kernel).  A cursor walks items 0 .. nact - 1 of chunks 0 .. nrc - 1 and
    // then runs on into the padding items of the last chunk, whose loads read
    // zeros, so no chunk restarts the pipeline.  Step j: the A loads of step
    // j + 1, the MFMAs of step j, the B loads of step j + 2.
    struct Cur {
      int rc, it;
    };
    auto advance = [&](Cur& c) {
      if (++c.it == nact && c.rc + 1 < nrc) {
        c.it = 0;
        ++c.rc;
      }
    };
    uint32_t bl[2][2];  // this lane's B offsets inside chunk 0 of an offset's slabs
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) bl[ks][nt] = bcol[nt] + uint32_t(ks * 2 + h) * slab_bytes;
    const uint32_t chunk_b = 4u * slab_bytes;  // B bytes per chunk of an offset
    auto entry = [&](int it) -> uint2 {
      return *reinterpret_cast<const uint2*>(s_src + (it * 32 + l32) * 2);
    };
    auto load_b = [&](uint32_t kb, int rc, frag (&b)[2][2]) {
      const uint32_t kr = kb + uint32_t(rc) * chunk_b;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) b[ks][nt] = buf_frag<T>(rb, kr + bl[ks][nt]);
    };
    if constexpr (VEC && SLOT && sizeof(T) == 2) {
      // A through a wave-private LDS slot (16-bit operands: with fp32 ones,
      // whose 64-clock MFMAs leave the gathers more time, it measured slower:
      // the LiDAR-like layer's mask-ordered direct GEMM 1 132 -> 1 250 us).  A gather fragment (lane l: row
      // l % 32, piece 2 ks + l / 32) reads 32 rows, 32 of their 64 bytes
      // each, and costs the L1 one tag per row; loaded row-contiguous
      // instead (lane l: row 16 ks + l / 4, piece l % 4: each load 16 whole
      // 64-byte rows) a step's 64 rows take half the tags.  The loads land in
      // registers, go through the slot (rows swizzled as in the staged
      // kernel) a step later, one 32-row block at a time, and come back as
      // the same MFMA fragments: the multiply and its result are unchanged.
      // LDS operations of one wave complete in order, so one slot serves
      // every block and step.  (A timing probe of the loads alone: the
      // unplanned 4-D 3^4 layer 273 -> 221 us.)
      unsigned char* aslot = smem + L.a_off + uint32_t(wave) * 2048u;
      const int rsub = lane >> 2, pc = lane & 3;  // this lane's row (within 16) and piece
      const int last_it = nact + kPad - 1;        // the cursors' reads stop at the last padding item
      // byte offsets in A of this lane's four rows (16 ks + rsub of block mt)
      auto bases = [&](int it) -> uint4 {
        const int i = it < last_it ? it : last_it;
        const uint2 r0 = *reinterpret_cast<const uint2*>(s_src + (i * 32 + rsub) * 2);
        const uint2 r1 = *reinterpret_cast<const uint2*>(s_src + (i * 32 + 16 + rsub) * 2);
        return make_uint4(r0.x, r0.y, r1.x, r1.y);  // [ks][mt]
      };
      auto gload_a = [&](const uint4& bs, int rc, uint4 (&raw)[2][2]) {
        const int e0 = rc * kChunk + pc * V;
        const uint32_t b4[2][2] = {{bs.x, bs.y}, {bs.z, bs.w}};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            const uint32_t base = b4[ks][mt];
            raw[ks][mt] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(
                           ra, (base != kOob && e0 < R) ? base + uint32_t(e0) * ES : kOob, 0, 0));
          }
      };
      // row r of the slot at chunk_base(r), its piece p at ^ (p << 4)
      const uint32_t wr_row = chunk_base(uint32_t(rsub)) ^ uint32_t(pc << 4);
      const uint32_t rd_row = chunk_base(uint32_t(l32));
      auto through_slot = [&](const uint4 (&raw)[2][2], frag (&a)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)  // rows 16 ks .. 16 ks + 15 (chunk_base(r + 16) = + 1024)
            *reinterpret_cast<uint4*>(aslot + wr_row + uint32_t(ks) * 1024u) = raw[ks][mt];
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
            a[ks][mt] = *reinterpret_cast<const frag*>(aslot +
                                                       (rd_row ^ uint32_t((ks * 2 + h) << 4)));
        }
      };
      frag b0[2][2], b1[2][2], b2[2][2], b3[2][2], a0[2][2], a1[2][2];
      uint4 q0[2][2], q1[2][2];  // row-contiguous A loads of a step
      Cur ca{0, 0}, cb{0, 0};    // the steps of the next A bases and the next B loads
      uint4 e_cur;               // bases of the next A loads' step
      int rc_cur;
      {
        const uint32_t k0 = s_kb[0];
        const int rc0 = cb.rc;
        advance(cb);
        const uint32_t k1 = s_kb[cb.it];
        const int rc1 = cb.rc;
        advance(cb);
        const uint4 e0 = bases(ca.it);
        const int ra0 = ca.rc;
        advance(ca);
        const uint4 e1 = bases(ca.it);
        const int ra1 = ca.rc;
        advance(ca);
        e_cur = bases(ca.it);
        rc_cur = ca.rc;
        advance(ca);
        __builtin_amdgcn_sched_barrier(0);
        gload_a(e0, ra0, q0);
        __builtin_amdgcn_sched_barrier(0);
        load_b(k0, rc0, b0);
        __builtin_amdgcn_sched_barrier(0);
        gload_a(e1, ra1, q1);
        __builtin_amdgcn_sched_barrier(0);
        load_b(k1, rc1, b1);
        __builtin_amdgcn_sched_barrier(0);
        through_slot(q0, a0);
        __builtin_amdgcn_sched_barrier(0);
      }
      // Step j: the A loads of step j + 2 (their bases read in step j - 1),
      // the MFMAs of step j (fragments from step j - 1), the fragments of
      // step j + 1 through the slot (loaded in step j - 1), the B loads of
      // step j + 2 and the A bases of step j + 3.
      auto step = [&](frag (&bc)[2][2], frag (&bn)[2][2], frag (&ac)[2][2], frag (&an)[2][2],
                      uint4 (&qn1)[2][2], uint4 (&qn2)[2][2]) {
        const uint32_t kb = s_kb[cb.it];
        const int rcb = cb.rc;
        advance(cb);
        gload_a(e_cur, rc_cur, qn2);
        const uint4 e_nxt = bases(ca.it);
        const int rc_nxt = ca.rc;
        advance(ca);
        __builtin_amdgcn_sched_barrier(0);
        mma_item<T>(ac, bc, acc);
        __builtin_amdgcn_sched_barrier(0);
        through_slot(qn1, an);
        __builtin_amdgcn_sched_barrier(0);
        load_b(kb, rcb, bn);
        __builtin_amdgcn_sched_barrier(0);
        e_cur = e_nxt;
        rc_cur = rc_nxt;
      };
      // Steps 0 .. 4 ceil(S / 4) - 1 for S = nrc * nact: the A and B loads
      // reach at most item nact + 4 of the last chunk, the last padding item
      // (the bases read ahead stop there).
      static_assert(kPad >= 5, "the loads run 4 items past the last one");
      const int n_steps = nrc * nact;
      for (int j = 0; j < n_steps; j += 4) {
        step(b0, b2, a0, a1, q1, q0);
        step(b1, b3, a1, a0, q0, q1);
        step(b2, b0, a0, a1, q1, q0);
        step(b3, b1, a1, a0, q0, q1);
      }
      continue;
    }
    auto load_a = [&](const uint2& e, int rc, frag (&a)[2][2]) {
      const uint32_t s2[2] = {e.x, e.y};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int e0 = rc * kChunk + (ks * 2 + h) * V;  // first element of this lane's piece
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const uint32_t base = s2[mt];
          if (VEC)
            a[ks][mt] =
                buf_frag<T>(ra, (base != kOob && e0 < R) ? base + uint32_t(e0) * ES : kOob);
          else
            a[ks][mt] = buf_frag_elems<T>(ra, base, e0, R);
        }
      }
    };
    frag b0[2][2], b1[2][2], b2[2][2], a0[2][2], a1[2][2], a2[2][2];
    Cur ca{0, 0}, cb{0, 0};  // the steps of the next A and the next B loads
    uint2 e_next;            // table entries of the next A loads' step
    {
      const uint32_t k0 = s_kb[0];
      const int rc0 = cb.rc;
      advance(cb);
      const uint32_t k1 = s_kb[cb.it];
      const int rc1 = cb.rc;
      advance(cb);
      const uint2 e0 = entry(0);
      advance(ca);
      __builtin_amdgcn_sched_barrier(0);
      load_b(k0, rc0, b0);
      __builtin_amdgcn_sched_barrier(0);
      load_b(k1, rc1, b1);
      __builtin_amdgcn_sched_barrier(0);
      load_a(e0, 0, a0);
      e_next = entry(ca.it);
      __builtin_amdgcn_sched_barrier(0);
    }
    auto step = [&](frag (&bc)[2][2], frag (&bn)[2][2], frag (&ac)[2][2], frag (&an)[2][2]) {
      load_a(e_next, ca.rc, an);
      advance(ca);
      const uint32_t kb = s_kb[cb.it];
      const int rcb = cb.rc;
      advance(cb);
      const uint2 e2 = entry(ca.it);
      __builtin_amdgcn_sched_barrier(0);
      mma_item<T>(ac, bc, acc);
      __builtin_amdgcn_sched_barrier(0);
      load_b(kb, rcb, bn);
      __builtin_amdgcn_sched_barrier(0);
      e_next = e2;
    };
    // Steps 0 .. 3 ceil(S / 3) - 1 for S = nrc * nact: the cursors reach at most
    // item nact + 3 of the last chunk, inside the kPad padding items.
    const int n_steps = nrc * nact;
    for (int j = 0; j < n_steps; j += 3) {
      step(b0, b2, a0, a1);
      step(b1, b0, a1, a2);
      step(b2, b1, a2, a0);
    }
  }
  __syncthreads();  // the tables are free for the epilogue
  store_tile<OutT>(acc, bias, ro, smem + L.src_off + uint32_t(wave) * 64u * epi_pitch(sizeof(OutT)),
                   slot0, n0, M, N, lane, order);
}

// A quarter of a (tile, 64-column block) by the direct path, the whole
// workgroup: rows 64 q .. 64 q + 63 of the tile, each wave a 32 x 32 block
// (row half w >> 1, column half w & 1).  A wave holds a quarter of
// direct_tile's work, so a tile whose waves carry many offsets can be spread
// over four workgroups.  Same per-row summation order as direct_tile (offset
// groups, chunks, offsets ascending, then the two K-steps of an item): results
// are bit-identical.  Uses direct_lds(min(kv, 64) + kPad) bytes of `smem`.
template <typename T, typename OutT, bool VEC>
__device__ __forceinline__ void direct_quarter(const T* __restrict__ A, const T* __restrict__ Bt,
                                               const int32_t* __restrict__ pairs,
                                               const float* __restrict__ bias,
                                               OutT* __restrict__ out, const GemmBufs& nb,
                                               int64_t n_src, int64_t M, int N, int R, int Rp,
                                               int kv, int64_t tile, int q, int n0,
                                               unsigned char* smem,
                                               const int32_t* __restrict__ order) {
  using frag = typename Mfma<T>::frag;
  constexpr int V = Mfma<T>::V;
  constexpr uint32_t ES = sizeof(T);
  constexpr int kChunk = kChunkBytes / int(ES);  // reduction elements per item

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t slot = tile * kTileRows + q * 64 + (wave >> 1) * 32 + l32;  // this lane's row
  const bool row_ok = slot < M;
  const int col = n0 + (wave & 1) * 32 + l32;  // this lane's B / output column

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, nb.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bt, nb.bt_bytes);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, nb.out_bytes);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(pairs, nb.pairs_bytes);

  const int G = kv < kGroupOffsets ? kv : kGroupOffsets;
  const int E = G + kPad;
  const DirectLds L = direct_lds(E, uint32_t(sizeof(OutT)));
  uint32_t* s_kb = reinterpret_cast<uint32_t*>(smem + L.kb_off) + wave * E;
  int32_t* s_src = reinterpret_cast<int32_t*>(smem + L.src_off) + wave * E * 64;

  const uint32_t row_bytes = uint32_t(R) * ES;
  const uint32_t slab_bytes = uint32_t(N) * V * ES;        // one (offset, r / V) slab of Bt
  const uint32_t k_bytes = uint32_t(Rp / V) * slab_bytes;  // one offset of Bt
  const int nrc = Rp / kChunk;                             // chunks per offset
  const uint32_t bcol = col < N ? uint32_t(col) * V * ES : kColOob;

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  for (int kc = 0; kc < kv; kc += G) {
    const int kn = kv - kc < G ? kv - kc : G;
    __syncthreads();  // the previous group's tables are no longer read
    // ---- this wave's table of the offsets with a pair in its 32 rows
    int nact = 0;
    constexpr int kTabBatch = 16;  // table loads in flight per lane
    for (int u0 = 0; u0 < kn; u0 += kTabBatch) {
      int32_t v[kTabBatch];
#pragma unroll
      for (int u = 0; u < kTabBatch; ++u) {
        const bool in = row_ok && u0 + u < kn;
        const int64_t e = int64_t(kc + u0 + u) * M + slot;
        v[u] = int32_t(__builtin_amdgcn_raw_buffer_load_b32(rp, in ? uint32_t(e * 4) : kOob, 0, 0));
      }
#pragma unroll
      for (int u = 0; u < kTabBatch; ++u) {
        const bool ok = row_ok && u0 + u < kn && v[u] >= 0 && v[u] < n_src;
        if (u0 + u < kn && __ballot(ok)) {  // wave-uniform (both lane halves hold the same rows)
          if (h == 0) s_src[nact * 32 + l32] = ok ? v[u] : -1;
          if (lane == 0) s_kb[nact] = uint32_t(kc + u0 + u) * k_bytes;
          ++nact;
        }
      }
    }
#pragma unroll
    for (int pi = 0; pi < kPad; ++pi) {  // padding items: no source row, out-of-range B
      if (h == 0) s_src[(nact + pi) * 32 + l32] = -1;
      if (lane == 0) s_kb[nact + pi] = kBOob;
    }
    if constexpr (sizeof(T) != 4) {
      // 16-bit operands: one pipeline per 64-byte chunk (32 channels).  With
      // 4-byte operands a chunk holds 16 channels, a row twice the chunks,
      // and one pipeline over the group's (chunk, item) steps, as in
      // direct_tile, measured faster: the reference-class fp32 layers' GEMM
      // (thin kernel, quarters) subm 0.106 -> 0.102 ms, strided 0.601 ->
      // 0.563, transposed 2.58 -> 2.50; the same for 16-bit operands made the
      // metric's split tail quarters 0.6 us slower.
      for (int rc = 0; rc < nrc; ++rc) {
        auto load = [&](int it, frag (&a)[2], frag (&b)[2]) {
          const int32_t src = s_src[it * 32 + l32];
          const uint32_t kb = s_kb[it];
          const uint32_t base = src >= 0 ? uint32_t(src) * row_bytes : kOob;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const int e0 = rc * kChunk + (ks * 2 + h) * V;
            if (VEC)
              a[ks] = buf_frag<T>(ra, (base != kOob && e0 < R) ? base + uint32_t(e0) * ES : kOob);
            else
              a[ks] = buf_frag_elems<T>(ra, base, e0, R);
            b[ks] = buf_frag<T>(rb, kb + bcol + uint32_t(rc * 4 + ks * 2 + h) * slab_bytes);
          }
        };
        // two items in flight: item it + 2 loads while item it multiplies
        frag a0[2], b0[2], a1[2], b1[2], a2[2], b2[2];
        load(0, a0, b0);
        load(1, a1, b1);
        auto step = [&](int it, frag (&ac)[2], frag (&bc)[2], frag (&an)[2], frag (&bn)[2]) {
          load(it + 2, an, bn);
          __builtin_amdgcn_sched_barrier(0);
          Mfma<T>::mma(ac[0], bc[0], acc);
          Mfma<T>::mma(ac[1], bc[1], acc);
          __builtin_amdgcn_sched_barrier(0);
        };
        for (int it = 0; it < nact; it += 3) {  // reads entries up to nact + 4 < nact + kPad
          step(it, a0, b0, a2, b2);
          step(it + 1, a1, b1, a0, b0);
          step(it + 2, a2, b2, a1, b1);
        }
      }
      continue;
    }
    nact = __builtin_amdgcn_readfirstlane(nact);  // wave-uniform: the cursor is scalar
    if (nact == 0) continue;                      // no pair in this wave's rows
    // The group's (chunk, item) steps as one pipeline, as in direct_tile: a
    // cursor walks items 0 .. nact - 1 of chunks 0 .. nrc - 1, then the
    // padding items after the last chunk.  Step j: the loads of step j + 2,
    // the MFMAs of step j.
    struct Cur {
      int rc, it;
    };
    auto advance = [&](Cur& c) {
      if (++c.it == nact && c.rc + 1 < nrc) {
        c.it = 0;
        ++c.rc;
      }
    };
    auto load = [&](const Cur& c, frag (&a)[2], frag (&b)[2]) {
      const int32_t src = s_src[c.it * 32 + l32];
      const uint32_t kb = s_kb[c.it];
      const uint32_t base = src >= 0 ? uint32_t(src) * row_bytes : kOob;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int e0 = c.rc * kChunk + (ks * 2 + h) * V;
        if (VEC)
          a[ks] = buf_frag<T>(ra, (base != kOob && e0 < R) ? base + uint32_t(e0) * ES : kOob);
        else
          a[ks] = buf_frag_elems<T>(ra, base, e0, R);
        b[ks] = buf_frag<T>(rb, kb + bcol + uint32_t(c.rc * 4 + ks * 2 + h) * slab_bytes);
      }
    };
    frag a0[2], b0[2], a1[2], b1[2], a2[2], b2[2];
    Cur cl{0, 0};  // the step of the next loads
    load(cl, a0, b0);
    advance(cl);
    load(cl, a1, b1);
    advance(cl);
    auto step = [&](frag (&ac)[2], frag (&bc)[2], frag (&an)[2], frag (&bn)[2]) {
      load(cl, an, bn);
      advance(cl);
      __builtin_amdgcn_sched_barrier(0);
      Mfma<T>::mma(ac[0], bc[0], acc);
      Mfma<T>::mma(ac[1], bc[1], acc);
      __builtin_amdgcn_sched_barrier(0);
    };
    // steps 0 .. 3 ceil(S / 3) - 1 for S = nrc * nact: the loads reach at most
    // item nact + 3 after the last chunk, inside the kPad padding items
    const int n_steps = nrc * nact;
    for (int j = 0; j < n_steps; j += 3) {
      step(a0, b0, a2, b2);
      step(a1, b1, a0, b0);
      step(a2, b2, a1, b1);
    }
  }
  // ---- epilogue: element stores (+ bias); rows past M and columns past N dropped
  const float bv = (bias && col < N) ? bias[col] : 0.f;
  auto out_row = [&](int64_t s) -> int64_t {
    if (!order || s >= M) return s;
    const int64_t r = order[s];
    return (r >= 0 && r < M) ? r : M;
  };
  const int64_t r0 = tile * kTileRows + q * 64 + (wave >> 1) * 32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = out_row(r0 + 8 * (i / 4) + 4 * h + (i % 4));
    const uint32_t off = (row < M && col < N) ? uint32_t((row * N + col) * int64_t(sizeof(OutT)))
                                              : kOob;
    buf_store<OutT>(from_f32<OutT>(acc[i] + bv), ro, off);
  }
}

// Every tile of an unplanned call, one workgroup per (tile, 64 columns).
// ORDERED instances take tile rows through `order` (the natural ones ignore
// the argument, so the pointer costs them no registers).
template <typename T, typename OutT, bool VEC, bool ORDERED>
__global__ __launch_bounds__(256, 2) void gather_gemm_direct(
    const T* __restrict__ A, const T* __restrict__ Bt, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ order, const float* __restrict__ bias, OutT* __restrict__ out,
    GemmBufs nb, int64_t n_src, int64_t M, int N, int R, int Rp, int kv,
    const uint32_t* __restrict__ words, int mic) {
  extern __shared__ __align__(16) unsigned char smem[];
  int64_t tile;
  int n0;
  if (!block_tile(M, N, &tile, &n0)) return;
  direct_tile<T, OutT, VEC>(A, Bt, pairs, bias, out, nb, n_src, M, N, R, Rp, kv, tile, n0, smem,
                            ORDERED ? order : nullptr, ORDERED ? words : nullptr, mic);
}

// ---------------------------------------------------------------------------
// staged kernel
// ---------------------------------------------------------------------------

constexpr int kRing = 4;  // B ring slots of the staged kernel (one item each)

// Dynamic LDS of the staged kernel: B offsets of the tile's items (E plus the
// read-ahead past the last group), the byte offsets of the tile's distinct rows
// in A, the staged rows (kLdsRows chunks) and the B ring; the epilogue tiles
// overlap the staged rows and the ring.
struct StagedLds {
  uint32_t kb_off, rowoff_off, rows_off, ring_off, total;
};

__host__ __device__ inline StagedLds staged_lds(int E, uint32_t out_size) {
  StagedLds l;
  l.kb_off = 0;
  l.rowoff_off = (4u * uint32_t(E + 2 * kItemGroup) + 255u) / 256u * 256u;
  l.rows_off = l.rowoff_off + uint32_t(kLdsRows) * 4u;
  l.ring_off = l.rows_off + uint32_t(kLdsRows * kChunkBytes);
  l.total = l.ring_off + uint32_t(kRing) * kSlabBytes;
  if (l.total < l.rows_off + epi_bytes(out_size)) l.total = l.rows_off + epi_bytes(out_size);
  return l;
}

// SPLIT instances (one column block, N <= 64) take the last n_split tiles,
// which would otherwise run as a round of their own on n_split CUs after the
// others have finished, in quarters by the direct path (direct_quarter,
// bit-identical): the grid's first staged_split_extra(n_split) workgroups take
// the quarters (starting first, they finish early), the rest the other tiles.
__host__ __device__ inline int64_t staged_split_extra(int n_split) {
  return 8 * ((4 * int64_t(n_split) + 7) / 8);  // a multiple of 8 keeps the XCD mapping
}

// Every tile of a planned call (kv <= kPlanMaxKv): staged when its distinct
// rows fit in LDS and its items (at most kPlanMaxItems, in one group of
// kGroupOffsets offsets) are listed, else (an overflow tile) by the direct
// path.  ORDERED as
// for the direct kernel.
template <typename T, typename OutT, bool VEC, bool ORDERED, bool SPLIT = false>
__global__ __launch_bounds__(256, 2) void gather_gemm_staged(
    const T* __restrict__ A, const T* __restrict__ Bt, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ order_arg, PlanDev plan, const float* __restrict__ bias,
    OutT* __restrict__ out, GemmBufs nb, int64_t n_src, int64_t M, int N, int R, int Rp,
    int kv, int n_split) {
  const int32_t* __restrict__ order = ORDERED ? order_arg : nullptr;
  using frag = typename Mfma<T>::frag;
  constexpr int V = Mfma<T>::V;
  constexpr uint32_t ES = sizeof(T);
  constexpr int kChunk = kChunkBytes / int(ES);  // reduction elements per item
  constexpr int kRowsPerLane = kLdsRows / 64;    // staged rows copied per thread and chunk
  static_assert(V * ES == 16, "fragments and B slab pieces are 16 bytes");
  static_assert(kLdsRows % 64 == 0, "rows are copied 64 per workgroup pass");
  static_assert(kItemGroup == 4 && kRing == 4, "the step loop is unrolled over 4 items");
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, l32 = lane & 31;
  int64_t tile;
  int n0;
  if constexpr (SPLIT) {  // one column block
    const int64_t n_extra = staged_split_extra(n_split);
    const int64_t nt_main = (M + kTileRows - 1) / kTileRows - n_split;
    if (blockIdx.x < n_extra) {  // whole workgroup (uniform)
      const int64_t e = blockIdx.x;
      if (e >= 4 * int64_t(n_split)) return;
      direct_quarter<T, OutT, VEC>(A, Bt, pairs, bias, out, nb, n_src, M, N, R, Rp, kv,
                                   nt_main + e / 4, int(e % 4), 0, smem, order);
      return;
    }
    tile = xcd_tile(int64_t(blockIdx.x) - n_extra, nt_main);
    n0 = 0;
  } else {
    if (!staged_tile(M, N, &tile, &n0)) return;
    // with a row order, tiles in reverse, as in the thin kernel: in mask
    // order the rows with the most mask bits come last, and their tiles (most
    // items, and the overflow tiles the direct path takes) should start first
    // rather than set the end
    if constexpr (ORDERED) tile = (M + kTileRows - 1) / kTileRows - 1 - tile;
  }
  const int64_t slot0 = tile * kTileRows + wave * 64;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, nb.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bt, nb.bt_bytes);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, nb.out_bytes);

  const int E = plan.E;
  const StagedLds L = staged_lds(E, uint32_t(sizeof(OutT)));
  uint32_t* s_kb = reinterpret_cast<uint32_t*>(smem + L.kb_off);
  unsigned char* rows_lds = smem + L.rows_off;
  unsigned char* ring = smem + L.ring_off;

  const uint32_t row_bytes = uint32_t(R) * ES;
  const uint32_t slab_bytes = uint32_t(N) * V * ES;        // one (offset, r / V) slab of Bt
  const uint32_t k_bytes = uint32_t(Rp / V) * slab_bytes;  // one offset of Bt
  const int nrc = Rp / kChunk;                             // chunks per offset

  // ---- prologue: every load below is independent of the others, so they
  // share one memory round trip (the row list is padded with -1, so its loads
  // need not wait for the count)
  const int p = tid & 3, ub = tid >> 2;  // this thread copies piece p of rows ub + 64 j
  const int U = plan.count[tile];
  int32_t rrow[kRowsPerLane];
  {
    const int32_t* rows = plan.rows + tile * kLdsRows;
#pragma unroll
    for (int j = 0; j < kRowsPerLane; ++j) rrow[j] = rows[ub + 64 * j];
  }
  const int nact = plan.nact[tile];
  const int32_t ko = tid < E ? plan.koff[tile * E + tid] : -1;
  if (U >= kLdsRows) {  // whole workgroup: an overflow tile
    // (the natural-order instances, whose tiles rarely overflow, keep the
    // gathers straight into fragments: the slot path's registers cost the
    // metric layer's staged steps 0.8 us)
    direct_tile<T, OutT, VEC, ORDERED>(A, Bt, pairs, bias, out, nb, n_src, M, N, R, Rp, kv, tile,
                                       n0, smem, order);
    return;
  }
  // byte offsets of the rows in A, kept in LDS (not registers) while the
  // K-loop runs; the four threads of a row write the same value
  uint32_t* s_rowoff = reinterpret_cast<uint32_t*>(smem + L.rowoff_off);
#pragma unroll
  for (int j = 0; j < kRowsPerLane; ++j)
    s_rowoff[ub + 64 * j] = rrow[j] >= 0 ? uint32_t(rrow[j]) * row_bytes : kOob;

  // Staging of a chunk: issue_stage(rc) loads chunk rc of this thread's rows
  // into registers, always all kRowsPerLane loads (out-of-range ones read
  // zeros) so that the compiler's load counts do not depend on U; put_stage()
  // writes them to LDS.  Chunk 0 is loaded now, chunk rc + 1 while chunk rc is
  // multiplied.
  frag st[kRowsPerLane];
  auto issue_stage = [&](int rc) {
    const int e0 = rc * kChunk + p * V;
#pragma unroll
    for (int j = 0; j < kRowsPerLane; ++j) {
      const uint32_t ro = s_rowoff[ub + 64 * j];
      if (VEC)
        st[j] = buf_frag<T>(ra, (ro != kOob && e0 < R) ? ro + uint32_t(e0) * ES : kOob);
      else
        st[j] = buf_frag_elems<T>(ra, ro, e0, R);
    }
  };
  auto put_stage = [&]() {
    const uint32_t wbase = L.rows_off + (chunk_base(uint32_t(ub)) ^ uint32_t(p << 4));
#pragma unroll
    for (int j = 0; j < kRowsPerLane; ++j)
      if (ub + 64 * j <= U)  // rows past the zero row are not stored
        *reinterpret_cast<frag*>(smem + wbase + 4096u * uint32_t(j)) = st[j];
  };
  issue_stage(0);
  // B offsets of the items; the entries past the tile's items (padding and
  // read-ahead) point past Bt, so their slabs read as zeros
  if (tid < E + 2 * kItemGroup)
    s_kb[tid] = (tid < E && ko >= 0) ? uint32_t(ko) * k_bytes : kBOob;
  floatx16 acc[2][2];
  zero_acc(acc);
  put_stage();
  __syncthreads();

  // this thread's 16-byte piece of every B slab: piece gp, column cp
  const int gp = tid >> 6, cp = n0 + (tid & 63);
  const uint32_t bpiece = cp < N ? uint32_t(cp) * V * ES : kColOob;
  // this lane's 4-byte A address record of item i (rows l32 and 32 + l32 of
  // its wave); items past the tile's last group read zeros (the staged row 0,
  // whose fragments are never multiplied)
  const int n_items = (nact + kItemGroup - 1) / kItemGroup * kItemGroup;
  const __amdgpu_buffer_rsrc_t rrec =
      make_rsrc(plan.addr + tile * E * kTileRows, uint32_t(E) * kTileRows * 2u);
  const uint32_t rec_lane = uint32_t(wave) * 128u + uint32_t(l32) * 4u;
  auto load_rec = [&](int i) -> uint32_t {
    return __builtin_amdgcn_raw_buffer_load_b32(
        rrec, i < n_items ? uint32_t(i) * 512u + rec_lane : kOob, 0, 0);
  };

  const uint32_t zaddr = chunk_base(uint32_t(U));  // the tile's zero row
  for (int rc = 0; rc < nrc; ++rc) {
    const uint32_t bofs = uint32_t(rc * 4 + gp) * slab_bytes + bpiece;
    auto gload = [&](uint32_t kb) -> uint4 {  // this thread's piece of an item's B slab
      return __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, kb + bofs, 0, 0));
    };
    auto ring_put = [&](int slot, const uint4& v) {
      *reinterpret_cast<uint4*>(ring + uint32_t(slot) * kSlabBytes + uint32_t(tid) * 16u) = v;
    };
    auto read_b = [&](int slot, frag (&b)[2][2]) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          b[ks][nt] = *reinterpret_cast<const frag*>(ring + uint32_t(slot) * kSlabBytes +
                                                     uint32_t(ks * 2 + h) * 1024u +
                                                     uint32_t(nt * 32 + l32) * 16u);
    };
    auto read_a = [&](uint32_t e, frag (&a)[2][2]) {
      const uint32_t t2[2] = {e & 0xffffu, e >> 16};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
          a[ks][mt] = *reinterpret_cast<const frag*>(rows_lds +
                                                     (t2[mt] ^ (uint32_t(ks * 2 + h) << 4)));
    };

    // ---- pipeline.  Item i's B piece is loaded from global memory in step
    // i-6, written to ring slot i % 4 in step i-3 and read into registers in
    // step i-1; its A address record is loaded in step i-5 and its A fragments
    // are read in step i-1; its MFMAs run in step i.  Step `it`:
    //   1. ring write of item it+3,
    //   2. the 8 MFMAs of item it, and between them the LDS reads of item
    //      it+1's A and B fragments, the B offset of item it+6, and the global
    //      loads of item it+5's A record and item it+6's B piece,
    //   3. after odd steps, a barrier: a ring slot is written two steps after
    //      its last read and read two steps after its write, so one barrier in
    //      every two steps separates both.
    // The loop is unrolled over one group (4 steps), so every register and
    // ring index is static.
    frag fa[2][2][2], fb[2][2][2];  // [item parity][ks][mt or nt]
    uint4 q[4];                     // B pieces loaded, not yet in the ring: item i in q[i % 4]
    uint32_t r[4];                  // A address records: item i in r[i % 4]
    // A 32-row block of an item whose rows all read the zero row (no pair in
    // the block, or a padding item) multiplies zeros.  With fp32 operands
    // (4 MFMAs of 64 clocks per fragment pair, the MFMA pipe is the limit)
    // its MFMAs are skipped; the test is a wave ballot, so the branch is
    // uniform.  For 16-bit operands the MFMAs are not the limit and the test
    // costs more than it saves (measured at the metric shape), so it is
    // compiled out.
    constexpr bool kSkipDead = sizeof(T) == 4;
    bool live[2][2] = {{true, true}, {true, true}};  // [item parity][mt]
    auto block_live = [&](uint32_t addr) -> bool {
      return !kSkipDead || __builtin_amdgcn_ballot_w64(addr != zaddr) != 0;
    };
    {
      const uint4 p0 = gload(s_kb[0]), p1 = gload(s_kb[1]), p2 = gload(s_kb[2]);
      r[0] = load_rec(0);
      r[1] = load_rec(1);
      r[2] = load_rec(2);
      r[3] = load_rec(3);
      q[3] = gload(s_kb[3]);
      q[0] = gload(s_kb[4]);
      q[1] = gload(s_kb[5]);
      ring_put(0, p0);
      ring_put(1, p1);
      ring_put(2, p2);
      lds_barrier();
      read_b(0, fb[0]);
      read_a(r[0], fa[0]);
      if constexpr (kSkipDead) {
        live[0][0] = block_live(r[0] & 0xffffu);
        live[0][1] = block_live(r[0] >> 16);
      }
      r[0] = load_rec(4);
      lds_barrier();  // the prologue counts as an odd step (slot 0 is rewritten in step 1)
    }
    // One MFMA at a time with the step's other work between them: a wave
    // that issues its eight MFMAs back to back waits for the MFMA pipe (which
    // it shares with the other workgroup's wave on its SIMD) and then does its
    // LDS, global and barrier work while the pipe idles; interleaved, that
    // work is issued in the shadow of the MFMAs.
    auto step = [&](int it, auto jc) {
      constexpr int j = decltype(jc)::value;  // it % 4
      const frag(&ac)[2][2] = fa[j % 2];
      const frag(&bc)[2][2] = fb[j % 2];
      frag(&an)[2][2] = fa[(j + 1) % 2];
      frag(&bn)[2][2] = fb[(j + 1) % 2];
      const uint32_t e = r[(j + 1) % 4];
      const uint32_t t2[2] = {e & 0xffffu, e >> 16};
      const unsigned char* slot_b = ring + uint32_t((j + 1) % 4) * kSlabBytes;
      auto rd_a = [&](int ks, int mt) {
        an[ks][mt] = *reinterpret_cast<const frag*>(rows_lds +
                                                   (t2[mt] ^ (uint32_t(ks * 2 + h) << 4)));
      };
      auto rd_b = [&](int ks, int nt) {
        bn[ks][nt] = *reinterpret_cast<const frag*>(slot_b + uint32_t(ks * 2 + h) * 1024u +
                                                   uint32_t(nt * 32 + l32) * 16u);
      };
      auto mma = [&](int ks, int mt, int nt) {
        if (!kSkipDead || live[j % 2][mt]) Mfma<T>::mma(ac[ks][mt], bc[ks][nt], acc[mt][nt]);
        __builtin_amdgcn_sched_barrier(0);
      };
      if constexpr (kSkipDead) {
        live[(j + 1) % 2][0] = block_live(t2[0]);
        live[(j + 1) % 2][1] = block_live(t2[1]);
      }
      // first LDS operation of the step: the B load below waits for it, and
      // LDS operations complete in order, so issued last it would make that
      // wait drain every fragment read of the step
      const uint32_t kb = s_kb[it + 6];
      ring_put((j + 3) % 4, q[(j + 3) % 4]);
      __builtin_amdgcn_sched_barrier(0);
      // fragment reads in the order the next step's MFMAs consume them
      mma(0, 0, 0);
      rd_a(0, 0);
      rd_b(0, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(0, 0, 1);
      rd_b(0, 1);
      rd_a(0, 1);
      __builtin_amdgcn_sched_barrier(0);
      mma(0, 1, 0);
      rd_a(1, 0);
      rd_b(1, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(0, 1, 1);
      rd_b(1, 1);
      rd_a(1, 1);
      __builtin_amdgcn_sched_barrier(0);
      mma(1, 0, 0);
      mma(1, 0, 1);
      r[(j + 1) % 4] = load_rec(it + 5);
      __builtin_amdgcn_sched_barrier(0);
      mma(1, 1, 0);
      q[(j + 2) % 4] = gload(kb);
      __builtin_amdgcn_sched_barrier(0);
      mma(1, 1, 1);
      // the ring write and the B reads must be complete before the barrier
      // (the ring slots are shared)
      if constexpr (j % 2 == 1) lds_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    step(0, I0{});
    step(1, I1{});
    // next chunk's rows: issued after the first steps' loads, so the waits of
    // the next steps do not cover them (past the last chunk the loads read
    // zeros and are dropped)
    issue_stage(rc + 1);
    step(2, I2{});
    step(3, I3{});
    for (int it = 4; it < n_items; it += kItemGroup) {
      step(it, I0{});
      step(it + 1, I1{});
      step(it + 2, I2{});
      step(it + 3, I3{});
    }
    // The loads in flight are read here on every path, so that the compiler
    // cannot sink the ones issued before the loop (only the loop reads them)
    // to the loop's entry, which would issue them late.
    using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;
    asm volatile("" ::"v"(__builtin_bit_cast(u32x4, q[0])), "v"(__builtin_bit_cast(u32x4, q[1])),
                 "v"(__builtin_bit_cast(u32x4, q[2])), "v"(__builtin_bit_cast(u32x4, q[3])),
                 "v"(r[0]), "v"(r[1]), "v"(r[2]), "v"(r[3]));
    if (rc + 1 < nrc) {
      put_stage();  // every wave is past the last barrier of chunk rc
      __syncthreads();
    }
  }
  __syncthreads();  // staged rows and ring are free for the epilogue
  store_tile<OutT>(acc, bias, ro, rows_lds + uint32_t(wave) * 64u * epi_pitch(sizeof(OutT)), slot0,
                   n0, M, N, lane, order);
}

// ---------------------------------------------------------------------------
// thin kernel
// ---------------------------------------------------------------------------
//
// Tables with about one pair per row, taken in mask order (a transposed or
// strided convolution of sparse voxels, a submanifold one of isolated voxels):
// a tile's rows share one mask, so a tile holds one to four live offsets and
// each of its chunks only a few MFMA steps.  The staged kernel issues a
// chunk's rows two steps before it stores them, so there every chunk waits
// for a memory round trip.  Here the plan's item list (at most kThinItems
// items, its A address records read once per tile) is the same for every
// chunk, and a chunk's rows and weight slabs are loaded three chunks ahead
// into registers: chunk c + 3's loads are issued when chunk c starts and
// stored to LDS when chunk c + 2 ends, so every wait in the loop is for loads
// issued two chunks' work earlier.  Items past the tile's own are not multiplied at all.
// Tiles with more items or more distinct rows than the thin layout holds take
// the direct path, as overflow tiles do in the staged kernel.  Same
// summation order as the staged kernel (items ascending inside each chunk,
// chunks ascending), so results are bit-identical.

constexpr int kThinRows = 320;   // staged rows per tile, including the zero row
constexpr int kThinItems = 4;    // items a thin tile may hold
// The thin kernel's QUARTER instances take the direct path in quarters
// (direct_quarter) and spread those of the last kThinSplitTiles tiles over
// four workgroups.  The host picks them for fp32 operands (whose MFMAs are
// slow enough that a wave of a heavy tile sets the kernel's end) and for
// 16-bit grids of at most kThinQuarterGrid workgroups (where the heavy tiles'
// waves run after most others are done); elsewhere a quarter's 32 x 32 waves,
// which load twice the bytes per MFMA of direct_tile's 64 x 64 ones, cost
// more than the split saves.  The two paths are never compiled into one
// instance: together they outgrow the instruction cache.
constexpr int kThinSplitTiles = 16;
constexpr int64_t kThinQuarterGrid = 1024;

// Workgroups in front of the thin grid for quarters 1..3 of the last n_split
// tiles' gy column blocks, rounded up to 8 so that the XCD mapping holds.
__host__ __device__ inline int64_t thin_split_extra(int n_split, int gy) {
  return 8 * ((3 * int64_t(n_split) * gy + 7) / 8);
}

struct ThinLds {
  uint32_t rows_off, slab_off, total;
};

__host__ __device__ inline ThinLds thin_lds(uint32_t out_size) {
  ThinLds l;
  l.rows_off = 0;
  l.slab_off = l.rows_off + uint32_t(kThinRows * kChunkBytes);
  l.total = l.slab_off + uint32_t(kThinItems) * kSlabBytes;
  if (l.total < l.rows_off + epi_bytes(out_size)) l.total = l.rows_off + epi_bytes(out_size);
  return l;
}

template <typename T, typename OutT, bool VEC, bool ORDERED, bool QUARTER>
__global__ __launch_bounds__(256, 2) void gather_gemm_thin(
    const T* __restrict__ A, const T* __restrict__ Bt, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ order_arg, PlanDev plan, const float* __restrict__ bias,
    OutT* __restrict__ out, GemmBufs nb, int64_t n_src, int64_t M, int N, int R, int Rp,
    int kv, int n_split) {
  const int32_t* __restrict__ order = ORDERED ? order_arg : nullptr;
  using frag = typename Mfma<T>::frag;
  constexpr int V = Mfma<T>::V;
  constexpr uint32_t ES = sizeof(T);
  constexpr int kChunk = kChunkBytes / int(ES);  // reduction elements per item
  constexpr int kPerLane = kThinRows / 64;       // staged rows copied per thread and chunk
  static_assert(V * ES == 16, "fragments and B slab pieces are 16 bytes");
  static_assert(kThinRows % 64 == 0 && kThinRows <= kLdsRows, "thin rows");
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, l32 = lane & 31;
  // Tiles the thin layout does not hold (the rows with the most mask bits,
  // last in mask order) take the direct path, and their waves carry many
  // offsets.  QUARTER instances: among the last n_split tiles each such (tile,
  // 64-column block) is spread over four workgroups of a quarter of its rows:
  // the grid's first n_extra workgroups (3 per (tile, column block) of those
  // tiles, rounded up to 8 so that the XCD mapping below holds) take quarters
  // 1..3 and exit at once for other tiles; the rest take the tiles as below,
  // with quarter 0 of a split tile and all four quarters of an earlier one.
  int64_t tile;
  int n0;
  if constexpr (QUARTER) {
    const int64_t nt_all = (M + kTileRows - 1) / kTileRows;
    const int gy = (N + 63) / 64;
    const int64_t n_extra = thin_split_extra(n_split, gy);
    auto direct_heavy = [&](int64_t t) -> bool {
      return plan.count[t] >= kThinRows || plan.nact[t] > kThinItems;
    };
    int q_lo = 0, q_hi = 0;  // quarters [q_lo, q_hi) by the direct path
    if (blockIdx.x < n_extra) {
      const int64_t e = blockIdx.x;
      if (e >= 3 * int64_t(n_split) * gy) return;
      const int64_t tc = e / 3;  // (tile, column block), heaviest tiles first
      tile = nt_all - 1 - tc / gy;
      if (!direct_heavy(tile)) return;
      n0 = int(tc % gy) * 64;
      q_lo = 1 + int(e % 3);
      q_hi = q_lo + 1;
    } else {
      if (!staged_tile_of(blockIdx.x - n_extra, gridDim.x - n_extra, M, N, &tile, &n0)) return;
      tile = nt_all - 1 - tile;  // reverse order, as below
      if (direct_heavy(tile)) q_hi = tile >= nt_all - n_split ? 1 : 4;
    }
    if (q_hi > 0) {  // whole workgroup (uniform)
      for (int qr = q_lo; qr < q_hi; ++qr)
        direct_quarter<T, OutT, VEC>(A, Bt, pairs, bias, out, nb, n_src, M, N, R, Rp, kv, tile,
                                     qr, n0, smem, order);
      return;
    }
  } else {
    if (!staged_tile(M, N, &tile, &n0)) return;
    // tiles in reverse order: in mask order the rows with the most bits come
    // last, and their tiles (the ones the direct path takes, many times
    // longer than a thin one) should start first rather than set the end
    tile = (M + kTileRows - 1) / kTileRows - 1 - tile;
  }
  const int64_t slot0 = tile * kTileRows + wave * 64;

  const int U = plan.count[tile];
  const int nact = plan.nact[tile];
  if constexpr (!QUARTER) {
    if (U >= kThinRows || nact > kThinItems) {  // whole workgroup (uniform)
      direct_tile<T, OutT, VEC>(A, Bt, pairs, bias, out, nb, n_src, M, N, R, Rp, kv, tile, n0,
                                smem, order);
      return;
    }
  }

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, nb.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bt, nb.bt_bytes);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, nb.out_bytes);
  const ThinLds L = thin_lds(uint32_t(sizeof(OutT)));
  unsigned char* rows_lds = smem + L.rows_off;
  unsigned char* slabs = smem + L.slab_off;

  const uint32_t row_bytes = uint32_t(R) * ES;
  const uint32_t slab_bytes = uint32_t(N) * V * ES;        // one (offset, r / V) slab of Bt
  const uint32_t k_bytes = uint32_t(Rp / V) * slab_bytes;  // one offset of Bt
  const int nrc = Rp / kChunk;                             // chunks per offset
  const int E = plan.E;

  // ---- per tile: source rows (as A byte offsets), the items' B offsets and
  // this lane's A address records
  const int p = tid & 3, ub = tid >> 2;  // this thread copies piece p of rows ub + 64 j
  uint32_t rowoff[kPerLane];
  {
    const int32_t* rows = plan.rows + tile * kLdsRows;
    int32_t rr[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) rr[j] = rows[ub + 64 * j];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) rowoff[j] = rr[j] >= 0 ? uint32_t(rr[j]) * row_bytes : kOob;
  }
  uint32_t kb[kThinItems];  // B offset of each item (uniform)
#pragma unroll
  for (int i = 0; i < kThinItems; ++i) {
    const int32_t ko = i < nact ? plan.koff[tile * E + i] : -1;
    kb[i] = ko >= 0 ? uint32_t(ko) * k_bytes : kBOob;
  }
  uint32_t rec[kThinItems];  // A address records: rows l32 and 32 + l32 of this wave
  {
    const __amdgpu_buffer_rsrc_t rrec =
        make_rsrc(plan.addr + tile * E * kTileRows, uint32_t(E) * kTileRows * 2u);
    const uint32_t rec_lane = uint32_t(wave) * 128u + uint32_t(l32) * 4u;
#pragma unroll
    for (int i = 0; i < kThinItems; ++i)
      rec[i] = __builtin_amdgcn_raw_buffer_load_b32(
          rrec, i < nact ? uint32_t(i) * 512u + rec_lane : kOob, 0, 0);
  }

  // ---- loads of one chunk into registers, and their stores into LDS
  // this thread's piece of every item's B slab: piece gp, column cp
  const int gp = tid >> 6, cp = n0 + (tid & 63);
  const uint32_t bpiece = (cp < N ? uint32_t(cp) * V * ES : kColOob) + uint32_t(gp) * slab_bytes;
  struct Chunk {
    frag st[kPerLane];
    uint4 q[kThinItems];
  };
  auto load_chunk = [&](int rc, Chunk& ch) {  // past the last chunk: zeros, never stored
    const int e0 = rc * kChunk + p * V;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const uint32_t o = rowoff[j];
      if (VEC)
        ch.st[j] = buf_frag<T>(ra, (o != kOob && e0 < R && rc < nrc) ? o + uint32_t(e0) * ES : kOob);
      else
        ch.st[j] = buf_frag_elems<T>(ra, rc < nrc ? o : kOob, e0, R);
    }
    const uint32_t cofs = uint32_t(rc) * 4u * slab_bytes + bpiece;
#pragma unroll
    for (int i = 0; i < kThinItems; ++i)
      ch.q[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, rc < nrc ? kb[i] + cofs : kOob, 0, 0));
  };
  auto store_chunk = [&](const Chunk& ch) {
    const uint32_t wbase = chunk_base(uint32_t(ub)) ^ uint32_t(p << 4);
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (ub + 64 * j <= U)  // rows past the zero row are not stored
        *reinterpret_cast<frag*>(rows_lds + wbase + 4096u * uint32_t(j)) = ch.st[j];
#pragma unroll
    for (int i = 0; i < kThinItems; ++i)
      if (i < nact)
        *reinterpret_cast<uint4*>(slabs + uint32_t(i) * kSlabBytes + uint32_t(tid) * 16u) = ch.q[i];
  };

  // ---- one chunk's MFMAs: the tile's items in ascending order
  const uint32_t zaddr = chunk_base(uint32_t(U));  // the tile's zero row
  constexpr bool kSkipDead = sizeof(T) == 4;       // as in the staged kernel
  floatx16 acc[2][2];
  zero_acc(acc);
  auto multiply = [&]() {
#pragma unroll
    for (int i = 0; i < kThinItems; ++i) {
      if (i < nact) {  // uniform
        const uint32_t t2[2] = {rec[i] & 0xffffu, rec[i] >> 16};
        bool live[2] = {true, true};
        if constexpr (kSkipDead) {
          live[0] = __builtin_amdgcn_ballot_w64(t2[0] != zaddr) != 0;
          live[1] = __builtin_amdgcn_ballot_w64(t2[1] != zaddr) != 0;
        }
        frag a[2][2], b[2][2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            a[ks][mt] = *reinterpret_cast<const frag*>(rows_lds +
                                                      (t2[mt] ^ (uint32_t(ks * 2 + h) << 4)));
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            b[ks][nt] = *reinterpret_cast<const frag*>(slabs + uint32_t(i) * kSlabBytes +
                                                      uint32_t(ks * 2 + h) * 1024u +
                                                      uint32_t(nt * 32 + l32) * 16u);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            if (!kSkipDead || live[mt])
#pragma unroll
              for (int nt = 0; nt < 2; ++nt) Mfma<T>::mma(a[ks][mt], b[ks][nt], acc[mt][nt]);
      }
    }
  };

  // ---- the chunk loop, unrolled by three so that the register sets are
  // static: while chunk c is multiplied, chunks c + 1 and c + 2 wait in two
  // sets (loaded when chunks c - 2 and c - 1 started) and chunk c + 3's loads
  // fill the third, so a load has three chunks' work to arrive in.  Every
  // store is unconditional, so no path reaches a load into a set whose
  // previous loads were not consumed (the compiler would wait for them
  // first); chunks past the last read zeros and are not multiplied.
  Chunk c0, c1, c2;
  load_chunk(0, c0);
  load_chunk(1, c1);
  load_chunk(2, c2);
  store_chunk(c0);
  __syncthreads();
  for (int rc = 0; rc < nrc; rc += 3) {
    load_chunk(rc + 3, c0);
    multiply();
    __syncthreads();  // chunk rc's LDS is no longer read
    store_chunk(c1);
    __syncthreads();
    load_chunk(rc + 4, c1);
    if (rc + 1 < nrc) multiply();
    __syncthreads();
    store_chunk(c2);
    __syncthreads();
    load_chunk(rc + 5, c2);
    if (rc + 2 < nrc) multiply();
    __syncthreads();
    store_chunk(c0);
    __syncthreads();
  }
  store_tile<OutT>(acc, bias, ro, rows_lds + uint32_t(wave) * 64u * epi_pitch(sizeof(OutT)), slot0,
                   n0, M, N, lane, order);
}
