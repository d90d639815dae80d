// Gather plans: per-tile staging tables of a gather table, for the staged
// gather-GEMM (sp_gather_gemm.h).
//
// The GEMM cuts the output rows into tiles of kTileRows (4 waves x 64 rows).
// Neighbouring output rows share most of their neighbours, so the (offset, row)
// entries of a tile reference ~3x fewer distinct source rows than it has pairs
// (a 256-row tile of a 200k-voxel surface cloud: ~2600 pairs, ~765 distinct
// rows).  The GEMM copies those distinct rows once per tile into LDS ("slots"
// 0..U-1 of the tile, slot U being a zero row) and reads every gather from
// there.  A plan holds what it needs for that, computed once per table:
//   * per tile: U and the ascending list of distinct source rows;
//   * per tile: the offsets with at least one pair among its rows ("items",
//     ascending), which the GEMM takes in groups of kItemGroup; at most
//     kPlanMaxItems, all in one group of kPlanGroupOffsets offsets (a tile
//     with more, or spanning two groups, is an overflow tile, below);
//   * for every (item, row) the LDS byte address of the row's staged chunk
//     (chunk_base(slot); the zero row for a row without a pair, a row past M
//     and the items that fill up the tile's last group).
//
// Layout of one plan buffer (256-byte aligned parts), E = min(kv, kPlanMaxItems)
// rounded up to a multiple of kItemGroup:
//   n_overflow                  int32   number of overflow tiles (below); it and
//                                       the overflow list are written only when
//                                       asked for (sp_gather_plan_overflow)
//   count[ntiles]               int32   U of the tile; U >= kLdsRows marks an
//                                       overflow tile, whose rows do not fit in
//                                       LDS or whose items are more than
//                                       kPlanMaxItems or span two groups of
//                                       kPlanGroupOffsets (nothing else is
//                                       written for it)
//   overflow[ntiles]            int32   ascending ids of the overflow tiles
//   rows[ntiles][kLdsRows]      int32   ascending distinct source rows, then -1
//   nact[ntiles]                int32   items of the tile
//   koff[ntiles][E]             int32   kernel offset of each item, then -1
//   addr[ntiles][E][4][32][2]   uint16  for item i and wave w, the address of
//                                       row w * 64 + mt * 32 + l32 of the tile,
//                                       stored at [i][w][l32][mt] (one 128-byte
//                                       record per wave and item; lane l of the
//                                       wave reads the 4 bytes at l % 32); the
//                                       items that fill up the last group are
//                                       written, later ones are not

#pragma once
#include "sp_common.h"

namespace sp {

constexpr int kTileRows = 256;      // output rows per GEMM workgroup (4 waves x 64)
constexpr int kLdsRows = 896;       // staged rows per tile, including one zero row
constexpr int kPlanMaxItems = 64;   // items per tile: kTileRows * 64 = 16384 entries sorted in LDS
constexpr int kPlanDenseKv = 64;    // kv up to which the builder reads every offset's entries
constexpr int kPlanMaxKv = 1024;    // kv range of plans (above kPlanDenseKv: live offsets first)
// The direct kernel sums a row's offsets 64 at a time (each group over all
// reduction chunks), the planned kernels their items chunk by chunk: the two
// orders agree, bit for bit, when a tile's items lie in one such group.
constexpr int kPlanGroupOffsets = 64;
constexpr int kItemGroup = 4;       // the GEMM runs whole groups of items
constexpr int kChunkBytes = 64;     // one MFMA K-step of one row (32 f16/bf16 or 16 f32)
constexpr int kSwizzleShift = 2;    // piece p of a row sits at piece p ^ ((slot >> 2) & 3)

// LDS byte address (within the staged rows) of piece 0 of row `slot`; piece p
// of the row is at chunk_base(slot) ^ (p << 4), as bits 4-5 of slot * 64 are
// zero.  The swizzle spreads the rows that the lanes of one ds_read_b128 read
// over all banks when their slots are consecutive, and because it reads slot
// bits 2-3 only, row slot + 64 j sits at chunk_base(slot) + 4096 j.
__host__ __device__ inline uint32_t chunk_base(uint32_t slot) {
  return slot * kChunkBytes + (((slot >> kSwizzleShift) & 3u) << 4);
}
static_assert(kSwizzleShift + 2 <= 6, "the swizzle must not depend on slot bits >= 6");
static_assert(kLdsRows * kChunkBytes <= 65536, "LDS addresses are stored as uint16");

struct PlanLayout {
  int64_t ntiles;
  int E;
  size_t count_off, overflow_off, rows_off, nact_off, koff_off, addr_off, total;
};

inline PlanLayout plan_layout(int64_t M, int64_t kv) {
  PlanLayout p;
  const int64_t m = M > 0 ? M : 1;
  p.ntiles = cdiv(m, kTileRows);
  const int64_t items = kv < kPlanMaxItems ? kv : kPlanMaxItems;
  p.E = int((items + kItemGroup - 1) / kItemGroup * kItemGroup);
  const size_t nt = size_t(p.ntiles);
  p.count_off = 256;
  p.overflow_off = align_up(p.count_off + nt * 4, 256);
  p.rows_off = align_up(p.overflow_off + nt * 4, 256);
  p.nact_off = align_up(p.rows_off + nt * kLdsRows * 4, 256);
  p.koff_off = align_up(p.nact_off + nt * 4, 256);
  p.addr_off = align_up(p.koff_off + nt * size_t(p.E) * 4, 256);
  p.total = align_up(p.addr_off + nt * size_t(p.E) * kTileRows * 2, 256);
  return p;
}

// Device view of a plan.
struct PlanDev {
  const int32_t* n_overflow;
  const int32_t* count;
  const int32_t* overflow;
  const int32_t* rows;
  const int32_t* nact;
  const int32_t* koff;
  const uint16_t* addr;
  int E;
};

inline PlanDev plan_view(const void* plan, int64_t M, int64_t kv) {
  const PlanLayout l = plan_layout(M, kv);
  const char* b = static_cast<const char*>(plan);
  return PlanDev{reinterpret_cast<const int32_t*>(b),
                 reinterpret_cast<const int32_t*>(b + l.count_off),
                 reinterpret_cast<const int32_t*>(b + l.overflow_off),
                 reinterpret_cast<const int32_t*>(b + l.rows_off),
                 reinterpret_cast<const int32_t*>(b + l.nact_off),
                 reinterpret_cast<const int32_t*>(b + l.koff_off),
                 reinterpret_cast<const uint16_t*>(b + l.addr_off),
                 l.E};
}

}  // namespace sp
