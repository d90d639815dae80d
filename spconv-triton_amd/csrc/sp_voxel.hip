// Point-cloud voxelisation (PointToVoxel) on gfx950.
//
// The reference (spconv_triton/pytorch/utils.py:72-163) quantises every point
// to a voxel, orders the voxels by the first point that falls in them
// ("first come, first served"), caps their number at max_num_voxels, and
// stores up to max_num_points_per_voxel points per voxel in arrival order,
// with torch.unique, scatter_reduce, argsort and cumsum.  Here:
//   1. insert: every in-range point's linear voxel key goes into an
//      open-addressing hash (sp_hash.h) with the point index as value; the
//      table keeps the smallest index, i.e. the voxel's first point;
//   2. first: a point is "first" when the table holds its own index; an
//      exclusive scan over the first flags, in point order, numbers the
//      voxels in order of first occurrence (the FCFS ids), and the ids are
//      written back into the table;
//   3. assign: every point reads its voxel id; points of voxels past the cap
//      get -1; per-voxel point counts by atomic adds (order-free);
//   4. a stable radix sort of the kept points by voxel id keeps arrival order
//      inside every voxel; an exclusive scan of the counts gives each voxel's
//      first position, so a point's slot is its sorted position minus that;
//   5. scatter: points with slot < max_points_per_voxel are copied into their
//      voxel; per voxel the clamped count and the coordinates (decoded from
//      the key of its first point, ZYX order) are written.
// The only host synchronisation is the final read of the voxel count, which
// sizes the returned views (the reference reads it too: uniq.numel()).
#include "sp_common.h"
#include "sp_hash.h"
#include "sp_sort.h"

namespace sp {

struct P2VGeom {
  int ndim;
  double vsize[4];
  double cmin[4];
  int64_t gsize[4];
};

template <typename F>
__global__ __launch_bounds__(256) void p2v_insert(const F* __restrict__ pc, int64_t n,
                                                  int64_t cols, P2VGeom g, Table64 t,
                                                  int64_t* __restrict__ keys) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  bool ok = true;
  int64_t lin = 0;
  for (int d = 0; d < g.ndim; ++d) {
    // (p - cmin) / vsize in the points' precision, as the reference computes
    // it with tensors of pc.dtype; the comparisons reject NaN as out of range
    const F q = floor((pc[i * cols + d] - F(g.cmin[d])) / F(g.vsize[d]));
    ok = ok && q >= F(0) && q < F(g.gsize[d]);
    lin = lin * g.gsize[d] + (ok ? int64_t(q) : 0);
  }
  keys[i] = ok ? lin : -1;
  if (ok) t.insert(uint64_t(lin), int32_t(i));
}

__global__ __launch_bounds__(256) void p2v_first(const int64_t* __restrict__ keys, int64_t n,
                                                 Table64 t, uint32_t* __restrict__ first) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t k = keys[i];
  first[i] = (k >= 0 && t.find(uint64_t(k)) == int32_t(i)) ? 1u : 0u;
}

__global__ __launch_bounds__(256) void p2v_set_ids(const int64_t* __restrict__ keys, int64_t n,
                                                   Table64 t, const uint32_t* __restrict__ first,
                                                   const uint32_t* __restrict__ rank) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n || !first[i]) return;
  t.set_value(t.find_slot(uint64_t(keys[i])), int32_t(rank[i]));
}

__global__ __launch_bounds__(256) void p2v_assign(const int64_t* __restrict__ keys, int64_t n,
                                                  Table64 t, int64_t max_vox,
                                                  int64_t* __restrict__ pc_voxel_id,
                                                  uint32_t* __restrict__ sort_key,
                                                  uint32_t* __restrict__ counts) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t k = keys[i];
  const int32_t vid = k >= 0 ? t.find(uint64_t(k)) : -1;
  const bool kept = vid >= 0 && vid < max_vox;
  pc_voxel_id[i] = kept ? int64_t(vid) : -1;
  sort_key[i] = kept ? uint32_t(vid) : uint32_t(max_vox);  // dropped points sort last
  if (kept) atomicAdd(&counts[vid], 1u);
}

template <typename F>
__global__ __launch_bounds__(256) void p2v_scatter(
    const F* __restrict__ pc, int64_t cols, int nfeat, const uint32_t* __restrict__ perm,
    const uint32_t* __restrict__ sort_key, const uint32_t* __restrict__ start, int64_t n,
    int64_t max_vox, int maxpts, float* __restrict__ voxels) {
  const int64_t p = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t i = perm[p];
  const uint32_t v = sort_key[i];
  if (int64_t(v) >= max_vox) return;
  const int64_t slot = p - int64_t(start[v]);
  if (slot >= maxpts) return;
  float* dst = voxels + (int64_t(v) * maxpts + slot) * nfeat;
  for (int f = 0; f < nfeat; ++f) dst[f] = float(pc[int64_t(i) * cols + f]);
}

__global__ __launch_bounds__(256) void p2v_voxels(
    const uint32_t* __restrict__ counts, const uint32_t* __restrict__ start,
    const uint32_t* __restrict__ perm, const int64_t* __restrict__ keys,
    const uint32_t* __restrict__ n_unique, int64_t max_vox, int maxpts, P2VGeom g,
    int32_t* __restrict__ npv, int32_t* __restrict__ indices) {
  const int64_t v = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t nv = int64_t(*n_unique) < max_vox ? int64_t(*n_unique) : max_vox;
  if (v >= nv) return;
  const uint32_t c = counts[v];
  npv[v] = int32_t(c < uint32_t(maxpts) ? c : uint32_t(maxpts));
  int64_t key = keys[perm[start[v]]];  // the voxel's first point
  for (int d = g.ndim - 1; d >= 0; --d) {
    indices[v * g.ndim + (g.ndim - 1 - d)] = int32_t(key % g.gsize[d]);  // ZYX order
    key /= g.gsize[d];
  }
}

// Empty slots of every voxel get the mean over all max_points_per_voxel slots
// divided by the point count (reference utils.py:145-152), summed in slot order.
__global__ __launch_bounds__(256) void p2v_empty_mean(float* __restrict__ voxels,
                                                      const int32_t* __restrict__ npv,
                                                      const uint32_t* __restrict__ n_unique,
                                                      int64_t max_vox, int maxpts, int nfeat) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t nv = int64_t(*n_unique) < max_vox ? int64_t(*n_unique) : max_vox;
  if (t >= nv * nfeat) return;
  const int64_t v = t / nfeat;
  const int f = int(t % nfeat);
  float* base = voxels + v * maxpts * nfeat + f;
  float sum = 0.f;
  for (int s = 0; s < maxpts; ++s) sum += base[int64_t(s) * nfeat];
  const int cnt = npv[v];
  const float mean = sum / float(cnt > 1 ? cnt : 1);
  for (int s = cnt; s < maxpts; ++s) base[int64_t(s) * nfeat] = mean;
}

struct P2VWs {
  int64_t* keys;
  uint32_t* first;
  uint32_t* rank;
  uint32_t* sort_key;
  uint32_t* counts;
  uint32_t* start;
  uint32_t* n_unique;
  uint64_t* tkeys;
  int32_t* tvals;
  int* overflow;
  void* sort_ws;
  void* scan_ws;
  uint64_t cap;
};

template <class W>
static void p2v_layout(W& w, int64_t n, int64_t max_vox, P2VWs* out) {
  uint64_t cap = 1024;
  while (cap < uint64_t(n) * 2) cap <<= 1;
  const int64_t scan_len = n > max_vox ? n : max_vox;
  auto* keys = w.template take<int64_t>(size_t(n));
  auto* first = w.template take<uint32_t>(size_t(n));
  auto* rank = w.template take<uint32_t>(size_t(n));
  auto* sort_key = w.template take<uint32_t>(size_t(n));
  auto* counts = w.template take<uint32_t>(size_t(max_vox));
  auto* start = w.template take<uint32_t>(size_t(max_vox));
  auto* flags = w.template take<uint32_t>(64);
  auto* tkeys = w.template take<uint64_t>(size_t(cap));
  auto* tvals = w.template take<int32_t>(size_t(cap));
  void* sws = w.template take<char>(sort_rows_ws_bytes(n));
  void* cws = w.template take<char>(scan_workspace_bytes(scan_len));
  if (out) {
    out->keys = reinterpret_cast<int64_t*>(keys);
    out->first = reinterpret_cast<uint32_t*>(first);
    out->rank = reinterpret_cast<uint32_t*>(rank);
    out->sort_key = reinterpret_cast<uint32_t*>(sort_key);
    out->counts = reinterpret_cast<uint32_t*>(counts);
    out->start = reinterpret_cast<uint32_t*>(start);
    out->n_unique = reinterpret_cast<uint32_t*>(flags);
    out->overflow = reinterpret_cast<int*>(reinterpret_cast<uint32_t*>(flags) + 16);
    out->tkeys = reinterpret_cast<uint64_t*>(tkeys);
    out->tvals = reinterpret_cast<int32_t*>(tvals);
    out->sort_ws = sws;
    out->scan_ws = cws;
    out->cap = cap;
  }
}

// The size-only pass: WsSizer::take returns nothing, so the layout is walked
// with a cursor over a null base and only its final offset is used.
static size_t p2v_ws_bytes(int64_t n, int64_t max_vox) {
  WsCursor c(nullptr, ~size_t(0));
  p2v_layout(c, n, max_vox, nullptr);
  return c.off;
}

template <typename F>
static int p2v_run(const F* pc, int64_t n, int64_t cols, const P2VGeom& g, int nfeat,
                   int64_t max_vox, int maxpts, bool clear, bool empty_mean, float* voxels,
                   int32_t* indices, int32_t* npv, int64_t* pc_voxel_id, int64_t* n_voxels,
                   const P2VWs& w, hipStream_t s) {
  const unsigned blocks = unsigned(cdiv(n, 256));
  Table64 t{w.tkeys, w.tvals, w.cap - 1, w.overflow};
  SP_HIP(hipMemsetAsync(w.n_unique, 0, 256, s));
  SP_HIP(hipMemsetAsync(w.counts, 0, size_t(max_vox) * 4, s));
  int rc = launch_fill_u64(w.tkeys, int64_t(w.cap), kEmpty64, s);
  if (rc) return rc;
  rc = launch_fill_i32(w.tvals, int64_t(w.cap), 0x7fffffff, s);
  if (rc) return rc;
  if (clear) {
    rc = launch_fill<float>(voxels, max_vox * maxpts * nfeat, 0.f, s);
    if (rc) return rc;
  }
  p2v_insert<F><<<blocks, 256, 0, s>>>(pc, n, cols, g, t, w.keys);
  SP_LAUNCHED();
  p2v_first<<<blocks, 256, 0, s>>>(w.keys, n, t, w.first);
  SP_LAUNCHED();
  rc = exclusive_scan_u32(w.first, w.rank, n, w.n_unique, w.scan_ws, s);
  if (rc) return rc;
  p2v_set_ids<<<blocks, 256, 0, s>>>(w.keys, n, t, w.first, w.rank);
  SP_LAUNCHED();
  p2v_assign<<<blocks, 256, 0, s>>>(w.keys, n, t, max_vox, pc_voxel_id, w.sort_key, w.counts);
  SP_LAUNCHED();
  // stable sort of the points by voxel id (sort_key <= max_vox)
  int bits = 0;
  while ((uint64_t(1) << bits) <= uint64_t(max_vox)) ++bits;
  const uint32_t mask = bits >= 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
  uint32_t* perm = nullptr;
  rc = sort_rows_by_words(w.sort_key, n, 1, bits, mask, &perm, w.sort_ws, s);
  if (rc) return rc;
  rc = exclusive_scan_u32(w.counts, w.start, max_vox, nullptr, w.scan_ws, s);
  if (rc) return rc;
  p2v_scatter<F><<<blocks, 256, 0, s>>>(pc, cols, nfeat, perm, w.sort_key, w.start, n, max_vox,
                                        maxpts, voxels);
  SP_LAUNCHED();
  const unsigned vblocks = unsigned(cdiv(max_vox, 256));
  p2v_voxels<<<vblocks, 256, 0, s>>>(w.counts, w.start, perm, w.keys, w.n_unique, max_vox, maxpts,
                                     g, npv, indices);
  SP_LAUNCHED();
  if (empty_mean) {
    const unsigned eblocks = unsigned(cdiv(max_vox * nfeat, 256));
    p2v_empty_mean<<<eblocks, 256, 0, s>>>(voxels, npv, w.n_unique, max_vox, maxpts, nfeat);
    SP_LAUNCHED();
  }
  uint32_t h[2] = {0, 0};
  SP_HIP(hipMemcpyAsync(&h[0], w.n_unique, 4, hipMemcpyDeviceToHost, s));
  SP_HIP(hipMemcpyAsync(&h[1], w.overflow, 4, hipMemcpyDeviceToHost, s));
  SP_HIP(hipStreamSynchronize(s));
  if (h[1]) return set_error(SP_ERR_HASH_FULL, "point2voxel: voxel hash overflowed");
  *n_voxels = int64_t(h[0]) < max_vox ? int64_t(h[0]) : max_vox;
  return SP_OK;
}

}  // namespace sp

using namespace sp;

extern "C" {

size_t sp_point2voxel_workspace_size(int64_t n_points, int64_t max_voxels) {
  if (n_points < 0 || max_voxels < 1) return 0;
  return p2v_ws_bytes(n_points > 0 ? n_points : 1, max_voxels);
}

int sp_point2voxel(const void* points, int32_t dtype, int64_t n_points, int64_t point_cols,
                   int32_t ndim, const double* vsize_xyz, const double* coors_min_xyz,
                   const int64_t* grid_size_xyz, int32_t num_point_features, int64_t max_voxels,
                   int32_t max_points_per_voxel, int32_t clear_voxels, int32_t empty_mean,
                   float* voxels, int32_t* indices, int32_t* num_per_voxel,
                   int64_t* pc_voxel_id, int64_t* num_voxels, void* ws, size_t ws_bytes,
                   void* stream) {
  SP_CHECK_ARG(ndim >= 1 && ndim <= 4, "point2voxel: ndim %d not in 1..4", ndim);
  SP_CHECK_ARG(dtype == SP_F32 || dtype == SP_F64, "point2voxel: points must be f32 or f64");
  SP_CHECK_ARG(n_points >= 0 && n_points < (int64_t(1) << 31), "point2voxel: bad point count");
  SP_CHECK_ARG(max_voxels >= 1 && max_voxels < (int64_t(1) << 31) && max_points_per_voxel >= 1,
               "point2voxel: bad capacities");
  SP_CHECK_ARG(num_point_features >= 1 && num_point_features <= point_cols && point_cols >= ndim,
               "point2voxel: %d point features of %lld columns", num_point_features,
               (long long)point_cols);
  SP_CHECK_ARG(vsize_xyz && coors_min_xyz && grid_size_xyz && num_voxels, "null pointer");
  *num_voxels = 0;
  P2VGeom g{};
  g.ndim = ndim;
  for (int d = 0; d < ndim; ++d) {
    SP_CHECK_ARG(grid_size_xyz[d] >= 1, "point2voxel: grid size %lld", (long long)grid_size_xyz[d]);
    g.vsize[d] = vsize_xyz[d];
    g.cmin[d] = coors_min_xyz[d];
    g.gsize[d] = grid_size_xyz[d];
  }
  hipStream_t s = as_stream(stream);
  if (n_points == 0) {
    if (clear_voxels)
      return launch_fill<float>(voxels, max_voxels * max_points_per_voxel * num_point_features,
                                0.f, s);
    return SP_OK;
  }
  SP_CHECK_ARG(points && voxels && indices && num_per_voxel && pc_voxel_id, "null pointer");
  const size_t need = p2v_ws_bytes(n_points, max_voxels);
  if (!ws || ws_bytes < need)
    return set_error(SP_ERR_WORKSPACE, "point2voxel: workspace %zu < %zu", ws_bytes, need);
  WsCursor c(ws, ws_bytes);
  P2VWs w;
  p2v_layout(c, n_points, max_voxels, &w);
  if (dtype == SP_F32)
    return p2v_run<float>(static_cast<const float*>(points), n_points, point_cols, g,
                          num_point_features, max_voxels, max_points_per_voxel, clear_voxels != 0,
                          empty_mean != 0, voxels, indices, num_per_voxel, pc_voxel_id, num_voxels,
                          w, s);
  return p2v_run<double>(static_cast<const double*>(points), n_points, point_cols, g,
                         num_point_features, max_voxels, max_points_per_voxel, clear_voxels != 0,
                         empty_mean != 0, voxels, indices, num_per_voxel, pc_voxel_id, num_voxels,
                         w, s);
}

}  // extern "C"
