// Device hash table behind spconv_triton.pytorch.hash.HashTable.
//
// The reference keeps the table as sorted key/value arrays and rebuilds them
// with torch.sort on every insert (spconv_triton/pytorch/hash.py:38-110).
// Here it is an open-addressing table in one device buffer (linear probing
// from a mixed home slot, as the pair-generation tables in sp_hash.h):
//   header   64 uint32: [0] occupied slots, [1] overflow flag
//   keys[cap]   uint64  stored key (all ones: empty)
//   owner[cap]  uint64  (epoch << 32 | input position) of the value's writer
//   vals[cap]   uint64  the value's raw bytes (4 or 8 of them)
// Stored keys are the user's keys with the sign bit flipped (int32 keys
// zero-extended first), so unsigned order equals signed order and only the
// int64 key INT64_MAX collides with the empty pattern (inserting it fails
// with SP_ERR_INVALID_ARG).
// Semantics kept from the reference:
//   * insert: a key given several times in one call takes the value of its
//     last occurrence, and a later call overwrites an earlier one -- every
//     writer raises owner to (epoch, position) with atomicMax and only the
//     maximum writes its value (the host increments epoch per call);
//   * items / assign_arange: entries enumerated in ascending key order
//     (compaction of the occupied slots, then a stable radix sort of their
//     stored keys), assign_arange numbering them 0..n-1 in that order.
#include "sp_common.h"
#include "sp_hash.h"
#include "sp_sort.h"

namespace sp {

constexpr int kHtHeader = 64;  // uint32 words

struct HtDev {
  uint32_t* header;
  uint64_t* keys;
  uint64_t* owner;
  uint64_t* vals;
  uint64_t mask;
};

static HtDev ht_view(void* table, int64_t cap) {
  char* b = static_cast<char*>(table);
  HtDev t;
  t.header = reinterpret_cast<uint32_t*>(b);
  t.keys = reinterpret_cast<uint64_t*>(b + 256);
  t.owner = t.keys + cap;
  t.vals = t.owner + cap;
  t.mask = uint64_t(cap) - 1;
  return t;
}

__device__ __forceinline__ uint64_t ht_store_key(const void* keys, int64_t i, bool key64) {
  if (key64) return uint64_t(static_cast<const int64_t*>(keys)[i]) ^ 0x8000000000000000ull;
  return uint64_t(uint32_t(static_cast<const int32_t*>(keys)[i]) ^ 0x80000000u);
}

__device__ __forceinline__ uint64_t ht_home(const HtDev& t, uint64_t k) { return mix64(k) & t.mask; }

__device__ __forceinline__ int64_t ht_find(const HtDev& t, uint64_t k) {
  uint64_t s = ht_home(t, k);
  for (uint64_t i = 0; i <= t.mask; ++i) {
    const uint64_t v = t.keys[s];
    if (v == k) return int64_t(s);
    if (v == kEmpty64) return -1;
    s = (s + 1) & t.mask;
  }
  return -1;
}

__device__ __forceinline__ uint64_t ht_load_value(const void* vals, int64_t i, int vsize) {
  if (vsize == 8) return static_cast<const uint64_t*>(vals)[i];
  return uint64_t(static_cast<const uint32_t*>(vals)[i]);
}

__device__ __forceinline__ void ht_store_value(void* out, int64_t i, int vsize, uint64_t v) {
  if (vsize == 8) static_cast<uint64_t*>(out)[i] = v;
  else static_cast<uint32_t*>(out)[i] = uint32_t(v);
}

__global__ void ht_clear(HtDev t, int64_t cap) {
  const int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s < kHtHeader) t.header[s] = 0u;
  if (s >= cap) return;
  t.keys[s] = kEmpty64;
  t.owner[s] = 0;
  t.vals[s] = 0;
}

// Claims (or finds) the slot of every key and raises its owner word.
__global__ __launch_bounds__(256) void ht_insert_keys(HtDev t, const void* __restrict__ keys,
                                                      int64_t n, bool key64, uint32_t epoch,
                                                      int64_t* __restrict__ slot_of) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t k = ht_store_key(keys, i, key64);
  if (k == kEmpty64) {  // the int64 key INT64_MAX: reserved
    atomicMax(&t.header[1], 2u);
    slot_of[i] = -1;
    return;
  }
  uint64_t s = ht_home(t, k);
  for (uint64_t probe = 0; probe <= t.mask; ++probe) {
    const uint64_t prev = atomicCAS(reinterpret_cast<unsigned long long*>(&t.keys[s]),
                                    (unsigned long long)kEmpty64, (unsigned long long)k);
    if (prev == kEmpty64 || prev == k) {
      if (prev == kEmpty64) atomicAdd(&t.header[0], 1u);
      atomicMax(reinterpret_cast<unsigned long long*>(&t.owner[s]),
                (unsigned long long)((uint64_t(epoch) << 32) | uint64_t(i)));
      slot_of[i] = int64_t(s);
      return;
    }
    s = (s + 1) & t.mask;
  }
  atomicMax(&t.header[1], 1u);
  slot_of[i] = -1;
}

// Finds the slot of every key; found ones raise their owner word.
__global__ __launch_bounds__(256) void ht_claim_existing(HtDev t, const void* __restrict__ keys,
                                                         int64_t n, bool key64, uint32_t epoch,
                                                         int64_t* __restrict__ slot_of,
                                                         uint8_t* __restrict__ found) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = ht_find(t, ht_store_key(keys, i, key64));
  if (s >= 0)
    atomicMax(reinterpret_cast<unsigned long long*>(&t.owner[s]),
              (unsigned long long)((uint64_t(epoch) << 32) | uint64_t(i)));
  slot_of[i] = s;
  if (found) found[i] = s >= 0 ? 1 : 0;
}

// The last writer of every slot stores its value (zero without values).
__global__ __launch_bounds__(256) void ht_write_values(HtDev t, const void* __restrict__ vals,
                                                       int vsize, int64_t n, uint32_t epoch,
                                                       const int64_t* __restrict__ slot_of) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = slot_of[i];
  if (s < 0) return;
  if (t.owner[s] == ((uint64_t(epoch) << 32) | uint64_t(i)))
    t.vals[s] = vals ? ht_load_value(vals, i, vsize) : 0;
}

__global__ __launch_bounds__(256) void ht_query(HtDev t, const void* __restrict__ keys, int64_t n,
                                                bool key64, void* __restrict__ out, int vsize,
                                                uint8_t* __restrict__ is_empty) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = ht_find(t, ht_store_key(keys, i, key64));
  ht_store_value(out, i, vsize, s >= 0 ? t.vals[s] : 0);
  is_empty[i] = s >= 0 ? 0 : 1;
}

__global__ __launch_bounds__(256) void ht_occupied(HtDev t, int64_t cap, uint32_t* __restrict__ f) {
  const int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s < cap) f[s] = t.keys[s] != kEmpty64 ? 1u : 0u;
}

__global__ __launch_bounds__(256) void ht_fill_words(uint32_t* __restrict__ words, int64_t n) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j < n) words[j] = 0xFFFFFFFFu;
}

__global__ __launch_bounds__(256) void ht_compact(HtDev t, int64_t cap,
                                                  const uint32_t* __restrict__ f,
                                                  const uint32_t* __restrict__ pos,
                                                  uint32_t* __restrict__ slot,
                                                  uint32_t* __restrict__ words) {
  const int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s >= cap || !f[s]) return;
  const uint32_t j = pos[s];
  slot[j] = uint32_t(s);
  const uint64_t k = t.keys[s];
  words[2 * int64_t(j)] = uint32_t(k);
  words[2 * int64_t(j) + 1] = uint32_t(k >> 32);
}

// Entry j of the sorted order: key, value (or the rank j, converted to the
// value type, for assign_arange).
__global__ __launch_bounds__(256) void ht_emit(HtDev t, const uint32_t* __restrict__ count,
                                               const uint32_t* __restrict__ perm,
                                               const uint32_t* __restrict__ slot, bool key64,
                                               int vkind, int64_t limit, void* __restrict__ keys_out,
                                               void* __restrict__ vals_out, bool arange) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = int64_t(*count) < limit ? int64_t(*count) : limit;
  if (j >= n) return;
  const uint32_t s = slot[perm[j]];
  if (arange) {
    uint64_t v;
    switch (vkind) {  // 0 int32, 1 int64, 2 float32, 3 float64
      case 0: v = uint32_t(int32_t(j)); break;
      case 1: v = uint64_t(j); break;
      case 2: v = __builtin_bit_cast(uint32_t, float(j)); break;
      default: v = __builtin_bit_cast(uint64_t, double(j)); break;
    }
    t.vals[s] = v;
    return;
  }
  const uint64_t k = t.keys[s];
  if (key64) static_cast<int64_t*>(keys_out)[j] = int64_t(k ^ 0x8000000000000000ull);
  else static_cast<int32_t*>(keys_out)[j] = int32_t(uint32_t(k) ^ 0x80000000u);
  ht_store_value(vals_out, j, (vkind == 1 || vkind == 3) ? 8 : 4, t.vals[s]);
}

static int ht_check(int64_t cap, int32_t vkind) {
  SP_CHECK_ARG(cap >= 1 && (cap & (cap - 1)) == 0, "hash table: capacity %lld is not a power of 2",
               (long long)cap);
  SP_CHECK_ARG(vkind >= 0 && vkind <= 3, "hash table: value kind %d", vkind);
  return SP_OK;
}

static int vsize_of(int32_t vkind) { return (vkind == 1 || vkind == 3) ? 8 : 4; }

template <class W>
static void ht_enum_layout(W& w, int64_t cap) {
  w.template take<uint32_t>(size_t(cap));        // occupied flags
  w.template take<uint32_t>(size_t(cap));        // positions
  w.template take<uint32_t>(size_t(cap));        // slot of entry
  w.template take<uint32_t>(size_t(cap) * 2);    // stored keys as words
  w.template take<char>(scan_workspace_bytes(cap));
  w.template take<char>(sort_rows_ws_bytes(cap));
}

// Sorted enumeration of the table (count on the device, perm/slot in ws).
static int ht_enumerate(const HtDev& t, int64_t cap, bool key64, void* ws, uint32_t** perm,
                        uint32_t** slot, hipStream_t s) {
  WsCursor c(ws, ~size_t(0));
  uint32_t* f = c.take<uint32_t>(size_t(cap));
  uint32_t* pos = c.take<uint32_t>(size_t(cap));
  *slot = c.take<uint32_t>(size_t(cap));
  uint32_t* words = c.take<uint32_t>(size_t(cap) * 2);
  void* scan_ws = c.take<char>(scan_workspace_bytes(cap));
  void* sort_ws = c.take<char>(sort_rows_ws_bytes(cap));
  const unsigned blocks = unsigned(cdiv(cap, 256));
  ht_occupied<<<blocks, 256, 0, s>>>(t, cap, f);
  SP_LAUNCHED();
  // positions past the count keep all-ones keys: they sort after every
  // stored key (a stored key is never all ones) and, stably, after ties
  ht_fill_words<<<unsigned(cdiv(cap * 2, 256)), 256, 0, s>>>(words, cap * 2);
  SP_LAUNCHED();
  // the count of occupied slots goes to header[2]
  int rc = exclusive_scan_u32(f, pos, cap, t.header + 2, scan_ws, s);
  if (rc) return rc;
  ht_compact<<<blocks, 256, 0, s>>>(t, cap, f, pos, *slot, words);
  SP_LAUNCHED();
  // the sort covers the whole capacity; only the first `count` positions of
  // its result are used
  return sort_rows_by_words(words, cap, 2, key64 ? 64 : 32, 0xFFFFFFFFu, perm, sort_ws, s);
}

}  // namespace sp

using namespace sp;

extern "C" {

size_t sp_hash_table_bytes(int64_t capacity) {
  if (capacity < 1) return 0;
  return 256 + size_t(capacity) * 24;
}

size_t sp_hash_workspace_size(int64_t capacity, int64_t n) {
  if (capacity < 1 || n < 0) return 0;
  WsSizer z;
  z.take<int64_t>(size_t(n > 0 ? n : 1));  // slot of each input key
  ht_enum_layout(z, capacity);
  return z.off;
}

int sp_hash_clear(void* table, int64_t capacity, void* stream) {
  int rc = ht_check(capacity, 0);
  if (rc) return rc;
  SP_CHECK_ARG(table, "hash table: null table");
  HtDev t = ht_view(table, capacity);
  const int64_t m = capacity > kHtHeader ? capacity : kHtHeader;
  ht_clear<<<unsigned(cdiv(m, 256)), 256, 0, as_stream(stream)>>>(t, capacity);
  SP_LAUNCHED();
  return SP_OK;
}

int sp_hash_insert(void* table, int64_t capacity, const void* keys, int32_t key64,
                   const void* values, int32_t vkind, int64_t n, uint32_t epoch,
                   int64_t* n_entries, void* ws, size_t ws_bytes, void* stream) {
  int rc = ht_check(capacity, vkind);
  if (rc) return rc;
  SP_CHECK_ARG(table && n_entries, "hash table: null pointer");
  SP_CHECK_ARG(n >= 0 && n < (int64_t(1) << 31), "hash table: %lld keys", (long long)n);
  HtDev t = ht_view(table, capacity);
  hipStream_t s = as_stream(stream);
  if (n > 0) {
    SP_CHECK_ARG(keys, "hash table: null keys");
    if (!ws || ws_bytes < sp_hash_workspace_size(capacity, n))
      return set_error(SP_ERR_WORKSPACE, "hash insert: workspace too small");
    int64_t* slot_of = static_cast<int64_t*>(ws);
    const unsigned blocks = unsigned(cdiv(n, 256));
    ht_insert_keys<<<blocks, 256, 0, s>>>(t, keys, n, key64 != 0, epoch, slot_of);
    SP_LAUNCHED();
    ht_write_values<<<blocks, 256, 0, s>>>(t, values, vsize_of(vkind), n, epoch, slot_of);
    SP_LAUNCHED();
  }
  uint32_t h[2] = {0, 0};
  SP_HIP(hipMemcpyAsync(h, t.header, 8, hipMemcpyDeviceToHost, s));
  SP_HIP(hipStreamSynchronize(s));
  if (h[1] == 2) return set_error(SP_ERR_INVALID_ARG, "hash table: the key INT64_MAX is reserved");
  if (h[1]) return set_error(SP_ERR_HASH_FULL, "hash table full");
  *n_entries = h[0];
  return SP_OK;
}

int sp_hash_insert_existing(void* table, int64_t capacity, const void* keys, int32_t key64,
                            const void* values, int32_t vkind, int64_t n, uint32_t epoch,
                            uint8_t* found, void* ws, size_t ws_bytes, void* stream) {
  int rc = ht_check(capacity, vkind);
  if (rc) return rc;
  SP_CHECK_ARG(table, "hash table: null table");
  if (n <= 0) return SP_OK;
  SP_CHECK_ARG(keys && values && found, "hash table: null pointer");
  if (!ws || ws_bytes < sp_hash_workspace_size(capacity, n))
    return set_error(SP_ERR_WORKSPACE, "hash insert_exist_keys: workspace too small");
  HtDev t = ht_view(table, capacity);
  hipStream_t s = as_stream(stream);
  int64_t* slot_of = static_cast<int64_t*>(ws);
  const unsigned blocks = unsigned(cdiv(n, 256));
  ht_claim_existing<<<blocks, 256, 0, s>>>(t, keys, n, key64 != 0, epoch, slot_of, found);
  SP_LAUNCHED();
  ht_write_values<<<blocks, 256, 0, s>>>(t, values, vsize_of(vkind), n, epoch, slot_of);
  SP_LAUNCHED();
  return SP_OK;
}

int sp_hash_query(const void* table, int64_t capacity, const void* keys, int32_t key64,
                  int32_t vkind, int64_t n, void* values_out, uint8_t* is_empty, void* stream) {
  int rc = ht_check(capacity, vkind);
  if (rc) return rc;
  if (n <= 0) return SP_OK;
  SP_CHECK_ARG(table && keys && values_out && is_empty, "hash table: null pointer");
  HtDev t = ht_view(const_cast<void*>(table), capacity);
  ht_query<<<unsigned(cdiv(n, 256)), 256, 0, as_stream(stream)>>>(t, keys, n, key64 != 0,
                                                                  values_out, vsize_of(vkind),
                                                                  is_empty);
  SP_LAUNCHED();
  return SP_OK;
}

int sp_hash_items(void* table, int64_t capacity, int32_t key64, int32_t vkind, int64_t max_items,
                  void* keys_out, void* values_out, int32_t assign_arange, void* ws,
                  size_t ws_bytes, void* stream) {
  int rc = ht_check(capacity, vkind);
  if (rc) return rc;
  SP_CHECK_ARG(table, "hash table: null table");
  SP_CHECK_ARG(assign_arange || (keys_out && values_out) || max_items == 0,
               "hash table: null outputs");
  if (!ws || ws_bytes < sp_hash_workspace_size(capacity, 0))
    return set_error(SP_ERR_WORKSPACE, "hash items: workspace too small");
  HtDev t = ht_view(table, capacity);
  hipStream_t s = as_stream(stream);
  uint32_t *perm = nullptr, *slot = nullptr;
  // the enumeration layout starts after the per-key slot area of size 1
  WsCursor c(ws, ws_bytes);
  c.take<int64_t>(1);
  rc = ht_enumerate(t, capacity, key64 != 0, static_cast<char*>(ws) + align_up(c.off, 256), &perm,
                    &slot, s);
  if (rc) return rc;
  const int64_t limit = assign_arange ? capacity : max_items;
  if (limit > 0) {
    ht_emit<<<unsigned(cdiv(limit, 256)), 256, 0, s>>>(t, t.header + 2, perm, slot, key64 != 0,
                                                       vkind, limit, keys_out, values_out,
                                                       assign_arange != 0);
    SP_LAUNCHED();
  }
  return SP_OK;
}

}  // extern "C"
