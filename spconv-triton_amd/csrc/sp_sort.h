// Stable LSD radix sort on gfx950 (8-bit digits, one histogram + scan +
// scatter per digit).  Ranking inside a 64-wide wave uses ballot-based peer
// matching, so the scatter is stable without any atomics on global memory.
#pragma once

#include "sp_common.h"

namespace sp {

// Rows 0..n-1 sorted stably by their mask words (word mic-1 most significant,
// word 0 ANDed with split).  kv bounds the meaningful bits.  The sorted
// permutation is returned through *perm_out (points into the workspace).
size_t sort_rows_ws_bytes(int64_t n);
int sort_rows_by_words(const uint32_t* words, int64_t n, int mic, int kv, uint32_t split,
                       uint32_t** perm_out, void* ws, hipStream_t stream);

// Ascending sort of n keys whose values fit in `bits` bits.  keys and tmp both
// hold n items; the sorted keys end in *result (keys or tmp).
size_t sort_keys_ws_bytes(int64_t n);
int sort_keys_u32(uint32_t* keys, uint32_t* tmp, int64_t n, int bits, uint32_t** result,
                  void* ws, hipStream_t stream);
int sort_keys_u64(uint64_t* keys, uint64_t* tmp, int64_t n, int bits, uint64_t** result,
                  void* ws, hipStream_t stream);

}  // namespace sp
