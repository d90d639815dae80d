/*
 * spconv_hip.h -- C ABI of the MI355X (gfx950) sparse-convolution library
 * libspconv_hip.so.
 *
 * Every entry point takes plain device pointers, element counts, small host
 * structs and a HIP stream (passed as void*, i.e. a hipStream_t), and returns
 * an int status (SP_OK == 0).  Nothing here allocates device memory: callers
 * pass a workspace whose size they query first (sp_conv_fwd_noalloc uses a
 * library-held device array instead).  All work is enqueued on the
 * given stream; only sp_pairgen_conv_build() blocks the host, once, to read
 * the data-dependent output count (the reference synchronises at the same
 * point: torch.unique in spconv_triton/pytorch/_impl/pairs.py:206-209).
 *
 * The reference (spconv-Triton) has no FFI: its boundary is the Python
 * module spconv_triton/pytorch/_impl/{pairs,pair_kernels,gemm,pool}.py,
 * called from spconv_triton/pytorch/ops.py.  Each declaration below names the
 * reference function (file:line, paths relative to the reference repository)
 * whose result it reproduces.  The Python mirror of that module in this
 * repository binds these symbols with ctypes.
 *
 * Index tensors are int32.  Feature tensors are row-major [rows, channels].
 * Weights are KRSC, i.e. [K_out, kv, C_in] contiguous
 * (spconv_triton/pytorch/ops.py:76-83).
 */
#ifndef SPCONV_HIP_H
#define SPCONV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define SP_OK 0
#define SP_ERR_INVALID_ARG 1  /* bad size / null pointer / misaligned table */
#define SP_ERR_UNSUPPORTED 2  /* dtype or shape the library does not handle */
#define SP_ERR_WORKSPACE 3    /* workspace smaller than the queried size */
#define SP_ERR_HIP 4          /* a HIP runtime call failed */
#define SP_ERR_HASH_FULL 5    /* coordinate hash overflowed its capacity */

/* ---- element types ----------------------------------------------------- */
#define SP_F16 0
#define SP_BF16 1
#define SP_F32 2
#define SP_F64 3
/* fp32 operands as bf16 parts (split-bf16, for SPCONV_ALLOW_TF32): a packed
 * weight of this type is the SP_BF16 packing of [hi | lo | hi] along the
 * reduction axis (3*C forward, 3*K input gradient), hi = bf16(w),
 * lo = bf16(w - hi); the GEMM then runs as SP_BF16 over a reduction three
 * times as long, with features split by sp_split_bf16x3 (pattern 0). */
#define SP_BF16X3 4

/* ---- pair-generation modes (spconv_triton/pytorch/_impl/pairs.py:6-22) -- */
#define SP_PAIR_SUBM 0       /* o = x + (k//2)*d - kpos*d, o must be an input */
#define SP_PAIR_REGULAR 1    /* o = (x + p - kpos*d) / s, exact division     */
#define SP_PAIR_TRANSPOSE 2  /* o = x*s - p + kpos*d                         */

/* Convolution geometry, host memory.  ndim in 1..4.  For SP_PAIR_SUBM the
 * library derives padding = (ksize//2)*dilation and stride 1 itself
 * (pairs.py:186-191); out_shape must equal in_shape. */
typedef struct sp_geom {
  int32_t ndim;
  int32_t mode;
  int64_t batch_size;
  int64_t in_shape[4];
  int64_t out_shape[4];
  int32_t ksize[4];
  int32_t stride[4];
  int32_t padding[4];
  int32_t dilation[4];
} sp_geom;

/* ---- library info ------------------------------------------------------ */
/* Revision of the argument lists declared here.  It changes whenever an
 * entry point's arguments change (revision 2: sp_pairgen_conv_build,
 * sp_gather_plan_build, sp_conv_gemm_ordered and sp_permute_table took their
 * current forms).  A caller compares sp_abi_version() with the value it was
 * compiled against and must not call into a library of another revision. */
#define SP_ABI_VERSION 2
int sp_abi_version(void);
int sp_version(void);              /* (major << 16) | (minor << 8) | patch */
const char* sp_arch(void);         /* offload target the code objects hold */
const char* sp_last_error(void);   /* message of the last failing call (thread-local) */

/* 1 when the key volume needs 64-bit linear keys: batch*prod(out_shape)
 * (and, for subm, batch*prod(in_shape)) >= 2^31.
 * Replaces the lin_dtype pick of compute_candidates, pairs.py:166-171. */
int sp_geom_key64(const sp_geom* g);

/* ---- pair generation --------------------------------------------------- */

/* Workspace bytes for sp_pairgen_subm / sp_pairgen_conv_build+fill on n input
 * rows.  The same workspace must be passed, untouched, from build to fill; it
 * must be 16-byte aligned (device allocations are). */
size_t sp_pairgen_workspace_size(const sp_geom* g, int64_t n);

/* Submanifold rulebook.  pair_fwd [kv, n] (nullable if pair_bwd is given):
 * pair_fwd[k, r] = input row j whose coordinate is the k-th neighbour of row
 * r, or -1.  pair_bwd [kv, n]
 * (nullable) is the transposed table, pair_bwd[k, j] = r or -1.  mask_words
 * [n, ceil(kv/32)] (nullable): bit k%32 of word k/32 set iff pair_fwd[k,r]>=0.
 * Reproduces compute_candidates(subm) + scatter_igemm_pairs + pack_mask_words:
 *   spconv_triton/pytorch/_impl/pairs.py:126-204, :318-340
 *   spconv_triton/pytorch/_impl/pair_kernels.py:37-94, :159-183, :220-261, :398-446 */
int sp_pairgen_subm(const sp_geom* g, const int32_t* indices, int64_t n,
                    int32_t* pair_fwd, int32_t* pair_bwd, uint32_t* mask_words,
                    void* ws, size_t ws_bytes, void* stream);

/* Int32 entries of the dense cell -> row grid buffer that sp_pairgen_subm_grid
 * needs for this geometry and n rows (the cells plus 4 guard entries on either
 * side), or 0 when that path does not apply (volume above 2^26 cells or 256
 * cells per row, n >= 2^24, kv > 512, not subm). */
int64_t sp_pairgen_subm_grid_cells(const sp_geom* g, int64_t n);

/* sp_pairgen_subm on a caller-kept grid, without clearing it: the grid
 * (grid_cells >= sp_pairgen_subm_grid_cells int32 cells) holds stamps of
 * earlier builds, each below `epoch` (1..255) in its top byte -- the caller
 * zero-fills a new grid, then uses epochs 1, 2, ... and fills it again before
 * reusing epoch values.  Writes the same pair_fwd / pair_bwd / mask_words as
 * sp_pairgen_subm and, when npl is not null, zeros npl[kv] (the
 * indice_num_per_loc of the implicit-GEMM tuple).  Calls that share a grid must
 * not overlap (one grid per stream).  Replaces the same reference functions as
 * sp_pairgen_subm (spconv_triton/pytorch/_impl/pairs.py:126-220, :281-426),
 * without the per-build clear of the lookup structure. */
int sp_pairgen_subm_grid(const sp_geom* g, const int32_t* indices, int64_t n, int32_t* pair_fwd,
                         int32_t* pair_bwd, uint32_t* mask_words, int32_t* npl, int32_t* grid,
                         int64_t grid_cells, uint32_t epoch, void* stream);

/* Regular / transposed convolution, phase 1: deduplicate the candidate output
 * keys, sort them ascending (batch-major linear key), and rank them.  Blocks
 * until the count is known and stores it in *n_out (0 = every point vanished).
 * *n_pairs (nullable) receives the number of candidates, i.e. the valid
 * entries of the gather table (before any n_keep truncation in phase 2),
 * read back in the same synchronisation.
 * Replaces K1 + out_lin[valid] + torch.unique + K3 of
 *   spconv_triton/pytorch/_impl/pairs.py:126-220 (regular/transpose branch)
 *   spconv_triton/pytorch/_impl/pair_kernels.py:37-94, :298-392 */
int sp_pairgen_conv_build(const sp_geom* g, const int32_t* indices, int64_t n,
                          void* ws, size_t ws_bytes, int64_t* n_out, int64_t* n_pairs,
                          void* stream);

/* Phase 2: output coordinates and gather tables for the first n_keep outputs
 * (n_keep <= n_out; smaller values implement num_out_act_bound,
 * pairs.py:318-323).  out_indices [n_keep, ndim+1]; pair_fwd [kv, n_keep]
 * (nullable if pair_bwd is given);
 * pair_bwd [kv, n] (nullable); mask_words_bwd [n, ceil(kv/32)] (nullable).
 * Replaces _delinearize + scatter_igemm_pairs, pairs.py:98-111, :318-340,
 * pair_kernels.py:220-261. */
int sp_pairgen_conv_fill(const sp_geom* g, const int32_t* indices, int64_t n,
                         const void* ws, size_t ws_bytes, int64_t n_keep,
                         int32_t* out_indices, int32_t* pair_fwd, int32_t* pair_bwd,
                         uint32_t* mask_words_bwd, void* stream);

/* Per-row offset bitmask of a gather table [kv, n] -> words [n, ceil(kv/32)].
 * Replaces pack_mask_words, spconv_triton/pytorch/_impl/pair_kernels.py:147-213. */
int sp_mask_words(const int32_t* table, int64_t kv, int64_t n, uint32_t* words,
                  void* stream);

/* Mask split + stable sort of mask words (make_mask_splits, pairs.py:356-392).
 * words [n, mic]; word 0 is ANDed with split_mask.  With do_sort, rows are
 * stably sorted ascending by the unsigned value, the highest word most
 * significant.  pair_mask [n, mic] (int32, wrapped) receives the sorted
 * words, argsort [n] the original row of each sorted entry. */
size_t sp_mask_sort_workspace_size(int64_t n, int32_t mic);
int sp_mask_sort(const uint32_t* words, int64_t n, int32_t mic, int32_t kv,
                 uint32_t split_mask, int32_t do_sort, int32_t* pair_mask,
                 int32_t* argsort, void* ws, size_t ws_bytes, void* stream);

/* Positions the radix-sort scatters of this device dropped because they fell
 * outside 0..n-1 (an inconsistent histogram; 0 unless the library has a bug),
 * since the process started or the last reset.  Synchronises the device.  No
 * counterpart in the reference (its sorts are torch's); tests read it after
 * the sorts they check. */
int sp_sort_dropped_positions(uint64_t* count, int32_t reset);

/* Per-row compaction of a table [kv, n]: for every k, the columns i with
 * table[k, i] >= 0 in ascending order go to pos_out[k, p] = i and
 * val_out[k, p] = table[k, i]; the tail of each row is filled with -1.
 * counts[k] = number of entries; npl[k] = counts[k] for k < npl_limit, else 0
 * (npl nullable).  Serves the Native [2, kv, N] format (pos = input rows,
 * val = output rows: _scatter_pairs_native + native_pairs, pairs.py:223-278)
 * and the compacted weight-gradient signal (gemm.py:661-669). */
size_t sp_compact_workspace_size(int64_t kv, int64_t n);
int sp_compact_table(const int32_t* table, int64_t kv, int64_t n, int32_t* pos_out,
                     int32_t* val_out, int32_t* counts, int32_t* npl, int32_t npl_limit,
                     void* ws, size_t ws_bytes, void* stream);

/* Native pair tensor [2, kv, n_pairs] -> gather tables.  pf [kv, n_out]
 * (-1 filled), pb [kv, n_in] (nullable).  inverse swaps the two rows of the
 * pair tensor.  Replaces native_pair_to_tables, pairs.py:429-469. */
int sp_native_to_tables(const int32_t* pair, int64_t kv, int64_t n_pairs, int32_t inverse,
                        int64_t n_in, int64_t n_out, int32_t* pf, int32_t* pb,
                        void* stream);

/* ---- gather-GEMM ------------------------------------------------------- */

/* Workspace for sp_conv_fwd / sp_conv_dgrad (relaid weights + fp32 bias). */
size_t sp_conv_workspace_size(int64_t K, int64_t kv, int64_t C, int32_t dtype);

/* Pre-packed weights: the KRSC weight (and optional bias) relaid once into the
 * MFMA operand layout of `dtype`, for the forward (transpose = 0, output
 * channels K) or the input gradient (transpose = 1, output channels C).  A
 * packed buffer stays valid while the weight is unchanged, so inference runs
 * the gather-GEMM as a single kernel launch.  Same computation as the weight
 * handling inside conv_forward / conv_backward_input, gemm.py:501-631. */
size_t sp_conv_packed_bytes(int64_t K, int64_t kv, int64_t C, int32_t dtype, int32_t transpose);
int sp_conv_pack_weight(const void* w, int32_t w_dtype, const void* bias, int64_t K, int64_t kv,
                        int64_t C, int32_t dtype, int32_t transpose, void* packed,
                        void* stream);
/* Gather-GEMM with packed weights: out[m, n] = bias[n] + sum_k sum_r
 * A[pairs[k, m], r] * W[k](n, r), A [n_src, R] dtype, pairs [kv, M],
 * out [M, N] out_dtype; N = K (forward) or C (dgrad), R the other one.
 * has_bias selects the bias packed with the weight. */
int sp_conv_gemm_packed(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                        int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                        const int32_t* pairs, int64_t M, const int32_t* pair_mask,
                        const int32_t* mask_argsort, void* out, int32_t out_dtype, void* stream);

/* Gather plan of a pair table pairs [kv, M] (values in [0, n_src) or -1):
 * for every tile of 256 consecutive rows, the ascending distinct source rows
 * it references and, per entry, the position of its row in that list.  The
 * planned GEMM stages those rows in LDS once per tile instead of gathering
 * every pair from memory.  A plan depends only on the table: build it once per
 * table, like the reference memoises its tables on the indice data
 * (spconv_triton/pytorch/_impl/pairs.py:429-469 native_pair_to_tables,
 * gemm.py:661-669 valid_signal).  No reference entry point corresponds to it.
 * sp_gather_plan_bytes returns 0 when kv is outside 1..1024 (no plan: use
 * sp_conv_gemm_packed).  A tile lists at most 64 offsets with a pair among
 * its rows; a tile with more is gathered directly, like one whose rows do not
 * fit in LDS (an overflow tile).  sp_gather_plan_build is asynchronous; n_overflow
 * (nullable) requests the number of tiles whose distinct rows do not fit in
 * LDS (the GEMM gathers those directly from memory), which costs one stream
 * synchronization.  row_words (nullable): the rows' mask words, words_per_row
 * (>= ceil(kv / 32)) per row (bit k of row r set iff pairs[k, r] >= 0); the
 * builder then reads only the entries of the offsets some row of a tile has
 * (the same plan, built faster for tables with few pairs per row). */
size_t sp_gather_plan_bytes(int64_t M, int64_t kv);
int sp_gather_plan_build(const int32_t* pairs, int64_t kv, int64_t M, int64_t n_src,
                         const uint32_t* row_words, int32_t words_per_row, void* plan,
                         size_t plan_bytes, int64_t* n_overflow, void* stream);
/* The number of overflow tiles of a built plan (same kv and M as its build),
 * for callers that choose a row order by it; one kernel launch and one stream
 * synchronization.  No reference entry point corresponds to it. */
int sp_gather_plan_overflow(void* plan, size_t plan_bytes, int64_t kv, int64_t M,
                            int64_t* n_overflow, void* stream);

/* sp_conv_gemm_packed with a gather plan of `pairs` (built for the same kv, M
 * and n_src); no mask tables.  One kernel launch.  Results are bit-identical
 * to sp_conv_gemm_packed's.  Replaces the same reference kernels as
 * sp_conv_fwd / sp_conv_dgrad (gemm.py:206-321). */
int sp_conv_gemm_planned(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                         int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                         const int32_t* pairs, int64_t M, const void* plan, size_t plan_bytes,
                         void* out, int32_t out_dtype, void* stream);

/* The gather-GEMM with the output rows taken in a given order: tile row i is
 * output row row_order[i] (a permutation of 0..M-1, here the stable mask
 * argsort), pairs_perm is the table permuted by it (sp_permute_table) and
 * plan (nullable, kv <= 1024) a gather plan of pairs_perm.  Results are
 * bit-identical to the natural order's.  This is the reference's masked
 * traversal, which visits rows in mask_argsort order so that a row tile holds
 * rows with similar masks (gemm.py:282-296, the mask_argsort operand of
 * _gather_gemm_kernel :501-568); with the table permuted up front the kernel
 * reads it coalesced.  thin_tiles 1 (with a plan): most tiles of
 * pairs_perm hold at most 4 live offsets (tables of about one pair per row);
 * a kernel that loads each chunk's rows and weights three chunks ahead runs
 * them (the others take the direct path inside it).  thin_tiles 2: the same
 * kernel with every tile it hands to the direct path spread over four
 * workgroups of a quarter of its rows each (fp32 operands on tables whose
 * tiles mostly hold more offsets).  0: the staged kernel.  Results are the
 * same; other values are an error.
 * row_words (nullable): the mask words of pairs_perm's rows, words_per_row
 * (>= ceil(kv / 32)) per row (bit k of row i set iff pairs_perm[k, i] >= 0,
 * e.g. the sorted pair_mask of sp_mask_sort whose argsort is row_order); an
 * unplanned call then reads the table entries of only the offsets set in a
 * wave's rows (tables with few pairs per row and kv > 64 gain most).  A clear
 * bit whose entry holds a pair drops that pair. */
int sp_conv_gemm_ordered(const void* a, int32_t dtype, int64_t n_src, const void* packed,
                         int64_t K, int64_t kv, int64_t C, int32_t transpose, int32_t has_bias,
                         const int32_t* pairs_perm, int64_t M, const int32_t* row_order,
                         const void* plan, size_t plan_bytes, int32_t thin_tiles,
                         const uint32_t* row_words, int32_t words_per_row, void* out,
                         int32_t out_dtype, void* stream);

/* out[k, i] = pairs[k, order[i]] for a gather table pairs [kv, M] (-1 where
 * order[i] is outside 0..M-1).  order_words (nullable, kv <= 32): the mask
 * word of row order[i] at [i] (bit k set iff pairs[k, order[i]] >= 0, e.g. the
 * sorted pair_mask of sp_mask_sort); entries of clear bits are then written
 * as -1 without being read.  Builds the pairs_perm of sp_conv_gemm_ordered
 * (the reference indexes the table through mask_argsort inside its kernel,
 * gemm.py:501-568). */
int sp_permute_table(const int32_t* pairs, int64_t kv, int64_t M, const int32_t* order,
                     const uint32_t* order_words, int32_t* out, void* stream);

/* Work statistics of a gather table [kv, M] (kv <= 512) in its own row order, added into
 * stats[0..2] (int64, zeroed by the caller): the pairs (entries in
 * 0..n_src-1), the (256-row tile, offset) pairs with at least one pair and
 * the (64-row block, offset) pairs with at least one pair.  pairs / (256 *
 * stats[1]) is the share of the staged GEMM's MFMA work spent on pairs, which
 * decides whether a table is worth reordering.  No reference counterpart: the
 * reference always takes the mask-sorted order (gemm.py:282-296). */
int sp_table_stats(const int32_t* pairs, int64_t kv, int64_t M, int64_t n_src, int64_t* stats,
                   void* stream);

/* Forward: out[m, n] = bias[n] + sum_k sum_c X[pf[k, m], c] * W[n, k, c].
 * X [n_in, C] dtype; W [K, kv, C] w_dtype; pf [kv, n_out]; bias [K] of
 * w_dtype (nullable); out [n_out, K] out_dtype.  pair_mask/mask_argsort [n_out]
 * (both nullable, kv <= 32) select the masked path: rows are visited in
 * argsort order and offsets empty across a row tile are skipped (identical
 * result).  Accumulation is fp32.  Replaces conv_forward + _gather_gemm_kernel,
 * spconv_triton/pytorch/_impl/gemm.py:206-321, :501-568. */
int sp_conv_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C,
                const void* w, int32_t w_dtype, int64_t K, int64_t kv,
                const int32_t* pf, int64_t n_out, const void* bias,
                const int32_t* pair_mask, const int32_t* mask_argsort,
                void* out, int32_t out_dtype, void* ws, size_t ws_bytes, void* stream);

/* sp_conv_fwd without the workspace argument: the relaid weights and fp32
 * bias go into a library-held device array of SP_NOALLOC_SCRATCH_BYTES (one
 * per GPU, kept until the process ends), so the call allocates nothing, and
 * calls no allocating routine: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and result as sp_conv_fwd, bit for bit.  Weights
 * whose relaid size exceeds the array (K * kv * C padded, times the element
 * size, plus 4 * K bytes of bias) are rejected with SP_ERR_UNSUPPORTED.
 * Every call on a GPU reuses that GPU's array: calls that overlap on one GPU
 * (two streams, or host threads) race and must be serialised by the caller.
 * No counterpart in the reference; it serves callers that cannot allocate. */
#define SP_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)
int sp_conv_fwd_noalloc(const void* x, int32_t dtype, int64_t n_in, int64_t C,
                        const void* w, int32_t w_dtype, int64_t K, int64_t kv,
                        const int32_t* pf, int64_t n_out, const void* bias,
                        const int32_t* pair_mask, const int32_t* mask_argsort,
                        void* out, int32_t out_dtype, void* stream);

/* Input gradient: dX[j, c] = sum_k sum_n G[pb[k, j], n] * W[n, k, c].
 * G [n_out, K]; pb [kv, n_in]; dX [n_in, C] in dtype.
 * Replaces conv_backward_input, gemm.py:571-631. */
int sp_conv_dgrad(const void* g, int32_t dtype, int64_t n_out, int64_t K,
                  const void* w, int32_t w_dtype, int64_t kv, int64_t C,
                  const int32_t* pb, int64_t n_in,
                  const int32_t* pair_mask, const int32_t* mask_argsort,
                  void* dx, void* ws, size_t ws_bytes, void* stream);

/* Split of fp32 rows into bf16 parts for the split-bf16 products that serve
 * SPCONV_ALLOW_TF32 (the reference runs tl.dot with input_precision="tf32" on
 * fp32 GEMMs: gemm.py:46-71, :456-463, used by conv_forward :564,
 * conv_backward_input :627 and conv_backward_weight :708).  x [rows, cols] f32
 * -> out [rows, parts * cols] bf16 with hi = bf16(x), lo = bf16(x - hi):
 * pattern 0 = [hi | hi | lo] (forward / input-gradient operand against a
 * SP_BF16X3 packed weight: hi*hi + hi*lo + lo*hi), 1 = [hi | lo | hi],
 * 2 = [hi | lo] (weight-gradient operands, SP_BF16X3 of sp_conv_wgrad).
 * Each product is recovered to about 2^-16 relative (TF32: 2^-11); method of
 * Henry, Tang & Heinecke, ARITH 2019. */
int sp_split_bf16x3(const float* x, int64_t rows, int64_t cols, int32_t pattern, void* out,
                    void* stream);

/* Weight gradient over compacted pairs (sp_compact_table of pair_fwd):
 * dW[n, k, c] = sum_{p < counts[k]} X[in_rows[k, p], c] * G[out_rows[k, p], n].
 * X [n_in, C], G [n_out, K]; in_rows/out_rows [kv, row_stride].  Split-P fp32 partials reduced in a fixed
 * order (deterministic).  dW [K, kv, C] in dtype.  dtype SP_BF16X3: x [n_in, 2C]
 * and g [n_out, 2K] are the bf16 [hi | lo] halves of fp32 tensors (sp_split_bf16x3
 * pattern 2), dW is fp32 (the four half products summed), and the workspace is
 * sp_wgrad_workspace_size(2K, kv, 2C, n_rows).
 * Replaces conv_backward_weight + _dweight_masked_kernel, gemm.py:324-453, :634-713. */
size_t sp_wgrad_workspace_size(int64_t K, int64_t kv, int64_t C, int64_t n_rows);
int sp_conv_wgrad(const void* x, int64_t n_in, const void* g, int64_t n_out, int32_t dtype,
                  int64_t C, int64_t K, int64_t kv, const int32_t* in_rows,
                  const int32_t* out_rows, const int32_t* counts, int64_t row_stride,
                  void* dw, void* ws, size_t ws_bytes, void* stream);

/* ---- pooling (spconv_triton/pytorch/_impl/pool.py) --------------------- */

/* out[m, c] = max(0, max_{k: pf[k,m] >= 0} X[pf[k,m], c]); fp32 accumulator
 * (fp64 for SP_F64).  Replaces maxpool_forward, pool.py:45-91, :260-284. */
int sp_maxpool_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C,
                   const int32_t* pf, int64_t kv, int64_t n_out, void* out, void* stream);

/* dX[j, c] = sum_{k: pb[k,j] >= 0, out[pb,c] == X[j,c]} G[pb[k,j], c].
 * Replaces maxpool_backward, pool.py:94-154, :287-330. */
int sp_maxpool_bwd(const void* x, const void* out, const void* gout, int32_t dtype,
                   int64_t n_in, int64_t C, const int32_t* pb, int64_t kv, int64_t n_out,
                   void* dx, void* stream);

/* Mean over present inputs; count [n_out] int32 (nullable).
 * Replaces avgpool_forward, pool.py:157-208, :333-367. */
int sp_avgpool_fwd(const void* x, int32_t dtype, int64_t n_in, int64_t C,
                   const int32_t* pf, int64_t kv, int64_t n_out, void* out,
                   int32_t* count, void* stream);

/* dX[j, c] = sum_{k: pb[k,j] >= 0} G[pb[k,j], c] * count[pb[k,j]] (the
 * reference multiplies by the count).  Replaces avgpool_backward,
 * pool.py:211-257, :370-397. */
int sp_avgpool_bwd(const void* gout, const int32_t* count, int32_t dtype, int64_t n_out,
                   int64_t C, const int32_t* pb, int64_t kv, int64_t n_in, void* dx,
                   void* stream);

/* ---- point-cloud voxelisation ------------------------------------------ */

/* Workspace bytes of sp_point2voxel (0 for bad sizes). */
size_t sp_point2voxel_workspace_size(int64_t n_points, int64_t max_voxels);

/* PointToVoxel.generate_voxel_with_id (spconv_triton/pytorch/utils.py:72-163).
 * points [n_points, point_cols] f32 or f64 (dtype), the first ndim columns x,
 * y, z, ...; a point's voxel is floor((p - coors_min) / vsize) per axis,
 * computed in the points' precision, kept when inside grid_size_xyz.  Voxels
 * are numbered in order of their first point, at most max_voxels of them;
 * each stores up to max_points_per_voxel points (num_point_features columns,
 * as f32) in point order.  Outputs, caller-owned, sized for max_voxels:
 * voxels [max_voxels, max_points_per_voxel, num_point_features] f32 (zeroed
 * first when clear_voxels; with empty_mean the empty slots of every voxel get
 * its mean, utils.py:145-152), indices [max_voxels, ndim] int32 in ZYX order,
 * num_per_voxel [max_voxels] int32 (clamped counts), pc_voxel_id [n_points]
 * int64 (voxel of every point, -1 when dropped) and *num_voxels.  Blocks the
 * host once, to read the voxel count. */
int sp_point2voxel(const void* points, int32_t dtype, int64_t n_points, int64_t point_cols,
                   int32_t ndim, const double* vsize_xyz, const double* coors_min_xyz,
                   const int64_t* grid_size_xyz, int32_t num_point_features, int64_t max_voxels,
                   int32_t max_points_per_voxel, int32_t clear_voxels, int32_t empty_mean,
                   float* voxels, int32_t* indices, int32_t* num_per_voxel,
                   int64_t* pc_voxel_id, int64_t* num_voxels, void* ws, size_t ws_bytes,
                   void* stream);

/* ---- hash table (spconv_triton/pytorch/hash.py:15-110) ----------------- */
/* A table of `capacity` (a power of two) slots lives in one caller-owned
 * device buffer of sp_hash_table_bytes(capacity).  Keys are int32 (key64 = 0)
 * or int64 (key64 = 1; the key INT64_MAX is reserved); values hold 4 or 8
 * bytes, vkind 0 int32, 1 int64, 2 f32, 3 f64.  `epoch` must grow with every
 * insert call on a table: among writers of one key the last call, and in it
 * the last position, wins (the reference's sort-based insert, hash.py:38-59). */
size_t sp_hash_table_bytes(int64_t capacity);
/* Workspace of an insert of n keys (n = 0: of items / assign_arange). */
size_t sp_hash_workspace_size(int64_t capacity, int64_t n);
/* Empties the table. */
int sp_hash_clear(void* table, int64_t capacity, void* stream);
/* HashTable.insert (hash.py:38-59); values may be NULL (zeros).  Blocks the
 * host once: *n_entries receives the number of stored keys, and a full table
 * fails with SP_ERR_HASH_FULL. */
int sp_hash_insert(void* table, int64_t capacity, const void* keys, int32_t key64,
                   const void* values, int32_t vkind, int64_t n, uint32_t epoch,
                   int64_t* n_entries, void* ws, size_t ws_bytes, void* stream);
/* HashTable.insert_exist_keys (hash.py:79-89): updates stored keys only;
 * found [n] uint8 receives 1 where the key was stored. */
int sp_hash_insert_existing(void* table, int64_t capacity, const void* keys, int32_t key64,
                            const void* values, int32_t vkind, int64_t n, uint32_t epoch,
                            uint8_t* found, void* ws, size_t ws_bytes, void* stream);
/* HashTable.query (hash.py:61-77): values_out [n] (0 where absent) and
 * is_empty [n] uint8. */
int sp_hash_query(const void* table, int64_t capacity, const void* keys, int32_t key64,
                  int32_t vkind, int64_t n, void* values_out, uint8_t* is_empty, void* stream);
/* HashTable.items / assign_arange_ (hash.py:91-110): the stored entries in
 * ascending key order.  assign_arange = 0: the first min(count, max_items)
 * keys and values go to keys_out / values_out; assign_arange = 1: the value
 * of the i-th key becomes i (in the value type).  The count is left in the
 * table's header word 2 (device memory, byte offset 8). */
int sp_hash_items(void* table, int64_t capacity, int32_t key64, int32_t vkind, int64_t max_items,
                  void* keys_out, void* values_out, int32_t assign_arange, void* ws,
                  size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPCONV_HIP_H */
