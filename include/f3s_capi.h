/*
 * f3s_capi.h -- C-ABI of libf3s_hip.so, the MI355X (gfx950) implementation of
 * the fused3S hot path: CSR -> 16x16 block-sparse conversion, window ordering
 * and the fused SDDMM -> online softmax -> SpMM pass.
 *
 * Plain C: no HIP or torch types.  Device buffers are `void*`/typed pointers
 * obtained from f3s_malloc (or any HIP allocation in the same process);
 * streams are `void*` (a hipStream_t, NULL = the default stream).  Every
 * function returns f3s_status (0 = F3S_OK) and never exits the process; the
 * detail of the last failure on the calling thread is f3s_last_error().
 *
 * Layouts:
 *   CSR            row_ptr int32[n+1], col_idx int32[nnz] (columns < n)
 *   block-sparse   W = ceil(n/16) row windows; window_offsets int32[W+1];
 *                  block_col int32[T] (ascending per window);
 *                  tile_mask uint16[T][16]: bit c of row r <=> edge
 *                  (16w + r, 16*block_col + c)
 *   features       Q, K, V: IEEE binary16 bits, node-major [n][H][d];
 *                  O: float32 [n][H][d].  Buffers need n rows (a reference-
 *                  style buffer padded to 16W rows also works).
 *
 * Thread safety: calls on different streams may run concurrently; the
 * library's only mutable global state is the per-thread last error and the
 * per-device cache of freed device memory (below; one mutex guards it).
 * A plan owns the partial-result buffers of its split windows, so one plan
 * must not serve two overlapping calls.
 */
#ifndef F3S_CAPI_H
#define F3S_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t f3s_status;

#define F3S_OK 0
#define F3S_EINVAL 1        /* bad size, pointer or argument */
#define F3S_ENOMEM 2        /* device allocation failed */
#define F3S_EHIP 3          /* a HIP runtime call failed (detail in f3s_last_error) */
#define F3S_ENODEV 4        /* no usable GPU */
#define F3S_EUNSUPPORTED 5  /* valid but not implemented here (e.g. d != 64) */
#define F3S_EDATA 6         /* input data violates the format (e.g. column >= n) */

#define F3S_ABI_VERSION 1

/* Semantics of f3s_attention_fwd*: tile_mask == NULL selects TILE_DENSE
 * (every column < n of every active tile is attended: the reference kernel
 * and test ground truth, tests/test_fused_3s_v2.cu:17-59); a mask selects
 * MASKED (edge-exact, baselines/cpu_baseline.cpp:16-91). */

const char* f3s_status_string(f3s_status s);
const char* f3s_last_error(void);
int32_t f3s_abi_version(void);

/* Loads the library's GPU code onto the current device now rather than at
 * the first launch of each kernel (HIP loads code objects lazily), so the
 * first timed call is not charged for it.  Optional; idempotent.  The
 * reference has no counterpart (CUDA contexts load modules the same way). */
f3s_status f3s_init(void);

/* ---- device plumbing (replaces the CUDA_CHECK'ed runtime calls of the
 *      reference harness, tests/test_fused_3s_v2.cu:93-120,139,157-159) ---- */
f3s_status f3s_device_count(int32_t* count);
f3s_status f3s_set_device(int32_t device);
f3s_status f3s_device_name(char* buf, int32_t buflen);
/* Device memory comes from a caching allocator over hipMalloc: blocks the
 * library frees (scratch of a call, in stream order; a destroyed plan's
 * buffers) are kept per device and size class for reuse, so repeated
 * conversions, plans and calls skip the driver's allocation and page
 * mapping.  Idle cached memory is capped per device at 1 GiB, or at the
 * F3S_CACHE_LIMIT_MB environment variable's value read at the first
 * allocation (0 keeps nothing); on an allocation failure the cache goes back
 * to the driver and the allocation is retried.  f3s_malloc'd memory is usable
 * on every stream on return; f3s_free waits for the device first, as hipFree
 * does, and returns the block to the cache (f3s_release_cached_memory hands
 * every idle block back to the driver). */
f3s_status f3s_malloc(void** ptr, uint64_t bytes);
f3s_status f3s_free(void* ptr);
/* Returns every idle cached block to the driver (waits for every device
 * first).  No reference counterpart; for processes that share the GPU with
 * another allocator, e.g. torch's. */
f3s_status f3s_release_cached_memory(void);
f3s_status f3s_memcpy_h2d(void* dst, const void* src, uint64_t bytes, void* stream);
f3s_status f3s_memcpy_d2h(void* dst, const void* src, uint64_t bytes, void* stream);
f3s_status f3s_memcpy_d2d(void* dst, const void* src, uint64_t bytes, void* stream);
f3s_status f3s_memset(void* ptr, int32_t value, uint64_t bytes, void* stream);
f3s_status f3s_synchronize(void* stream);            /* NULL: whole device */
f3s_status f3s_stream_create(void** stream);
f3s_status f3s_stream_destroy(void* stream);
f3s_status f3s_event_create(void** event);
f3s_status f3s_event_destroy(void* event);
f3s_status f3s_event_record(void* event, void* stream);
f3s_status f3s_event_elapsed_ms(void* start, void* stop, float* ms);  /* waits for stop */

/* float2half_kernel (tests/test_fused_3s_v2.cu:61-64): IEEE round to
 * nearest even, elementwise. */
f3s_status f3s_cast_f32_to_f16(const float* d_in, uint16_t* d_out, int64_t count, void* stream);

/* convert_csr_to_block_sparse (src/converter.cu:13-44), on the GPU.
 * d_window_offsets[W+1] is always written and *T_out receives T (the call
 * synchronises `stream` to read it).  When d_block_col is non-NULL the tile
 * lists are written too (it must hold T entries), and when d_tile_mask is
 * non-NULL the 16 row masks of each tile (T*16 entries).  Typical use is two
 * calls: sizes first (d_block_col = NULL), then the lists.  Output is
 * bit-exact with the reference converter.  F3S_EDATA if row_ptr is not
 * monotone from 0 to nnz or a column is outside [0, n) (the offsets written
 * are then meaningless).  A CSR may repeat an entry (a multigraph): the
 * reference converter accepts that, and so does this one -- the tile lists
 * are those of the deduplicated CSR and the masks record each (row, column)
 * pair once, so nnz - mask_bits (f3s_bsf_stats) counts the repeated entries.
 * The masked pass then attends each edge once, whereas the reference's
 * cpu_sparse_attention_csr (baselines/cpu_baseline.cpp:38-50) counts a
 * repeated entry once per repeat; the tile-dense pass is unaffected.  Each
 * call makes one host round trip (to read T and the error bits); scratch
 * comes from the library's cache. */
f3s_status f3s_convert_csr_to_bsf(const int32_t* d_row_ptr, const int32_t* d_col_idx,
                                  int32_t n, int64_t nnz,
                                  int32_t* d_window_offsets, int32_t* d_block_col,
                                  uint16_t* d_tile_mask, int64_t* T_out, void* stream);

/* generate_balanced_window_order (include/utils.cuh:48-59), on the GPU:
 * windows by descending tile count, ties by ascending window index. */
f3s_status f3s_window_order(const int32_t* d_window_offsets, int32_t W,
                            int32_t* d_order, void* stream);

/* Figures behind the algorithmic byte model (no reference counterpart):
 * occ_sum = sum over tiles of the columns the fused pass gathers (popcount of
 * the OR of the row masks if d_tile_mask, else the tile's columns < n);
 * mask_bits = popcount of all masks, the distinct edges: mask_bits < nnz iff
 * the CSR repeats entries.  Synchronises `stream`. */
f3s_status f3s_bsf_stats(const int32_t* d_block_col, const uint16_t* d_tile_mask,
                         int64_t T, int32_t n, int64_t* occ_sum, int64_t* mask_bits,
                         void* stream);

/* f3s_1tb1rw_kernel (src/fused3s_v2.cu:81-90) and its launch
 * (tests/test_fused_3s_v2.cu:124-131): one fused pass, each row window
 * handled whole, over the windows d_window_order names (NULL = all).
 * O[i] = sum_j softmax_j(scale * Q[i].K[j]) V[j] per head; rows with no
 * attended column get 0; rows of windows the order does not name are not
 * written.  Requires d == 64 and 1 <= H <= 64 heads in node-major [n][H][64]
 * layout, of any size (tensors past ~4 GiB are read with 64-bit addresses);
 * scale = 1 reproduces the reference (which has no scaling, and one head).
 * Small graphs run each window on a team of 4 or 16 waves of one workgroup
 * (masked: W*H <= 1024, teams of 4; tile-dense: W*H <= 512, teams of 16, up
 * to 2048, teams of 4), each wave taking an even share of the window's
 * tiles, merged in LDS in a fixed order, in the order's sequence.  On larger
 * graphs (W > 512), given d_window_order on a launch of fewer than 2^18
 * window-heads (W x H), windows run in the order's sequence: the heavy
 * windows (more than max(1024, 8 x mean) tiles) among its first 512 entries
 * as teams of 16 waves in a launch of their own, every other entry on one
 * wave.  In natural order, and with an order from 2^18 window-heads on, the
 * order only names the windows -- each named window is computed once;
 * invalid entries are skipped -- and the library schedules them itself,
 * identically for every order: the heavy windows, heaviest first, the first
 * 512 of them as teams of 16 waves in a launch of their own; every other
 * window on one wave, by octave of its tile count, heaviest first, each
 * octave in index order and cut into eight contiguous shares interleaved
 * slot by slot across the XCDs (longest windows first for the tail, each
 * share's contiguous windows on one or a few XCDs for the L2; on a
 * community-ordered graph the reference's descending order would scatter
 * each community over the whole run).  With W <= 1024 no window can be heavy
 * (one tile per block column at most) and no team launch is made.  Three
 * small kernels (four given an order; ~15-30 us) build the schedule in
 * scratch of about 9 bytes per window taken from the
 * library's cache and returned to it in stream order on `stream` (the call
 * does not wait).  Tensors past ~4 GiB take the sequence of the order, as
 * small graphs do.  Every other path allocates nothing. */
f3s_status f3s_attention_fwd(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                             float* O, const int32_t* d_window_offsets,
                             const int32_t* d_block_col, const uint16_t* d_tile_mask,
                             const int32_t* d_window_order, int32_t W, int32_t n,
                             int32_t d, int32_t H, float scale, void* stream);

/* f3s_attention_fwd without any device allocation.  No counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * semantics, kernels and results (bit for bit) as f3s_attention_fwd; the
 * schedule's scratch (tables, team list, class counts, one-wave slots and an
 * order's inverse: 16.5 MiB) is a fixed device array of the library, one per
 * GPU, held until the process ends.  Limit: W <= 2,097,152 row windows
 * (n <= 33,554,432 nodes); larger W returns F3S_EUNSUPPORTED.  Every call on
 * one GPU shares that GPU's array and overwrites it, so calls that overlap in
 * time on one GPU (e.g. on two streams) race; serialise them.  Allocates
 * nothing, clears no memory and never waits for the device. */
f3s_status f3s_attention_fwd_noalloc(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                     float* O, const int32_t* d_window_offsets,
                                     const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                     const int32_t* d_window_order, int32_t W, int32_t n,
                                     int32_t d, int32_t H, float scale, void* stream);

/* The timed launch of tests/test_fused_3s_v2.cu:126-136 (events recorded
 * around the kernel on the launch stream): `reps` back-to-back calls of
 * f3s_attention_fwd with the same arguments, timed with HIP events on
 * `stream`; *us_out = mean microseconds per call.  Synchronises `stream`. */
f3s_status f3s_attention_fwd_timed(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                   float* O, const int32_t* d_window_offsets,
                                   const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                   const int32_t* d_window_order, int32_t W, int32_t n,
                                   int32_t d, int32_t H, float scale, void* stream,
                                   int32_t reps, float* us_out);

/* f3s_naive_baseline_kernel (baselines/gpu_baseline.cu:28-116): the naive
 * edge-exact comparator, one thread per node, fp32 Q/K/V/O [n][d], CSR
 * neighbours as stored (a duplicate entry counts twice, as in
 * cpu_sparse_attention_csr).  No device-heap allocation (the reference
 * mallocs per thread).  1 <= d <= 64. */
f3s_status f3s_naive_attention_fwd(const float* Q, const float* K, const float* V, float* O,
                                   const int32_t* d_row_ptr, const int32_t* d_col_idx,
                                   int32_t n, int32_t d, float scale, void* stream);

/* Planned execution (no reference counterpart; the reference relies on the
 * window sort alone, include/utils.cuh:48-59).  A plan splits windows with
 * more than `seg_tiles` tiles into segments processed by separate waves; the
 * last segment of each split window to finish merges its segments in a fixed
 * order (deterministic), inside the same launch, so hub windows do not
 * serialise.  seg_tiles = 0 chooses
 * automatically: on small graphs (W*H <= 2048) the teams of f3s_attention_fwd
 * (same items, same bits), else segment sizes from T*H.  Windows run in d_window_order (the reference's descending
 * sort) or, when it is NULL, in natural order with consecutive windows kept
 * on one XCD (for community-ordered graphs).  Build once per graph; reuse for
 * every forward pass; one plan must not serve two overlapping calls (it owns
 * the partial-result buffers).  From 2^18 window-heads (W x H) on, a plan
 * whose items run one wave each follows the library's schedule of
 * f3s_attention_fwd instead of the order's sequence (the order then only
 * names the windows), keeping a community-ordered graph's L2 reuse under the
 * reference's descending order. */
typedef struct f3s_plan f3s_plan;
f3s_status f3s_plan_create(const int32_t* d_window_offsets, const int32_t* d_window_order,
                           int32_t W, int32_t H, int32_t seg_tiles, void* stream,
                           f3s_plan** plan_out);
f3s_status f3s_plan_destroy(f3s_plan* plan);
/* Lists, once per graph, the columns each planned item attends under the
 * masked semantics (32 row offsets + 32 row masks per 32-column chunk), so
 * masked passes read 8 bytes per attended column instead of expanding 36
 * bytes of tile metadata on every pass.  Later masked calls of
 * f3s_attention_fwd_planned with these same d_block_col / d_tile_mask
 * pointers and n use the lists; the structure they point to must not change
 * afterwards (compile again if it does).  Other calls are unaffected. */
f3s_status f3s_plan_compile(f3s_plan* plan, const int32_t* d_block_col,
                            const uint16_t* d_tile_mask, int32_t n, void* stream);
f3s_status f3s_plan_info(const f3s_plan* plan, int64_t* num_items, int64_t* num_split_windows,
                         int64_t* T, int32_t* seg_tiles);
/* The sizes behind a planned pass's memory traffic (no reference
 * counterpart): compiled column chunks (256 bytes each; 0 before
 * f3s_plan_compile), and for the item sets of masked and of tile-dense
 * passes their work items (16 bytes each) and split-window partial slots
 * (per head, 4,224 bytes written by the pass and read by its merge).  Any
 * output pointer may be NULL. */
f3s_status f3s_plan_stats(const f3s_plan* plan, int64_t* num_chunks, int64_t* masked_items,
                          int64_t* masked_slots, int64_t* dense_items, int64_t* dense_slots);
f3s_status f3s_attention_fwd_planned(const f3s_plan* plan, const uint16_t* Q,
                                     const uint16_t* K, const uint16_t* V, float* O,
                                     const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                     int32_t n, int32_t d, int32_t H, float scale,
                                     void* stream);

/* Measurement only (no reference counterpart): the device's random-gather
 * ceiling for the fused pass's access pattern.  For each of `count` columns
 * (a multiple of 32) it loads the 128-byte row at byte offset
 * d_idx[i] * row_stride of K and of V (eight lanes x 16 bytes per row, 32
 * columns per step, `cpw` steps per wave: the fused pass's load shape) and
 * folds the bytes into d_out, one word per wave: ceil(count / 32 / cpw)
 * words.  Tables hold `rows` rows (rows * row_stride <= 0xffff0000 bytes);
 * a negative row or one past the table reads zero.  Asynchronous on
 * `stream`. */
f3s_status f3s_probe_gather(const uint16_t* K, const uint16_t* V, int64_t rows,
                            int32_t row_stride, const int32_t* d_idx, int64_t count,
                            int32_t cpw, uint32_t* d_out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
