/*
 * f3s_oracle.h -- CPU restatement of the fused3S hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline).  The product path (fused3s_amd/,
 * libf3s_hip.so, libf3s_host.so) never links or calls it.
 *
 * Each function cites the reference file:line it restates.  How every
 * function is pinned (golden fixtures, the reference's own CPU baseline
 * compiled under oracle/_ref, closed forms, brute force) is listed in
 * tests/test_oracle.py; a function without such a check would be marked
 * "parity unpinned" here -- there is none.
 *
 * Layouts: row-major, node-major features [n][H][d]; CSR int32.
 */
#ifndef F3S_ORACLE_H
#define F3S_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary32 -> binary16, round to nearest even (the semantics of
 * __float2half used by float2half_kernel, tests/test_fused_3s_v2.cu:61-64). */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
void orc_cast_f32_to_f16(const float* in, uint16_t* out, int64_t count);
void orc_cast_f16_to_f32(const uint16_t* in, float* out, int64_t count);

/* load_csr_graph (include/utils.cuh:26-40), with F1 fixed: reads
 * meta.txt, row_ptr.txt and col_idx.txt (col_ind.txt accepted as fallback).
 * Returns 0 on success, nonzero if a file is missing or short.  Arrays are
 * malloc'ed; release with orc_free. */
int orc_load_csr(const char* dir, int32_t* n, int64_t* nnz,
                 int32_t** row_ptr, int32_t** col_idx);
void orc_free(void* p);

/* convert_csr_to_block_sparse (src/converter.cu:13-44).
 * Pass 1: fills window_offsets[W+1] (W = ceil(n/16)), returns T.
 * Pass 2: fills block_col[T] (ascending unique c/16 per window) and, if
 * tile_mask != NULL, tile_mask[T][16] with bit c of row r set iff edge
 * (16w+r, 16*block_col+c) exists (new output; closed form from the CSR). */
int64_t orc_convert_count(int32_t n, const int32_t* row_ptr, const int32_t* col_idx,
                          int32_t* window_offsets);
void orc_convert_fill(int32_t n, const int32_t* row_ptr, const int32_t* col_idx,
                      const int32_t* window_offsets, int32_t* block_col,
                      uint16_t* tile_mask);

/* generate_balanced_window_order (include/utils.cuh:48-59): windows by
 * descending tile count.  The reference sort is unstable; this one is stable
 * (ties by ascending window index), the tie rule of f3s_window_order. */
void orc_window_order(const int32_t* window_offsets, int32_t W, int32_t* order);

/* cpu_sparse_attention_csr (baselines/cpu_baseline.cpp:16-91), MASKED
 * (edge-exact) semantics, generalised to H heads and a logit scale
 * (scale = 1 reproduces the reference).  Computes rows [r0, r1) of O.
 * threads <= 1 runs single-threaded like the reference. */
void orc_masked_attention(int32_t n, int32_t d, int32_t H,
                          const float* Q, const float* K, const float* V,
                          const int32_t* row_ptr, const int32_t* col_idx,
                          float scale, int32_t r0, int32_t r1, float* O,
                          int32_t threads);

/* cpu_block_sparse_attention (tests/test_fused_3s_v2.cu:17-59), TILE_DENSE
 * semantics: every column < n of every active tile of the row's window enters
 * the softmax (columns >= n get -1e9 there, i.e. are excluded).  Rows
 * [r0, r1); rows of an empty window are left at 0. */
void orc_tile_dense_attention(int32_t n, int32_t d, int32_t H,
                              const float* Q, const float* K, const float* V,
                              const int32_t* window_offsets, const int32_t* block_col,
                              float scale, int32_t r0, int32_t r1, float* O,
                              int32_t threads);

/* The same TILE_DENSE truth with each window's 16 rows in SIMD lanes: the
 * scalar restatement's operations in its order, lane by lane, hence
 * bit-identical to orc_tile_dense_attention (checked by tests/test_oracle.py);
 * fast enough to check every row of the large configurations. */
void orc_tile_dense_attention_fast(int32_t n, int32_t d, int32_t H,
                                   const float* Q, const float* K, const float* V,
                                   const int32_t* window_offsets, const int32_t* block_col,
                                   float scale, int32_t r0, int32_t r1, float* O,
                                   int32_t threads);

/* Occupancy figures behind the algorithmic byte model: occ_sum = sum over
 * tiles of occ(t), where occ(t) = popcount of the OR of the tile's 16 row
 * masks (masked) or the number of the tile's columns < n (tile-dense);
 * mask_bits = total popcount of all masks (= nnz for a simple graph). */
void orc_bsf_occupancy(int32_t n, int64_t T, const int32_t* block_col,
                       const uint16_t* tile_mask, int masked,
                       int64_t* occ_sum, int64_t* mask_bits);

#ifdef __cplusplus
}
#endif
#endif
