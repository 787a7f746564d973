/*
 * f3s_host.h -- C-ABI of libf3s_host.so: host-side parts of the path that
 * the reference keeps on the CPU, plus deterministic synthetic inputs.
 *
 * The C++ drop-in API with the reference's own signatures
 * (load_csr_graph, convert_csr_to_block_sparse,
 * generate_balanced_window_order) is in include/f3s/graph.hpp; the entry
 * points below are the plain-C view of the same functions for FFI callers
 * (ctypes in fused3s_amd/_lib.py).
 *
 * All returned arrays are allocated by the library and released with
 * f3s_host_free.  Functions return 0 on success.
 */
#ifndef F3S_HOST_H
#define F3S_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void f3s_host_free(void* p);
const char* f3s_host_last_error(void);

/* load_csr_graph (include/utils.cuh:26-40), with the file-name bug fixed:
 * reads <dir>/meta.txt ("n nnz"), row_ptr.txt (n+1 ints) and col_idx.txt
 * (nnz ints; col_ind.txt, the name the reference opens, is accepted as a
 * fallback).  Unlike the reference, a missing or short file or an invalid
 * CSR is an error (return 1), never a silent all-zero graph. */
int32_t f3s_host_load_csr(const char* dir, int32_t* n, int64_t* nnz, int32_t** row_ptr,
                          int32_t** col_idx);

/* Binary graph file (no counterpart in the reference, which keeps only the
 * text files read by load_csr_graph, include/utils.cuh:26-40): the CSR and,
 * when window_offsets is given, its block-sparse form (W = ceil(n/16) windows,
 * T tiles, and the 16 row masks per tile when tile_mask is given), in one
 * checksummed file with 64-byte-aligned arrays.  The file is written to
 * <path>.tmp and renamed, so a reader never sees a partial file.
 * f3s_host_load_graph validates header, size, checksum, CSR and block-sparse
 * invariants and returns library-allocated arrays (window_offsets,
 * block_col and tile_mask are NULL, W and T 0, when the file has none). */
int32_t f3s_host_save_graph(const char* path, int32_t n, int64_t nnz, const int32_t* row_ptr,
                            const int32_t* col_idx, int32_t W, int64_t T,
                            const int32_t* window_offsets, const int32_t* block_col,
                            const uint16_t* tile_mask);
int32_t f3s_host_load_graph(const char* path, int32_t* n, int64_t* nnz, int32_t** row_ptr,
                            int32_t** col_idx, int32_t* W, int64_t* T, int32_t** window_offsets,
                            int32_t** block_col, uint16_t** tile_mask);

/* generate_balanced_window_order (include/utils.cuh:48-59): std::sort of
 * iota(W) by descending tile count with the reference's comparator. */
int32_t f3s_host_window_order(const int32_t* window_offsets, int32_t W, int32_t* order);

/* Synthetic graphs (undirected, symmetric CSR, sorted unique columns,
 * optional self-loop on every node).  Deterministic for a seed on any host
 * and thread count (counter-based random streams).
 *
 * Chung-Lu power law: expected degrees proportional to (i + i0)^(-1/(gamma-1))
 * with i0 chosen so the largest expected degree is ~max_degree; about
 * target_edges directed edges before self-loops; node ids randomly permuted
 * when `permute` (so 16x16 tiles are mostly 1-3 nnz).
 *
 * SBM: communities of `community` consecutive node ids (the last one may be
 * partial); each sampled pair picks u uniformly, then v uniformly from u's
 * community with probability p_intra, else uniformly from all nodes;
 * n*mean_degree/2 pairs are sampled. */
int32_t f3s_gen_powerlaw(int32_t n, int64_t target_edges, double gamma, double max_degree,
                         int32_t permute, int32_t self_loops, uint64_t seed, int32_t** row_ptr,
                         int32_t** col_idx, int64_t* nnz);
int32_t f3s_gen_sbm(int32_t n, int32_t community, double mean_degree, double p_intra,
                    int32_t self_loops, uint64_t seed, int32_t** row_ptr, int32_t** col_idx,
                    int64_t* nnz);

/* Feature values as IEEE binary16 bits (round to nearest even from an fp32
 * draw).  Element i of tensor `tensor` (0 = Q, 1 = K, 2 = V) uses stream
 * position 3*i + tensor, i.e. the three tensors are drawn interleaved like
 * tests/test_fused_3s_v2.cu:86-88.  dist 0: U[-1, 1); dist 1: N(0, 1). */
int32_t f3s_gen_features_f16(uint64_t seed, int32_t tensor, int64_t count, int32_t dist,
                             uint16_t* out);

/* binary16 bits -> float32 (exact). */
void f3s_host_f16_to_f32(const uint16_t* in, float* out, int64_t count);

#ifdef __cplusplus
}
#endif
#endif
