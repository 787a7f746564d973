// graph.hpp -- drop-in C++ host API of the fused3S hot path.
//
// Same names, argument meaning and return types as the reference's
// include/utils.cuh:19-59 and src/converter.cu:13, so a caller of the
// reference links libf3s_host.so instead.  Differences, all deliberate:
//   * load_csr_graph reads col_idx.txt (the exporter's name) and throws
//     std::runtime_error on a missing or malformed file instead of returning
//     an all-zero graph (utils.cuh:36 opens col_ind.txt and never checks);
//   * blockSparseFormat carries the new intra-tile row masks and the count of
//     repeated CSR entries;
//   * convert_csr_to_block_sparse runs on the GPU through libf3s_hip.so
//     (bit-exact with the reference's host converter) and throws if no GPU
//     is usable; it prints the same two lines as the reference (:42-43), and
//     a notice on stderr when the CSR repeats entries;
//   * F3S_CHECK replaces CUDA_CHECK (utils.cuh:9-17) for f3s_status codes.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "../f3s_capi.h"

#define F3S_CHECK(call)                                                                  \
    do {                                                                                 \
        f3s_status f3s_chk_ = (call);                                                    \
        if (f3s_chk_ != F3S_OK) {                                                        \
            f3s_report_failure(f3s_chk_, #call, __FILE__, __LINE__);                     \
        }                                                                                \
    } while (0)

// Prints the status, the library's detail message and the call site, then
// exits with EXIT_FAILURE (the behaviour of CUDA_CHECK, utils.cuh:13-15).
[[noreturn]] void f3s_report_failure(f3s_status s, const char* call, const char* file, int line);

// include/utils.cuh:19-24
struct GraphData {
    int num_nodes = 0;
    int num_edges = 0;
    std::vector<int> row_ptr;
    std::vector<int> col_ind;
};

// include/utils.cuh:26-40
GraphData load_csr_graph(const std::string& dataset_dir);

// include/utils.cuh:42-46, plus tile_masks (16 uint16 per active tile: bit c
// of entry r <=> edge (16w + r, 16*block_col + c)) and duplicate_entries: CSR
// entries that repeat an earlier (row, column) pair (nnz minus the masks'
// popcount).  A CSR with repeats (a multigraph) gives the tile lists of its
// deduplicated form, as the reference converter does; its masks, and so the
// masked (edge-exact) pass, count each edge once, whereas the reference's
// cpu_sparse_attention_csr (baselines/cpu_baseline.cpp:38-50) counts a
// repeated entry once per repeat.
struct blockSparseFormat {
    int num_row_windows = 0;
    std::vector<int> window_offsets;
    std::vector<int> block_col_indices;
    std::vector<uint16_t> tile_masks;
    int64_t duplicate_entries = 0;
};

// src/converter.cu:13-44
blockSparseFormat convert_csr_to_block_sparse(int num_nodes, const std::vector<int>& row_ptr,
                                              const std::vector<int>& col_ind);

// include/utils.cuh:48-59
std::vector<int> generate_balanced_window_order(const blockSparseFormat& format);

// Binary graph file (f3s_host_save_graph / f3s_host_load_graph; no
// counterpart in the reference, which reads text only): the CSR and,
// optionally, its block-sparse form with row masks.  Both throw
// std::runtime_error on failure; load fills *bsf when it is not NULL and the
// file holds a block-sparse section (else leaves it empty).
void save_graph_binary(const std::string& path, const GraphData& graph,
                       const blockSparseFormat* bsf = nullptr);
GraphData load_graph_binary(const std::string& path, blockSparseFormat* bsf = nullptr);
