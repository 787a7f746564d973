// graph.cpp -- host side of the path: CSR loader, window order, the C++
// drop-in API of include/f3s/graph.hpp and the C view of include/f3s_host.h.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <fstream>
#include <iostream>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../../include/f3s/graph.hpp"
#include "../../../include/f3s_capi.h"
#include "../../../include/f3s_host.h"

namespace f3s_host {

static thread_local std::string g_error;
void set_error(const std::string& s) { g_error = s; }

// Reads `count` integers; false if the file is missing or short.
static bool read_ints(const std::string& path, int64_t count, std::vector<int>& out)
{
    std::ifstream f(path);
    if (!f) return false;
    out.resize((size_t)count);
    for (int64_t i = 0; i < count; ++i) {
        long long v;
        if (!(f >> v)) return false;
        if (v < INT32_MIN || v > INT32_MAX) return false;
        out[(size_t)i] = (int)v;
    }
    return true;
}

// include/utils.cuh:26-40 with validation.
static GraphData load(const std::string& dir)
{
    GraphData g;
    std::ifstream meta(dir + "/meta.txt");
    long long n = -1, e = -1;
    if (!meta || !(meta >> n >> e) || n < 0 || e < 0 || n > INT32_MAX || e > INT32_MAX)
        throw std::runtime_error("load_csr_graph: cannot read " + dir + "/meta.txt");
    g.num_nodes = (int)n;
    g.num_edges = (int)e;
    if (!read_ints(dir + "/row_ptr.txt", n + 1, g.row_ptr))
        throw std::runtime_error("load_csr_graph: missing or short " + dir + "/row_ptr.txt");
    if (!read_ints(dir + "/col_idx.txt", e, g.col_ind) &&
        !read_ints(dir + "/col_ind.txt", e, g.col_ind))
        throw std::runtime_error("load_csr_graph: missing or short " + dir +
                                 "/col_idx.txt (or col_ind.txt)");
    if (g.row_ptr[0] != 0 || g.row_ptr[(size_t)n] != e)
        throw std::runtime_error("load_csr_graph: row_ptr must run from 0 to nnz");
    for (long long i = 0; i < n; ++i)
        if (g.row_ptr[(size_t)i + 1] < g.row_ptr[(size_t)i])
            throw std::runtime_error("load_csr_graph: row_ptr is not monotone");
    for (int c : g.col_ind)
        if (c < 0 || c >= n) throw std::runtime_error("load_csr_graph: column outside [0, n)");
    return g;
}

// include/utils.cuh:48-59: std::sort, descending tile count, same comparator.
static void order(const int* offs, int W, int* out)
{
    std::iota(out, out + W, 0);
    std::sort(out, out + W, [offs](int a, int b) {
        int blocks_a = offs[a + 1] - offs[a];
        int blocks_b = offs[b + 1] - offs[b];
        return blocks_a > blocks_b;
    });
}

// RAII device allocation for the drop-in converter.
struct DevPtr {
    void* p = nullptr;
    ~DevPtr() { f3s_free(p); }
};

static void check(f3s_status s, const char* what)
{
    if (s != F3S_OK)
        throw std::runtime_error(std::string(what) + ": " + f3s_status_string(s) + " (" +
                                 f3s_last_error() + ")");
}

}  // namespace f3s_host

using namespace f3s_host;

[[noreturn]] void f3s_report_failure(f3s_status s, const char* call, const char* file, int line)
{
    std::cerr << "f3s error in " << file << ":" << line << " code=" << s << ": "
              << f3s_status_string(s) << " [" << call << "] " << f3s_last_error() << std::endl;
    exit(EXIT_FAILURE);
}

GraphData load_csr_graph(const std::string& dataset_dir) { return load(dataset_dir); }

void save_graph_binary(const std::string& path, const GraphData& g, const blockSparseFormat* bsf)
{
    const bool has = bsf && !bsf->window_offsets.empty();
    const bool masks = has && !bsf->block_col_indices.empty() &&
                       bsf->tile_masks.size() == 16 * bsf->block_col_indices.size();
    if (f3s_host_save_graph(path.c_str(), g.num_nodes, (int64_t)g.col_ind.size(),
                            g.row_ptr.data(), g.col_ind.data(), has ? bsf->num_row_windows : 0,
                            has ? (int64_t)bsf->block_col_indices.size() : 0,
                            has ? bsf->window_offsets.data() : nullptr,
                            has ? bsf->block_col_indices.data() : nullptr,
                            masks ? bsf->tile_masks.data() : nullptr) != 0)
        throw std::runtime_error(f3s_host_last_error());
}

// Distinct (row, column) pairs the masks record (a tile's 16 masks are 32
// bytes, so the array is a whole number of 64-bit words).
static int64_t mask_popcount(const std::vector<uint16_t>& masks)
{
    int64_t bits = 0;
    const size_t words = masks.size() / 4;
    const unsigned char* b = reinterpret_cast<const unsigned char*>(masks.data());
    for (size_t i = 0; i < words; ++i) {
        uint64_t x;
        memcpy(&x, b + 8 * i, sizeof x);
        bits += __builtin_popcountll(x);
    }
    for (size_t i = 4 * words; i < masks.size(); ++i) bits += __builtin_popcount(masks[i]);
    return bits;
}

GraphData load_graph_binary(const std::string& path, blockSparseFormat* bsf)
{
    int32_t n = 0, W = 0;
    int64_t nnz = 0, T = 0;
    int32_t *rp = nullptr, *ci = nullptr, *wo = nullptr, *bc = nullptr;
    uint16_t* tm = nullptr;
    if (f3s_host_load_graph(path.c_str(), &n, &nnz, &rp, &ci, &W, &T, &wo, &bc, &tm) != 0)
        throw std::runtime_error(f3s_host_last_error());
    GraphData g;
    g.num_nodes = n;
    g.num_edges = (int)nnz;
    g.row_ptr.assign(rp, rp + n + 1);
    g.col_ind.assign(ci, ci + nnz);
    if (bsf) {
        *bsf = blockSparseFormat{};
        if (wo) {
            bsf->num_row_windows = W;
            bsf->window_offsets.assign(wo, wo + W + 1);
            bsf->block_col_indices.assign(bc, bc + T);
            if (tm) {
                bsf->tile_masks.assign(tm, tm + 16 * T);
                bsf->duplicate_entries = nnz - mask_popcount(bsf->tile_masks);
            }
        }
    }
    for (void* p : {(void*)rp, (void*)ci, (void*)wo, (void*)bc, (void*)tm}) free(p);
    return g;
}

blockSparseFormat convert_csr_to_block_sparse(int num_nodes, const std::vector<int>& row_ptr,
                                              const std::vector<int>& col_ind)
{
    if (num_nodes < 0 || row_ptr.size() != (size_t)num_nodes + 1)
        throw std::invalid_argument("convert_csr_to_block_sparse: row_ptr must hold n+1 entries");
    const int64_t nnz = (int64_t)col_ind.size();
    if (row_ptr[(size_t)num_nodes] != nnz)
        throw std::invalid_argument("convert_csr_to_block_sparse: row_ptr[n] != col_ind.size()");
    blockSparseFormat bsf;
    bsf.num_row_windows = (num_nodes + 15) / 16;
    const int W = bsf.num_row_windows;
    DevPtr rp, ci, offs, bcol, mask;
    check(f3s_malloc(&rp.p, sizeof(int) * row_ptr.size()), "f3s_malloc");
    check(f3s_malloc(&ci.p, sizeof(int) * (size_t)(nnz > 0 ? nnz : 1)), "f3s_malloc");
    check(f3s_malloc(&offs.p, sizeof(int) * ((size_t)W + 1)), "f3s_malloc");
    check(f3s_memcpy_h2d(rp.p, row_ptr.data(), sizeof(int) * row_ptr.size(), nullptr), "h2d");
    if (nnz) check(f3s_memcpy_h2d(ci.p, col_ind.data(), sizeof(int) * (size_t)nnz, nullptr), "h2d");
    int64_t T = 0;
    check(f3s_convert_csr_to_bsf((const int32_t*)rp.p, (const int32_t*)ci.p, num_nodes, nnz,
                                 (int32_t*)offs.p, nullptr, nullptr, &T, nullptr),
          "f3s_convert_csr_to_bsf (count)");
    check(f3s_malloc(&bcol.p, sizeof(int) * (size_t)(T > 0 ? T : 1)), "f3s_malloc");
    check(f3s_malloc(&mask.p, 32 * (size_t)(T > 0 ? T : 1)), "f3s_malloc");
    int64_t T2 = 0;
    check(f3s_convert_csr_to_bsf((const int32_t*)rp.p, (const int32_t*)ci.p, num_nodes, nnz,
                                 (int32_t*)offs.p, (int32_t*)bcol.p, (uint16_t*)mask.p, &T2,
                                 nullptr),
          "f3s_convert_csr_to_bsf (fill)");
    // the distinct (row, column) pairs, counted on the device
    int64_t occ = 0, mask_bits = 0;
    check(f3s_bsf_stats((const int32_t*)bcol.p, (const uint16_t*)mask.p, T, num_nodes, &occ,
                        &mask_bits, nullptr),
          "f3s_bsf_stats");
    bsf.window_offsets.resize((size_t)W + 1);
    bsf.block_col_indices.resize((size_t)T);
    bsf.tile_masks.resize((size_t)T * 16);
    check(f3s_memcpy_d2h(bsf.window_offsets.data(), offs.p, sizeof(int) * ((size_t)W + 1), nullptr),
          "d2h");
    if (T) {
        check(f3s_memcpy_d2h(bsf.block_col_indices.data(), bcol.p, sizeof(int) * (size_t)T, nullptr),
              "d2h");
        check(f3s_memcpy_d2h(bsf.tile_masks.data(), mask.p, 32 * (size_t)T, nullptr), "d2h");
    }
    bsf.duplicate_entries = nnz - mask_bits;
    std::cout << "Row Windows: " << bsf.num_row_windows << std::endl;
    std::cout << "Total Active Blocks: " << bsf.block_col_indices.size() << std::endl;
    if (bsf.duplicate_entries > 0)
        std::cerr << "convert_csr_to_block_sparse: the CSR repeats " << bsf.duplicate_entries
                  << " entries; tile lists are unaffected, masked attention counts each edge "
                     "once (cpu_sparse_attention_csr counts every repeat)"
                  << std::endl;
    return bsf;
}

std::vector<int> generate_balanced_window_order(const blockSparseFormat& format)
{
    std::vector<int> out((size_t)format.num_row_windows);
    if (format.num_row_windows > 0) {
        if (format.window_offsets.size() != (size_t)format.num_row_windows + 1)
            throw std::invalid_argument("generate_balanced_window_order: window_offsets size");
        order(format.window_offsets.data(), format.num_row_windows, out.data());
    }
    return out;
}

extern "C" {

void f3s_host_free(void* p) { free(p); }

const char* f3s_host_last_error(void) { return g_error.c_str(); }

int32_t f3s_host_load_csr(const char* dir, int32_t* n, int64_t* nnz, int32_t** row_ptr,
                          int32_t** col_idx)
{
    if (!dir || !n || !nnz || !row_ptr || !col_idx) {
        set_error("f3s_host_load_csr: NULL argument");
        return 1;
    }
    try {
        GraphData g = load(dir);
        int32_t* rp = (int32_t*)malloc(sizeof(int32_t) * g.row_ptr.size());
        int32_t* ci = (int32_t*)malloc(sizeof(int32_t) * (g.col_ind.size() + 1));
        if (!rp || !ci) {
            free(rp);
            free(ci);
            set_error("f3s_host_load_csr: out of host memory");
            return 1;
        }
        memcpy(rp, g.row_ptr.data(), sizeof(int32_t) * g.row_ptr.size());
        if (!g.col_ind.empty()) memcpy(ci, g.col_ind.data(), sizeof(int32_t) * g.col_ind.size());
        *n = g.num_nodes;
        *nnz = g.num_edges;
        *row_ptr = rp;
        *col_idx = ci;
        return 0;
    } catch (const std::exception& e) {
        set_error(e.what());
        return 1;
    }
}

int32_t f3s_host_window_order(const int32_t* window_offsets, int32_t W, int32_t* out)
{
    if (W < 0 || (W > 0 && (!window_offsets || !out))) {
        set_error("f3s_host_window_order: bad arguments");
        return 1;
    }
    order(window_offsets, W, out);
    return 0;
}

void f3s_host_f16_to_f32(const uint16_t* in, float* out, int64_t count)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        const uint32_t h = in[i];
        const uint32_t s = (h & 0x8000u) << 16;
        const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
        uint32_t x;
        if (e == 0x1fu) {
            x = s | 0x7f800000u | (m << 13);
        } else if (e == 0) {
            float f = (float)m * 0x1.0p-24f;
            memcpy(&x, &f, 4);
            x |= s;
        } else {
            x = s | ((e + 112u) << 23) | (m << 13);
        }
        memcpy(&out[i], &x, 4);
    }
}

}  // extern "C"
