// test_fused_3s.cpp -- launch/verify harness of the fused pass, the
// counterpart of the reference's tests/test_fused_3s_v2.cu:66-161.
//
// Same flow through the drop-in host API: load_csr_graph ->
// convert_csr_to_block_sparse -> generate_balanced_window_order -> seeded
// Q/K/V -> CPU ground truth -> device buffers -> fused pass (one cold
// launch timed with events, then repeated launches) -> copy back -> verify.
// Differences (deliberate): independent Q/K/V streams; both sides consume the
// same fp16-rounded inputs; the converter output is also checked bit-exact
// against the CPU oracle; the tolerance is max abs 2e-3 and normwise max rel
// 1e-2; the exit code is non-zero on failure.
//
//   test_fused_3s [dataset_dir] [--semantics masked|tile_dense] [--reps R]
//                 [--config N]   (synthetic config 1-5 instead of a directory; configs
//                 4 and 5 with their N(0,1) features, at one head as the reference)
//                 [--zero-columns]  (every column index read as 0: the graph the
//                 reference's as-shipped loader produces, include/utils.cuh:36,
//                 on which its published kernel times were measured)
//                 [--save-graph FILE]  (write the graph and its block-sparse form
//                 to a binary graph file; a dataset path ending in .f3sg is read
//                 as such a file instead of a text directory)
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <iostream>
#include <string>
#include <thread>
#include <vector>

#include "f3s/graph.hpp"
#include "f3s_capi.h"
#include "f3s_host.h"
#include "f3s_oracle.h"

namespace {

struct Dev {
    void* p = nullptr;
    explicit Dev(size_t bytes) { F3S_CHECK(f3s_malloc(&p, bytes ? bytes : 1)); }
    ~Dev() { f3s_free(p); }
    template <typename T>
    T* as() const { return static_cast<T*>(p); }
};

GraphData synthetic(int cfg)
{
    int32_t* rp = nullptr;
    int32_t* ci = nullptr;
    int64_t nnz = 0;
    int32_t n = 0, rc = 1;
    if (cfg == 1 || cfg == 2) {
        n = 2708;
        rc = f3s_gen_powerlaw(n, 10556, 2.5, 170, 1, 1, 42, &rp, &ci, &nnz);
    } else if (cfg == 3) {
        n = 3327;
        rc = f3s_gen_powerlaw(n, 9104, 2.8, 99, 1, 1, 43, &rp, &ci, &nnz);
    } else if (cfg == 4) {
        n = 1000000;
        rc = f3s_gen_powerlaw(n, 16000000, 2.2, 16384, 1, 1, 44, &rp, &ci, &nnz);
    } else if (cfg == 5) {
        n = 2400000;
        rc = f3s_gen_sbm(n, 4096, 50.0, 0.8, 1, 45, &rp, &ci, &nnz);
    }
    if (rc != 0) {
        std::cerr << "cannot generate config " << cfg << ": " << f3s_host_last_error() << std::endl;
        exit(EXIT_FAILURE);
    }
    GraphData g;
    g.num_nodes = n;
    g.num_edges = (int)nnz;
    g.row_ptr.assign(rp, rp + n + 1);
    g.col_ind.assign(ci, ci + nnz);
    f3s_host_free(rp);
    f3s_host_free(ci);
    return g;
}

}  // namespace

int main(int argc, char** argv)
{
    std::string dataset_path = "tests/golden/cora";
    bool masked = true;
    int reps = 20, cfg = 0;
    bool zero_columns = false;
    std::string save_path;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        if (a == "--semantics" && i + 1 < argc) masked = std::string(argv[++i]) != "tile_dense";
        else if (a == "--reps" && i + 1 < argc) reps = atoi(argv[++i]);
        else if (a == "--config" && i + 1 < argc) cfg = atoi(argv[++i]);
        else if (a == "--zero-columns") zero_columns = true;
        else if (a == "--save-graph" && i + 1 < argc) save_path = argv[++i];
        else dataset_path = a;
    }
    const int feat_dim = 64;
    int32_t ndev = 0;
    f3s_device_count(&ndev);
    if (ndev < 1) {
        std::cerr << "FAILURE: no GPU visible (the fused pass runs only on the GPU)" << std::endl;
        return 2;
    }

    F3S_CHECK(f3s_init());   // load the GPU code before the first (cold) timed launch
    std::cout << "=== fused3s_amd (gfx950) " << (masked ? "masked" : "tile-dense") << " ===" << std::endl;
    GraphData graph;
    try {
        if (cfg) {
            std::cout << "Synthetic config " << cfg << std::endl;
            graph = synthetic(cfg);
        } else {
            std::cout << "Loading graph from: " << dataset_path << std::endl;
            const std::string ext = ".f3sg";
            const bool binary = dataset_path.size() > ext.size() &&
                                dataset_path.compare(dataset_path.size() - ext.size(),
                                                     ext.size(), ext) == 0;
            graph = binary ? load_graph_binary(dataset_path) : load_csr_graph(dataset_path);
        }
    } catch (const std::exception& e) {
        std::cerr << "FAILURE: " << e.what() << std::endl;
        return 1;
    }
    if (zero_columns) std::fill(graph.col_ind.begin(), graph.col_ind.end(), 0);
    const int n = graph.num_nodes;
    blockSparseFormat format = convert_csr_to_block_sparse(n, graph.row_ptr, graph.col_ind);
    std::vector<int> window_order = generate_balanced_window_order(format);
    if (!save_path.empty()) {
        try {
            save_graph_binary(save_path, graph, &format);
            std::cout << "Saved graph file: " << save_path << std::endl;
        } catch (const std::exception& e) {
            std::cerr << "FAILURE: " << e.what() << std::endl;
            return 1;
        }
    }
    const int W = format.num_row_windows;
    const int64_t T = (int64_t)format.block_col_indices.size();

    // Converter bit-exact against the CPU restatement.
    std::vector<int32_t> o_offs(W + 1), o_bcol(T > 0 ? T : 1);
    std::vector<uint16_t> o_mask((T > 0 ? T : 1) * 16);
    int64_t oT = orc_convert_count(n, graph.row_ptr.data(), graph.col_ind.data(), o_offs.data());
    orc_convert_fill(n, graph.row_ptr.data(), graph.col_ind.data(), o_offs.data(), o_bcol.data(),
                     o_mask.data());
    bool conv_ok = oT == T &&
                   memcmp(o_offs.data(), format.window_offsets.data(), 4 * (W + 1)) == 0 &&
                   memcmp(o_bcol.data(), format.block_col_indices.data(), 4 * T) == 0 &&
                   memcmp(o_mask.data(), format.tile_masks.data(), 32 * T) == 0;
    std::cout << "Converter vs CPU oracle: " << (conv_ok ? "bit-exact" : "MISMATCH") << std::endl;

    // Seeded fp16 inputs; the CPU truth widens the same fp16 values.
    const size_t feat = (size_t)n * feat_dim;
    std::vector<uint16_t> hQ(feat), hK(feat), hV(feat);
    const int dist = cfg >= 4 ? 1 : 0;                  // N(0, 1) for configs 4, 5; else U[-1, 1)
    const uint64_t seed = cfg >= 4 ? (uint64_t)(40 + cfg) : 42;
    if (f3s_gen_features_f16(seed, 0, (int64_t)feat, dist, hQ.data()) ||
        f3s_gen_features_f16(seed, 1, (int64_t)feat, dist, hK.data()) ||
        f3s_gen_features_f16(seed, 2, (int64_t)feat, dist, hV.data())) {
        std::cerr << "FAILURE: feature generation" << std::endl;
        return 1;
    }
    std::vector<float> fQ(feat), fK(feat), fV(feat), O_cpu(feat, 0.f), O_gpu(feat, 0.f);
    orc_cast_f16_to_f32(hQ.data(), fQ.data(), (int64_t)feat);
    orc_cast_f16_to_f32(hK.data(), fK.data(), (int64_t)feat);
    orc_cast_f16_to_f32(hV.data(), fV.data(), (int64_t)feat);

    // the truth on the host's cores (at most 16, a one-GPU box's share)
    const int threads = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::cout << "Computing CPU ground truth (" << threads << " threads)..." << std::endl;
    if (masked)
        orc_masked_attention(n, feat_dim, 1, fQ.data(), fK.data(), fV.data(), graph.row_ptr.data(),
                             graph.col_ind.data(), 1.0f, 0, n, O_cpu.data(), threads);
    else
        orc_tile_dense_attention(n, feat_dim, 1, fQ.data(), fK.data(), fV.data(),
                                 format.window_offsets.data(), format.block_col_indices.data(),
                                 1.0f, 0, n, O_cpu.data(), threads);

    Dev dQ(2 * feat), dK(2 * feat), dV(2 * feat), dO(4 * feat);
    Dev dOffs(4 * (W + 1)), dBcol(4 * (T > 0 ? T : 1)), dMask(32 * (T > 0 ? T : 1)), dOrder(4 * (W > 0 ? W : 1));
    F3S_CHECK(f3s_memcpy_h2d(dQ.p, hQ.data(), 2 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dK.p, hK.data(), 2 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dV.p, hV.data(), 2 * feat, nullptr));
    F3S_CHECK(f3s_memset(dO.p, 0, 4 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dOffs.p, format.window_offsets.data(), 4 * (W + 1), nullptr));
    if (T) {
        F3S_CHECK(f3s_memcpy_h2d(dBcol.p, format.block_col_indices.data(), 4 * T, nullptr));
        F3S_CHECK(f3s_memcpy_h2d(dMask.p, format.tile_masks.data(), 32 * T, nullptr));
    }
    if (W) F3S_CHECK(f3s_memcpy_h2d(dOrder.p, window_order.data(), 4 * W, nullptr));

    void *ev0 = nullptr, *ev1 = nullptr;
    F3S_CHECK(f3s_event_create(&ev0));
    F3S_CHECK(f3s_event_create(&ev1));
    auto launch = [&]() {
        F3S_CHECK(f3s_attention_fwd(dQ.as<uint16_t>(), dK.as<uint16_t>(), dV.as<uint16_t>(),
                                    dO.as<float>(), dOffs.as<int32_t>(), dBcol.as<int32_t>(),
                                    masked ? dMask.as<uint16_t>() : nullptr, dOrder.as<int32_t>(),
                                    W, n, feat_dim, 1, 1.0f, nullptr));
    };
    std::cout << "Launching fused kernel (" << W << " row windows)..." << std::endl;
    F3S_CHECK(f3s_event_record(ev0, nullptr));
    launch();
    F3S_CHECK(f3s_event_record(ev1, nullptr));
    float cold_ms = 0.f;
    F3S_CHECK(f3s_event_elapsed_ms(ev0, ev1, &cold_ms));
    std::cout << "Kernel Time (cold): " << cold_ms << " ms" << std::endl;
    if (reps > 0) {
        float us = 0.f;
        F3S_CHECK(f3s_attention_fwd_timed(dQ.as<uint16_t>(), dK.as<uint16_t>(),
                                          dV.as<uint16_t>(), dO.as<float>(), dOffs.as<int32_t>(),
                                          dBcol.as<int32_t>(),
                                          masked ? dMask.as<uint16_t>() : nullptr,
                                          dOrder.as<int32_t>(), W, n, feat_dim, 1, 1.0f, nullptr,
                                          reps, &us));
        const double ms = us * 1e-3;
        std::cout << "Kernel Time (mean of " << reps << "): " << ms << " ms, "
                  << (double)graph.num_edges / (ms * 1e-3) << " edges/s" << std::endl;
    }
    F3S_CHECK(f3s_memcpy_d2h(O_gpu.data(), dO.p, 4 * feat, nullptr));
    f3s_event_destroy(ev0);
    f3s_event_destroy(ev1);

    double max_abs = 0.0, max_ref = 0.0;
    int mismatches = 0;
    for (size_t i = 0; i < feat; ++i) {
        double dlt = fabs((double)O_cpu[i] - (double)O_gpu[i]);
        if (!(dlt <= 2e-3)) {
            if (++mismatches <= 5)
                std::cerr << "MISMATCH [" << i / feat_dim << "," << i % feat_dim << "]: cpu=" << O_cpu[i]
                          << " gpu=" << O_gpu[i] << std::endl;
        }
        if (!(dlt <= max_abs)) max_abs = dlt;
        max_ref = fmax(max_ref, fabs((double)O_cpu[i]));
    }
    const double max_rel = max_ref > 0 ? max_abs / max_ref : max_abs;
    std::cout << "max_abs=" << max_abs << " max_rel=" << max_rel << std::endl;
    const bool passed = conv_ok && max_abs <= 2e-3 && max_rel <= 1e-2;
    std::cout << (passed ? "SUCCESS" : "FAILURE") << std::endl;
    return passed ? 0 : 1;
}
