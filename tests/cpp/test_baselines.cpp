// test_baselines.cpp -- the baseline harness, counterpart of the reference's
// tests/test_baselines.cu:37-138: load a graph, time the CPU edge-exact
// attention (one call, steady clock, as :82-89), run the naive GPU comparator
// (one warm-up launch, then a timed launch, as :100-116), verify within
// 1e-4 (:27) and print the speedup.  Differences (deliberate): Q, K and V are
// independent draws unless --same-qkv reproduces the reference's three
// identically seeded matrices (:56-58); the exit code is non-zero on failure;
// the fused fp16 pass on the same graph is timed as well, for reference.
//
//   test_baselines [dataset_dir] [--same-qkv]
#include <math.h>

#include <chrono>
#include <iostream>
#include <string>
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
};
}  // namespace

int main(int argc, char** argv)
{
    std::string dataset_path = "tests/golden/citeseer";
    bool same_qkv = false;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        if (a == "--same-qkv") same_qkv = true;
        else dataset_path = a;
    }
    const int feat_dim = 64;
    int32_t ndev = 0;
    f3s_device_count(&ndev);
    if (ndev < 1) {
        std::cerr << "FAILURE: no GPU visible" << std::endl;
        return 2;
    }
    F3S_CHECK(f3s_init());

    std::cout << "Loading graph from: " << dataset_path << std::endl;
    GraphData graph;
    try {
        graph = load_csr_graph(dataset_path);
    } catch (const std::exception& e) {
        std::cerr << "FAILURE: " << e.what() << std::endl;
        return 1;
    }
    const int n = graph.num_nodes;
    std::cout << "Nodes: " << n << ", Edges: " << graph.num_edges << std::endl;
    const size_t feat = (size_t)n * feat_dim;

    // fp32 inputs in U[-1, 1) (the reference draws U(-1, 1), :20), taken as
    // the fp32 widening of fp16 draws so the fused pass sees the same values.
    std::vector<uint16_t> h16(3 * feat);
    for (int t = 0; t < 3; ++t)
        if (f3s_gen_features_f16(42, same_qkv ? 0 : t, (int64_t)feat, 0, h16.data() + t * feat)) {
            std::cerr << "FAILURE: feature generation" << std::endl;
            return 1;
        }
    std::vector<float> f32(3 * feat);
    orc_cast_f16_to_f32(h16.data(), f32.data(), (int64_t)(3 * feat));
    const float* hQ = f32.data();
    const float* hK = f32.data() + feat;
    const float* hV = f32.data() + 2 * feat;
    std::vector<float> out_cpu(feat, 0.f), out_gpu(feat, 0.f), out_fused(feat, 0.f);

    std::cout << "\n=== SPARSE ATTENTION BASELINE ===" << std::endl;
    auto t0 = std::chrono::steady_clock::now();
    orc_masked_attention(n, feat_dim, 1, hQ, hK, hV, graph.row_ptr.data(), graph.col_ind.data(),
                         1.0f, 0, n, out_cpu.data(), 1);
    auto t1 = std::chrono::steady_clock::now();
    const double cpu_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    std::cout << "CPU Sparse Attention Time (1 thread): " << cpu_ms << " ms" << std::endl;

    Dev dQ(4 * feat), dK(4 * feat), dV(4 * feat), dO(4 * feat);
    Dev dRp(4 * (n + 1)), dCi(4 * (size_t)graph.num_edges);
    F3S_CHECK(f3s_memcpy_h2d(dQ.p, hQ, 4 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dK.p, hK, 4 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dV.p, hV, 4 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dRp.p, graph.row_ptr.data(), 4 * (n + 1), nullptr));
    if (graph.num_edges)
        F3S_CHECK(f3s_memcpy_h2d(dCi.p, graph.col_ind.data(), 4 * (size_t)graph.num_edges, nullptr));
    auto naive = [&]() {
        F3S_CHECK(f3s_naive_attention_fwd((const float*)dQ.p, (const float*)dK.p,
                                          (const float*)dV.p, (float*)dO.p,
                                          (const int32_t*)dRp.p, (const int32_t*)dCi.p, n,
                                          feat_dim, 1.0f, nullptr));
    };
    void *e0 = nullptr, *e1 = nullptr;
    F3S_CHECK(f3s_event_create(&e0));
    F3S_CHECK(f3s_event_create(&e1));
    std::cout << "\nRunning GPU naive sparse attention..." << std::endl;
    naive();                                      // warm-up
    F3S_CHECK(f3s_synchronize(nullptr));
    F3S_CHECK(f3s_memset(dO.p, 0, 4 * feat, nullptr));
    F3S_CHECK(f3s_event_record(e0, nullptr));
    naive();
    F3S_CHECK(f3s_event_record(e1, nullptr));
    float naive_ms = 0.f;
    F3S_CHECK(f3s_event_elapsed_ms(e0, e1, &naive_ms));
    std::cout << "GPU Naive Time: " << naive_ms << " ms" << std::endl;
    F3S_CHECK(f3s_memcpy_d2h(out_gpu.data(), dO.p, 4 * feat, nullptr));

    // the fused fp16 pass on the same graph (masked = edge-exact semantics)
    blockSparseFormat fmt = convert_csr_to_block_sparse(n, graph.row_ptr, graph.col_ind);
    const int W = fmt.num_row_windows;
    const size_t T = fmt.block_col_indices.size();
    Dev dQ16(2 * feat), dK16(2 * feat), dV16(2 * feat), dOffs(4 * (W + 1)), dB(4 * (T ? T : 1)),
        dM(32 * (T ? T : 1));
    F3S_CHECK(f3s_memcpy_h2d(dQ16.p, h16.data(), 2 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dK16.p, h16.data() + feat, 2 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dV16.p, h16.data() + 2 * feat, 2 * feat, nullptr));
    F3S_CHECK(f3s_memcpy_h2d(dOffs.p, fmt.window_offsets.data(), 4 * (W + 1), nullptr));
    if (T) {
        F3S_CHECK(f3s_memcpy_h2d(dB.p, fmt.block_col_indices.data(), 4 * T, nullptr));
        F3S_CHECK(f3s_memcpy_h2d(dM.p, fmt.tile_masks.data(), 32 * T, nullptr));
    }
    auto fused = [&]() {
        F3S_CHECK(f3s_attention_fwd((const uint16_t*)dQ16.p, (const uint16_t*)dK16.p,
                                    (const uint16_t*)dV16.p, (float*)dO.p, (const int32_t*)dOffs.p,
                                    (const int32_t*)dB.p, (const uint16_t*)dM.p, nullptr, W, n,
                                    feat_dim, 1, 1.0f, nullptr));
    };
    fused();
    F3S_CHECK(f3s_event_record(e0, nullptr));
    fused();
    F3S_CHECK(f3s_event_record(e1, nullptr));
    float fused_ms = 0.f;
    F3S_CHECK(f3s_event_elapsed_ms(e0, e1, &fused_ms));
    std::cout << "GPU Fused (fp16, MFMA) Time: " << fused_ms << " ms" << std::endl;
    F3S_CHECK(f3s_memcpy_d2h(out_fused.data(), dO.p, 4 * feat, nullptr));
    f3s_event_destroy(e0);
    f3s_event_destroy(e1);

    bool ok = true;
    double worst = 0.0, worst_fused = 0.0;
    for (size_t i = 0; i < feat; ++i) {
        const double dd = fabs((double)out_cpu[i] - (double)out_gpu[i]);
        worst = dd > worst ? dd : worst;
        const double df = fabs((double)out_cpu[i] - (double)out_fused[i]);
        worst_fused = df > worst_fused ? df : worst_fused;
        if (!(dd <= 1e-4)) {
            if (ok)
                std::cerr << "Mismatch at index " << i << ": CPU=" << out_cpu[i]
                          << ", GPU=" << out_gpu[i] << std::endl;
            ok = false;
        }
    }
    ok = ok && worst_fused <= 2e-3;
    std::cout << "max |naive - cpu| = " << worst << ", max |fused - cpu| = " << worst_fused
              << std::endl;
    if (ok) {
        std::cout << "\nSUCCESS: GPU results match CPU baseline!" << std::endl;
        std::cout << "Speedup naive: " << cpu_ms / naive_ms << "x, fused: " << cpu_ms / fused_ms
                  << "x" << std::endl;
    } else {
        std::cout << "\nFAILURE: GPU results do not match." << std::endl;
    }
    return ok ? 0 : 1;
}
