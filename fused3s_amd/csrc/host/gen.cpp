// gen.cpp -- deterministic synthetic graphs and features (host, OpenMP).
//
// Every random draw is a pure function of (seed, stream id, counter): a
// SplitMix64 finaliser applied to a keyed Weyl sequence (Steele, Lea and
// Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014).
// Results therefore do not depend on the thread count or the host, which the
// parity tests rely on: the GPU and the CPU oracle see bit-identical inputs.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../../include/f3s_host.h"

namespace f3s_host {

void set_error(const std::string& s);

static inline uint64_t mix64(uint64_t z)
{
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}

struct Stream {
    uint64_t key;
    Stream(uint64_t seed, uint64_t id) : key(mix64(seed ^ mix64(id * 0xD1B54A32D192ED03ULL + 1))) {}
    uint64_t at(uint64_t i) const { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL); }
};

static inline double u01(uint64_t x) { return (double)(x >> 11) * 0x1.0p-53; }

// binary32 -> binary16 bits, round to nearest even.
static inline uint16_t to_half(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u;
    const int32_t e = (int32_t)((x >> 23) & 0xff);
    uint32_t mant = x & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(s | 0x7c00u | (mant ? 0x200u : 0u));
    const int32_t he = e - 112;   // rebias 127 -> 15
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)s;
        mant |= 0x800000u;
        const int sh = 14 - he;
        uint32_t v = mant >> sh;
        const uint32_t rem = mant & ((1u << sh) - 1u), halfway = 1u << (sh - 1);
        if (rem > halfway || (rem == halfway && (v & 1u))) ++v;
        return (uint16_t)(s | v);
    }
    uint32_t v = ((uint32_t)he << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
    return (uint16_t)(s | v);
}

// Builds a symmetric CSR with sorted unique columns from undirected pairs
// (u[k], v[k]); pairs with u == v are ignored; a self-loop per node is added
// when requested.  Deterministic: the per-row sort fixes the order.
static int build_csr(int32_t n, const std::vector<int32_t>& pu, const std::vector<int32_t>& pv,
                     bool self_loops, int32_t** row_ptr_out, int32_t** col_out, int64_t* nnz_out)
{
    const int64_t S = (int64_t)pu.size();
    std::vector<int64_t> deg(n + 1, 0);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < S; ++k) {
        if (pu[k] == pv[k]) continue;
        __atomic_fetch_add(&deg[pu[k]], 1, __ATOMIC_RELAXED);
        __atomic_fetch_add(&deg[pv[k]], 1, __ATOMIC_RELAXED);
    }
    std::vector<int64_t> start(n + 1, 0);
    for (int32_t i = 0; i < n; ++i) start[i + 1] = start[i] + deg[i];
    std::vector<int32_t> tmp((size_t)start[n] + 1);
    std::vector<int64_t> cur(start.begin(), start.end() - 1);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < S; ++k) {
        const int32_t a = pu[k], b = pv[k];
        if (a == b) continue;
        tmp[__atomic_fetch_add(&cur[a], 1, __ATOMIC_RELAXED)] = b;
        tmp[__atomic_fetch_add(&cur[b], 1, __ATOMIC_RELAXED)] = a;
    }
    std::vector<int64_t> ucount(n, 0);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int32_t i = 0; i < n; ++i) {
        int32_t* b = tmp.data() + start[i];
        int32_t* e = tmp.data() + start[i + 1];
        std::sort(b, e);
        ucount[i] = (int64_t)(std::unique(b, e) - b) + (self_loops ? 1 : 0);
    }
    int64_t total = 0;
    int32_t* rp = (int32_t*)malloc(sizeof(int32_t) * ((size_t)n + 1));
    if (!rp) return 1;
    rp[0] = 0;
    for (int32_t i = 0; i < n; ++i) {
        total += ucount[i];
        if (total > INT32_MAX) {
            free(rp);
            set_error("generated graph exceeds the int32 CSR range");
            return 1;
        }
        rp[i + 1] = (int32_t)total;
    }
    int32_t* col = (int32_t*)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    if (!col) {
        free(rp);
        return 1;
    }
#pragma omp parallel for schedule(dynamic, 1024)
    for (int32_t i = 0; i < n; ++i) {
        const int32_t* b = tmp.data() + start[i];
        const int64_t u = ucount[i] - (self_loops ? 1 : 0);
        int32_t* o = col + rp[i];
        int64_t j = 0;
        bool placed = !self_loops;
        for (int64_t x = 0; x < u; ++x) {
            if (!placed && b[x] > i) {
                o[j++] = i;
                placed = true;
            }
            o[j++] = b[x];
        }
        if (!placed) o[j++] = i;
    }
    *row_ptr_out = rp;
    *col_out = col;
    *nnz_out = total;
    return 0;
}

static int64_t count_unique_directed(int32_t n, const std::vector<int32_t>& pu,
                                     const std::vector<int32_t>& pv)
{
    int32_t *rp = nullptr, *col = nullptr;
    int64_t nnz = 0;
    if (build_csr(n, pu, pv, false, &rp, &col, &nnz) != 0) return -1;
    free(rp);
    free(col);
    return nnz;
}

}  // namespace f3s_host

using namespace f3s_host;

namespace {
// Runs `body` (which returns 0 or 1); an exception (std::bad_alloc from a
// large sample, say) becomes an error return instead of crossing the C ABI.
template <typename F>
int32_t guarded(const char* name, F&& body)
{
    try {
        return body();
    } catch (const std::exception& e) {
        set_error(std::string(name) + ": " + e.what());
        return 1;
    }
}
}  // namespace

extern "C" {

int32_t f3s_gen_powerlaw(int32_t n, int64_t target_edges, double gamma, double max_degree,
                         int32_t permute, int32_t self_loops, uint64_t seed, int32_t** row_ptr,
                         int32_t** col_idx, int64_t* nnz)
{
    if (n <= 1 || target_edges < 0 || gamma <= 1.0 || !row_ptr || !col_idx || !nnz) {
        set_error("f3s_gen_powerlaw: bad arguments");
        return 1;
    }
    return guarded("f3s_gen_powerlaw", [&]() -> int32_t {
    const double alpha = 1.0 / (gamma - 1.0);
    // Expected degree of node 0 relative to the total, from the integral of
    // x^-alpha (midpoint rule); bisection on the offset i0.
    auto top_share = [&](double i0) {
        auto F = [&](double x) {
            return fabs(alpha - 1.0) < 1e-12 ? log(x) : pow(x, 1.0 - alpha) / (1.0 - alpha);
        };
        const double lo = i0 + 0.5 > 1e-9 ? i0 + 0.5 : 1e-9;
        const double sum = pow(i0 > 1e-9 ? i0 : 1e-9, -alpha) + (F(i0 + n - 0.5) - F(lo));
        return pow(i0 > 1e-9 ? i0 : 1e-9, -alpha) / sum;
    };
    const double want = max_degree / (double)target_edges;
    double lo = 1e-3, hi = (double)n * 16.0;
    for (int it = 0; it < 200; ++it) {
        const double mid = sqrt(lo * hi);
        if (top_share(mid) > want) lo = mid; else hi = mid;
    }
    const double i0 = sqrt(lo * hi);
    std::vector<double> cdf(n);
    double acc = 0.0;
    for (int32_t i = 0; i < n; ++i) {
        acc += pow((double)i + i0, -alpha);
        cdf[i] = acc;
    }
    std::vector<int32_t> perm(n);
    for (int32_t i = 0; i < n; ++i) perm[i] = i;
    if (permute) {
        Stream ps(seed, 7);
        for (int32_t i = n - 1; i > 0; --i) {
            const int32_t j = (int32_t)(u01(ps.at((uint64_t)i)) * (double)(i + 1));
            std::swap(perm[i], perm[j < i ? j : i]);
        }
    }
    const Stream es(seed, 1);
    auto draw = [&](int64_t k, std::vector<int32_t>& pu, std::vector<int32_t>& pv) {
        const double a = u01(es.at(2 * (uint64_t)k)) * acc;
        const double b = u01(es.at(2 * (uint64_t)k + 1)) * acc;
        int32_t u = (int32_t)(std::upper_bound(cdf.begin(), cdf.end(), a) - cdf.begin());
        int32_t v = (int32_t)(std::upper_bound(cdf.begin(), cdf.end(), b) - cdf.begin());
        if (u >= n) u = n - 1;
        if (v >= n) v = n - 1;
        pu[k] = perm[u];
        pv[k] = perm[v];
    };
    // Sample pairs; top up (at most 3 times) until ~target unique directed
    // edges.  The pair list only grows, so the result is a function of the
    // final sample count.
    int64_t S = target_edges / 2;
    std::vector<int32_t> pu, pv;
    int64_t have = 0;
    for (int round = 0; round < 4; ++round) {
        const int64_t old = (int64_t)pu.size();
        pu.resize(S);
        pv.resize(S);
#pragma omp parallel for schedule(static)
        for (int64_t k = old; k < S; ++k) draw(k, pu, pv);
        if (round == 3) break;
        have = count_unique_directed(n, pu, pv);
        if (have < 0) return 1;
        if ((double)have >= 0.995 * (double)target_edges || have == 0) break;
        const double per_sample = (double)have / (double)S;
        S += (int64_t)ceil(((double)target_edges - (double)have) / per_sample);
    }
    return build_csr(n, pu, pv, self_loops != 0, row_ptr, col_idx, nnz);
    });
}

int32_t f3s_gen_sbm(int32_t n, int32_t community, double mean_degree, double p_intra,
                    int32_t self_loops, uint64_t seed, int32_t** row_ptr, int32_t** col_idx,
                    int64_t* nnz)
{
    if (n <= 1 || community <= 1 || mean_degree < 0 || p_intra < 0 || p_intra > 1 || !row_ptr ||
        !col_idx || !nnz) {
        set_error("f3s_gen_sbm: bad arguments");
        return 1;
    }
    return guarded("f3s_gen_sbm", [&]() -> int32_t {
    const int64_t S = (int64_t)((double)n * mean_degree / 2.0);
    std::vector<int32_t> pu(S), pv(S);
    const Stream es(seed, 2);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < S; ++k) {
        const int32_t u = (int32_t)(u01(es.at(3 * (uint64_t)k)) * (double)n);
        const bool intra = u01(es.at(3 * (uint64_t)k + 1)) < p_intra;
        const double y = u01(es.at(3 * (uint64_t)k + 2));
        int32_t v;
        if (intra) {
            const int32_t c0 = (u / community) * community;
            const int32_t size = std::min(community, n - c0);
            v = c0 + (int32_t)(y * (double)size);
        } else {
            v = (int32_t)(y * (double)n);
        }
        pu[k] = std::min(u, n - 1);
        pv[k] = std::min(v, n - 1);
    }
    return build_csr(n, pu, pv, self_loops != 0, row_ptr, col_idx, nnz);
    });
}

int32_t f3s_gen_features_f16(uint64_t seed, int32_t tensor, int64_t count, int32_t dist,
                             uint16_t* out)
{
    if (count < 0 || !out || tensor < 0 || tensor > 2 || (dist != 0 && dist != 1)) {
        set_error("f3s_gen_features_f16: bad arguments");
        return 1;
    }
    const Stream fs(seed, 3);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        const uint64_t x = fs.at(3 * (uint64_t)i + (uint64_t)tensor);
        float f;
        if (dist == 0) {
            f = 2.0f * ((float)(x >> 40) * 0x1.0p-24f) - 1.0f;
        } else {
            const double a = ((double)(x >> 32) + 0.5) * 0x1.0p-32;
            const double b = (double)(x & 0xffffffffu) * 0x1.0p-32;
            f = (float)(sqrt(-2.0 * log(a)) * cos(6.283185307179586 * b));
        }
        out[i] = to_half(f);
    }
    return 0;
}

}  // extern "C"
