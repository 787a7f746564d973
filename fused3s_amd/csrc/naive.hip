// naive.hip -- the naive, edge-exact GPU comparator of the fused pass.
//
// Semantics of f3s_naive_baseline_kernel (baselines/gpu_baseline.cu:28-116):
// one thread per node, fp32 Q/K/V/O [n][d], CSR neighbours in stored order
// (duplicate entries count twice), scores Q[i].K[j], max from -1e9
// (:67-70), exp and sum (:72-76), O[i] = sum_j (e_j / sum) V[j] (:79-100);
// a node without neighbours gets 0 (:33-38).  The reference keeps the scores
// in a per-thread device malloc (:58); here the scores are recomputed in a
// second pass instead, so nothing is allocated on the device heap.  The
// accumulator (d floats) lives in registers, hence d <= 64.
#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

constexpr int kNaiveMaxD = 64;

__global__ void __launch_bounds__(256)
naive_attention_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                       const float* __restrict__ V, float* __restrict__ O,
                       const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
                       int32_t n, int32_t d, float scale)
{
    const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t s = row_ptr[i], e = row_ptr[i + 1];
    float* o = O + (int64_t)i * d;
    if (e <= s) {
        for (int f = 0; f < d; ++f) o[f] = 0.0f;
        return;
    }
    const float* q = Q + (int64_t)i * d;
    auto score = [&](int32_t j) {
        const float* k = K + (int64_t)j * d;
        float dot = 0.0f;
        for (int f = 0; f < d; ++f) dot += q[f] * k[f];
        return dot * scale;
    };
    float mx = -1e9f;
    for (int32_t x = s; x < e; ++x) mx = fmaxf(mx, score(col_idx[x]));
    float acc[kNaiveMaxD];
#pragma unroll
    for (int f = 0; f < kNaiveMaxD; ++f) acc[f] = 0.0f;
    float sum = 0.0f;
    for (int32_t x = s; x < e; ++x) {
        const int32_t j = col_idx[x];
        const float w = expf(score(j) - mx);
        sum += w;
        const float* v = V + (int64_t)j * d;
#pragma unroll
        for (int f = 0; f < kNaiveMaxD; ++f)
            if (f < d) acc[f] += w * v[f];
    }
    const float inv = 1.0f / sum;
#pragma unroll
    for (int f = 0; f < kNaiveMaxD; ++f)
        if (f < d) o[f] = acc[f] * inv;
}

__global__ void warm_naive_kernel() {}

hipError_t warm_naive(hipStream_t s)
{
    hipLaunchKernelGGL(warm_naive_kernel, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

}  // namespace f3s

extern "C" f3s_status f3s_naive_attention_fwd(const float* Q, const float* K, const float* V,
                                              float* O, const int32_t* d_row_ptr,
                                              const int32_t* d_col_idx, int32_t n, int32_t d,
                                              float scale, void* stream)
{
    using namespace f3s;
    F3S_REQUIRE(n >= 0, "f3s_naive_attention_fwd: negative n");
    if (d < 1 || d > kNaiveMaxD) {
        set_error("f3s_naive_attention_fwd: 1 <= d <= 64 required");
        return F3S_EUNSUPPORTED;
    }
    if (n == 0) return F3S_OK;
    F3S_REQUIRE(Q && K && V && O && d_row_ptr, "f3s_naive_attention_fwd: NULL pointer");
    F3S_TRY(require_device());
    clear_error();
    hipLaunchKernelGGL(naive_attention_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0,
                       as_stream(stream), Q, K, V, O, d_row_ptr, d_col_idx, n, d, scale);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}
