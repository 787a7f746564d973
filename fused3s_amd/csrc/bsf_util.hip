// bsf_util.hip -- window ordering and block-sparse statistics on the GPU.
#include <rocprim/device/device_radix_sort.hpp>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

__global__ void window_counts(const int32_t* __restrict__ offs, int32_t W,
                              uint32_t* __restrict__ counts, int32_t* __restrict__ iota)
{
    const int32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    const int32_t c = offs[w + 1] - offs[w];
    counts[w] = c > 0 ? (uint32_t)c : 0u;
    iota[w] = w;
}

__global__ void __launch_bounds__(256)
bsf_stats_kernel(const int32_t* __restrict__ block_col, const uint16_t* __restrict__ tile_mask,
                 int64_t T, int32_t n, unsigned long long* __restrict__ out)
{
    __shared__ unsigned long long lds[2][256 / kWave];
    unsigned long long occ = 0, bits = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < T; t += stride) {
        const int64_t left = (int64_t)n - (int64_t)block_col[t] * 16;
        const uint32_t valid = left >= 16 ? 0xffffu : (left <= 0 ? 0u : ((1u << left) - 1u));
        if (tile_mask) {
            const uint4* mp = reinterpret_cast<const uint4*>(tile_mask + t * 16);
            const uint4 a = mp[0], b = mp[1];
            const uint32_t o = a.x | a.y | a.z | a.w | b.x | b.y | b.z | b.w;
            occ += __popc((o | (o >> 16)) & valid);
            bits += __popc(a.x) + __popc(a.y) + __popc(a.z) + __popc(a.w) + __popc(b.x) +
                    __popc(b.y) + __popc(b.z) + __popc(b.w);
        } else {
            occ += __popc(valid);
        }
    }
    occ = wave_sum(occ);
    bits = wave_sum(bits);
    const int wid = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
        lds[0][wid] = occ;
        lds[1][wid] = bits;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long a = 0, b = 0;
        for (int i = 0; i < 256 / kWave; ++i) {
            a += lds[0][i];
            b += lds[1][i];
        }
        atomicAdd(out, a);
        atomicAdd(out + 1, b);
    }
}

__global__ void warm_bsf_util_kernel() {}

hipError_t warm_bsf_util(hipStream_t s)
{
    hipLaunchKernelGGL(warm_bsf_util_kernel, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

}  // namespace f3s

using namespace f3s;

extern "C" {

f3s_status f3s_window_order(const int32_t* d_window_offsets, int32_t W, int32_t* d_order,
                            void* stream)
{
    F3S_REQUIRE(W >= 0, "f3s_window_order: negative W");
    if (W == 0) return F3S_OK;
    F3S_REQUIRE(d_window_offsets && d_order, "f3s_window_order: NULL pointer");
    F3S_TRY(require_device());
    clear_error();
    hipStream_t st = as_stream(stream);
    StreamBuffer keys_in(st), keys_out(st), vals_in(st), tmp(st);
    F3S_TRY(keys_in.reserve(sizeof(uint32_t) * (size_t)W));
    F3S_TRY(keys_out.reserve(sizeof(uint32_t) * (size_t)W));
    F3S_TRY(vals_in.reserve(sizeof(int32_t) * (size_t)W));
    auto* ki = reinterpret_cast<uint32_t*>(keys_in.ptr);
    auto* ko = reinterpret_cast<uint32_t*>(keys_out.ptr);
    auto* vi = reinterpret_cast<int32_t*>(vals_in.ptr);
    hipLaunchKernelGGL(window_counts, dim3((unsigned)ceil_div(W, 256)), dim3(256), 0, st,
                       d_window_offsets, W, ki, vi);
    F3S_HIP(hipGetLastError());
    // A window's tile count never exceeds W (one tile per block column).
    unsigned end_bit = 1;
    while (end_bit < 32 && ((uint64_t)1 << end_bit) <= (uint64_t)W) ++end_bit;
    size_t bytes = 0;
    F3S_HIP(rocprim::radix_sort_pairs_desc(nullptr, bytes, ki, ko, vi, d_order, (size_t)W, 0,
                                           end_bit, st));
    F3S_TRY(tmp.reserve(bytes));
    // Stable descending sort: equal counts keep ascending window order.
    F3S_HIP(rocprim::radix_sort_pairs_desc(tmp.ptr, bytes, ki, ko, vi, d_order, (size_t)W, 0,
                                           end_bit, st));
    F3S_HIP(hipStreamSynchronize(st));
    return F3S_OK;
}

f3s_status f3s_bsf_stats(const int32_t* d_block_col, const uint16_t* d_tile_mask, int64_t T,
                         int32_t n, int64_t* occ_sum, int64_t* mask_bits, void* stream)
{
    F3S_REQUIRE(T >= 0 && n >= 0, "f3s_bsf_stats: negative size");
    F3S_REQUIRE(occ_sum && mask_bits, "f3s_bsf_stats: NULL output");
    *occ_sum = 0;
    *mask_bits = 0;
    if (T == 0) return F3S_OK;
    F3S_REQUIRE(d_block_col != nullptr, "f3s_bsf_stats: NULL block_col");
    F3S_REQUIRE((((uintptr_t)d_tile_mask) & 15) == 0, "f3s_bsf_stats: tile_mask alignment");
    F3S_TRY(require_device());
    clear_error();
    hipStream_t st = as_stream(stream);
    StreamBuffer out(st);
    F3S_TRY(out.reserve(2 * sizeof(unsigned long long)));
    F3S_HIP(hipMemsetAsync(out.ptr, 0, 2 * sizeof(unsigned long long), st));
    int64_t blocks = ceil_div(T, 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(bsf_stats_kernel, dim3((unsigned)blocks), dim3(256), 0, st, d_block_col,
                       d_tile_mask, T, n, reinterpret_cast<unsigned long long*>(out.ptr));
    F3S_HIP(hipGetLastError());
    unsigned long long h[2] = {0, 0};
    F3S_HIP(hipMemcpyAsync(h, out.ptr, sizeof h, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    *occ_sum = (int64_t)h[0];
    *mask_bits = (int64_t)h[1];
    return F3S_OK;
}

}  // extern "C"
