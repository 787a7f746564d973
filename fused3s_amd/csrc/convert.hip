// convert.hip -- CSR -> 16x16 block-sparse conversion on the GPU.
//
// Semantics of convert_csr_to_block_sparse (src/converter.cu:13-44): W =
// ceil(n/16) row windows (:15); for window w the ascending unique set of
// c/16 over the edges (u, c) of rows [16w, min(16w+16, n)) (:19-36);
// window_offsets = exclusive prefix of the set sizes (:39).  New output: the
// 16 row masks of each tile (bit c of row r <=> edge (16w+r, 16b+c)).
//
// Design (one workgroup of 256 threads per window):
//   * windows with E <= kCap edges: keys (blockcol, row, col%16) are built in
//     LDS, bitonic-sorted, and tile heads (first key of each block column) are
//     counted (pass 1) or compacted in order with their masks (pass 2);
//   * heavier (hub) windows: the block-column range is swept in slices of
//     kRange tiles; each slice ORs edge bits into LDS masks with LDS atomics,
//     then non-empty tiles are counted / compacted in ascending order.
// Both paths give the same, deterministic output.  Counts are scanned into
// window_offsets with the device scan of runtime.hip.
#include <stdio.h>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

constexpr int kConvThreads = 256;
constexpr int kLdsBytes = 32768;   // key buffer / slice masks
constexpr int kRange = kLdsBytes / 32;   // tiles per slice in the hub path

enum ConvErr : int32_t { kErrNone = 0, kErrRowPtr = 1, kErrCol = 2, kErrCount = 4 };

template <typename Key>
struct KeyTraits;
template <>
struct KeyTraits<uint32_t> {
    static constexpr int kCap = kLdsBytes / 4;
    static __device__ __forceinline__ uint32_t pad() { return 0xffffffffu; }
};
template <>
struct KeyTraits<uint64_t> {
    static constexpr int kCap = kLdsBytes / 8;
    static __device__ __forceinline__ uint64_t pad() { return ~0ull; }
};

struct WindowRows {
    int32_t u0, nrows;
    int64_t e0, E;
};

// Loads the window's row pointers into LDS and validates them.
__device__ __forceinline__ WindowRows load_window_rows(const int32_t* __restrict__ row_ptr,
                                                       int32_t n, int64_t nnz, int32_t w,
                                                       int32_t* rp, int32_t* err)
{
    WindowRows wr;
    wr.u0 = w * 16;
    wr.nrows = min(16, n - wr.u0);
    if ((int)threadIdx.x <= wr.nrows) rp[threadIdx.x] = row_ptr[wr.u0 + threadIdx.x];
    __syncthreads();
    if ((int)threadIdx.x < wr.nrows) {
        int32_t a = rp[threadIdx.x], b = rp[threadIdx.x + 1];
        if (a < 0 || b < a || b > nnz) *err = kErrRowPtr;
    }
    wr.e0 = rp[0];
    wr.E = (int64_t)rp[wr.nrows] - wr.e0;
    return wr;
}

__device__ __forceinline__ int row_of_edge(const int32_t* rp, int nrows, int64_t e)
{
    int r = 0;
    while (r + 1 < nrows && e >= rp[r + 1]) ++r;
    return r;
}

// Pass kind: COUNT writes counts[w]; FILL writes block_col / tile_mask at
// window_offsets[w] and checks the count against the offsets.
template <typename Key, bool FILL>
__global__ void __launch_bounds__(kConvThreads)
convert_windows(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
                int32_t n, int64_t nnz, int32_t W, int32_t* __restrict__ counts,
                const int32_t* __restrict__ window_offsets, int32_t* __restrict__ block_col,
                uint16_t* __restrict__ tile_mask, int32_t* __restrict__ err)
{
    using Tr = KeyTraits<Key>;
    __shared__ __align__(16) unsigned char lds_raw[kLdsBytes];
    __shared__ int32_t rp[17];
    __shared__ int32_t scan_lds[kConvThreads / kWave];
    __shared__ int32_t bad;

    const int32_t w = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid == 0) bad = 0;
    WindowRows wr = load_window_rows(row_ptr, n, nnz, w, rp, err);
    __syncthreads();
    if (wr.E < 0 || wr.e0 < 0 || wr.e0 + wr.E > nnz) {
        if (tid == 0) *err = kErrRowPtr;
        return;
    }
    int32_t out_base = 0, expect = 0;
    if (FILL) {
        // The caller's offsets must describe this CSR (checked against the
        // tile count found below) and stay inside [0, window_offsets[W]],
        // the size of block_col / tile_mask.
        const int32_t total = window_offsets[W];
        out_base = window_offsets[w];
        expect = window_offsets[w + 1] - out_base;
        if (out_base < 0 || expect < 0 || out_base > total - expect) {
            if (tid == 0) *err = kErrCount;
            return;
        }
    }

    int32_t found = 0;   // tiles of this window (meaningful in thread 0 / all after scans)
    if (wr.E <= Tr::kCap) {
        Key* keys = reinterpret_cast<Key*>(lds_raw);
        const int E = (int)wr.E;
        int P = 1;
        while (P < E) P <<= 1;
        for (int i = tid; i < P; i += kConvThreads) {
            Key k = Tr::pad();
            if (i < E) {
                const int64_t e = wr.e0 + i;
                const int32_t c = col_idx[e];
                if (c < 0 || c >= n) {
                    bad = 1;
                } else {
                    const int r = row_of_edge(rp, wr.nrows, e);
                    k = ((Key)(uint32_t)(c >> 4) << 8) | (Key)(r << 4) | (Key)(c & 15);
                }
            }
            keys[i] = k;
        }
        __syncthreads();
        // Bitonic sort, ascending.
        for (int k = 2; k <= P; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = tid; i < P / 2; i += kConvThreads) {
                    const int lo = 2 * i - (i & (j - 1));
                    const int hi = lo + j;
                    const bool up = (lo & k) == 0;
                    Key a = keys[lo], b = keys[hi];
                    if ((a > b) == up) {
                        keys[lo] = b;
                        keys[hi] = a;
                    }
                }
                __syncthreads();
            }
        }
        // Each thread owns a contiguous run of sorted keys.
        const int per = (E + kConvThreads - 1) / kConvThreads;
        const int s0 = min(E, tid * per), s1 = min(E, s0 + per);
        int local = 0;
        for (int i = s0; i < s1; ++i)
            local += (i == 0) || ((keys[i] >> 8) != (keys[i - 1] >> 8));
        int32_t total;
        int32_t before = block_exclusive_scan<kConvThreads>(local, scan_lds, total);
        found = total;
        if (FILL && total == expect) {
            int t = before;
            for (int i = s0; i < s1; ++i) {
                const Key bc = keys[i] >> 8;
                if (i != 0 && bc == (keys[i - 1] >> 8)) continue;
                uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int j = i; j < E && (keys[j] >> 8) == bc; ++j) {
                    const uint32_t r = (uint32_t)(keys[j] >> 4) & 15u;
                    const uint32_t c = (uint32_t)keys[j] & 15u;
                    m[r >> 1] |= (1u << c) << (16 * (r & 1));
                }
                const int64_t o = (int64_t)out_base + t;
                block_col[o] = (int32_t)bc;
                if (tile_mask) {
                    uint4* dst = reinterpret_cast<uint4*>(tile_mask + o * 16);
                    dst[0] = make_uint4(m[0], m[1], m[2], m[3]);
                    dst[1] = make_uint4(m[4], m[5], m[6], m[7]);
                }
                ++t;
            }
        }
    } else {
        // Hub window: sweep block columns in slices of kRange tiles.
        uint32_t* masks = reinterpret_cast<uint32_t*>(lds_raw);   // kRange x 8 words
        int32_t running = 0;
        for (int32_t lo = 0; lo < W; lo += kRange) {
            for (int i = tid; i < kRange * 8; i += kConvThreads) masks[i] = 0u;
            __syncthreads();
            for (int64_t i = tid; i < wr.E; i += kConvThreads) {
                const int64_t e = wr.e0 + i;
                const int32_t c = col_idx[e];
                if (c < 0 || c >= n) {
                    bad = 1;
                    continue;
                }
                const int32_t bc = c >> 4;
                if (bc < lo || bc >= lo + kRange) continue;
                const int r = row_of_edge(rp, wr.nrows, e);
                atomicOr(&masks[(bc - lo) * 8 + (r >> 1)], (1u << (c & 15)) << (16 * (r & 1)));
            }
            __syncthreads();
            constexpr int kPer = kRange / kConvThreads;
            int local = 0;
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                const int ti = tid * kPer + q;
                const uint32_t* mm = masks + ti * 8;
                local += (mm[0] | mm[1] | mm[2] | mm[3] | mm[4] | mm[5] | mm[6] | mm[7]) != 0u;
            }
            int32_t total;
            int32_t before = block_exclusive_scan<kConvThreads>(local, scan_lds, total);
            if (FILL && running + total <= expect) {
                int t = running + before;
#pragma unroll
                for (int q = 0; q < kPer; ++q) {
                    const int ti = tid * kPer + q;
                    const uint32_t* mm = masks + ti * 8;
                    if ((mm[0] | mm[1] | mm[2] | mm[3] | mm[4] | mm[5] | mm[6] | mm[7]) == 0u)
                        continue;
                    const int64_t o = (int64_t)out_base + t;
                    block_col[o] = lo + ti;
                    if (tile_mask) {
                        uint4* dst = reinterpret_cast<uint4*>(tile_mask + o * 16);
                        dst[0] = make_uint4(mm[0], mm[1], mm[2], mm[3]);
                        dst[1] = make_uint4(mm[4], mm[5], mm[6], mm[7]);
                    }
                    ++t;
                }
            }
            running += total;
            __syncthreads();   // masks are cleared by the next slice
        }
        found = running;
    }
    __syncthreads();
    if (tid == 0) {
        if (bad) *err = kErrCol;
        if (FILL) {
            if (found != expect) *err = kErrCount;
        } else {
            counts[w] = found;
        }
    }
}

__global__ void offsets_to_i32(const int64_t* __restrict__ in, int32_t* __restrict__ out,
                               int64_t count)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = (int32_t)in[i];
}

// Per-call workspace of the converter (counts, scan temporaries, flags).
struct ConvertScratch {
    DeviceBuffer counts, offs64, tmp, flags;
};

static f3s_status convert_impl(const int32_t* row_ptr, const int32_t* col_idx, int32_t n,
                               int64_t nnz, int32_t* window_offsets, int32_t* block_col,
                               uint16_t* tile_mask, int64_t* T_out, hipStream_t stream)
{
    const int32_t W = (int32_t)ceil_div(n, 16);
    ConvertScratch s;
    F3S_TRY(s.flags.reserve(sizeof(int32_t) * 2 + sizeof(int64_t)));
    int32_t* err = reinterpret_cast<int32_t*>(s.flags.ptr);
    F3S_HIP(hipMemsetAsync(err, 0, sizeof(int32_t), stream));

    const bool wide = W > (1 << 24) - 1;
    if (!block_col) {
        F3S_TRY(s.counts.reserve(sizeof(int32_t) * (size_t)W));
        F3S_TRY(s.offs64.reserve(sizeof(int64_t) * ((size_t)W + 1)));
        F3S_TRY(s.tmp.reserve(sizeof(int64_t) * (size_t)scan_tmp_elems(W)));
        int32_t* counts = reinterpret_cast<int32_t*>(s.counts.ptr);
        if (W > 0) {
            if (wide)
                hipLaunchKernelGGL((convert_windows<uint64_t, false>), dim3(W),
                                   dim3(kConvThreads), 0, stream, row_ptr, col_idx, n, nnz, W,
                                   counts, nullptr, nullptr, nullptr, err);
            else
                hipLaunchKernelGGL((convert_windows<uint32_t, false>), dim3(W),
                                   dim3(kConvThreads), 0, stream, row_ptr, col_idx, n, nnz, W,
                                   counts, nullptr, nullptr, nullptr, err);
            F3S_HIP(hipGetLastError());
        }
        int64_t* offs64 = reinterpret_cast<int64_t*>(s.offs64.ptr);
        F3S_TRY(exclusive_scan_i32_to_i64(counts, offs64, W,
                                          reinterpret_cast<int64_t*>(s.tmp.ptr), stream));
        int32_t h_err = 0;
        int64_t total = 0;
        F3S_HIP(hipMemcpyAsync(&h_err, err, sizeof h_err, hipMemcpyDeviceToHost, stream));
        F3S_HIP(hipMemcpyAsync(&total, offs64 + W, sizeof total, hipMemcpyDeviceToHost, stream));
        F3S_HIP(hipStreamSynchronize(stream));
        if (h_err & kErrRowPtr) {
            set_error("f3s_convert_csr_to_bsf: row_ptr is not monotone within [0, nnz]");
            return F3S_EDATA;
        }
        if (h_err & kErrCol) {
            set_error("f3s_convert_csr_to_bsf: a column index is outside [0, n)");
            return F3S_EDATA;
        }
        if (total > INT32_MAX) {
            set_error("f3s_convert_csr_to_bsf: more than 2^31-1 active tiles");
            return F3S_EUNSUPPORTED;
        }
        hipLaunchKernelGGL(offsets_to_i32, dim3((unsigned)ceil_div(W + 1, 256)), dim3(256), 0,
                           stream, offs64, window_offsets, (int64_t)W + 1);
        F3S_HIP(hipGetLastError());
        F3S_HIP(hipStreamSynchronize(stream));
        *T_out = total;
        return F3S_OK;
    }

    if (W > 0) {
        if (wide)
            hipLaunchKernelGGL((convert_windows<uint64_t, true>), dim3(W), dim3(kConvThreads), 0,
                               stream, row_ptr, col_idx, n, nnz, W, nullptr, window_offsets,
                               block_col, tile_mask, err);
        else
            hipLaunchKernelGGL((convert_windows<uint32_t, true>), dim3(W), dim3(kConvThreads), 0,
                               stream, row_ptr, col_idx, n, nnz, W, nullptr, window_offsets,
                               block_col, tile_mask, err);
        F3S_HIP(hipGetLastError());
    }
    int32_t h_err = 0, total = 0;
    F3S_HIP(hipMemcpyAsync(&h_err, err, sizeof h_err, hipMemcpyDeviceToHost, stream));
    F3S_HIP(hipMemcpyAsync(&total, window_offsets + W, sizeof total, hipMemcpyDeviceToHost,
                           stream));
    F3S_HIP(hipStreamSynchronize(stream));
    if (h_err & (kErrRowPtr | kErrCol)) {
        set_error("f3s_convert_csr_to_bsf: CSR violates the format (row_ptr or column range)");
        return F3S_EDATA;
    }
    if (h_err & kErrCount) {
        set_error("f3s_convert_csr_to_bsf: window_offsets do not match this CSR "
                  "(call once with d_block_col = NULL first)");
        return F3S_EINVAL;
    }
    *T_out = total;
    return F3S_OK;
}

__global__ void warm_convert_kernel() {}

hipError_t warm_convert(hipStream_t s)
{
    hipLaunchKernelGGL(warm_convert_kernel, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

}  // namespace f3s

extern "C" f3s_status f3s_convert_csr_to_bsf(const int32_t* d_row_ptr, const int32_t* d_col_idx,
                                             int32_t n, int64_t nnz, int32_t* d_window_offsets,
                                             int32_t* d_block_col, uint16_t* d_tile_mask,
                                             int64_t* T_out, void* stream)
{
    using namespace f3s;
    F3S_REQUIRE(n >= 0 && nnz >= 0, "f3s_convert_csr_to_bsf: negative size");
    F3S_REQUIRE(nnz <= INT32_MAX, "f3s_convert_csr_to_bsf: nnz exceeds int32 CSR range");
    F3S_REQUIRE(d_row_ptr && d_window_offsets && T_out, "f3s_convert_csr_to_bsf: NULL pointer");
    F3S_REQUIRE(nnz == 0 || d_col_idx, "f3s_convert_csr_to_bsf: NULL col_idx");
    F3S_REQUIRE(!d_tile_mask || d_block_col,
                "f3s_convert_csr_to_bsf: tile_mask requires block_col");
    F3S_TRY(require_device());
    clear_error();
    return convert_impl(d_row_ptr, d_col_idx, n, nnz, d_window_offsets, d_block_col,
                        d_tile_mask, T_out, as_stream(stream));
}
