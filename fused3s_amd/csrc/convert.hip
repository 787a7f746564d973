// convert.hip -- CSR -> 16x16 block-sparse conversion on the GPU.
//
// Semantics of convert_csr_to_block_sparse (src/converter.cu:13-44): W =
// ceil(n/16) row windows (:15); for window w the ascending unique set of
// c/16 over the edges (u, c) of rows [16w, min(16w+16, n)) (:19-36);
// window_offsets = exclusive prefix of the set sizes (:39).  New output: the
// 16 row masks of each tile (bit c of row r <=> edge (16w+r, 16b+c)).
//
// Design (one workgroup of 256 threads per window, no sort):
//   * the window's block columns are marked in an LDS bitmap (one bit per
//     block column, LDS atomic OR).  An edge that sets a new bit is a new
//     tile, so the count pass needs no scan at all;
//   * the fill pass also marks, in a 64-word summary, which bitmap words are
//     non-empty, lists those words in ascending order, and scans their
//     popcounts: a tile's rank (its output position) is the base of its word
//     plus the set bits below it.  Block columns are written while walking
//     the set bits; each edge then ORs its bit into the LDS mask of its tile
//     and the masks are streamed out, kMaskTiles tiles at a time;
//   * each thread owns a contiguous run of the window's edges and merges
//     consecutive edges that hit the same LDS word before its atomic, so rows
//     with sorted columns issue few atomics;
//   * graphs wider than one bitmap (kSliceCols block columns) are swept in
//     slices, and only slices that hold one of the window's edges are
//     visited; bitmap words are cleared edge by edge after use;
//   * edges stay in registers between phases when the window has at most
//     kRegEdges of them; heavier (hub) windows re-read them from memory.
// The per-window work is O(E) plus a few barriers; the output is
// deterministic and does not depend on the order of columns in a row.
// Counts are scanned into window_offsets with the device scan of runtime.hip.
#include <stdio.h>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

constexpr int kConvThreads = 256;
constexpr int kBitWords = 2048;                   // bitmap words per column slice
constexpr int kSumWords = kBitWords / 32;         // summary: one bit per bitmap word
constexpr int kSliceCols = kBitWords * 32;        // block columns per slice
constexpr int kMaxSlices = 2048;                  // >= ceil(2^27 / kSliceCols)
constexpr int kMaskTiles = 256;                   // tile masks staged in LDS at once
constexpr int kEPT = 8;                           // edges per thread kept in registers
constexpr int kRegEdges = kConvThreads * kEPT;
static_assert(kSumWords == kWave, "the summary is scanned by one wave");

enum ConvErr : int32_t { kErrNone = 0, kErrRowPtr = 1, kErrCol = 2, kErrCount = 4 };

// The count pass needs only the bitmap; its LDS stays small for occupancy.
template <bool FILL>
struct ConvLds {
    uint32_t bits[kBitWords];                  // block columns of the current slice
    uint32_t base[FILL ? kBitWords : 1];       // tiles before each non-empty word
    uint32_t masks[FILL ? kMaskTiles * 8 : 1]; // row masks of tiles [ms, ms + kMaskTiles)
    uint16_t list[FILL ? kBitWords : 2];       // non-empty words, ascending
    uint32_t summary[FILL ? kSumWords : 1];    // non-empty bitmap words
    uint32_t slices[kMaxSlices / 32];          // slices holding at least one edge
    int32_t rp[17];
    int32_t scan[kConvThreads / kWave];
    int32_t nlist;
    int32_t bad;
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

// Row of the window that holds edge e: the last r < nrows with rp[r] <= e
// (an empty row r has rp[r] == rp[r + 1], so the search passes over it).
__device__ __forceinline__ int row_of_edge(const int32_t* rp, int nrows, int32_t e)
{
    int r = 0;
#pragma unroll
    for (int step = 8; step > 0; step >>= 1)
        if (r + step < nrows && rp[r + step] <= e) r += step;
    return r;
}

// Pass kind: COUNT writes counts[w]; FILL writes block_col / tile_mask at
// window_offsets[w] and checks the count against the offsets.
template <bool FILL>
__global__ void __launch_bounds__(kConvThreads)
convert_windows(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
                int32_t n, int64_t nnz, int32_t W, int32_t* __restrict__ counts,
                const int32_t* __restrict__ window_offsets, int32_t* __restrict__ block_col,
                uint16_t* __restrict__ tile_mask, int32_t* __restrict__ err)
{
    __shared__ ConvLds<FILL> L;
    const int32_t w = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid == 0) L.bad = 0;
    if (tid < kMaxSlices / 32) L.slices[tid] = 0u;
    for (int g = tid; g < kBitWords / 4; g += kConvThreads)
        *reinterpret_cast<uint4*>(&L.bits[4 * g]) = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (FILL) {
        if (tid < kSumWords) L.summary[tid] = 0u;
    }
    WindowRows wr = load_window_rows(row_ptr, n, nnz, w, L.rp, err);
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
    const int E = (int)wr.E;
    const int32_t e0 = (int32_t)wr.e0;
    const int nrows = wr.nrows;
    // This thread's run of edges: e0 + [i0, i1).
    const int per = (E + kConvThreads - 1) / kConvThreads;
    const int i0 = min(E, tid * per), i1 = min(E, i0 + per);
    const bool in_regs = E <= kRegEdges;   // i.e. per <= kEPT

    // Visits the run's valid edges (column c, row r) in order.
    int32_t col[kEPT];
    uint32_t rows = 0;
    auto for_each_edge = [&](auto&& fn) {
        if (in_regs) {
#pragma unroll
            for (int j = 0; j < kEPT; ++j)
                if (col[j] >= 0) fn(col[j], (int)((rows >> (4 * j)) & 15u));
        } else {
            int r = i0 < i1 ? row_of_edge(L.rp, nrows, e0 + i0) : 0;
            for (int i = i0; i < i1; ++i) {
                while (r + 1 < nrows && e0 + i >= L.rp[r + 1]) ++r;
                const int32_t c = col_idx[e0 + i];
                if (c >= 0 && c < n) fn(c, r);
            }
        }
    };

    // ---- load (registers) or validate (hub), and mark the slices in use ----
    {
        int32_t last_sl = -1;
        auto mark = [&](int32_t c) {
            const int32_t sl = (c >> 4) / kSliceCols;
            if (sl != last_sl) {
                atomicOr(&L.slices[sl >> 5], 1u << (sl & 31));
                last_sl = sl;
            }
        };
        int r = i0 < i1 ? row_of_edge(L.rp, nrows, e0 + i0) : 0;
        if (in_regs) {
#pragma unroll
            for (int j = 0; j < kEPT; ++j) {
                const int i = i0 + j;
                int32_t c = -1;
                if (i < i1) {
                    while (r + 1 < nrows && e0 + i >= L.rp[r + 1]) ++r;
                    c = col_idx[e0 + i];
                    if (c < 0 || c >= n) {
                        L.bad = 1;
                        c = -1;
                    } else {
                        mark(c);
                    }
                }
                col[j] = c;
                rows |= (uint32_t)r << (4 * j);
            }
        } else {
            for (int i = i0; i < i1; ++i) {
                const int32_t c = col_idx[e0 + i];
                if (c < 0 || c >= n)
                    L.bad = 1;
                else
                    mark(c);
            }
        }
    }
    __syncthreads();

    const int32_t nslices = (W + kSliceCols - 1) / kSliceCols;
    int32_t running = 0;   // tiles of the slices already done
    for (int32_t sl = 0; sl < nslices; ++sl) {
        if (!((L.slices[sl >> 5] >> (sl & 31)) & 1u)) continue;   // block-uniform
        const int32_t lo = sl * kSliceCols;

        // ---- mark block columns; newly set bits are new tiles ----
        int32_t fresh = 0;
        {
            int32_t cur = -1;
            uint32_t acc = 0;
            auto flush = [&]() {
                if (cur < 0) return;
                const uint32_t old = atomicOr(&L.bits[cur], acc);
                fresh += __popc(acc & ~old);
                if constexpr (FILL) {
                    if (old == 0u) atomicOr(&L.summary[cur >> 5], 1u << (cur & 31));
                }
            };
            for_each_edge([&](int32_t c, int) {
                const int32_t q = (c >> 4) - lo;
                if (q < 0 || q >= kSliceCols) return;
                const int32_t wi = q >> 5;
                if (wi != cur) {
                    flush();
                    cur = wi;
                    acc = 0u;
                }
                acc |= 1u << (q & 31);
            });
            flush();
        }
        int32_t total;
        (void)block_exclusive_scan<kConvThreads>(fresh, L.scan, total);   // barriers inside

        if constexpr (FILL) {
            if (running + total <= expect) {
                // ---- ascending list of the non-empty words (one wave) ----
                if (tid < kSumWords) {
                    uint32_t sm = L.summary[tid];
                    const int cnt = __popc(sm);
                    const int incl = wave_inclusive_scan(cnt);
                    int pos = incl - cnt;
                    while (sm) {
                        const int b = __builtin_ctz(sm);
                        sm &= sm - 1u;
                        L.list[pos++] = (uint16_t)(tid * 32 + b);
                    }
                    if (tid == kSumWords - 1) L.nlist = incl;
                }
                __syncthreads();
                // ---- word bases and block columns, contiguous list entries ----
                const int nl = L.nlist;
                const int lper = (nl + kConvThreads - 1) / kConvThreads;
                const int a0 = min(nl, tid * lper), a1 = min(nl, a0 + lper);
                int32_t loc = 0;
                for (int a = a0; a < a1; ++a) loc += __popc(L.bits[L.list[a]]);
                int32_t tot2;
                int32_t t = block_exclusive_scan<kConvThreads>(loc, L.scan, tot2);
                for (int a = a0; a < a1; ++a) {
                    const int wi = L.list[a];
                    L.base[wi] = (uint32_t)t;
                    uint32_t m = L.bits[wi];
                    while (m) {
                        const int b = __builtin_ctz(m);
                        m &= m - 1u;
                        block_col[(int64_t)out_base + running + t] = lo + wi * 32 + b;
                        ++t;
                    }
                }
                __syncthreads();   // bases complete
                if (!in_regs) {
                    // ---- hub window: OR the edge bits straight into the zeroed
                    // output masks (one pass over the edges, not one per round) ----
                    if (tile_mask) {
                        uint4* dst = reinterpret_cast<uint4*>(
                            tile_mask + ((int64_t)out_base + running) * 16);
                        for (int i = tid; i < 2 * total; i += kConvThreads)
                            dst[i] = make_uint4(0u, 0u, 0u, 0u);
                        // the zeros reach L2, where the atomics act, before any OR
                        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                        __syncthreads();
                        uint32_t* gm = reinterpret_cast<uint32_t*>(
                            tile_mask + ((int64_t)out_base + running) * 16);
                        int32_t cur = -1;
                        uint32_t acc = 0;
                        for_each_edge([&](int32_t c, int r) {
                            const int32_t q = (c >> 4) - lo;
                            if (q < 0 || q >= kSliceCols) return;
                            const int32_t wi = q >> 5;
                            const uint32_t below = (1u << (q & 31)) - 1u;
                            const int32_t idx =
                                (int32_t)(L.base[wi] + __popc(L.bits[wi] & below)) * 8 + (r >> 1);
                            if (idx != cur) {
                                if (cur >= 0) atomicOr(&gm[cur], acc);
                                cur = idx;
                                acc = 0u;
                            }
                            acc |= (1u << (c & 15)) << (16 * (r & 1));
                        });
                        if (cur >= 0) atomicOr(&gm[cur], acc);
                    }
                    __syncthreads();
                }
                // ---- tile masks, kMaskTiles at a time ----
                for (int32_t ms = 0; in_regs && ms < total; ms += kMaskTiles) {
                    for (int i = tid; i < kMaskTiles * 2; i += kConvThreads)
                        *reinterpret_cast<uint4*>(&L.masks[4 * i]) = make_uint4(0u, 0u, 0u, 0u);
                    __syncthreads();
                    int32_t cur = -1;
                    uint32_t acc = 0;
                    for_each_edge([&](int32_t c, int r) {
                        const int32_t q = (c >> 4) - lo;
                        if (q < 0 || q >= kSliceCols) return;
                        const int32_t wi = q >> 5;
                        const uint32_t below = (1u << (q & 31)) - 1u;
                        const int32_t t2 =
                            (int32_t)(L.base[wi] + __popc(L.bits[wi] & below)) - ms;
                        if (t2 < 0 || t2 >= kMaskTiles) return;
                        const int32_t idx = t2 * 8 + (r >> 1);
                        if (idx != cur) {
                            if (cur >= 0) atomicOr(&L.masks[cur], acc);
                            cur = idx;
                            acc = 0u;
                        }
                        acc |= (1u << (c & 15)) << (16 * (r & 1));
                    });
                    if (cur >= 0) atomicOr(&L.masks[cur], acc);
                    __syncthreads();
                    if (tile_mask) {
                        const int32_t nt = min(kMaskTiles, total - ms);
                        for (int t3 = tid; t3 < nt; t3 += kConvThreads) {
                            const uint4* src = reinterpret_cast<const uint4*>(&L.masks[t3 * 8]);
                            uint4* dst = reinterpret_cast<uint4*>(
                                tile_mask + ((int64_t)out_base + running + ms + t3) * 16);
                            dst[0] = src[0];
                            dst[1] = src[1];
                        }
                    }
                    __syncthreads();   // masks are cleared by the next round
                }
            }
            if (tid < kSumWords) L.summary[tid] = 0u;
        }
        // ---- leave the bitmap clear for the next slice ----
        for_each_edge([&](int32_t c, int) {
            const int32_t q = (c >> 4) - lo;
            if (q >= 0 && q < kSliceCols) L.bits[q >> 5] = 0u;
        });
        running += total;
        __syncthreads();
    }
    if (tid == 0) {
        if (L.bad) *err = kErrCol;
        if (FILL) {
            if (running != expect) *err = kErrCount;
        } else {
            counts[w] = running;
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

    if (!block_col) {
        F3S_TRY(s.counts.reserve(sizeof(int32_t) * (size_t)W));
        F3S_TRY(s.offs64.reserve(sizeof(int64_t) * ((size_t)W + 1)));
        F3S_TRY(s.tmp.reserve(sizeof(int64_t) * (size_t)scan_tmp_elems(W)));
        int32_t* counts = reinterpret_cast<int32_t*>(s.counts.ptr);
        if (W > 0) {
            hipLaunchKernelGGL((convert_windows<false>), dim3(W), dim3(kConvThreads), 0, stream,
                               row_ptr, col_idx, n, nnz, W, counts, nullptr, nullptr, nullptr,
                               err);
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
        hipLaunchKernelGGL((convert_windows<true>), dim3(W), dim3(kConvThreads), 0, stream,
                           row_ptr, col_idx, n, nnz, W, nullptr, window_offsets, block_col,
                           tile_mask, err);
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
