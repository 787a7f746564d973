// convert.hip -- CSR -> 16x16 block-sparse conversion on the GPU.
//
// Semantics of convert_csr_to_block_sparse (src/converter.cu:13-44): W =
// ceil(n/16) row windows (:15); for window w the ascending unique set of
// c/16 over the edges (u, c) of rows [16w, min(16w+16, n)) (:19-36);
// window_offsets = exclusive prefix of the set sizes (:39).  New output: the
// 16 row masks of each tile (bit c of row r <=> edge (16w+r, 16b+c)).
//
// Design (no sort; an LDS bitmap with one bit per block column):
//   * convert_light, the main pass: a persistent kernel (as many 256-thread
//     workgroups as are resident at once) walks the windows of up to
//     kLightEdges edges on graphs whose block columns fit one bitmap sized
//     to the graph (up to 4.2 M nodes).  Every edge ORs its block column's
//     bit into the bitmap; a bit set for the first time is a new tile, so
//     the count pass needs no scan.  The fill pass marks non-empty bitmap
//     words in a summary and counts the new tiles under each summary word,
//     turns those into word bases (a tile's output rank is the base of its
//     word plus the set bits below it), stages the row masks
//     and block columns of up to kMaskTiles tiles in LDS and streams them
//     out in coalesced stores.  Each workgroup keeps the loads of its next
//     window in flight while it works on the current one, and its barriers
//     order LDS only, so they do not wait for those loads;
//   * count_waves: the count pass of graphs whose bitmap is small (W <=
//     65,536 windows): one window per wave with a bitmap of its own, no
//     workgroup barrier;
//   * the windows with more edges (hubs), which the main pass lists: when
//     counting, count_hubs takes each with a 512-thread workgroup (any
//     order); when filling, rank_hubs orders them heaviest first and
//     convert_hubs gives each a 1024-thread workgroup;
//   * convert_hubs, per window: on graphs too wide for one bitmap it takes
//     every window with 256 threads, the bitmap swept in column slices of
//     kSliceCols block columns (only slices holding an edge of the window
//     are visited).  Each thread owns a contiguous run of the window's edges
//     and merges consecutive edges that hit the same LDS word before its
//     atomic; windows with more than NT * kEPT edges re-read them from
//     memory and OR their masks straight into the zeroed output;
//   * the main passes clear bitmap words edge by edge after use, so no
//     window touches all W / 32 words.
// The per-window work is O(E) plus a few barriers; the output is
// deterministic and does not depend on the order of columns in a row.
// Counts become window_offsets through counts_to_offsets (two launches).
#include <stdio.h>

#include <mutex>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

constexpr int kConvThreads = 256;                 // persistent kernel; per-window fallback
constexpr int kHubThreads = 1024;                 // hub windows of the fill pass
constexpr int kBitWords = 2048;                  // bitmap words per column slice
constexpr int kSumWords = kBitWords / 32;         // summary: one bit per bitmap word
constexpr int kSliceCols = kBitWords * 32;        // block columns per slice
constexpr int kMaxSlices = 2048;                  // >= ceil(2^27 / kSliceCols)
constexpr int kMaskTiles = 256;                   // tile masks staged in LDS at once
constexpr int kEPT = 8;                           // edges per thread kept in registers
constexpr int kHubBatch = 4;                      // edge loads in flight per thread, wide windows
static_assert(kSumWords == kWave, "the summary is scanned by one wave");

enum ConvErr : int32_t { kErrNone = 0, kErrRowPtr = 1, kErrCol = 2, kErrCount = 4 };

// The count pass needs only the bitmap; its LDS stays small for occupancy.
// MT tile masks are staged at once (one per thread of the workgroup).
template <bool FILL, int MT>
struct ConvLds {
    uint32_t bits[kBitWords];                  // block columns of the current slice
    uint32_t base[FILL ? kBitWords : 1];       // tiles before each non-empty word
    uint32_t masks[FILL ? MT * 8 : 1];         // row masks of tiles [ms, ms + MT)
    uint16_t list[FILL ? kBitWords : 2];       // non-empty words, ascending
    uint32_t summary[FILL ? kSumWords : 1];    // non-empty bitmap words
    uint32_t slices[kMaxSlices / 32];          // slices holding at least one edge
    int32_t rp[17];
    int32_t scan[MT / kWave];
    int32_t nlist;
    int32_t bad;
};

struct WindowRows {
    int32_t u0, nrows;
    int64_t e0, E;
};

// Loads the window's row pointers into LDS and validates them (threads 0-16).
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
        if (a < 0 || b < a || b > nnz) atomicOr(err, kErrRowPtr);
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

// One window by one workgroup of NT threads, any edge count (every window of
// a graph too wide for the persistent kernel's bitmap).  Pass kind: COUNT
// writes counts[w]; FILL
// writes block_col / tile_mask at window_offsets[w] and checks the count
// against the offsets.
template <bool FILL, int NT>
__device__ __forceinline__ void
convert_one_window(ConvLds<FILL, NT>& L, int32_t w, const int32_t* __restrict__ row_ptr,
                   const int32_t* __restrict__ col_idx, int32_t n, int64_t nnz, int32_t W,
                   int32_t* __restrict__ counts, const int32_t* __restrict__ window_offsets,
                   int32_t* __restrict__ block_col, uint16_t* __restrict__ tile_mask,
                   int32_t* __restrict__ err)
{
    const int tid = threadIdx.x;
    __syncthreads();   // the previous window of this workgroup is done with L
    if (tid == 0) L.bad = 0;
    if (tid < kMaxSlices / 32) L.slices[tid] = 0u;
    for (int g = tid; g < kBitWords / 4; g += NT)
        *reinterpret_cast<uint4*>(&L.bits[4 * g]) = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (FILL) {
        if (tid < kSumWords) L.summary[tid] = 0u;
    }
    WindowRows wr = load_window_rows(row_ptr, n, nnz, w, L.rp, err);
    __syncthreads();
    if (wr.E < 0 || wr.e0 < 0 || wr.e0 + wr.E > nnz) {
        if (tid == 0) atomicOr(err, kErrRowPtr);
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
            if (tid == 0) atomicOr(err, kErrCount);
            return;
        }
    }
    constexpr int kRegEdgesNT = NT * kEPT;
    const int E = (int)wr.E;
    const int32_t e0 = (int32_t)wr.e0;
    const int nrows = wr.nrows;
    // This thread's run of edges: e0 + [i0, i1).
    const int per = (E + NT - 1) / NT;
    const int i0 = min(E, tid * per), i1 = min(E, i0 + per);
    const bool in_regs = E <= kRegEdgesNT;   // i.e. per <= kEPT

    // Visits the run's valid edges (column c, row r) in order.
    int32_t col[kEPT];
    uint32_t rows = 0;
    auto for_each_edge = [&](auto&& fn) {
        if (in_regs) {
#pragma unroll
            for (int j = 0; j < kEPT; ++j)
                if (col[j] >= 0) fn(col[j], (int)((rows >> (4 * j)) & 15u));
        } else {
            // kHubBatch loads in flight per thread, then their edges in order
            int r = i0 < i1 ? row_of_edge(L.rp, nrows, e0 + i0) : 0;
            for (int i = i0; i < i1; i += kHubBatch) {
                int32_t cb[kHubBatch];
#pragma unroll
                for (int j = 0; j < kHubBatch; ++j)
                    cb[j] = i + j < i1 ? col_idx[e0 + i + j] : -1;
#pragma unroll
                for (int j = 0; j < kHubBatch; ++j) {
                    if (i + j < i1) {
                        while (r + 1 < nrows && e0 + i + j >= L.rp[r + 1]) ++r;
                        if (cb[j] >= 0 && cb[j] < n) fn(cb[j], r);
                    }
                }
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
            for (int i = i0; i < i1; i += kHubBatch) {
                int32_t cb[kHubBatch];
#pragma unroll
                for (int j = 0; j < kHubBatch; ++j)
                    cb[j] = i + j < i1 ? col_idx[e0 + i + j] : 0;
#pragma unroll
                for (int j = 0; j < kHubBatch; ++j) {
                    if (cb[j] < 0 || cb[j] >= n)
                        L.bad = 1;
                    else
                        mark(cb[j]);
                }
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
        (void)block_exclusive_scan<NT>(fresh, L.scan, total);   // barriers inside

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
                const int lper = (nl + NT - 1) / NT;
                const int a0 = min(nl, tid * lper), a1 = min(nl, a0 + lper);
                int32_t loc = 0;
                for (int a = a0; a < a1; ++a) loc += __popc(L.bits[L.list[a]]);
                int32_t tot2;
                int32_t t = block_exclusive_scan<NT>(loc, L.scan, tot2);
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
                        for (int i = tid; i < 2 * total; i += NT)
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
                // ---- tile masks, NT at a time ----
                for (int32_t ms = 0; in_regs && ms < total; ms += NT) {
                    for (int i = tid; i < NT * 2; i += NT)
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
                        if (t2 < 0 || t2 >= NT) return;
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
                        const int32_t nt = min(NT, total - ms);
                        for (int t3 = tid; t3 < nt; t3 += NT) {
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
        if (L.bad) atomicOr(err, kErrCol);
        if (FILL) {
            if (running != expect) atomicOr(err, kErrCount);
        } else {
            counts[w] = running;
        }
    }
}

// The hub windows of the fill pass, heaviest first (hubs != NULL; listed by
// the main pass, ordered by rank_hubs), or every window (hubs == NULL:
// graphs too wide for convert_light's bitmap); a workgroup per window.
template <bool FILL, int NT>
__global__ void __launch_bounds__(NT)
convert_hubs(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
             int32_t n, int64_t nnz, int32_t W, int32_t* __restrict__ counts,
             const int32_t* __restrict__ window_offsets, int32_t* __restrict__ block_col,
             uint16_t* __restrict__ tile_mask, const int32_t* __restrict__ hubs,
             const int32_t* __restrict__ num_hubs, int32_t* __restrict__ err)
{
    __shared__ ConvLds<FILL, NT> L;
    // the main pass lists each window at most once (num_hubs <= W); the clamp
    // keeps the list read inside its W + 1 entries whatever the count holds
    const int32_t nh = hubs ? min(*num_hubs, W) : W;
    for (int32_t i = blockIdx.x; i < nh; i += gridDim.x) {
        const int32_t w = hubs ? hubs[i] : i;
        if (w < 0 || w >= W) continue;   // uniform
        convert_one_window<FILL, NT>(L, w, row_ptr, col_idx, n, nnz, W, counts, window_offsets,
                                     block_col, tile_mask, err);
    }
}

// ---------------------------------------------------------------------------
// Persistent kernel for the windows with at most kLightEdges edges, on graphs
// whose block columns fit one LDS bitmap (W <= 32 kLightMaxWords).
//
// Each workgroup walks windows w_i = blockIdx.x + i G (G = grid size) and
// keeps its memory traffic one window ahead of its work: while it works on
// w_i, the edges of w_{i+1} are in flight into a second register set, and
// the row pointers (and, when filling, output offsets) of w_{i+3} into a
// register; those of w_{i+2}, fetched one window earlier, go into a
// three-slot LDS ring.  The bitmap (one bit per block column, sized to the
// graph) stays clear between windows: each edge clears its own word after
// use.  Per window:
//   mark   every edge ORs its block column's bit into the bitmap; a bit set
//          for the first time is a new tile (count; filling, it adds one to
//          its summary word's tile count); the first setter of a word also
//          marks the word in the summary (fill);
//   base   (fill) wave 0 scans the summary words' tile counts and turns the
//          summary into word bases: a tile's output rank is the base of its
//          word plus the set bits below it;
//   stage  (fill) every edge ORs its bit into its tile's staged row masks and
//          records the tile's block column, kMaskTiles tiles per round; each
//          thread then streams out (and re-zeroes) the tiles it owns, so
//          block columns and masks leave in coalesced stores;
//   clear  every edge clears its bitmap word.
// The per-edge work is a handful of VALU operations and one or two LDS
// atomics: the passes are bound by instruction issue, and the fill pass also
// by the occupancy its LDS allows, so they keep no per-edge state beyond the
// column (and, filling, the row) and stage no more than kMaskTiles tiles.
// Windows with more edges are listed for the hub launches, so that one heavy
// window never holds up the windows queued behind it in this workgroup.
// ---------------------------------------------------------------------------
constexpr int kLightEPT = 4;                      // edges per thread, light windows
constexpr int kLightEdges = kConvThreads * kLightEPT;
constexpr int kLightMaxWords = 8192;              // bitmap words: W <= 262,144 (n <= 4,194,304)
constexpr int kHubCountThreads = 512;             // count_hubs workgroup

// The hub windows (more than kLightEdges edges), listed by the main passes:
// entry {window, first edge, edges, 0}, from the window description the
// main pass has already validated.
struct HubList {
    int32_t* count;   // entries listed (atomic; zeroed before the main pass)
    int4* hubs;       // [cap]
    int32_t cap;      // entries `hubs` holds (each window is listed at most once)
};

// Lists window w (edges [e0, e0 + E)).  One thread lists a window: a listing
// spread over a wave (a broadcast of the atomic's result) measured 40 %
// slower in convert_light's fill pass, whose other waves wait for it at a
// barrier.
__device__ __forceinline__ void list_hub(const HubList& hl, int32_t w, int32_t e0, int32_t E)
{
    const int32_t i = atomicAdd(hl.count, 1);
    if (i < hl.cap) hl.hubs[i] = make_int4(w, e0, E, 0);
}

constexpr int kMetaInts = 20;                     // rp[0..16], out_base, expect, flags
constexpr int kMetaSlots = 3;                     // windows w_i, w_{i+1}, w_{i+2}
constexpr int kMiscInts = 8;                      // cnt[2], total[2], bad
constexpr int kFlagLive = 1, kFlagRowsOk = 2, kFlagOutOk = 4;

// Dynamic LDS layout of convert_light (bytes; 16-byte aligned sections).
struct LightLayout {
    int32_t words;   // bitmap words, ceil(W / 32)
    int32_t sums;    // summary words, ceil(words / 32) (fill)
    uint32_t off_base, off_sum, off_masks, off_tcol, off_meta, bytes;
};

__host__ __device__ inline uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

__host__ __device__ inline LightLayout light_layout(int32_t W, bool fill)
{
    LightLayout l;
    l.words = (W + 31) / 32;
    l.sums = (l.words + 31) / 32;
    uint32_t o = align16(4u * (uint32_t)l.words);
    l.off_base = o;
    if (fill) o = align16(o + 2u * (uint32_t)l.words);
    l.off_sum = o;
    if (fill) o = align16(o + 8u * (uint32_t)l.sums);   // summary, then tiles per summary word
    l.off_masks = o;
    if (fill) o = align16(o + 4u * kMaskTiles * 8);
    l.off_tcol = o;
    if (fill) o = align16(o + 4u * kMaskTiles);
    l.off_meta = o;
    o = align16(o + 4u * (kMetaSlots * kMetaInts + kMiscInts));
    l.bytes = o;
    return l;
}

extern __shared__ __align__(16) unsigned char conv_lds[];

struct LightLds {
    uint32_t* bits;     // [words] block columns of the window
    uint16_t* base;     // [words] tiles before each word (fill)
    uint32_t* summary;  // [sums] non-empty bitmap words (fill)
    int32_t* scnt;      // [sums] tiles under each summary word (fill)
    uint32_t* masks;    // [kMaskTiles * 8] staged row masks, two rows per word (fill)
    int32_t* tcol;      // [kMaskTiles] staged block columns (fill)
    int32_t* meta;      // [kMetaSlots][kMetaInts] window descriptions (ring)
    int32_t* cnt;       // [2] count: tiles of a window, by parity
    int32_t* total;     // [2] fill: tiles of a window, by parity
    int32_t* bad;       // a column outside [0, n) was seen
    int32_t words, sums;
};

__device__ __forceinline__ LightLds light_lds(const LightLayout& lay)
{
    LightLds L;
    L.bits = reinterpret_cast<uint32_t*>(conv_lds);
    L.base = reinterpret_cast<uint16_t*>(conv_lds + lay.off_base);
    L.summary = reinterpret_cast<uint32_t*>(conv_lds + lay.off_sum);
    L.scnt = reinterpret_cast<int32_t*>(L.summary + lay.sums);
    L.masks = reinterpret_cast<uint32_t*>(conv_lds + lay.off_masks);
    L.tcol = reinterpret_cast<int32_t*>(conv_lds + lay.off_tcol);
    L.meta = reinterpret_cast<int32_t*>(conv_lds + lay.off_meta);
    L.cnt = L.meta + kMetaSlots * kMetaInts;
    L.total = L.cnt + 2;
    L.bad = L.cnt + 4;
    L.words = lay.words;
    L.sums = lay.sums;
    return L;
}

// What lane t (< 19) fetches for window wn: row_ptr[16 wn + t] for t <=
// nrows, window_offsets[wn] (t = 17) and [wn + 1] (t = 18) when filling.
// One vector load with a per-lane address (a uniform window_offsets load
// would become a scalar load into the same register, and that register
// write would have to wait for every load in flight).
template <bool FILL>
__device__ __forceinline__ int32_t fetch_meta(int32_t wn, int32_t W, int32_t n,
                                              const int32_t* __restrict__ row_ptr,
                                              const int32_t* __restrict__ window_offsets)
{
    const int t = threadIdx.x & (kWave - 1);
    const int32_t* p = nullptr;
    if (wn < W) {
        const int nrows = min(16, n - wn * 16);
        if (t <= nrows) p = row_ptr + (int64_t)wn * 16 + t;
        if (FILL && (t == 17 || t == 18)) p = window_offsets + wn + (t - 17);
    }
    int32_t v = 0;
    if (p) v = *p;
    return v;
}

// Wave 0 stores a fetched window description into ring slot `slot`, with
// flags: live (wn < W), row pointers usable (0 <= rp[0] <= ... <= rp[nrows]
// <= nnz) and output range usable ([out_base, out_base + expect) inside
// [0, total_tiles)).
template <bool FILL>
__device__ __forceinline__ void publish_meta(const LightLds& L, int slot, int32_t v, int32_t wn,
                                             int32_t W, int32_t n, int64_t nnz,
                                             int32_t total_tiles, int32_t* __restrict__ err)
{
    const int lane = threadIdx.x;   // wave 0 only
    const bool live = wn < W;
    const int nrows = live ? min(16, n - wn * 16) : 0;
    const int32_t rp0 = __shfl(v, 0, kWave), rpn = __shfl(v, nrows, kWave);
    const int32_t nxt = __shfl_down(v, 1, kWave);
    const bool back = lane < nrows && nxt < v;
    const bool rows_ok = live && !__any(back) && rp0 >= 0 && rpn >= rp0 && (int64_t)rpn <= nnz;
    bool out_ok = true;
    int32_t val = v;
    if (FILL) {
        // lanes 17 and 18 hold window_offsets[wn] and [wn + 1]
        const int32_t ob = __shfl(v, 17, kWave), end = __shfl(v, 18, kWave);
        out_ok = ob >= 0 && end >= ob && end <= total_tiles;
        if (lane == 18) val = out_ok ? end - ob : 0;   // expect
    }
    int32_t* dst = L.meta + slot * kMetaInts;
    if (lane < 19) dst[lane] = val;
    if (lane == 19)
        dst[19] = (live ? kFlagLive : 0) | (rows_ok ? kFlagRowsOk : 0) |
                  (out_ok ? kFlagOutOk : 0) | (nrows << 8);
    if (lane == 0 && live) {
        if (!rows_ok) atomicOr(err, kErrRowPtr);
        else if (!out_ok) atomicOr(err, kErrCount);
    }
}

struct LightWin {
    int32_t e0, E, nrows, out_base, expect, flags;
};

__device__ __forceinline__ LightWin read_meta(const LightLds& L, int slot)
{
    const int32_t* m0 = L.meta + slot * kMetaInts;
    LightWin m;
    m.flags = m0[19];
    m.nrows = m.flags >> 8;
    m.e0 = m0[0];
    m.E = (m.flags & kFlagRowsOk) ? m0[m.nrows] - m.e0 : 0;
    m.out_base = m0[17];
    m.expect = m0[18];
    return m;
}

// Issues the loads of this thread's run of edges of the window in ring slot
// `slot` (nothing for hub windows): col[j] for j < cnt, and (filling) the
// rows, packed 4 bits per edge.  The loaded values are not used here, so the
// loads stay in flight.
template <bool FILL>
__device__ __forceinline__ void issue_edges(const LightLds& L, int slot,
                                            const int32_t* __restrict__ col_idx,
                                            int32_t (&col)[kLightEPT], uint32_t& rows, int& cnt)
{
    const LightWin m = read_meta(L, slot);
    cnt = 0;
    rows = 0;
    if (m.E <= 0 || m.E > kLightEdges) return;
    const int per = (m.E + kConvThreads - 1) / kConvThreads;
    const int i0 = min(m.E, (int)threadIdx.x * per), i1 = min(m.E, i0 + per);
    cnt = i1 - i0;
#pragma unroll
    for (int j = 0; j < kLightEPT; ++j)
        if (j < cnt) col[j] = col_idx[m.e0 + i0 + j];
    if (FILL && cnt > 0) {
        const int32_t* rp = L.meta + slot * kMetaInts;
        int r = row_of_edge(rp, m.nrows, m.e0 + i0);
#pragma unroll
        for (int j = 0; j < kLightEPT; ++j) {
            const int32_t e = m.e0 + i0 + j;
            while (r + 1 < m.nrows && e >= rp[r + 1]) ++r;
            rows |= (uint32_t)r << (4 * j);
        }
    }
}

// One window (at most kLightEdges edges, in col / rows) described by ring
// slot `slot`.  Every thread runs the same sequence of barriers.  Nothing
// here waits for a load: the only loads in flight are the next window's.
template <bool FILL>
__device__ __forceinline__ void light_window(const LightLds& L, int slot, int32_t w,
                                             int32_t (&col)[kLightEPT], uint32_t rows, int cnt,
                                             int& round, int32_t n,
                                             int32_t* __restrict__ counts,
                                             int32_t* __restrict__ block_col,
                                             uint16_t* __restrict__ tile_mask,
                                             const HubList& hl,
                                             int32_t* __restrict__ err)
{
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wid = tid / kWave;
    const LightWin m = read_meta(L, slot);
    const bool usable = (m.flags & kFlagLive) && (m.flags & kFlagRowsOk) &&
                        (!FILL || (m.flags & kFlagOutOk));

    if (!usable || m.E > kLightEdges || m.E == 0) {
        // hub (listed for count_hubs / convert_hubs, which also write its
        // count or tiles), empty or rejected window: no tiles here
        if (usable && m.E > 0) {
            if (tid == 0) list_hub(hl, w, m.e0, m.E);
        } else if (tid == 0) {
            if (FILL) {
                if (usable && m.expect != 0) atomicOr(err, kErrCount);
            } else {
                counts[w] = 0;
            }
        }
        lds_barrier();   // the description published for window w + 2G is visible
        return;
    }

    // absent (j >= cnt) and invalid columns become -1; an invalid column
    // (outside [0, n)) is reported and left out
#pragma unroll
    for (int j = 0; j < kLightEPT; ++j) {
        const int32_t c = col[j];
        const bool present = j < cnt;
        const bool ok = present && c >= 0 && c < n;
        if (present && !ok) *L.bad = 1;
        col[j] = ok ? c : -1;
    }
    const int k = round & 1;
    ++round;

    // ---- mark ----
    int32_t fresh = 0;
#pragma unroll
    for (int j = 0; j < kLightEPT; ++j) {
        const int32_t c = col[j];
        if (c < 0) continue;
        const int32_t wi = c >> 9;
        const uint32_t bit = 1u << ((c >> 4) & 31);
        const uint32_t old = atomicOr(&L.bits[wi], bit);
        if (FILL) {
            if (old == 0u) atomicOr(&L.summary[wi >> 5], 1u << (wi & 31));
            if ((old & bit) == 0u) atomicAdd(&L.scnt[wi >> 5], 1);   // a new tile
        } else {
            fresh += (old & bit) == 0u;
        }
    }
    if (!FILL) {
        fresh = wave_sum(fresh);
        if (lane == 0 && fresh) atomicAdd(&L.cnt[k], fresh);
    }
    lds_barrier();   // B1: bitmap (+ summary) complete
    if (tid == 0) L.cnt[k ^ 1] = 0;   // read before B1 by the previous window

    int32_t total;
    if constexpr (!FILL) {
        total = L.cnt[k];
    } else {
        // ---- base (wave 0): lane l owns summary words [l spl, (l + 1) spl) ----
        if (wid == 0) {
            const int spl = (L.sums + kWave - 1) / kWave;
            const int s0 = min(L.sums, lane * spl), s1 = min(L.sums, s0 + spl);
            // the tiles under each summary word were counted while marking
            int32_t own = 0;
            for (int sw = s0; sw < s1; ++sw) own += L.scnt[sw];
            const int32_t incl = wave_inclusive_scan(own);
            int32_t t0 = incl - own;
            for (int sw = s0; sw < s1; ++sw) {
                uint32_t t = L.summary[sw];
                if (!t) continue;
                L.summary[sw] = 0u;
                L.scnt[sw] = 0;
                for (; t; t &= t - 1u) {
                    const int wi = sw * 32 + __builtin_ctz(t);
                    L.base[wi] = (uint16_t)t0;
                    t0 += __popc(L.bits[wi]);
                }
            }
            if (lane == kWave - 1) L.total[k] = incl;
        }
        lds_barrier();   // B2: bases and the window's tile count
        total = L.total[k];
        if (total <= m.expect) {
            // ---- stage, kMaskTiles tiles per round ----
            for (int32_t ms = 0; ms < total; ms += kMaskTiles) {
                if (ms > 0) lds_barrier();   // the previous round's tiles are re-zeroed
#pragma unroll
                for (int j = 0; j < kLightEPT; ++j) {
                    const int32_t c = col[j];
                    if (c < 0) continue;
                    const int32_t wi = c >> 9;
                    const uint32_t below = (1u << ((c >> 4) & 31)) - 1u;
                    const int32_t t2 = (int32_t)L.base[wi] + __popc(L.bits[wi] & below) - ms;
                    if (t2 < 0 || t2 >= kMaskTiles) continue;
                    const int r = (int)((rows >> (4 * j)) & 15u);
                    atomicOr(&L.masks[t2 * 8 + (r >> 1)], (1u << (c & 15)) << (16 * (r & 1)));
                    L.tcol[t2] = c >> 4;   // every edge of the tile writes the same value
                }
                lds_barrier();   // B3: the round's staged tiles are complete
                const int32_t nt = min(kMaskTiles, total - ms);
                for (int t3 = tid; t3 < nt; t3 += kConvThreads) {
                    const int64_t o = (int64_t)m.out_base + ms + t3;
                    block_col[o] = L.tcol[t3];
                    uint4* src = reinterpret_cast<uint4*>(&L.masks[t3 * 8]);
                    if (tile_mask) {
                        uint4* dst = reinterpret_cast<uint4*>(tile_mask + o * 16);
                        dst[0] = src[0];
                        dst[1] = src[1];
                    }
                    src[0] = make_uint4(0u, 0u, 0u, 0u);
                    src[1] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
    }
    // ---- clear (every reader of the bitmap is past B1, B2 or B3) ----
#pragma unroll
    for (int j = 0; j < kLightEPT; ++j)
        if (col[j] >= 0) L.bits[col[j] >> 9] = 0u;
    lds_barrier();   // B4: bitmap and staged masks clear for the next window
    if (tid == 0) {
        if (FILL) {
            if (total != m.expect) atomicOr(err, kErrCount);
        } else {
            counts[w] = total;
        }
    }
}

template <bool FILL>
__global__ void __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
convert_light(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
              int32_t n, int64_t nnz, int32_t W, int32_t* __restrict__ counts,
              const int32_t* __restrict__ window_offsets, int32_t* __restrict__ block_col,
              uint16_t* __restrict__ tile_mask, HubList hl, int32_t* __restrict__ err)
{
    const LightLayout lay = light_layout(W, FILL);
    const LightLds L = light_lds(lay);
    const int tid = threadIdx.x;
    const int wid = tid / kWave;
    const int32_t G = gridDim.x;
    int32_t w = blockIdx.x;
    if (w >= W) return;   // uniform
    for (int g = tid; g < (L.words + 3) / 4; g += kConvThreads)
        *reinterpret_cast<uint4*>(&L.bits[4 * g]) = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (FILL) {
        for (int g = tid; g < kMaskTiles * 2; g += kConvThreads)
            *reinterpret_cast<uint4*>(&L.masks[4 * g]) = make_uint4(0u, 0u, 0u, 0u);
        for (int g = tid; g < 2 * L.sums; g += kConvThreads) L.summary[g] = 0u;   // + scnt
    }
    if (tid < kMiscInts) L.cnt[tid] = 0;
    const int32_t total_tiles = FILL ? window_offsets[W] : 0;
    // descriptions in flight (every wave fetches them; wave 0 publishes)
    int32_t aheadX = 0, aheadY = 0;
    {
        const int32_t v0 = fetch_meta<FILL>(w, W, n, row_ptr, window_offsets);
        const int32_t v1 = fetch_meta<FILL>(w + G, W, n, row_ptr, window_offsets);
        aheadX = fetch_meta<FILL>(w + 2 * G, W, n, row_ptr, window_offsets);
        if (wid == 0) {
            publish_meta<FILL>(L, 0, v0, w, W, n, nnz, total_tiles, err);
            publish_meta<FILL>(L, 1, v1, w + G, W, n, nnz, total_tiles, err);
        }
    }
    lds_barrier();

    static_assert(kLightEPT == 4, "the register uses in the loop name every edge register");
    int32_t colA[kLightEPT], colB[kLightEPT];
    uint32_t rowsA = 0, rowsB = 0;
    int cntA = 0, cntB = 0;
    int round = 0;
    int slot = 0;   // ring slot of the current window
    issue_edges<FILL>(L, 0, col_idx, colA, rowsA, cntA);
    // Two windows per trip so that the register sets alternate without copies
    // (a copy would wait for the loads in flight).  Each half first uses the
    // registers loaded one window ago -- gfx950 counts loads and stores with
    // one counter, so once a store is pending any wait is a wait for
    // everything, and it must come before the next window's loads issue --
    // then publishes the description of w + 2G into the ring slot whose last
    // readers (window w - G) are past a barrier, issues the loads of w + G
    // and w + 3G, and works on w.
    while (true) {
        {
            const int s1 = slot == 2 ? 0 : slot + 1, s2 = s1 == 2 ? 0 : s1 + 1;
            asm volatile("" ::"v"(colA[0]), "v"(colA[1]), "v"(colA[2]), "v"(colA[3]), "v"(aheadX));
            if (wid == 0) publish_meta<FILL>(L, s2, aheadX, w + 2 * G, W, n, nnz, total_tiles, err);
            aheadY = fetch_meta<FILL>(w + 3 * G, W, n, row_ptr, window_offsets);
            issue_edges<FILL>(L, s1, col_idx, colB, rowsB, cntB);
            light_window<FILL>(L, slot, w, colA, rowsA, cntA, round, n, counts, block_col,
                               tile_mask, hl, err);
            w += G;
            slot = s1;
            if (w >= W) break;
        }
        {
            const int s1 = slot == 2 ? 0 : slot + 1, s2 = s1 == 2 ? 0 : s1 + 1;
            asm volatile("" ::"v"(colB[0]), "v"(colB[1]), "v"(colB[2]), "v"(colB[3]), "v"(aheadY));
            if (wid == 0) publish_meta<FILL>(L, s2, aheadY, w + 2 * G, W, n, nnz, total_tiles, err);
            aheadX = fetch_meta<FILL>(w + 3 * G, W, n, row_ptr, window_offsets);
            issue_edges<FILL>(L, s1, col_idx, colA, rowsA, cntA);
            light_window<FILL>(L, slot, w, colB, rowsB, cntB, round, n, counts, block_col,
                               tile_mask, hl, err);
            w += G;
            slot = s1;
            if (w >= W) break;
        }
    }
    if (tid == 0 && *L.bad) atomicOr(err, kErrCol);
}

// ---------------------------------------------------------------------------
// count_waves: the count pass of graphs whose bitmap is small (W <=
// 32 * kWaveCountMaxWords windows): one window per wave, each wave with a
// bitmap of its own in LDS, so a window costs no workgroup barrier.  A wave
// takes windows w, w + GW, w + 2 GW, ... (GW waves in the grid); while it
// marks one window, the columns of its next window and the row pointers of
// the one after are in flight.  Its counts leave 64 windows at a time (lane
// k keeps the count of the batch's k-th window): gfx950 counts loads and
// stores with one counter, so a store pending at every window would make
// each wait a wait for the prefetched loads too.  Windows of more than
// kLightEdges edges are listed for count_hubs, which writes their counts
// (the zero this pass leaves there is overwritten).  Same counts, same hub
// list and same error bits as convert_light<false>; on graphs of many block
// columns the bitmap per wave leaves fewer windows in flight per CU than
// convert_light's shared one, which is used there.
// ---------------------------------------------------------------------------
constexpr int kWaveCountWaves = 4;                   // waves per workgroup
constexpr int kWaveCountEPL = kLightEdges / kWave;   // edge slots per lane
constexpr int32_t kWaveCountMaxWords = 2048;         // 8 KB of bitmap per wave

struct WaveWin {
    int32_t e0, E;
    bool ok;   // row pointers usable
};

// Row pointers of window wn: lane t <= nrows holds row_ptr[16 wn + t]; the
// other lanes (and every lane past the last window) load past the end of
// the descriptor `rp` over row_ptr[0..n], which reads 0 -- one unconditional
// load, so nothing waits for it before its value is used.
__device__ __forceinline__ int32_t wave_fetch_rp(__amdgpu_buffer_rsrc_t rp, int32_t n, int32_t W,
                                                 int64_t wn, int lane)
{
    uint32_t off = 4u * ((uint32_t)n + 1u);   // out of range
    if (wn < W) {
        const int nrows = min(16, n - (int32_t)wn * 16);
        if (lane <= nrows) off = 4u * (uint32_t)(wn * 16 + lane);
    }
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, 0);
}

// The window's edge range, and whether its row pointers are usable (0 <=
// rp[0] <= ... <= rp[nrows] <= nnz), from the fetched row pointers; all
// wave-uniform (scalar).
__device__ __forceinline__ WaveWin wave_describe(int32_t v, int32_t n, int64_t nnz, int64_t wn,
                                                 int32_t W, int lane)
{
    WaveWin d{0, 0, false};
    if (wn >= W) return d;
    const int nrows = min(16, n - (int32_t)wn * 16);
    const int32_t rp0 = __builtin_amdgcn_readfirstlane(__shfl(v, 0, kWave));
    const int32_t rpn = __builtin_amdgcn_readfirstlane(__shfl(v, nrows, kWave));
    const int32_t nxt = __shfl_down(v, 1, kWave);
    const bool back = lane < nrows && nxt < v;
    d.ok = !__any(back) && rp0 >= 0 && rpn >= rp0 && (int64_t)rpn <= nnz;
    d.e0 = rp0;
    d.E = d.ok ? rpn - rp0 : 0;
    return d;
}

// Issues the loads of a light window's columns: edge lane + 64 j in col[j],
// through a buffer descriptor over the window's edges (32-bit offsets; a
// load past them reads 0 and touches no memory).  The values are not used
// here, so the loads stay in flight.
__device__ __forceinline__ void wave_issue_cols(const WaveWin& d,
                                                const int32_t* __restrict__ col_idx, int lane,
                                                int32_t (&col)[kWaveCountEPL])
{
    const int32_t E = d.E <= kLightEdges ? d.E : 0;   // hubs and unusable windows: none
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(col_idx) + (E > 0 ? d.e0 : 0), (short)0, 4 * E, 0x00020000);
#pragma unroll
    for (int j = 0; j < kWaveCountEPL; ++j) {
        if (kWave * j >= E) break;   // wave-uniform: the window has no edge here
        col[j] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, 4 * (lane + kWave * j), 0, 0);
    }
}

__global__ void __launch_bounds__(kWaveCountWaves * kWave)
count_waves(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx, int32_t n,
            int64_t nnz, int32_t W, int32_t* __restrict__ counts, HubList hl,
            int32_t* __restrict__ err)
{
    const int words = (W + 31) / 32;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    uint32_t* bits = reinterpret_cast<uint32_t*>(conv_lds) + (size_t)wave * words;
    for (int i = lane; i < words; i += kWave) bits[i] = 0u;
    F3S_WAVE_LDS_SYNC();
    const int64_t GW = (int64_t)gridDim.x * kWaveCountWaves;
    int64_t w = (int64_t)blockIdx.x * kWaveCountWaves + wave;
    if (w >= W) return;   // wave-uniform; the kernel has no workgroup barrier

    bool bad = false;           // a column outside [0, n) was seen
    int32_t mycount = 0;        // count of the batch's lane-th window
    int nb = 0;                 // windows in the batch
    int64_t wfirst = w;         // the batch's first window
    // Marks window wn's columns, leaves the bitmap clear again and returns
    // its tile count (0 for an unusable, empty or hub window).
    auto process = [&](const WaveWin& d, int64_t wn, const int32_t (&col)[kWaveCountEPL]) {
        int32_t cnt = 0;
        if (!d.ok) {
            if (lane == 0) atomicOr(err, kErrRowPtr);
        } else if (d.E > kLightEdges) {
            if (lane == 0) list_hub(hl, (int32_t)wn, d.e0, d.E);
        } else if (d.E > 0) {
            int fresh = 0;
#pragma unroll
            for (int j = 0; j < kWaveCountEPL; ++j) {
                if (kWave * j >= d.E) break;   // wave-uniform: no edge in this slot
                const int32_t c = col[j];
                if (lane + kWave * j < d.E) {
                    if (c < 0 || c >= n) {
                        bad = true;
                    } else {
                        const uint32_t bit = 1u << ((c >> 4) & 31);
                        fresh += (atomicOr(&bits[c >> 9], bit) & bit) == 0u;
                    }
                }
            }
            cnt = wave_sum(fresh);
            F3S_WAVE_LDS_SYNC();   // every mark is done before the clears
#pragma unroll
            for (int j = 0; j < kWaveCountEPL; ++j) {
                if (kWave * j >= d.E) break;
                const int32_t c = col[j];
                if (lane + kWave * j < d.E && c >= 0 && c < n) bits[c >> 9] = 0u;
            }
            F3S_WAVE_LDS_SYNC();
        }
        if (lane == nb) mycount = cnt;
        if (++nb == kWave) {
            counts[wfirst + lane * GW] = mycount;
            nb = 0;
            wfirst = wn + GW;
        }
    };

    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(row_ptr), (short)0, (int32_t)(4 * ((int64_t)n + 1)), 0x00020000);
    int32_t colA[kWaveCountEPL], colB[kWaveCountEPL];
    WaveWin dA = wave_describe(wave_fetch_rp(rp, n, W, w, lane), n, nnz, w, W, lane);
    int32_t rpN = wave_fetch_rp(rp, n, W, w + GW, lane);   // next window, in flight
    wave_issue_cols(dA, col_idx, lane, colA);
    WaveWin dB;
    // Two windows per trip so that the two column register sets alternate
    // without copies (a copy would wait for the loads in flight).
    while (true) {
        dB = wave_describe(rpN, n, nnz, w + GW, W, lane);
        wave_issue_cols(dB, col_idx, lane, colB);
        rpN = wave_fetch_rp(rp, n, W, w + 2 * GW, lane);
        process(dA, w, colA);
        w += GW;
        if (w >= W) break;
        dA = wave_describe(rpN, n, nnz, w + GW, W, lane);
        wave_issue_cols(dA, col_idx, lane, colA);
        rpN = wave_fetch_rp(rp, n, W, w + 2 * GW, lane);
        process(dB, w, colB);
        w += GW;
        if (w >= W) break;
    }
    if (lane < nb) counts[wfirst + lane * GW] = mycount;
    if (__any(bad) && lane == 0) atomicOr(err, kErrCol);
}

// ---------------------------------------------------------------------------
// count_hubs: the count pass of the hub windows the main pass listed, one
// kHubCountThreads workgroup per window (any order, a grid-stride loop over
// the list): every edge ORs its block column's bit into an LDS bitmap, and
// the bits set for the first time add up to the window's tile count.  The
// edges are read in coalesced chunks of kHubCountThreads * kHubCountEPT, all
// loads of a chunk in flight at once.  Measured on config 4's 1,310 hubs:
// 13 us, against 29 us with the fill pass's 1024-thread kernel plus 10 us to
// order the list first.
// ---------------------------------------------------------------------------
constexpr int kHubCountEPT = 8;

__global__ void __launch_bounds__(kHubCountThreads)
count_hubs(const int32_t* __restrict__ col_idx, int32_t n, int64_t nnz, int32_t W,
           int32_t* __restrict__ counts, HubList hl, int32_t* __restrict__ err)
{
    constexpr int NT = kHubCountThreads;
    constexpr int32_t kChunk = NT * kHubCountEPT;
    uint32_t* bits = reinterpret_cast<uint32_t*>(conv_lds);
    const int words4 = ((W + 31) / 32 + 3) & ~3;
    int32_t* scan = reinterpret_cast<int32_t*>(conv_lds) + words4;   // [NT / 64]
    int32_t* bad = scan + NT / kWave;
    const int tid = threadIdx.x;
    const int32_t nh = min(*hl.count, hl.cap);
    if ((int32_t)blockIdx.x >= nh) return;   // uniform
    for (int g = tid; g < words4 / 4; g += NT)
        reinterpret_cast<uint4*>(bits)[g] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) *bad = 0;
    for (int32_t i = blockIdx.x; i < nh; i += gridDim.x) {
        const int4 h = hl.hubs[i];
        const int32_t w = h.x, e0 = h.y, E = h.z;
        // (the main pass listed the window with usable row pointers; the
        // check keeps every access in bounds whatever the list holds)
        if ((uint32_t)w >= (uint32_t)W || e0 < 0 || E <= 0 || (int64_t)e0 + E > nnz)
            continue;   // uniform
        __syncthreads();   // the previous window's bitmap is clear
        int32_t fresh = 0;
        for (int64_t c0 = 0; c0 < E; c0 += kChunk) {
            int32_t col[kHubCountEPT];
#pragma unroll
            for (int j = 0; j < kHubCountEPT; ++j) {
                const int64_t e = c0 + tid + NT * j;
                col[j] = e < E ? col_idx[e0 + e] : 0;
            }
#pragma unroll
            for (int j = 0; j < kHubCountEPT; ++j) {
                const int64_t e = c0 + tid + NT * j;
                if (e >= E) continue;
                const int32_t c = col[j];
                if (c < 0 || c >= n) {
                    *bad = 1;
                    continue;
                }
                const uint32_t bit = 1u << ((c >> 4) & 31);
                fresh += (atomicOr(&bits[c >> 9], bit) & bit) == 0u;
            }
        }
        int32_t T;
        (void)block_exclusive_scan<NT>(fresh, scan, T);   // barriers inside: the marks are done
        if (tid == 0) counts[w] = T;
        for (int g = tid; g < words4 / 4; g += NT)
            reinterpret_cast<uint4*>(bits)[g] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    if (tid == 0 && *bad) atomicOr(err, kErrCol);
}

// Hub windows heaviest first, for the fill pass.  The main pass lists them
// in the order its workgroups find them; rank_hubs writes their windows again,
// ordered by descending edge count (ties: ascending window index, so the
// order is deterministic), and the hub launch that follows gives each listed
// window a workgroup of its own, dispatched in list order, so the longest
// windows start first.  Every workgroup of rank_hubs loads the keys of the
// whole list (up to kHubSortCap) into LDS and places 64 of them at their
// ranks, four lanes per entry each counting the smaller keys in a quarter of
// the list; keys are unique, so the ranks are a permutation.  A longer list
// is copied as listed.
constexpr int kHubSortCap = 4096;
constexpr int kHubLaunch = 2048;   // hub-launch workgroups (one per listed window up to this)

__global__ void __launch_bounds__(256)
rank_hubs(int32_t W, HubList hl, int32_t* __restrict__ sorted)
{
    __shared__ __align__(16) uint64_t key[kHubSortCap];
    const int32_t nh = min(*hl.count, hl.cap);
    const int tid = threadIdx.x;
    if (nh > kHubSortCap) {   // uniform: copy in listing order
        for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < nh; i += (int64_t)gridDim.x * 256)
            sorted[i] = hl.hubs[i].x;
        return;
    }
    const int32_t base = blockIdx.x * 64;
    if (base >= nh) return;   // uniform
    constexpr int kPer = kHubSortCap / 256;
    int4 h[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid + 256 * k;
        h[k] = i < nh ? hl.hubs[i] : make_int4(-1, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        // (~edges, window) ascending = edges descending, window ascending; an
        // entry naming no window sorts last, keyed by its position
        const int i = tid + 256 * k;
        if (i >= nh) break;
        uint64_t key_i = (0xffffffffull << 32) | (uint32_t)i;
        if ((uint32_t)h[k].x < (uint32_t)W) {
            const uint32_t edges = (uint32_t)max(1, h[k].z);
            key_i = ((uint64_t)(~edges) << 32) | (uint32_t)h[k].x;
        }
        key[i] = key_i;
    }
    __syncthreads();
    // lanes 4e..4e+3 of a wave rank entry base + tid / 4, each over a quarter
    // of the list in steps of eight keys (four 16-byte LDS reads, from a
    // multiple of 8); their counts add up with two lane swaps
    const int32_t i = base + tid / 4;
    const uint64_t ki = key[i < nh ? i : 0];
    const int32_t quarter = ((nh + 31) / 32) * 8;   // a multiple of 8
    const int32_t j0 = min(nh, (tid & 3) * quarter), j1 = min(nh, j0 + quarter);
    int32_t rank = 0;
    int32_t j = j0;
    for (; j + 8 <= j1; j += 8) {
        const ulonglong2* k2 = reinterpret_cast<const ulonglong2*>(&key[j]);
        const ulonglong2 a = k2[0], b = k2[1], c = k2[2], d = k2[3];
        rank += (a.x < ki) + (a.y < ki) + (b.x < ki) + (b.y < ki) + (c.x < ki) + (c.y < ki) +
                (d.x < ki) + (d.y < ki);
    }
    for (; j < j1; ++j) rank += key[j] < ki ? 1 : 0;
    rank += __shfl_xor(rank, 1, kWave);
    rank += __shfl_xor(rank, 2, kWave);
    if (i < nh && (tid & 3) == 0)
        sorted[rank] = (ki >> 32) == 0xffffffffull ? -1 : (int32_t)(uint32_t)ki;
}

// int64 window offsets -> the caller's int32 offsets; thread 0 also reports
// the error bits and the tile count for the host (status[0], status[1]).
// ---------------------------------------------------------------------------
// Counts -> window_offsets in two launches: block sums, then each workgroup
// adds up the sums of the blocks before its own (at most kOffsFusedBlocks of
// them; wider graphs scan the sums in one workgroup first), scans its block
// straight into the int32 offsets -- T <= nnz <= INT32_MAX, since a tile
// holds at least one edge -- and its last workgroup writes offsets[W] and the
// host's status words (error bits, T).
// ---------------------------------------------------------------------------
constexpr int kOffsThreads = 256;
constexpr int kOffsPerThread = 8;
constexpr int kOffsTile = kOffsThreads * kOffsPerThread;
constexpr int64_t kOffsFusedBlocks = 1024;

__global__ void __launch_bounds__(kOffsThreads)
offsets_block_sums(const int32_t* __restrict__ counts, int64_t W, int64_t* __restrict__ sums)
{
    __shared__ int64_t lds[kOffsThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kOffsTile + (int64_t)threadIdx.x * kOffsPerThread;
    int64_t s = 0;
#pragma unroll
    for (int i = 0; i < kOffsPerThread; ++i)
        if (base + i < W) s += counts[base + i];
    int64_t total;
    (void)block_exclusive_scan<kOffsThreads>(s, lds, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One workgroup: the block sums into exclusive prefix sums, in place.
__global__ void __launch_bounds__(kOffsThreads)
offsets_scan_sums(int64_t* __restrict__ sums, int64_t nblocks)
{
    __shared__ int64_t lds[kOffsThreads / kWave];
    int64_t carry = 0;
    for (int64_t b0 = 0; b0 < nblocks; b0 += kOffsThreads) {
        const int64_t i = b0 + threadIdx.x;
        const int64_t v = i < nblocks ? sums[i] : 0;
        int64_t total;
        const int64_t ex = block_exclusive_scan<kOffsThreads>(v, lds, total);
        if (i < nblocks) sums[i] = carry + ex;
        carry += total;
    }
}

__global__ void __launch_bounds__(kOffsThreads)
offsets_apply(const int32_t* __restrict__ counts, int64_t W, const int64_t* __restrict__ sums,
              bool scanned, int32_t* __restrict__ offsets, const int32_t* __restrict__ err,
              int64_t* __restrict__ status)
{
    __shared__ int64_t lds[kOffsThreads / kWave];
    int64_t before;
    if (scanned) {
        before = sums[blockIdx.x];
    } else {
        int64_t part = 0;
        for (int64_t i = threadIdx.x; i < (int64_t)blockIdx.x; i += kOffsThreads) part += sums[i];
        (void)block_exclusive_scan<kOffsThreads>(part, lds, before);
    }
    const int64_t base = (int64_t)blockIdx.x * kOffsTile + (int64_t)threadIdx.x * kOffsPerThread;
    int64_t v[kOffsPerThread];
    int64_t s = 0;
#pragma unroll
    for (int i = 0; i < kOffsPerThread; ++i) {
        v[i] = (base + i < W) ? counts[base + i] : 0;
        s += v[i];
    }
    int64_t total;
    int64_t ex = block_exclusive_scan<kOffsThreads>(s, lds, total) + before;
#pragma unroll
    for (int i = 0; i < kOffsPerThread; ++i) {
        if (base + i < W) offsets[base + i] = (int32_t)ex;
        ex += v[i];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
        offsets[W] = (int32_t)(before + total);
        status[0] = *err;
        status[1] = before + total;
    }
}

// `sums` holds offsets_sum_elems(W) elements.
static int64_t offsets_sum_elems(int64_t W) { return W > 0 ? ceil_div(W, kOffsTile) : 1; }

static f3s_status counts_to_offsets(const int32_t* counts, int32_t* offsets, int64_t W,
                                    int64_t* sums, const int32_t* err, int64_t* status,
                                    hipStream_t stream)
{
    const int64_t nb = offsets_sum_elems(W);
    hipLaunchKernelGGL(offsets_block_sums, dim3((unsigned)nb), dim3(kOffsThreads), 0, stream,
                       counts, W, sums);
    const bool scanned = nb > kOffsFusedBlocks;
    if (scanned)
        hipLaunchKernelGGL(offsets_scan_sums, dim3(1), dim3(kOffsThreads), 0, stream, sums, nb);
    hipLaunchKernelGGL(offsets_apply, dim3((unsigned)nb), dim3(kOffsThreads), 0, stream, counts,
                       W, sums, scanned, offsets, err, status);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}

// The fill pass's error bits and the tile count it was given (status[0..1]).
__global__ void fill_status(const int32_t* __restrict__ window_offsets, int32_t W,
                            const int32_t* __restrict__ err, int64_t* __restrict__ status)
{
    if (threadIdx.x == 0) {
        status[0] = *err;
        status[1] = window_offsets[W];
    }
}

// Per-call workspace of the converter, one allocation: status words (error
// bits, the hub count, two int64 results), the hub list as found and (fill)
// ordered heaviest first and, for the count pass, the counts, their int64
// scan and its temporaries.
struct ConvertScratch {
    int32_t* err;
    HubList hl;
    int32_t* hubs_sorted;
    int64_t* status;
    int32_t* counts;
    int64_t* tmp;
};

static f3s_status convert_scratch(StreamBuffer& buf, int32_t W, bool count, ConvertScratch& s)
{
    const size_t head = 32;   // err, hub count, pad, status[2]
    const size_t hubs = sizeof(int4) * ((size_t)W + 1);
    const size_t sorted = count ? 0 : sizeof(int32_t) * ((size_t)W + 1);
    const size_t counts = count ? sizeof(int32_t) * (size_t)W : 0;
    const size_t tmp = count ? sizeof(int64_t) * (size_t)offsets_sum_elems(W) : 0;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    F3S_TRY(buf.reserve(al(head) + al(hubs) + al(sorted) + al(counts) + al(tmp)));
    char* p = static_cast<char*>(buf.ptr);
    s.err = reinterpret_cast<int32_t*>(p);
    s.hl.count = s.err + 1;
    s.status = reinterpret_cast<int64_t*>(p + 16);
    p += al(head);
    s.hl.hubs = reinterpret_cast<int4*>(p);
    s.hl.cap = W + 1;
    p += al(hubs);
    s.hubs_sorted = reinterpret_cast<int32_t*>(p);
    p += al(sorted);
    s.counts = reinterpret_cast<int32_t*>(p);
    p += al(counts);
    s.tmp = reinterpret_cast<int64_t*>(p);
    return F3S_OK;
}

// Workgroups of `fn` (`threads` wide, `lds` bytes of dynamic LDS) resident
// on the current device at once: the grid of a persistent pass.  Cached per
// device, kernel and LDS size -- a conversion asks for three of them, and
// the runtime's occupancy query is host time on every call.
static f3s_status resident_workgroups(const void* fn, int threads, uint32_t lds, int64_t* out)
{
    struct Entry {
        int dev;
        const void* fn;
        int threads;
        uint32_t lds;
        int64_t resident;
    };
    constexpr int kEntries = 32;
    static std::mutex mu;
    static Entry cache[kEntries];
    static int used = 0, next = 0;
    int dev = 0;
    F3S_HIP(hipGetDevice(&dev));
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int i = 0; i < used; ++i) {
            const Entry& e = cache[i];
            if (e.dev == dev && e.fn == fn && e.threads == threads && e.lds == lds) {
                *out = e.resident;
                return F3S_OK;
            }
        }
    }
    int cus = 0, per_cu = 0;
    F3S_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    F3S_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds));
    const int64_t r = (int64_t)(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    {
        std::lock_guard<std::mutex> lock(mu);
        cache[next] = Entry{dev, fn, threads, lds, r};
        next = (next + 1) % kEntries;
        if (used < kEntries) ++used;
    }
    *out = r;
    return F3S_OK;
}

// One pass (count or fill) over all windows: the persistent kernel with as
// many workgroups as fit on the device at once, then the hub windows it
// listed (the hub count is known only on the device, so the hub launches
// have a fixed grid that walks the list).  Graphs too wide for one LDS
// bitmap run every window through the per-window kernel.
template <bool FILL>
static f3s_status launch_pass(const int32_t* row_ptr, const int32_t* col_idx, int32_t n,
                              int64_t nnz, int32_t W, int32_t* counts,
                              const int32_t* window_offsets, int32_t* block_col,
                              uint16_t* tile_mask, const HubList& hl, int32_t* hubs_sorted,
                              int32_t* err, hipStream_t stream)
{
    if (W <= 0) return F3S_OK;
    if ((int64_t)W > 32LL * kLightMaxWords) {
        hipLaunchKernelGGL((convert_hubs<FILL, kConvThreads>), dim3((unsigned)W), dim3(kConvThreads), 0,
                           stream, row_ptr, col_idx, n, nnz, W, counts, window_offsets,
                           block_col, tile_mask, nullptr, nullptr, err);
        F3S_HIP(hipGetLastError());
        return F3S_OK;
    }
    int64_t resident = 0;
    if (!FILL && (int64_t)W <= 32LL * kWaveCountMaxWords) {
        // small bitmap: the count pass with one window per wave
        const uint32_t lds = (uint32_t)(sizeof(uint32_t) * kWaveCountWaves * ((W + 31) / 32));
        F3S_TRY(resident_workgroups(reinterpret_cast<const void*>(count_waves),
                                    kWaveCountWaves * kWave, lds, &resident));
        const int64_t need = ceil_div(W, kWaveCountWaves);
        hipLaunchKernelGGL(count_waves, dim3((unsigned)(need < resident ? need : resident)),
                           dim3(kWaveCountWaves * kWave), lds, stream, row_ptr, col_idx, n, nnz,
                           W, counts, hl, err);
    } else {
        const LightLayout lay = light_layout(W, FILL);
        F3S_TRY(resident_workgroups(reinterpret_cast<const void*>(convert_light<FILL>),
                                    kConvThreads, lay.bytes, &resident));
        const unsigned grid = (unsigned)(W < resident ? W : resident);
        hipLaunchKernelGGL((convert_light<FILL>), dim3(grid), dim3(kConvThreads), lay.bytes,
                           stream, row_ptr, col_idx, n, nnz, W, counts, window_offsets, block_col,
                           tile_mask, hl, err);
    }
    F3S_HIP(hipGetLastError());
    if (!FILL) {
        const uint32_t lds = (uint32_t)(4 * ((((W + 31) / 32 + 3) & ~3) + kHubCountThreads / kWave + 4));
        F3S_TRY(resident_workgroups(reinterpret_cast<const void*>(count_hubs), kHubCountThreads,
                                    lds, &resident));
        hipLaunchKernelGGL(count_hubs, dim3((unsigned)(W < resident ? W : resident)),
                           dim3(kHubCountThreads), lds, stream, col_idx, n, nnz, W, counts, hl, err);
    } else {
        const int32_t rank_wgs = (int32_t)ceil_div(W < kHubSortCap ? W : kHubSortCap, 64);
        hipLaunchKernelGGL(rank_hubs, dim3((unsigned)rank_wgs), dim3(256), 0, stream, W, hl,
                           hubs_sorted);
        hipLaunchKernelGGL((convert_hubs<true, kHubThreads>),
                           dim3((unsigned)(W < kHubLaunch ? W : kHubLaunch)), dim3(kHubThreads), 0,
                           stream, row_ptr, col_idx, n, nnz, W, counts, window_offsets, block_col,
                           tile_mask, hubs_sorted, hl.count, err);
    }
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}

// Count call: tile counts, their scan into the caller's offsets, and one
// host round trip for the error bits and T.  Fill call: the lists, and one
// round trip for the error bits.
static f3s_status convert_impl(const int32_t* row_ptr, const int32_t* col_idx, int32_t n,
                               int64_t nnz, int32_t* window_offsets, int32_t* block_col,
                               uint16_t* tile_mask, int64_t* T_out, hipStream_t stream)
{
    const int32_t W = (int32_t)ceil_div(n, 16);
    const bool count = block_col == nullptr;
    StreamBuffer buf(stream);
    ConvertScratch s;
    F3S_TRY(convert_scratch(buf, W, count, s));
    F3S_HIP(hipMemsetAsync(s.err, 0, 2 * sizeof(int32_t), stream));   // err, hub count
    if (count) {
        F3S_TRY(launch_pass<false>(row_ptr, col_idx, n, nnz, W, s.counts, nullptr, nullptr,
                                   nullptr, s.hl, nullptr, s.err, stream));
        F3S_TRY(counts_to_offsets(s.counts, window_offsets, W, s.tmp, s.err, s.status, stream));
    } else {
        F3S_TRY(launch_pass<true>(row_ptr, col_idx, n, nnz, W, nullptr, window_offsets,
                                  block_col, tile_mask, s.hl, s.hubs_sorted, s.err, stream));
        hipLaunchKernelGGL(fill_status, dim3(1), dim3(64), 0, stream, window_offsets, W, s.err,
                           s.status);
    }
    F3S_HIP(hipGetLastError());
    int64_t* h = host_staging();
    F3S_HIP(hipMemcpyAsync(h, s.status, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    F3S_HIP(hipStreamSynchronize(stream));
    const int32_t h_err = (int32_t)h[0];
    const int64_t total = h[1];
    if (count) {
        // (on an error the offsets written are meaningless, as documented)
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
        *T_out = total;
        return F3S_OK;
    }
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
