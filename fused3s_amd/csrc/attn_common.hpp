// attn_common.hpp -- building blocks of the fused attention kernels
// (attention.hip): operand types and layouts, row references, the per-row
// online-softmax state and the 32-column MFMA chunk step.
#pragma once

#include <math.h>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kD = 64;             // feature dim per head (FEAT_DIM_FIXED, fused3s_v2.cu:41)
constexpr int kRowBytes = kD * 2;  // one fp16 K/V/Q row of one head
constexpr int kChunk = 32;         // attended columns per MFMA step
constexpr int kRing = 256;         // column ring entries per wave
constexpr int kPartialFloats = 16 * kD + 32;   // O[16][64], m[16], l[16]
constexpr int kXcds = 8;           // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr int kMaxHeads = 64;
// Word 3 of a raw buffer descriptor for the gfx9 family (incl. gfx950):
// 32-bit data format, no swizzle.  Offsets >= num_records read as 0.
constexpr int32_t kBufferFlags = 0x00020000;
// Row-mask layout in the ring: bit k = row 2k, bit 16 + k = row 2k + 1.

struct Item {
    int32_t w, tb, te, slot;       // slot < 0: whole window, write O directly;
                                   // w < 0: no window (an invalid order entry), skipped
};

struct SplitInfo {
    int32_t w, first_slot, nseg, pad;
};

// Staging rows of 144 bytes: the 16 lanes that read one 16-byte piece of
// 16 consecutive rows then hit 64 distinct LDS banks.
constexpr int kStageRow = kD + 8;   // halves

// The epilogue stages O (16 rows of 64 floats) through a wave's stage, rows
// 68 floats apart so the 16 rows start in different LDS banks.
constexpr int kOutStride = kD + 4;   // floats
// O stores of the epilogue: whole rows (four per instruction, see
// fused_attention_kernel), non-temporal -- O is written once and never read
// by the pass, so its lines should not displace the K/V rows in the caches.
__device__ __forceinline__ void store_out(float* dst, f4 v)
{
    __builtin_nontemporal_store(v, reinterpret_cast<f4*>(dst));
}

struct __align__(16) WaveLds {
    uint32_t off[kRing];   // byte offset of the slot's K/V row for this wave's head
    uint32_t rm[kRing];    // rows of the window that attend the slot
    _Float16 stage[kChunk * kStageRow];   // the chunk's K rows, then its V rows; O at the end
};
static_assert(sizeof(_Float16) * kChunk * kStageRow >= sizeof(float) * 16 * kOutStride,
              "the stage holds a window's O rows");

struct AttnParams {
    const _Float16* Q;
    const _Float16* K;
    const _Float16* V;
    float* O;
    const int32_t* window_offsets;   // unplanned launch only
    const int32_t* block_col;
    const uint16_t* tile_mask;       // NULL: tile-dense semantics
    const int32_t* window_order;     // unplanned launch only (NULL: natural order)
    const Item* items;               // planned launch (NULL: one item per window)
    int64_t num_items;
    int32_t W, n;
    int32_t H;                       // heads, 1 <= H <= kMaxHeads
    float scale_log2;
    int32_t xcd_contiguous;          // map consecutive items to the same XCD
    uint32_t feat_bytes;             // bytes of Q (= K = V) in a narrow launch, else 0
    float* partials;
    const SplitInfo* splits;
    int64_t num_split;
    const int32_t* chunk_base;       // compiled plan: item i owns chunks [cb[i], cb[i+1])
    const uint32_t* columns;         // compiled plan: per chunk 32 row offsets, 32 row masks
    int32_t team;                    // waves per window (1, or kTeamSmall / kTeamLarge)
    int32_t heavy_mode;              // order-sequence launches: 0 every entry; 1 all but the
                                     // heavy windows among the first kHeavyMaxWindows
                                     // entries; 2 only those (teams)
    const int32_t* slot_split;       // planned launch: the split window of each partial slot
    int32_t* counters;               // planned launch: segments arrived per (split window,
                                     // head); zero between passes
};

// A window is heavy for the unplanned launch's teams when its tiles exceed
// both kHeavyMinTiles and kHeavyMeanFactor x the mean window; on the
// library's schedule the first kHeavyMaxWindows of them (heaviest first),
// in an order's sequence those among its first kHeavyMaxWindows entries, run
// as 16-wave teams.
constexpr int32_t kHeavyMinTiles = 1024;
constexpr int32_t kHeavyMeanFactor = 8;
constexpr int32_t kHeavyMaxWindows = 512;
__host__ __device__ __forceinline__ int32_t heavy_tiles(int32_t T, int32_t W, int32_t min_tiles,
                                                        int32_t factor)
{
    const int64_t mean = W > 0 ? ((int64_t)T + W - 1) / W : 0;
    const int64_t thr = mean * factor;
    return (int32_t)(thr > min_tiles ? thr : min_tiles);
}

// Small graphs: a team of waves in one workgroup shares each row window, each
// wave taking an even share of the window's tiles (cut at tile pairs, the
// tile-dense chunk), and the team merges its (m, l, O) states through LDS, so
// the heaviest window no longer runs as one wave's serial chain and no merge
// launch is needed.  A window of fewer tile pairs than waves has only as many
// parts, on waves 0.. (the others have nothing to do and publish nothing).
// Number of non-empty parts of [tb, te):
__host__ __device__ __forceinline__ int32_t team_parts(int32_t tb, int32_t te, int32_t team)
{
    const int64_t pairs = ((int64_t)te - tb + 1) / 2;
    return (int32_t)(pairs < team ? pairs : team);
}
// Start of part k of a window's tiles [tb, te) (part k = [part(k), part(k + 1))):
__host__ __device__ __forceinline__ int32_t team_part(int32_t tb, int32_t te, int32_t k,
                                                      int32_t team)
{
    const int64_t pairs = ((int64_t)te - tb + 1) / 2;
    const int64_t parts = pairs < team ? pairs : team;
    if (k >= parts) return te;
    const int64_t a = tb + 2 * ((pairs * k) / parts);
    return (int32_t)(a < te ? a : te);
}
constexpr int kTeamSmall = 4;
constexpr int kTeamLarge = 16;

// Team size for W windows of H heads (measured on MI355X over graphs of
// 170 to 62,500 windows): masked windows hold a few chunks each, so teams
// of 4 pay while the windows leave most SIMDs idle; a tile-dense window is
// ~15x the work, so teams of 16 pay on the smallest graphs and teams of 4
// a little further.  1 = one wave per window or segment.
static inline int32_t team_for(int64_t W, int32_t H, bool masked)
{
    const int64_t units = W * H;
    if (masked) return units <= 1024 ? kTeamSmall : 1;
    if (units <= 512) return kTeamLarge;
    return units <= 2048 ? kTeamSmall : 1;
}

// Workgroup index -> logical block.  The dispatcher deals workgroups to the
// 8 XCDs round-robin; with `xcd_contiguous` each XCD instead receives one
// contiguous range of logical blocks, so windows that share neighbours
// (community-ordered graphs) share one XCD's L2.
__device__ __forceinline__ int64_t logical_block(int32_t xcd_contiguous)
{
    const int64_t b = blockIdx.x;
    if (!xcd_contiguous) return b;
    const int64_t G = gridDim.x;
    const int64_t x = b % kXcds, q = G / kXcds, rem = G % kXcds;
    return x * q + min(x, rem) + b / kXcds;
}

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kBufferFlags);
}

// One 16-byte piece of a row; AUX is the load's cache-policy immediate (0,
// or kStreamLoad: non-temporal, for rows read once).
template <int AUX = 0>
__device__ __forceinline__ h8 load_h8(__amdgpu_buffer_rsrc_t rs, uint32_t off)
{
    u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, AUX);
    return __builtin_bit_cast(h8, v);
}

// Cache policy of the tile-dense pass.  A tile whose block column lies
// within kNearCols block columns of its window's own (4,096 nodes either
// side) is "near": on a graph whose windows mostly attend near tiles (a
// community-ordered graph) the neighbouring windows, which run on the same
// XCD at about the same time, read its rows again, while a far tile's rows
// are read once.  There the far tiles' rows are loaded non-temporally, so
// they stream past the L2 instead of evicting the near rows (config 5
// tile-dense: 27 % fewer bytes below the L2, 12 % faster).  Where fewer
// than a quarter of an item's tiles are near (a random graph, whose rows
// nothing reuses in time) every load keeps the default policy:
// non-temporal loads over the whole pass measured much slower there.
constexpr int kStreamLoad = 2;      // the `nt` bit of a buffer load's cache policy
constexpr int32_t kNearCols = 256;

// Cache policy sc0 | sc1 (system coherence) of a buffer load or store: the
// store writes through to memory and the load does not take a line another
// XCD's L2 may hold stale.  The segments of a split window hand their
// partials to the last of them this way (each XCD has its own L2), instead
// of device-scope fences, which on gfx950 write back and invalidate the
// whole L2 of the XCD.
constexpr int kCoherent = 1 | 16;
// s_waitcnt immediate (gfx9 encoding) for vmcnt(0), expcnt and lgkmcnt left
// open: wait until every vector memory operation of the wave is done.
constexpr int kWaitVmcnt0 = 0x0F70;

// Inclusive prefix sum over the wave with DPP row shifts and row broadcasts.
__device__ __forceinline__ int wave_scan_incl(int x)
{
    int s = x;
    s += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    s += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    s += __builtin_amdgcn_update_dpp(0, x, 0x113, 0xf, 0xf, true);   // row_shr:3
    s += __builtin_amdgcn_update_dpp(0, s, 0x114, 0xf, 0xe, true);   // row_shr:4, lanes 4-15
    s += __builtin_amdgcn_update_dpp(0, s, 0x118, 0xf, 0xc, true);   // row_shr:8, lanes 8-15
    s += __builtin_amdgcn_update_dpp(0, s, 0x142, 0xa, 0xf, true);   // row_bcast:15 -> rows 1, 3
    s += __builtin_amdgcn_update_dpp(0, s, 0x143, 0xc, 0xf, true);   // row_bcast:31 -> rows 2, 3
    return s;
}

// Rows of a tile that attend its column c, from the tile's 16 row masks
// packed two per word (word k = rows 2k | 2k+1 << 16).
__device__ __forceinline__ uint32_t column_rows(const uint32_t (&wd)[8], int c)
{
    uint32_t x = (wd[0] >> c) & 0x00010001u;
#pragma unroll
    for (int k = 1; k < 8; ++k) x |= ((wd[k] >> c) & 0x00010001u) << k;
    return x;
}

// max over the lanes r, r+16, r+32, r+48 (the four lanes that hold row r),
// with the gfx950 row and half-wave swaps (no LDS crossbar).
__device__ __forceinline__ float row_max4(float x)
{
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __builtin_fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __builtin_fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Slot order of the 8 logits a lane holds (lane group g): S^T tile 0 rows
// 4g..4g+3, then tile 1 rows 16+4g..16+4g+3.  Used as the k order of P.V.
__device__ __forceinline__ int slot_of(int g, int j) { return (j < 4) ? 4 * g + j : 16 + 4 * g + (j - 4); }

// Out-of-range buffer offset for slots with no row: loads read 0.  The
// largest offset added to it (head offset + piece + 64 for Q's second half,
// under 8,256 bytes at 64 heads) cannot wrap past 2^32, and the feature
// tensors are required to end at or below it.
constexpr uint32_t kNoRow = 0xffffc000u;
// Wide launches (feature tensors beyond kNoRow bytes) address rows by node
// index with 64-bit loads; kNoIdx marks a slot with no row.
constexpr uint32_t kNoIdx = 0xffffffffu;

// A row reference is the node's byte offset (node * row stride) in a narrow
// launch and the node index in a wide one; `extra` adds the head and piece.
template <bool WIDE>
__device__ __forceinline__ h8 load_ref(__amdgpu_buffer_rsrc_t rs, const _Float16* base,
                                       uint32_t ref, uint32_t row_stride, uint32_t extra)
{
    if constexpr (!WIDE) {
        return load_h8<0>(rs, ref + extra);
    } else {
        h8 v = {};
        if (ref != kNoIdx)
            v = *reinterpret_cast<const h8*>(reinterpret_cast<const char*>(base) +
                                             (uint64_t)ref * row_stride + extra);
        return v;
    }
}

// Online-softmax state of one row (lane (g, r) holds row r).  The running
// max m (log2 domain) is moved only when a chunk's max exceeds it by more
// than kLazy, so most chunks skip the rescale; weights exp2(x - m) then stay
// <= 2^kLazy, well inside fp16 range, and numerator and denominator share m.
struct RowState {
    float m;
    float l;        // this lane's share of the running sum of row r
    f4 acc[4];      // O^T accumulators: dims 16g + 4v + t of row r (t = index, v = lane element)
};
constexpr float kLazy = 8.0f;

// The masked online-softmax update of row r for one chunk's logits S^T (s0:
// slots 4g..4g+3, s1: slots 16+4g..16+4g+3 of the lane's group g); returns
// the fp16 weights P^T in B-operand layout for the P.V product.
__device__ __forceinline__ h8 softmax_update(RowState& st, const f4 s0, const f4 s1,
                                             uint32_t valid, float scale_log2)
{
    float x[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        x[v] = ((valid >> v) & 1u) ? s0[v] * scale_log2 : -INFINITY;
        x[4 + v] = ((valid >> (4 + v)) & 1u) ? s1[v] * scale_log2 : -INFINITY;
    }
    float cm = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) cm = __builtin_fmaxf(cm, x[j]);
    cm = row_max4(cm);
    if (__ballot(cm > st.m + kLazy)) {
        if (cm > st.m + kLazy) {
            const float corr = fast_exp2(st.m - cm);   // m = -inf -> 0
            st.l *= corr;
#pragma unroll
            for (int t = 0; t < 4; ++t) st.acc[t] *= corr;
            st.m = cm;
        }
    }
    const float mu = (st.m == -INFINITY) ? 0.f : st.m;
    h8 pb;
#pragma unroll
    for (int j = 0; j < 8; ++j) pb[j] = (_Float16)fast_exp2(x[j] - mu);
    // the sum uses the rounded weights P.V uses
    const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    st.l = __builtin_amdgcn_fdot2(h2{pb[0], pb[1]}, ones, st.l, false);
    st.l = __builtin_amdgcn_fdot2(h2{pb[2], pb[3]}, ones, st.l, false);
    st.l = __builtin_amdgcn_fdot2(h2{pb[4], pb[5]}, ones, st.l, false);
    st.l = __builtin_amdgcn_fdot2(h2{pb[6], pb[7]}, ones, st.l, false);
    return pb;
}

// One chunk of 32 attended columns for the wave: S^T = K.Q^T, the masked
// online-softmax update of row r, and O^T += V^T.P^T.  `valid` bit j says
// whether the lane's j-th logit (slot slot_of(g, j)) is attended by row r.
// krow[i] / vrow[i] hold 16 bytes (piece lane & 7) of the K / V row of slot
// (lane >> 3) + 8i: gathered in this layout, eight consecutive lanes read one
// 128-byte row, which the vector-memory address unit coalesces; the LDS
// stage then hands K out in MFMA A-operand layout (lane (g, r): slots r and
// 16 + r, dims 8g.. and 32 + 8g..) and V transposed.
__device__ __forceinline__ void chunk_step(RowState& st, const h8 (&krow)[4],
                                           const h8 q0, const h8 q1, uint32_t valid,
                                           const h8 (&vrow)[4], _Float16* __restrict__ stage,
                                           int lane, float scale_log2)
{
    const int g = lane >> 4, r = lane & 15;
    F3S_WAVE_LDS_SYNC();   // previous chunk's V reads are complete
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = (lane >> 3) + 8 * i;
        *reinterpret_cast<h8*>(&stage[s * kStageRow + 8 * (lane & 7)]) = krow[i];
    }
    F3S_WAVE_LDS_SYNC();
    const h8 ka0 = *reinterpret_cast<const h8*>(&stage[r * kStageRow + 8 * g]);
    const h8 ka1 = *reinterpret_cast<const h8*>(&stage[r * kStageRow + 32 + 8 * g]);
    const h8 kb0 = *reinterpret_cast<const h8*>(&stage[(16 + r) * kStageRow + 8 * g]);
    const h8 kb1 = *reinterpret_cast<const h8*>(&stage[(16 + r) * kStageRow + 32 + 8 * g]);
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    s0 = mfma16x16x32(ka0, q0, s0);
    s0 = mfma16x16x32(ka1, q1, s0);
    s1 = mfma16x16x32(kb0, q0, s1);
    s1 = mfma16x16x32(kb1, q1, s1);
    const h8 pb = softmax_update(st, s0, s1, valid, scale_log2);

    // V through the same stage, transposed into A operands
    F3S_WAVE_LDS_SYNC();   // K reads are complete
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = (lane >> 3) + 8 * i;
        *reinterpret_cast<h8*>(&stage[s * kStageRow + 8 * (lane & 7)]) = vrow[i];
    }
    F3S_WAVE_LDS_SYNC();
    h8 va[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const h4 q = *reinterpret_cast<const h4*>(&stage[slot_of(g, j) * kStageRow + 4 * r]);
#pragma unroll
        for (int t = 0; t < 4; ++t) va[t][j] = q[t];
    }
    // A row i of output tile t is dim 4i + t, so lane (g, r) holds dims
    // 16g + 4v + t of row r.
#pragma unroll
    for (int t = 0; t < 4; ++t) st.acc[t] = mfma16x16x32(va[t], pb, st.acc[t]);
}

// Feature tensors whose bytes exceed the 32-bit offset range of the narrow
// path (kNoRow, just under 4 GiB) are addressed with 64-bit loads.
static inline bool wide_features(int32_t n, int32_t H)
{
    return (int64_t)n * H * kRowBytes > (int64_t)kNoRow;
}

}  // namespace f3s
