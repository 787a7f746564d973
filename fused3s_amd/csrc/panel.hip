// panel.hip -- masked passes over community-ordered graphs, with the K/V rows
// that several row windows share staged once in LDS.
//
// The gathered pass (attention.hip) fetches every attended column's K and V
// rows once per row window; on large graphs it is bound by the per-CU
// vector-memory path (rows fetched per CU per cycle), not by HBM bytes.  On
// community-ordered graphs neighbouring windows attend many of the same
// columns.  A panel is kPanel = 16 consecutive windows, processed by one
// 16-wave workgroup per (panel, head), one wave per window:
//   * columns attended by at least two windows of the panel are "staged":
//     the workgroup loads their K and V rows into LDS once, kBlockSlots rows
//     at a time, and every wave runs its chunks over them from LDS;
//   * every other attended column is "direct": the wave gathers it as the
//     gathered pass does.
// Each wave's online softmax runs over its window's staged chunks block by
// block, then over its direct chunks, and writes the window's O rows.  The
// per-window chunk lists (32 columns each, LDS row offsets or global row
// references plus the rows that attend each column) are compiled once per
// graph by panel_compile; f3s_plan_compile builds them when the graph's
// panels fetch enough fewer rows this way (config 5: 1.9x fewer), and keeps
// the plain compiled lists otherwise.
//
// The reference has no counterpart (its kernel gathers per window,
// src/fused3s_v2.cu:81-246); results follow the same masked semantics
// (baselines/cpu_baseline.cpp:16-91) as the gathered pass.
#include <algorithm>
#include <new>

#include "attn_common.hpp"
#include "attn_plan.hpp"

namespace f3s {

constexpr int kPanel = 16;                    // windows per panel = waves per workgroup
constexpr int kPanelThreads = kPanel * kWave;
constexpr int kBlockSlots = 256;              // staged rows per LDS block
constexpr int kBlockRows = kBlockSlots + 1;   // + a row of zeros read by padding slots
constexpr int kMaxBlocks = 24;                // staged rows per panel <= 6,144
constexpr int kTableStride = kMaxBlocks + 1;  // per window: chunks of blocks 0..23, direct
constexpr int kPanelTiles = 8192;             // tiles of one panel the compile holds in LDS
constexpr int kTilesPerThread = kPanelTiles / kPanelThreads;
// Panels are used when they cut the plan's K/V row fetches by this factor.
constexpr double kPanelMinGain = 1.3;
static_assert(kTilesPerThread * kPanelThreads == kPanelTiles, "tile ranges per thread");
static_assert(kBlockSlots % 128 == 0, "block loads: 128 rows per workgroup pass");
static_assert(kMaxBlocks * kBlockSlots == 6144, "staged rows per panel");

struct PanelParams {
    const int32_t* nslots;      // [panel]: staged rows
    const int64_t* slot_base;   // [panel]: first staged row reference
    const uint32_t* slot_refs;  // staged rows' references (byte offsets of head 0)
    const int64_t* chunk_base;  // [(panel * 16 + window) * 25 + j], j = block or 24 = direct
    const uint32_t* records;    // 256-byte chunk records (32 references, 32 row masks)
    int64_t num_panels;
};

// ------------------------------------------------------------------ compile

struct PanelCompileLds {
    int32_t bc[kPanelTiles];      // block column of each tile of the panel
    uint16_t cm[kPanelTiles];     // columns the tile attends (OR of its row masks, < n)
    uint16_t twos[kPanelTiles];   // at an owner: columns of its block column attended by >= 2 windows
    int16_t own[kPanelTiles];     // owner tile (the first window's tile of this block column),
                                  // or -1 - (first staged slot) at the owner itself
    int32_t wb[kPanel + 1];       // window tile ranges, panel-local
    int32_t scan[kPanelThreads / kWave];
};

// Column mask of tile t: the columns < n that some row of the tile attends,
// and the tile's row masks (word k = rows 2k | 2k+1 << 16).
__device__ __forceinline__ uint32_t tile_columns(const int32_t* __restrict__ block_col,
                                                 const uint16_t* __restrict__ tile_mask,
                                                 int64_t t, int32_t n, int32_t& bc,
                                                 uint32_t (&wd)[8])
{
    const int32_t nbc = (n + 15) >> 4;
    bc = block_col[t];
#pragma unroll
    for (int k = 0; k < 8; ++k) wd[k] = 0;
    if ((uint32_t)bc >= (uint32_t)nbc) return 0;
    const int32_t left = n - bc * 16;
    const uint32_t vmask = left >= 16 ? 0xffffu : ((1u << left) - 1u);
    const uint4* mp = reinterpret_cast<const uint4*>(tile_mask + t * 16);
    const uint4 a = mp[0], b = mp[1];
    wd[0] = a.x; wd[1] = a.y; wd[2] = a.z; wd[3] = a.w;
    wd[4] = b.x; wd[5] = b.y; wd[6] = b.z; wd[7] = b.w;
    const uint32_t o = a.x | a.y | a.z | a.w | b.x | b.y | b.z | b.w;
    return (o | (o >> 16)) & vmask;
}

// Index of `key` in the ascending list s[lo, hi), or -1.
__device__ __forceinline__ int32_t find_sorted(const int32_t* s, int32_t lo, int32_t hi, int32_t key)
{
    while (lo < hi) {
        const int32_t mid = (lo + hi) >> 1;
        const int32_t v = s[mid];
        if (v == key) return mid;
        if (v < key) lo = mid + 1;
        else hi = mid;
    }
    return -1;
}

// Columns of `twos` whose rank (position among its set bits) is below k.
__device__ __forceinline__ uint32_t first_bits(uint32_t twos, int32_t k)
{
    uint32_t m = 0;
    for (int32_t i = 0; i < k && twos; ++i) {
        m |= twos & (0u - twos);
        twos &= twos - 1;
    }
    return m;
}

// One workgroup per panel.  Pass 1 (FILL = false) counts each window's
// chunks per block and direct chunks, the staged rows of the panel and the
// row fetches with and without staging; pass 2 writes the staged rows'
// references and the chunk records.  Panels with more than kPanelTiles tiles
// or more than kMaxBlocks blocks of shared columns keep every column direct.
template <bool FILL>
__global__ void __launch_bounds__(kPanelThreads)
panel_compile(const Item* __restrict__ items, int32_t W, const int32_t* __restrict__ block_col,
              const uint16_t* __restrict__ tile_mask, int32_t n, uint32_t ref_stride,
              uint32_t no_ref, int32_t* __restrict__ counts, int32_t* __restrict__ nslots,
              unsigned long long* __restrict__ stats, const int64_t* __restrict__ chunk_base,
              const int64_t* __restrict__ slot_base, uint32_t* __restrict__ slot_refs,
              uint32_t* __restrict__ records)
{
    __shared__ PanelCompileLds L;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int64_t P = blockIdx.x;
    if (tid == 0) {
        // window tile ranges from the plan's items (one whole window per
        // item, in window order), made monotone
        int32_t prev = 0;
        for (int k = 0; k <= kPanel; ++k) {
            const int64_t w = P * kPanel + k;
            const int32_t v = std::max(prev, w < W ? items[w].tb : items[W - 1].te);
            L.wb[k] = v;
            prev = v;
        }
    }
    __syncthreads();
    const int32_t t0 = L.wb[0];
    const int32_t nt = L.wb[kPanel] - t0;
    bool staged = nt <= kPanelTiles;

    if (staged) {
        // ---- tiles of the panel into LDS ----
        for (int32_t i = tid; i < nt; i += kPanelThreads) {
            int32_t bc;
            uint32_t wd[8];
            const uint32_t cm = tile_columns(block_col, tile_mask, (int64_t)t0 + i, n, bc, wd);
            L.bc[i] = bc;
            L.cm[i] = (uint16_t)cm;
        }
        __syncthreads();
        // ---- per tile: which columns >= 2 windows attend, and the owner ----
        for (int32_t i = tid; i < nt; i += kPanelThreads) {
            const int32_t bc = L.bc[i];
            uint32_t ones = 0, twos = 0;
            int32_t owner = -1;
            for (int k = 0; k < kPanel; ++k) {
                const int32_t lo = L.wb[k] - t0, hi = L.wb[k + 1] - t0;
                const int32_t idx = (i >= lo && i < hi) ? i : find_sorted(L.bc, lo, hi, bc);
                if (idx < 0) continue;
                const uint32_t m = L.cm[idx];
                if (owner < 0) owner = idx;
                twos |= ones & m;
                ones |= m;
            }
            L.twos[i] = (uint16_t)twos;
            L.own[i] = (int16_t)(owner == i ? -1 : owner);
        }
        __syncthreads();
        // ---- staged slots: owners in tile order ----
        const int32_t tb = tid * kTilesPerThread;
        int32_t mine = 0;
        for (int32_t k = 0; k < kTilesPerThread; ++k) {
            const int32_t i = tb + k;
            if (i < nt && L.own[i] == -1) mine += __popc(L.twos[i]);
        }
        int32_t S = 0;
        int32_t base = block_exclusive_scan<kPanelThreads>(mine, L.scan, S);
        staged = S <= kMaxBlocks * kBlockSlots;   // uniform over the workgroup
        if (staged) {
            for (int32_t k = 0; k < kTilesPerThread; ++k) {
                const int32_t i = tb + k;
                if (i < nt && L.own[i] == -1) {
                    const uint32_t tw = L.twos[i];
                    if (FILL) {
                        const int32_t bc = L.bc[i];
                        uint32_t* dst = slot_refs + slot_base[P] + base;
                        uint32_t rest = tw;
                        int32_t q = 0;
                        while (rest) {
                            const int c = __ffs(rest) - 1;
                            rest &= rest - 1;
                            dst[q++] = (uint32_t)(bc * 16 + c) * ref_stride;
                        }
                    }
                    L.own[i] = (int16_t)(-1 - base);
                    base += __popc(tw);
                }
            }
        }
        if (!FILL && tid == 0) {
            nslots[P] = staged ? S : 0;
            if (staged && S > 0) atomicAdd(&stats[1], (unsigned long long)S);
        }
        __syncthreads();
    } else if (!FILL && tid == 0) {
        nslots[P] = 0;
    }

    // ---- per window: chunk lists, staged per block, then direct ----
    const int32_t w = (int32_t)(P * kPanel + wave);
    const int64_t trow = (P * kPanel + wave) * kTableStride;
    if (w >= W) {
        if (!FILL && lane < kTableStride) counts[trow + lane] = 0;
        return;
    }
    const int rowstride = 64;   // u32 per record
    int64_t dpos = 0;
    int32_t bpos[kMaxBlocks];
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) bpos[j] = 0;
    unsigned long long all_cols = 0, direct_cols = 0;
    const int32_t wbeg = L.wb[wave], wend = L.wb[wave + 1];
    for (int32_t tt = wbeg; tt < wend; tt += kWave) {
        const int32_t t = tt + lane;
        int32_t bc = 0;
        uint32_t wd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t cm = 0, twos = 0;
        int32_t sbase = 0;
        if (t < wend) {
            cm = tile_columns(block_col, tile_mask, t, n, bc, wd);
            if (staged) {
                const int32_t i = t - t0;
                const int32_t o = L.own[i] < 0 ? i : L.own[i];
                twos = L.twos[o];
                sbase = -1 - L.own[o];
            }
        }
        const uint32_t dcols = cm & ~twos, scols = cm & twos;
        all_cols += __popc(cm);
        direct_cols += __popc(dcols);
        // direct columns: global row references
        {
            const int occ = __popc(dcols);
            const int incl = wave_scan_incl(occ);
            if (FILL && occ) {
                uint32_t* rec0 = records + chunk_base[trow + kMaxBlocks] * rowstride;
                int64_t q = dpos + incl - occ;
                uint32_t rest = dcols;
                while (rest) {
                    const int c = __ffs(rest) - 1;
                    rest &= rest - 1;
                    uint32_t* rec = rec0 + (q >> 5) * rowstride;
                    rec[q & 31] = (uint32_t)(bc * 16 + c) * ref_stride;
                    rec[32 + (q & 31)] = column_rows(wd, c);
                    ++q;
                }
            }
            dpos += __builtin_amdgcn_readlane(incl, kWave - 1);
        }
        if (staged) {
            // The tile's staged columns have consecutive slots sbase + rank
            // (rank among `twos`), so they fall into at most two blocks.
            const int32_t jlo = sbase / kBlockSlots;
            const uint32_t lo_mask = first_bits(twos, (jlo + 1) * kBlockSlots - sbase);
            const uint32_t s_lo = scols & lo_mask, s_hi = scols & ~lo_mask;
#pragma unroll
            for (int j = 0; j < kMaxBlocks; ++j) {
                const uint32_t mine = (j == jlo) ? s_lo : (j == jlo + 1 ? s_hi : 0u);
                const int occ = __popc(mine);
                const int incl = wave_scan_incl(occ);
                const int added = __builtin_amdgcn_readlane(incl, kWave - 1);
                if (added == 0) continue;
                if (FILL && occ) {
                    uint32_t* rec0 = records + chunk_base[trow + j] * rowstride;
                    int32_t q = bpos[j] + incl - occ;
                    uint32_t rest = mine;
                    while (rest) {
                        const int c = __ffs(rest) - 1;
                        rest &= rest - 1;
                        const int32_t slot = sbase + __popc(twos & ((1u << c) - 1u));
                        uint32_t* rec = rec0 + (q >> 5) * rowstride;
                        rec[q & 31] = (uint32_t)(slot - j * kBlockSlots);
                        rec[32 + (q & 31)] = column_rows(wd, c);
                        ++q;
                    }
                }
                bpos[j] += added;
            }
        }
    }
    if (!FILL) {
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < kMaxBlocks; ++j) counts[trow + j] = (bpos[j] + kChunk - 1) / kChunk;
            counts[trow + kMaxBlocks] = (int32_t)((dpos + kChunk - 1) / kChunk);
        }
        const unsigned long long a = wave_sum(all_cols), d = wave_sum(direct_cols);
        if (lane == 0) {
            atomicAdd(&stats[0], a);
            atomicAdd(&stats[1], d);
        }
        return;
    }
    // pad each list to whole chunks: staged with the zero row, direct out of range
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
        const int32_t nch = (bpos[j] + kChunk - 1) / kChunk;
        uint32_t* rec0 = records + chunk_base[trow + j] * rowstride;
        for (int32_t q = bpos[j] + lane; q < nch * kChunk; q += kWave) {
            uint32_t* rec = rec0 + (q >> 5) * rowstride;
            rec[q & 31] = (uint32_t)kBlockSlots;
            rec[32 + (q & 31)] = 0u;
        }
    }
    {
        const int64_t nch = (dpos + kChunk - 1) / kChunk;
        uint32_t* rec0 = records + chunk_base[trow + kMaxBlocks] * rowstride;
        for (int64_t q = dpos + lane; q < nch * kChunk; q += kWave) {
            uint32_t* rec = rec0 + (q >> 5) * rowstride;
            rec[q & 31] = no_ref;
            rec[32 + (q & 31)] = 0u;
        }
    }
}

// ----------------------------------------------------------------- the pass

// The wave's row-mask bits of one record's 32 slots (see kModeList).
__device__ __forceinline__ uint32_t record_valid(const uint32_t* m, int g, int rbit)
{
    const uint4 ra = *reinterpret_cast<const uint4*>(&m[32 + 4 * g]);
    const uint4 rb = *reinterpret_cast<const uint4*>(&m[48 + 4 * g]);
    return ((ra.x >> rbit) & 1u) | (((ra.y >> rbit) & 1u) << 1) | (((ra.z >> rbit) & 1u) << 2) |
           (((ra.w >> rbit) & 1u) << 3) | (((rb.x >> rbit) & 1u) << 4) |
           (((rb.y >> rbit) & 1u) << 5) | (((rb.z >> rbit) & 1u) << 6) |
           (((rb.w >> rbit) & 1u) << 7);
}

// Staged rows are 128 bytes, unpadded (the asynchronous LDS loads below fill
// 16 bytes per lane at consecutive addresses), with the 16-byte pieces of
// row s stored at position piece ^ (s & 7), so that the sixteen rows the
// lanes of one group read for an MFMA operand spread over the LDS banks.
__device__ __forceinline__ int piece_pos(uint32_t s, int piece) { return piece ^ (int)(s & 7u); }

// One chunk whose K and V rows are already in LDS: `m` holds the slots'
// rows in the block (K rows at kb, V rows at vb).
__device__ __forceinline__ void chunk_step_staged(RowState& st, const _Float16* __restrict__ kb,
                                                  const _Float16* __restrict__ vb,
                                                  const uint32_t* m, const h8 q0, const h8 q1,
                                                  uint32_t valid, int lane, float scale_log2)
{
    const int g = lane >> 4, r = lane & 15;
    const uint32_t sa = m[r], sb = m[16 + r];
    const h8 ka0 = *reinterpret_cast<const h8*>(&kb[sa * kD + 8 * piece_pos(sa, g)]);
    const h8 ka1 = *reinterpret_cast<const h8*>(&kb[sa * kD + 8 * piece_pos(sa, 4 + g)]);
    const h8 kb0 = *reinterpret_cast<const h8*>(&kb[sb * kD + 8 * piece_pos(sb, g)]);
    const h8 kb1 = *reinterpret_cast<const h8*>(&kb[sb * kD + 8 * piece_pos(sb, 4 + g)]);
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    s0 = mfma16x16x32(ka0, q0, s0);
    s0 = mfma16x16x32(ka1, q1, s0);
    s1 = mfma16x16x32(kb0, q0, s1);
    s1 = mfma16x16x32(kb1, q1, s1);
    const h8 pb = softmax_update(st, s0, s1, valid, scale_log2);
    // V^T operands: dims 4r..4r+3 of each slot, i.e. half of piece r / 2
    h8 va[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t sv = m[slot_of(g, j)];
        const h4 q = *reinterpret_cast<const h4*>(
            &vb[sv * kD + 8 * piece_pos(sv, r >> 1) + 4 * (r & 1)]);
#pragma unroll
        for (int t = 0; t < 4; ++t) va[t][j] = q[t];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) st.acc[t] = mfma16x16x32(va[t], pb, st.acc[t]);
}

// One block buffer (K rows, then V rows).  The kernel holds two, as two
// distinct LDS objects, and alternates them in code unrolled by two: the
// compiler then sees that the chunks read one object while the asynchronous
// loads write the other, and does not make the reads wait for those loads.
struct __align__(16) PanelBuf {
    _Float16 rows[2][kBlockRows * kD];
};
struct __align__(16) PanelMeta {
    uint32_t meta[kPanel][4 * 64];          // four chunk records per wave
};
static_assert(2 * sizeof(PanelBuf) + sizeof(PanelMeta) <= 160 * 1024, "LDS budget");
static_assert(kPanel / 2 * kChunk * kStageRow <= 2 * kBlockRows * kD,
              "direct-phase stages of half the waves fit in one block buffer");

// Loads one block's K and V rows (head h) into LDS buffer B without
// registers: 16 waves x 8 rows per round, lane l fetching piece
// (l & 7) ^ (row & 7) of row (l >> 3) so that it lands at position l & 7.
__device__ __forceinline__ void load_block_async(PanelBuf& B, __amdgpu_buffer_rsrc_t kres,
                                                 __amdgpu_buffer_rsrc_t vres, const uint32_t (&refs)[2],
                                                 uint32_t head_off, int wave, int lane)
{
    typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
    for (int i = 0; i < kBlockSlots / 128; ++i) {
        const int r0 = 128 * i + 8 * wave;
        const int piece = (lane & 7) ^ (lane >> 3);   // (r0 + (lane >> 3)) & 7 == lane >> 3
        const uint32_t off = refs[i] + head_off + 16 * piece;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kres, (lds_void*)(&B.rows[0][r0 * kD]), 16, off,
                                                 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, (lds_void*)(&B.rows[1][r0 * kD]), 16, off,
                                                 0, 0, 0);
    }
}

// References of this lane's rows of block j (row 8 * wave + lane / 8 + 128 i).
__device__ __forceinline__ void block_refs(const PanelParams& q, int64_t sb, int32_t S, int j,
                                           int wave, int lane, uint32_t (&refs)[2])
{
#pragma unroll
    for (int i = 0; i < kBlockSlots / 128; ++i) {
        const int row = 128 * i + 8 * wave + (lane >> 3);
        const int32_t slot = j * kBlockSlots + row;
        refs[i] = slot < S ? q.slot_refs[sb + slot] : kNoRow;
    }
}

// One 16-wave workgroup per (panel, head); wave k owns window 16 * panel + k.
// Staged blocks are double-buffered: while the waves run block j's chunks,
// block j + 1 streams into the other buffer.  The loads a wave needs during
// block j (its first four chunk records) are issued before block j + 1's
// asynchronous loads, which vmcnt would otherwise make them wait behind.
__global__ void __launch_bounds__(kPanelThreads) __attribute__((amdgpu_waves_per_eu(4)))
panel_attention_kernel(const AttnParams p, const PanelParams q)
{
    // distinct objects: reads of one need not wait for loads into another
    __shared__ PanelBuf buf0, buf1;
    __shared__ PanelMeta M;
    const int H = p.H;
    // wave-uniform values in scalar registers: their loads stay off vmcnt
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int g = lane >> 4, r = lane & 15;
    const uint32_t gb = (uint32_t)logical_block(p.xcd_contiguous);
    const int64_t P = (int64_t)(gb / (uint32_t)H);
    const int h = (int)(gb % (uint32_t)H);
    if (P >= q.num_panels) return;   // uniform over the workgroup
    const int32_t n = p.n;
    const int32_t w = (int32_t)(P * kPanel + wave);   // >= W: no window (last panel)
    const __amdgpu_buffer_rsrc_t qres = make_rsrc(p.Q, p.feat_bytes);
    const __amdgpu_buffer_rsrc_t kres = make_rsrc(p.K, p.feat_bytes);
    const __amdgpu_buffer_rsrc_t vres = make_rsrc(p.V, p.feat_bytes);
    const uint32_t head_off = (uint32_t)h * kRowBytes;
    const uint32_t row_stride = H * kRowBytes;
    const uint32_t piece_off = head_off + 16 * (lane & 7);
    const int rbit = (r & 1) ? 16 + (r >> 1) : (r >> 1);

    const int32_t qrow = w < p.W ? w * 16 + r : n;
    const uint32_t qref = qrow < n ? (uint32_t)qrow * row_stride : kNoRow;
    const h8 q0 = load_h8(qres, qref + head_off + 16 * g);
    const h8 q1 = load_h8(qres, qref + head_off + 16 * g + 64);

    RowState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) st.acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    // rows of zeros that padding slots of staged chunks read, in both buffers
    if (threadIdx.x < 4 * (kD / 8)) {
        const int which = threadIdx.x / (kD / 8), piece = threadIdx.x % (kD / 8);
        PanelBuf& zb = (which >> 1) ? buf1 : buf0;
        *reinterpret_cast<h8*>(&zb.rows[which & 1][kBlockSlots * kD + 8 * piece]) = h8{};
    }
    const int32_t S = q.nslots[P];
    const int64_t sb = q.slot_base[P];
    const int nb = (S + kBlockSlots - 1) / kBlockSlots;
    const int64_t trow = (P * kPanel + wave) * kTableStride;
    uint32_t* meta = M.meta[wave];
    const uint4* __restrict__ rec = reinterpret_cast<const uint4*>(q.records);
    // this wave's chunk ranges, one entry per lane (read back with readlane:
    // loads issued after the asynchronous ones would wait behind them)
    const int64_t my_cb = lane <= kTableStride ? q.chunk_base[trow + lane] : 0;
    auto chunk_at = [&](int j) -> int64_t {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)my_cb, j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(my_cb >> 32), j);
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };

    // ---- staged blocks ----
    uint32_t refs[2];
    uint4 first = make_uint4(0u, 0u, 0u, 0u);   // first four records of (window, block j)
    if (nb > 0) {
        block_refs(q, sb, S, 0, wave, lane, refs);
        const int64_t cb = chunk_at(0);
        if (cb < chunk_at(1)) first = rec[cb * 16 + lane];
        F3S_VMEM_SYNC();
        load_block_async(buf0, kres, vres, refs, head_off, wave, lane);
        if (nb > 1) block_refs(q, sb, S, 1, wave, lane, refs);
    }
    // Block j + 1's loads are issued before block j's chunks run; so that no
    // load the chunks need waits behind them (vmcnt counts in order), the
    // chunks' first four records are loaded in the iteration before.
    // block j: runs its chunks from `cur` while block j + 1 loads into `nxt`
    auto staged_block = [&](int j, const PanelBuf& cur, PanelBuf& nxt) {
        F3S_VMEM_SYNC();   // this wave's share of block j is in LDS
        __syncthreads();   // ... everyone's; and block j - 1's reads are done
        F3S_WAVE_LDS_SYNC();
        *reinterpret_cast<uint4*>(&meta[4 * lane]) = first;   // records loaded with block j
        F3S_WAVE_LDS_SYNC();
        const int64_t cb = chunk_at(j), ce = chunk_at(j + 1);
        if (j + 1 < nb) {
            const int64_t nb1 = chunk_at(j + 2);
            if (ce < nb1) first = rec[ce * 16 + lane];
            load_block_async(nxt, kres, vres, refs, head_off, wave, lane);
            if (j + 2 < nb) block_refs(q, sb, S, j + 2, wave, lane, refs);
        }
        for (int64_t c0 = cb; c0 < ce; c0 += 4) {
            if (c0 > cb) {   // records past the first four: loaded now, behind block j + 1
                const uint4 more = rec[c0 * 16 + lane];
                F3S_WAVE_LDS_SYNC();
                *reinterpret_cast<uint4*>(&meta[4 * lane]) = more;
                F3S_WAVE_LDS_SYNC();
            }
            const int nk = (int)min((int64_t)4, ce - c0);
            for (int k = 0; k < nk; ++k) {
                const uint32_t* m = meta + 64 * k;
                chunk_step_staged(st, cur.rows[0], cur.rows[1], m, q0, q1,
                                  record_valid(m, g, rbit), lane, p.scale_log2);
            }
        }
    };
    for (int j = 0; j < nb; j += 2) {
        staged_block(j, buf0, buf1);
        if (j + 1 < nb) staged_block(j + 1, buf1, buf0);
    }
    __syncthreads();   // every wave is done with the blocks: their rows become per-wave stages

    // ---- direct columns: gathered as in the compiled-list pass ----
    {
        _Float16* stage = &(wave < kPanel / 2 ? buf0 : buf1).rows[0][0] +
                          (wave % (kPanel / 2)) * kChunk * kStageRow;
        const int64_t cb = chunk_at(kMaxBlocks), ce = chunk_at(kMaxBlocks + 1);
        uint4 blk = cb < ce ? rec[cb * 16 + lane] : make_uint4(0u, 0u, 0u, 0u);
        for (int64_t c0 = cb; c0 < ce; c0 += 4) {
            F3S_WAVE_LDS_SYNC();
            *reinterpret_cast<uint4*>(&meta[4 * lane]) = blk;
            F3S_WAVE_LDS_SYNC();
            if (c0 + 4 < ce) blk = rec[(c0 + 4) * 16 + lane];
            const int nk = (int)min((int64_t)4, ce - c0);
            for (int k = 0; k < nk; ++k) {
                const uint32_t* m = meta + 64 * k;
                h8 krow[4], vrow[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t ref = m[(lane >> 3) + 8 * i];
                    krow[i] = load_h8(kres, ref + piece_off);
                    vrow[i] = load_h8(vres, ref + piece_off);
                }
                chunk_step(st, krow, q0, q1, record_valid(m, g, rbit), vrow, stage, lane,
                           p.scale_log2);
            }
        }
    }

    // ---- epilogue ----
    if (w >= p.W) return;
    const int32_t orow = w * 16 + r;
    float lrow = st.l + __shfl_xor(st.l, 16, kWave);
    lrow += __shfl_xor(lrow, 32, kWave);
    const float inv = lrow > 0.f ? 1.0f / lrow : 0.f;
    if (orow < n) {
        float* op = p.O + ((int64_t)orow * H + h) * kD + 16 * g;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float4 o4 = make_float4(st.acc[0][v] * inv, st.acc[1][v] * inv,
                                          st.acc[2][v] * inv, st.acc[3][v] * inv);
            *reinterpret_cast<float4*>(op + 4 * v) = o4;
        }
    }
}

// ------------------------------------------------------------------ host

// Compiles the plan's panels if they pay: returns F3S_OK with plan->panels
// set when built, F3S_OK with it clear when the graph does not qualify.
f3s_status panel_compile_plan(f3s_plan* plan, const int32_t* d_block_col,
                              const uint16_t* d_tile_mask, int32_t n, hipStream_t st)
{
    plan->panels = false;
    const int32_t W = plan->W;
    if (W == 0 || plan->T == 0 || !plan->natural_order || plan->masked.team != 1 ||
        plan->masked.num_split != 0 || wide_features(n, plan->H))
        return F3S_OK;
    const int64_t np = ceil_div(W, kPanel);
    const int64_t entries = np * kPanel * kTableStride;
    const auto* items = reinterpret_cast<const Item*>(plan->masked.items.ptr);
    DeviceBuffer counts, stats, tmp;
    F3S_TRY(counts.reserve(sizeof(int32_t) * (size_t)entries));
    F3S_TRY(plan->pn_nslots.reserve(sizeof(int32_t) * (size_t)np));
    F3S_TRY(stats.reserve(2 * sizeof(unsigned long long)));
    F3S_TRY(tmp.reserve(sizeof(int64_t) * (size_t)scan_tmp_elems(entries > np ? entries : np)));
    F3S_HIP(hipMemsetAsync(stats.ptr, 0, 2 * sizeof(unsigned long long), st));
    const uint32_t ref_stride = (uint32_t)plan->H * kRowBytes;
    auto* cnt = reinterpret_cast<int32_t*>(counts.ptr);
    auto* ns = reinterpret_cast<int32_t*>(plan->pn_nslots.ptr);
    auto* sts = reinterpret_cast<unsigned long long*>(stats.ptr);
    hipLaunchKernelGGL(panel_compile<false>, dim3((unsigned)np), dim3(kPanelThreads), 0, st,
                       items, W, d_block_col, d_tile_mask, n, ref_stride, kNoRow, cnt,
                       ns, sts, nullptr, nullptr, nullptr, nullptr);
    F3S_HIP(hipGetLastError());
    unsigned long long h_stats[2] = {0, 0};
    F3S_HIP(hipMemcpyAsync(h_stats, sts, sizeof h_stats, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    // stats[0]: (window, column) pairs = row fetches of the gathered pass;
    // stats[1]: staged rows + direct columns = row fetches with panels
    plan->pn_rows_gathered = (int64_t)h_stats[0];
    plan->pn_rows_fetched = (int64_t)h_stats[1];
    if (h_stats[1] == 0 || (double)h_stats[0] < kPanelMinGain * (double)h_stats[1]) {
        plan->pn_nslots.release();
        return F3S_OK;
    }
    F3S_TRY(plan->pn_chunk_base.reserve(sizeof(int64_t) * (size_t)(entries + 1)));
    F3S_TRY(plan->pn_slot_base.reserve(sizeof(int64_t) * (size_t)(np + 1)));
    auto* cb = reinterpret_cast<int64_t*>(plan->pn_chunk_base.ptr);
    auto* sbp = reinterpret_cast<int64_t*>(plan->pn_slot_base.ptr);
    auto* tp = reinterpret_cast<int64_t*>(tmp.ptr);
    F3S_TRY(exclusive_scan_i32_to_i64(cnt, cb, entries, tp, st));
    F3S_TRY(exclusive_scan_i32_to_i64(ns, sbp, np, tp, st));
    int64_t totals[2] = {0, 0};
    F3S_HIP(hipMemcpyAsync(&totals[0], cb + entries, 8, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipMemcpyAsync(&totals[1], sbp + np, 8, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    // four records of padding: the pass reads records in blocks of four
    F3S_TRY(plan->pn_records.reserve(sizeof(uint32_t) * 64 * (size_t)(totals[0] + 4)));
    F3S_TRY(plan->pn_slot_refs.reserve(sizeof(uint32_t) * (size_t)(totals[1] + 1)));
    hipLaunchKernelGGL(panel_compile<true>, dim3((unsigned)np), dim3(kPanelThreads), 0, st,
                       items, W, d_block_col, d_tile_mask, n, ref_stride, kNoRow,
                       nullptr, nullptr, nullptr, cb, sbp,
                       reinterpret_cast<uint32_t*>(plan->pn_slot_refs.ptr),
                       reinterpret_cast<uint32_t*>(plan->pn_records.ptr));
    F3S_HIP(hipGetLastError());
    F3S_HIP(hipStreamSynchronize(st));
    plan->num_panels = np;
    plan->num_panel_chunks = totals[0];
    plan->panels = true;
    return F3S_OK;
}

void panel_launch(const f3s_plan* plan, const AttnParams& p, hipStream_t st)
{
    PanelParams q;
    q.nslots = reinterpret_cast<const int32_t*>(plan->pn_nslots.ptr);
    q.slot_base = reinterpret_cast<const int64_t*>(plan->pn_slot_base.ptr);
    q.slot_refs = reinterpret_cast<const uint32_t*>(plan->pn_slot_refs.ptr);
    q.chunk_base = reinterpret_cast<const int64_t*>(plan->pn_chunk_base.ptr);
    q.records = reinterpret_cast<const uint32_t*>(plan->pn_records.ptr);
    q.num_panels = plan->num_panels;
    hipLaunchKernelGGL(panel_attention_kernel, dim3((unsigned)(plan->num_panels * p.H)),
                       dim3(kPanelThreads), 0, st, p, q);
}

}  // namespace f3s
