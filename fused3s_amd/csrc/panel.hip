// panel.hip -- tile-dense passes over community-ordered graphs, with the
// tiles that several row windows share staged once in LDS.
//
// Under the tile-dense semantics (the reference kernel's, tests/
// test_fused_3s_v2.cu:17-59) a window attends every column < n of each of
// its active tiles, so a block column active in several windows costs the
// gathered pass (attention.hip) its 16 K and V rows once per window; on large
// graphs that pass is bound by the rows each CU fetches.  On community-ordered
// graphs most tiles of neighbouring windows share block columns (config 5:
// ~60 % of the tiles, each shared by ~15 of 16 windows).  A panel is
// kPanel = 16 consecutive windows, processed by one 16-wave workgroup per
// (panel, head), one wave per window:
//   * block columns active in at least two windows of the panel are staged:
//     the workgroup loads their K and V rows into LDS once, kBlockSlots rows
//     at a time (double-buffered asynchronous LDS loads), and every wave
//     runs its window's chunks over them;
//   * each wave writes its window's (m, l, unnormalised O) partial;
//   * the remaining ("residual") tiles of each window run through the
//     gathered tile-dense pass, which folds the partial in before writing O.
// The staging lists (per window and block: chunks of 32 staged columns) and
// the residual tile lists are compiled once per graph by panel_compile, and
// f3s_plan_compile keeps them only when they cut the K/V row fetches by
// kPanelMinGain.
//
// Masked passes gain nothing from this: the same scheme fetched 1.9x fewer
// rows on config 5 and ran slower (LDS holds too few bytes in flight).
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
constexpr int kPanelTiles = 8192;             // tiles of one panel the compile holds in LDS
constexpr int kTilesPerThread = kPanelTiles / kPanelThreads;
// Rows 0-15 in the records' row-mask layout (bit k = row 2k, 16 + k = row 2k + 1).
constexpr uint32_t kAllRows = 0x00ff00ffu;
// Panels are used when they cut the pass's K/V row fetches by this factor.
constexpr double kPanelMinGain = 1.5;
static_assert(kTilesPerThread * kPanelThreads == kPanelTiles, "tile ranges per thread");
static_assert(kBlockSlots % 128 == 0, "block loads: 128 rows per workgroup pass");
static_assert(kMaxBlocks * kBlockSlots == 6144, "staged rows per panel");
static_assert(kMaxBlocks + 1 <= kWave, "chunk ranges are held one per lane");

struct PanelParams {
    const int32_t* nslots;      // [panel]: staged rows
    const int64_t* slot_base;   // [panel]: first staged row reference
    const uint32_t* slot_refs;  // staged rows' references (byte offsets of head 0)
    const int64_t* chunk_base;  // [(panel * 16 + window) * kMaxBlocks + block]
    const uint32_t* records;    // 256-byte chunk records (32 slots, 32 row masks)
    float* partials;            // [window][head]: (O, m, l) of the staged tiles
    int64_t num_panels;
};

// ------------------------------------------------------------------ compile

struct PanelCompileLds {
    int32_t bc[kPanelTiles];      // block column of each tile of the panel
    uint16_t cm[kPanelTiles];     // the tile's columns < n (0 for an invalid block column)
    uint16_t twos[kPanelTiles];   // at an owner: its columns active in >= 2 windows
    int16_t own[kPanelTiles];     // owner tile (the first window's tile of this block column),
                                  // or -1 - (first staged slot) at the owner itself
    int32_t wb[kPanel + 1];       // window tile ranges, panel-local
    int32_t scan[kPanelThreads / kWave];
};

__device__ __forceinline__ uint32_t dense_columns(int32_t bc, int32_t n)
{
    const int32_t nbc = (n + 15) >> 4;
    if ((uint32_t)bc >= (uint32_t)nbc) return 0;
    const int32_t left = n - bc * 16;
    return left >= 16 ? 0xffffu : ((1u << left) - 1u);
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
// staged chunks per block and residual tiles, the staged rows of the panel
// and the K/V row fetches with and without staging; pass 2 writes the staged
// rows' references, the chunk records and the residual tile lists.  Panels
// with more than kPanelTiles tiles or more than kMaxBlocks blocks of shared
// columns stage nothing.  Window tile ranges come from the plan's items, in
// window order: `team` consecutive items per window, no split windows.
template <bool FILL>
__global__ void __launch_bounds__(kPanelThreads)
panel_compile(const Item* __restrict__ items, int32_t team, int32_t W,
              const int32_t* __restrict__ block_col, int32_t n, uint32_t ref_stride,
              int32_t* __restrict__ counts,
              int32_t* __restrict__ res_counts, int32_t* __restrict__ nslots,
              unsigned long long* __restrict__ stats, const int64_t* __restrict__ chunk_base,
              const int64_t* __restrict__ res_base, const int64_t* __restrict__ slot_base,
              uint32_t* __restrict__ slot_refs, uint32_t* __restrict__ records,
              int32_t* __restrict__ res_block_col)
{
    __shared__ PanelCompileLds L;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int64_t P = blockIdx.x;
    if (tid == 0) {   // window tile ranges, made monotone
        int32_t prev = 0;
        for (int k = 0; k <= kPanel; ++k) {
            const int64_t w = P * kPanel + k;
            const int32_t v =
                std::max(prev, w < W ? items[w * team].tb : items[(int64_t)W * team - 1].te);
            L.wb[k] = v;
            prev = v;
        }
    }
    __syncthreads();
    const int32_t t0 = L.wb[0];
    const int32_t nt = L.wb[kPanel] - t0;
    bool staged = nt <= kPanelTiles;

    if (staged) {
        for (int32_t i = tid; i < nt; i += kPanelThreads) {
            const int32_t bc = block_col[(int64_t)t0 + i];
            L.bc[i] = bc;
            L.cm[i] = (uint16_t)dense_columns(bc, n);
        }
        __syncthreads();
        // per tile: the columns of its block column active in >= 2 windows
        // (all of them or none), and the owner
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
        // staged slots: owners in tile order
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

    // ---- per window: staged chunks per block, residual tiles ----
    const int32_t w = (int32_t)(P * kPanel + wave);
    const int64_t trow = (P * kPanel + wave) * kMaxBlocks;
    if (w >= W) {
        if (!FILL && lane < kMaxBlocks) counts[trow + lane] = 0;
        return;
    }
    constexpr int kRec = 64;   // u32 per record
    int32_t rpos = 0;
    int32_t bpos[kMaxBlocks];
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) bpos[j] = 0;
    unsigned long long all_cols = 0, res_cols = 0;
    const int32_t wbeg = L.wb[wave], wend = L.wb[wave + 1];
    for (int32_t tt = wbeg; tt < wend; tt += kWave) {
        const int32_t t = tt + lane;
        int32_t bc = -1;
        uint32_t cm = 0, twos = 0;
        int32_t sbase = 0;
        if (t < wend) {
            bc = block_col[t];
            cm = dense_columns(bc, n);
            if (staged) {
                const int32_t i = t - t0;
                const int32_t o = L.own[i] < 0 ? i : L.own[i];
                twos = L.twos[o];
                sbase = -1 - L.own[o];
            }
        }
        const uint32_t scols = cm & twos;
        const bool residual = cm != 0 && scols == 0;
        all_cols += __popc(cm);
        res_cols += residual ? __popc(cm) : 0;
        // residual tiles, in tile order
        {
            const int occ = residual ? 1 : 0;
            const int incl = wave_scan_incl(occ);
            if (FILL && residual) res_block_col[res_base[w] + rpos + incl - 1] = bc;
            rpos += __builtin_amdgcn_readlane(incl, kWave - 1);
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
                    uint32_t* rec0 = records + chunk_base[trow + j] * kRec;
                    int32_t q = bpos[j] + incl - occ;
                    uint32_t rest = mine;
                    while (rest) {
                        const int c = __ffs(rest) - 1;
                        rest &= rest - 1;
                        const int32_t slot = sbase + __popc(twos & ((1u << c) - 1u));
                        uint32_t* rec = rec0 + (q >> 5) * kRec;
                        rec[q & 31] = (uint32_t)(slot - j * kBlockSlots);
                        rec[32 + (q & 31)] = kAllRows;
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
            res_counts[w] = rpos;
        }
        const unsigned long long a = wave_sum(all_cols), d = wave_sum(res_cols);
        if (lane == 0) {
            atomicAdd(&stats[0], a);
            atomicAdd(&stats[1], d);
        }
        return;
    }
    // pad each list to whole chunks with the zero row, attended by no row
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
        const int32_t nch = (bpos[j] + kChunk - 1) / kChunk;
        uint32_t* rec0 = records + chunk_base[trow + j] * kRec;
        for (int32_t q = bpos[j] + lane; q < nch * kChunk; q += kWave) {
            uint32_t* rec = rec0 + (q >> 5) * kRec;
            rec[q & 31] = (uint32_t)kBlockSlots;
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

// Staged rows are 128 bytes, unpadded (the asynchronous LDS loads fill 16
// bytes per lane at consecutive addresses), with the 16-byte pieces of row s
// stored at position piece ^ (s & 7), so that the sixteen rows the lanes of
// one group read for an MFMA operand spread over the LDS banks.
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
    uint32_t meta[kPanel][4 * 64];   // four chunk records per wave
};
static_assert(2 * sizeof(PanelBuf) + sizeof(PanelMeta) <= 160 * 1024, "LDS budget");

// Waits until every vector-memory load this wave issued has completed,
// including those that write LDS directly.
#define F3S_VMEM_SYNC() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")

// Loads one block's K and V rows (head h) into LDS buffer B without
// registers: 16 waves x 8 rows per round, lane l fetching piece
// (l & 7) ^ (row & 7) of row (l >> 3) so that it lands at position l & 7.
__device__ __forceinline__ void load_block_async(PanelBuf& B, __amdgpu_buffer_rsrc_t kres,
                                                 __amdgpu_buffer_rsrc_t vres,
                                                 const uint32_t (&refs)[2], uint32_t head_off,
                                                 int wave, int lane)
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

// One 16-wave workgroup per (panel, head); wave k owns window 16 * panel + k
// and writes the (m, l, O) partial of its window's staged tiles.  Block
// j + 1 streams into one buffer while the waves run block j's chunks from
// the other; the loads a wave needs during block j (its first four chunk
// records) are issued before block j + 1's asynchronous loads, which vmcnt
// would otherwise make them wait behind.
__global__ void __launch_bounds__(kPanelThreads) __attribute__((amdgpu_waves_per_eu(4)))
panel_attention_kernel(const AttnParams p, const PanelParams q)
{
    // distinct objects: reads of one need not wait for loads into another
    __shared__ PanelBuf buf0, buf1;
    __shared__ PanelMeta M;
    const int H = p.H;
    // wave-uniform values in scalar registers
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

    // rows of zeros that padding slots read, in both buffers
    if (threadIdx.x < 4 * (kD / 8)) {
        const int which = threadIdx.x / (kD / 8), piece = threadIdx.x % (kD / 8);
        PanelBuf& zb = (which >> 1) ? buf1 : buf0;
        *reinterpret_cast<h8*>(&zb.rows[which & 1][kBlockSlots * kD + 8 * piece]) = h8{};
    }
    const int32_t S = q.nslots[P];
    const int64_t sb = q.slot_base[P];
    const int nb = (S + kBlockSlots - 1) / kBlockSlots;
    const int64_t trow = (P * kPanel + wave) * kMaxBlocks;
    uint32_t* meta = M.meta[wave];
    const uint4* __restrict__ rec = reinterpret_cast<const uint4*>(q.records);
    // this wave's chunk ranges, one entry per lane (read back with readlane:
    // loads issued after the asynchronous ones would wait behind them)
    const int64_t my_cb = lane <= kMaxBlocks ? q.chunk_base[trow + lane] : 0;
    auto chunk_at = [&](int j) -> int64_t {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)my_cb, j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(my_cb >> 32), j);
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };

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

    // ---- the staged tiles' partial: (O^T unnormalised, m, l) ----
    if (w >= p.W) return;
    float lrow = st.l + __shfl_xor(st.l, 16, kWave);
    lrow += __shfl_xor(lrow, 32, kWave);
    float* part = q.partials + ((int64_t)w * H + h) * kPartialFloats;
    float* op = part + r * kD + 16 * g;
#pragma unroll
    for (int v = 0; v < 4; ++v)
        *reinterpret_cast<float4*>(op + 4 * v) =
            make_float4(st.acc[0][v], st.acc[1][v], st.acc[2][v], st.acc[3][v]);
    if (g == 0) {
        part[16 * kD + r] = st.m;
        part[16 * kD + 16 + r] = lrow;
    }
}

// ------------------------------------------------------------------ host

__global__ void residual_items(const int64_t* __restrict__ base, int32_t W, Item* __restrict__ items)
{
    const int32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w < W) items[w] = Item{w, (int32_t)base[w], (int32_t)base[w + 1], -1};
}

f3s_status panel_compile_plan(f3s_plan* plan, const int32_t* d_block_col, int32_t n,
                              hipStream_t st)
{
    plan->panels = false;
    const int32_t W = plan->W;
    if (W == 0 || plan->T == 0 || !plan->natural_order || plan->masked.num_split != 0 ||
        wide_features(n, plan->H))
        return F3S_OK;
    const int32_t team = plan->masked.team;
    const int64_t np = ceil_div(W, kPanel);
    const int64_t entries = np * kPanel * kMaxBlocks;
    const auto* items = reinterpret_cast<const Item*>(plan->masked.items.ptr);
    DeviceBuffer counts, rcounts, stats, tmp;
    F3S_TRY(counts.reserve(sizeof(int32_t) * (size_t)entries));
    F3S_TRY(rcounts.reserve(sizeof(int32_t) * (size_t)W));
    F3S_TRY(plan->pn_nslots.reserve(sizeof(int32_t) * (size_t)np));
    F3S_TRY(stats.reserve(2 * sizeof(unsigned long long)));
    F3S_TRY(tmp.reserve(sizeof(int64_t) * (size_t)scan_tmp_elems(std::max<int64_t>(entries, W))));
    F3S_HIP(hipMemsetAsync(stats.ptr, 0, 2 * sizeof(unsigned long long), st));
    const uint32_t ref_stride = (uint32_t)plan->H * kRowBytes;
    auto* cnt = reinterpret_cast<int32_t*>(counts.ptr);
    auto* rcnt = reinterpret_cast<int32_t*>(rcounts.ptr);
    auto* ns = reinterpret_cast<int32_t*>(plan->pn_nslots.ptr);
    auto* sts = reinterpret_cast<unsigned long long*>(stats.ptr);
    hipLaunchKernelGGL(panel_compile<false>, dim3((unsigned)np), dim3(kPanelThreads), 0, st,
                       items, team, W, d_block_col, n, ref_stride, cnt, rcnt, ns, sts, nullptr,
                       nullptr, nullptr, nullptr, nullptr, nullptr);
    F3S_HIP(hipGetLastError());
    unsigned long long h_stats[2] = {0, 0};
    F3S_HIP(hipMemcpyAsync(h_stats, sts, sizeof h_stats, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    // stats[0]: tile columns = K/V row fetches per head of the gathered pass;
    // stats[1]: staged rows + residual tile columns = row fetches with panels
    plan->pn_rows_gathered = (int64_t)h_stats[0];
    plan->pn_rows_fetched = (int64_t)h_stats[1];
    if (h_stats[1] == 0 || (double)h_stats[0] < kPanelMinGain * (double)h_stats[1]) {
        plan->pn_nslots.release();
        return F3S_OK;
    }
    F3S_TRY(plan->pn_chunk_base.reserve(sizeof(int64_t) * (size_t)(entries + 1)));
    F3S_TRY(plan->pn_slot_base.reserve(sizeof(int64_t) * (size_t)(np + 1)));
    DeviceBuffer rbase;
    F3S_TRY(rbase.reserve(sizeof(int64_t) * (size_t)(W + 1)));
    auto* cb = reinterpret_cast<int64_t*>(plan->pn_chunk_base.ptr);
    auto* sbp = reinterpret_cast<int64_t*>(plan->pn_slot_base.ptr);
    auto* rb = reinterpret_cast<int64_t*>(rbase.ptr);
    auto* tp = reinterpret_cast<int64_t*>(tmp.ptr);
    F3S_TRY(exclusive_scan_i32_to_i64(cnt, cb, entries, tp, st));
    F3S_TRY(exclusive_scan_i32_to_i64(ns, sbp, np, tp, st));
    F3S_TRY(exclusive_scan_i32_to_i64(rcnt, rb, W, tp, st));
    int64_t totals[3] = {0, 0, 0};
    F3S_HIP(hipMemcpyAsync(&totals[0], cb + entries, 8, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipMemcpyAsync(&totals[1], sbp + np, 8, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipMemcpyAsync(&totals[2], rb + W, 8, hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    // four records of padding: the pass reads records in blocks of four
    F3S_TRY(plan->pn_records.reserve(sizeof(uint32_t) * 64 * (size_t)(totals[0] + 4)));
    F3S_TRY(plan->pn_slot_refs.reserve(sizeof(uint32_t) * (size_t)(totals[1] + 1)));
    F3S_TRY(plan->pn_res_block_col.reserve(sizeof(int32_t) * (size_t)(totals[2] + 1)));
    F3S_TRY(plan->pn_res_items.reserve(sizeof(Item) * (size_t)W));
    F3S_TRY(plan->pn_partials.reserve(sizeof(float) * kPartialFloats * (size_t)W * plan->H));
    hipLaunchKernelGGL(panel_compile<true>, dim3((unsigned)np), dim3(kPanelThreads), 0, st,
                       items, team, W, d_block_col, n, ref_stride, nullptr, nullptr, nullptr,
                       nullptr, cb, rb, sbp, reinterpret_cast<uint32_t*>(plan->pn_slot_refs.ptr),
                       reinterpret_cast<uint32_t*>(plan->pn_records.ptr),
                       reinterpret_cast<int32_t*>(plan->pn_res_block_col.ptr));
    F3S_HIP(hipGetLastError());
    hipLaunchKernelGGL(residual_items, dim3((unsigned)ceil_div(W, 256)), dim3(256), 0, st, rb, W,
                       reinterpret_cast<Item*>(plan->pn_res_items.ptr));
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
    q.partials = reinterpret_cast<float*>(plan->pn_partials.ptr);
    q.num_panels = plan->num_panels;
    hipLaunchKernelGGL(panel_attention_kernel, dim3((unsigned)(plan->num_panels * p.H)),
                       dim3(kPanelThreads), 0, st, p, q);
}

}  // namespace f3s
