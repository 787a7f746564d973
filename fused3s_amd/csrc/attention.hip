// attention.hip -- fused SDDMM -> online softmax -> SpMM over the 16x16
// block-sparse row windows, written for gfx950 (wave64, MFMA 16x16x32 f16).
//
// Computes what f3s_1tb1rw_kernel computes (src/fused3s_v2.cu:81-246):
// per row window, streaming over its active tiles in order, raw logits
// S = Q.K^T (no 1/sqrt(d) unless `scale` says so), an online softmax with a
// running max and sum, P rounded to fp16 before P.V, and a final
// O * (sum > 0 ? 1/sum : 0) (:235-245).  Two semantics:
//   TILE_DENSE (tile_mask == NULL): all columns < n of an active tile are
//     attended (the reference kernel and tests/test_fused_3s_v2.cu:17-59,
//     with padded columns excluded as on the reference CPU side);
//   MASKED: only the edges named by the tile's row masks
//     (baselines/cpu_baseline.cpp:16-91).
//
// Work decomposition (one wave = one (item, head)):
//   An item is a row window or, in a plan, a segment of a heavy window; on
//   small graphs a team of 4 or 16 waves of one workgroup shares a window
//   (each wave a part of its tiles) and merges in LDS.
//   MASKED, unplanned: the wave expands its tiles into a list of attended
//   columns ("slots"), each with the mask of the window rows that attend it,
//   held in a per-wave LDS ring: 64 tiles per step, one tile per lane,
//   positions from a DPP wave prefix sum.  Columns no row attends are never
//   gathered (column compaction).  MASKED with a compiled plan: the same
//   lists, built once per graph, are read 32 columns per record.
//   TILE_DENSE: a chunk is simply two whole tiles, i.e. 32 columns in two
//   runs of 16 contiguous K/V rows.  Slots are consumed 32 at a time
//   (chunk_step), their K and V rows gathered eight lanes per 128-byte row
//   and handed to the matrix cores through a per-wave LDS stage:
//     S^T[32 x 16] = K_slots[32 x 64] . Q_w^T    4 MFMA 16x16x32
//     masked online softmax, row r in lanes r, r+16, r+32, r+48
//     O^T[64 x 16] += V_slots^T . P^T            4 MFMA
//   Computing S^T instead of S puts each lane's logits for row r = lane%16
//   exactly where the B operand of the P.V product needs them, and the O^T
//   accumulator rows of a lane are also row r, so the per-row rescale
//   (scale_fragment_by_row, src/fused3s_v2.cu:54-71) is a plain multiply by
//   the lane's own correction: no shuffles, no LDS round trip for P.
//   Q stays in registers in B-operand layout for the whole item.
//   Segments of split windows write (m, l, O) partials; the last segment of
//   a window to finish combines them in slot order, in the same launch.
//
// MFMA 16x16x32 f16 operand layout used (CDNA3/CDNA4 16x16 family): lane l
// supplies row l%16 of A and column l%16 of B, 8 consecutive k per lane in
// lane group l/16; C/D: lane l holds rows 4*(l/16)+v, column l%16, v=0..3.
// The k order inside a lane group is the same for A and B, so any consistent
// assignment of k indices to (group, element) gives the same product; the
// code relies only on that and on the row/column/C mapping.
#include <algorithm>
#include <math.h>
#include <mutex>
#include <new>
#include <stdio.h>

#include "attn_common.hpp"
#include "attn_plan.hpp"

namespace f3s {

// WPG waves per workgroup; each wave processes one (item, head), the H heads
// of an item in adjacent waves of one workgroup: their K/V rows are adjacent
// in memory ([n][H][d]), which measured faster on config 5 than visiting the
// heads one after another (smaller per-head L2 working set, but scattered
// 128-byte fetches).  The register budget is capped for 4 waves per SIMD.
enum Mode : int {
    kModeRing = 0,    // masked, tiles expanded on every pass (unplanned launch)
    kModeList = 1,    // masked, compiled column lists (planned + compiled)
    kModeDense = 2,   // tile-dense semantics
};

// Combines the partials of split window `si` for head h, in slot order
// (deterministic): M = max m_k, O = sum O_k 2^(m_k - M) / sum l_k 2^(m_k - M),
// and writes its O rows.  Lane (g, r) owns row r, dims 16g..16g+15.  An
// online merge over the segments, KB segments' loads in flight at a time:
// (m, l, O) of a batch are rescaled to the batch's running max, so one pass
// suffices.  The partials were written through to memory by segments that
// may have run on other XCDs, and are read the same way (kCoherent).
template <int KB>
__device__ __forceinline__ void merge_split(const AttnParams& p, const SplitInfo si, int h,
                                            int lane)
{
    const int H = p.H;
    const int g = lane >> 4, r = lane & 15;
    float M = -INFINITY, Ls = 0.f;
    float4 o[4] = {make_float4(0, 0, 0, 0), make_float4(0, 0, 0, 0), make_float4(0, 0, 0, 0),
                   make_float4(0, 0, 0, 0)};
    for (int k0 = 0; k0 < si.nseg; k0 += KB) {
        float mk[KB], lk[KB];
        float4 a[KB][4];
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const bool in = k0 + j < si.nseg;
            // one descriptor per partial: 32-bit offsets inside it
            const float* pk =
                p.partials + ((int64_t)(si.first_slot + (in ? k0 + j : k0)) * H + h) * kPartialFloats;
            const __amdgpu_buffer_rsrc_t pr = make_rsrc(pk, sizeof(float) * kPartialFloats);
            mk[j] = in ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                             pr, sizeof(float) * (16 * kD + r), 0, kCoherent))
                       : -INFINITY;
            lk[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                pr, sizeof(float) * (16 * kD + 16 + r), 0, kCoherent));
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const u4 x = __builtin_amdgcn_raw_buffer_load_b128(
                    pr, sizeof(float) * (r * kD + 16 * g + 4 * v), 0, kCoherent);
                a[j][v] = make_float4(__uint_as_float(x.x), __uint_as_float(x.y),
                                      __uint_as_float(x.z), __uint_as_float(x.w));
            }
        }
        float Mb = M;
#pragma unroll
        for (int j = 0; j < KB; ++j) Mb = __builtin_fmaxf(Mb, mk[j]);
        if (Mb == -INFINITY) continue;   // all rows of these segments empty
        const float c = fast_exp2(M - Mb);   // 0 while M is still -inf
        Ls *= c;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            o[v].x *= c;
            o[v].y *= c;
            o[v].z *= c;
            o[v].w *= c;
        }
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const float f = fast_exp2(mk[j] - Mb);   // 0 for absent / empty segments
            Ls += lk[j] * f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                o[v].x += a[j][v].x * f;
                o[v].y += a[j][v].y * f;
                o[v].z += a[j][v].z * f;
                o[v].w += a[j][v].w * f;
            }
        }
        M = Mb;
    }
    const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
    const int32_t row = si.w * 16 + r;
    if (row < p.n) {
        float* dst = p.O + ((int64_t)row * H + h) * kD + 16 * g;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            *reinterpret_cast<float4*>(dst + 4 * v) =
                make_float4(o[v].x * inv, o[v].y * inv, o[v].z * inv, o[v].w * inv);
    }
}

// The pass is bound by memory throughput, not latency: keeping a second
// chunk's gathers in flight per wave (double-buffered registers, 3 waves per
// SIMD) measured no faster than one chunk per wave at 4-5 waves per SIMD, so
// the simpler single-buffered loop is kept.
template <int MODE, int WPG, bool WIDE, int TEAM>
__global__ void __launch_bounds__(kWave * WPG) __attribute__((amdgpu_waves_per_eu(4)))
fused_attention_kernel(const AttnParams p)
{
    static_assert(TEAM == 1 || TEAM == WPG, "a team fills its workgroup");
    const int H = p.H;
    __shared__ WaveLds lds_all[WPG];
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int g = lane >> 4;                          // lane group
    const int r = lane & 15;                          // row of the window this lane owns
    WaveLds& L = lds_all[wave];

    const int32_t n = p.n;
    // wave -> (item, head); the launch keeps num_items * H < 2^31.  A team's
    // workgroup is one (window, head); its waves take the window's TEAM
    // consecutive items, so every exit below is uniform over the workgroup
    // (num_items is a multiple of TEAM).
    int64_t item_idx;
    int h;
    if constexpr (TEAM == 1) {
        const uint32_t gw = (uint32_t)(logical_block(p.xcd_contiguous) * WPG + wave);
        item_idx = (int64_t)(gw / (uint32_t)H);
        h = (int)(gw % (uint32_t)H);
    } else {
        const uint32_t gb = (uint32_t)logical_block(p.xcd_contiguous);
        item_idx = (int64_t)(gb / (uint32_t)H) * TEAM + wave;
        h = (int)(gb % (uint32_t)H);
    }
    if (item_idx >= p.num_items) return;

    // ---- item decode (wave-uniform) ----
    int32_t w, tb, te, slot;
    int32_t team_n = 1;   // teams: non-empty parts of the window (uniform over the team)
    if (p.items) {
        const Item it = p.items[item_idx];
        w = it.w;
        tb = it.tb;
        te = it.te;
        slot = it.slot;
        if (w < 0 || w >= p.W) return;   // an invalid order entry (a whole team's items)
        if constexpr (TEAM > 1) {
            // the window's tiles run from its first part's start to its last
            // part's end
            const int64_t ib = item_idx - wave;
            team_n = team_parts(p.items[ib].tb, p.items[ib + TEAM - 1].te, TEAM);
        }
    } else {
        const int64_t wi = item_idx / TEAM;
        w = p.window_order ? p.window_order[wi] : (int32_t)wi;
        if (w < 0 || w >= p.W) return;   // an empty slot or an invalid order entry
        const int32_t T = p.window_offsets[p.W];
        tb = max(0, min(p.window_offsets[w], T));
        te = max(tb, min(p.window_offsets[w + 1], T));
        if (p.heavy_mode) {
            // in an order's sequence, the heavy windows among its first
            // kHeavyMaxWindows entries belong to the team launch (mode 2), all
            // others to the one-wave launch (mode 1); uniform over a team
            const bool heavy =
                wi < kHeavyMaxWindows &&
                te - tb > heavy_tiles(T, p.W, kHeavyMinTiles, kHeavyMeanFactor);
            if (heavy != (p.heavy_mode == 2)) return;
        }
        if constexpr (TEAM > 1) {
            team_n = team_parts(tb, te, TEAM);
            const int32_t a = team_part(tb, te, wave, TEAM), b = team_part(tb, te, wave + 1, TEAM);
            tb = a;
            te = b;
        }
        slot = -1;
    }
    // a window of at most one part is wave 0's alone: no merge, no barrier
    if (TEAM > 1 && team_n <= 1 && wave != 0) return;
    const int32_t nbc = (n + 15) >> 4;   // valid block columns
    const int32_t* __restrict__ block_col = p.block_col;
    const __amdgpu_buffer_rsrc_t qres = make_rsrc(p.Q, p.feat_bytes);
    const __amdgpu_buffer_rsrc_t kres = make_rsrc(p.K, p.feat_bytes);
    const __amdgpu_buffer_rsrc_t vres = make_rsrc(p.V, p.feat_bytes);
    const uint32_t head_off = (uint32_t)h * kRowBytes;
    const uint32_t row_stride = H * kRowBytes;
    const uint32_t ref_stride = WIDE ? 1u : row_stride;   // node -> row reference
    const uint32_t no_ref = WIDE ? kNoIdx : kNoRow;

    // ---- Q tile in registers, B-operand layout ----
    const int32_t qrow = w * 16 + r;
    const uint32_t qref = qrow < n ? (uint32_t)qrow * ref_stride : no_ref;
    const h8 q0 = load_ref<WIDE>(qres, p.Q, qref, row_stride, head_off + 16 * g);
    const h8 q1 = load_ref<WIDE>(qres, p.Q, qref, row_stride, head_off + 16 * g + 64);

    RowState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) st.acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    if constexpr (MODE == kModeList) {
      {
        // ---- compiled plan: the attended columns were listed once per graph ----
        // Chunk records (32 offsets, 32 row masks: 256 bytes) are read four at
        // a time with one coalesced 16-byte load per lane, one block ahead,
        // and handed out through LDS: the vector-memory address path, not
        // HBM, bounds this pass, so metadata costs a quarter instruction per
        // chunk.  The plan pads its record array by four records, so a block
        // read at an item's last chunks stays inside it.
        const int rbit = (r & 1) ? 16 + (r >> 1) : (r >> 1);
        const int64_t cb = p.chunk_base[item_idx], ce = p.chunk_base[item_idx + 1];
        const uint32_t piece_off = head_off + 16 * (lane & 7);
        uint32_t* meta = reinterpret_cast<uint32_t*>(L.off);   // 4 records of this wave
        const u4* __restrict__ rec = reinterpret_cast<const u4*>(p.columns);
        u4 blk = cb < ce ? rec[cb * 16 + lane] : u4{0u, 0u, 0u, 0u};
        for (int64_t c0 = cb; c0 < ce; c0 += 4) {
            F3S_WAVE_LDS_SYNC();   // the previous block's reads of meta are done
            *reinterpret_cast<u4*>(&meta[4 * lane]) = blk;
            F3S_WAVE_LDS_SYNC();
            if (c0 + 4 < ce) blk = rec[(c0 + 4) * 16 + lane];   // next block, in flight
            const int nk = (int)min((int64_t)4, ce - c0);
            for (int k = 0; k < nk; ++k) {
                const uint32_t* m = meta + 64 * k;
                h8 krow[4], vrow[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t ref = m[(lane >> 3) + 8 * i];
                    krow[i] = load_ref<WIDE>(kres, p.K, ref, row_stride, piece_off);
                    vrow[i] = load_ref<WIDE>(vres, p.V, ref, row_stride, piece_off);
                }
                const uint4 ra = *reinterpret_cast<const uint4*>(&m[32 + 4 * g]);
                const uint4 rb = *reinterpret_cast<const uint4*>(&m[48 + 4 * g]);
                const uint32_t valid =
                    ((ra.x >> rbit) & 1u) | (((ra.y >> rbit) & 1u) << 1) |
                    (((ra.z >> rbit) & 1u) << 2) | (((ra.w >> rbit) & 1u) << 3) |
                    (((rb.x >> rbit) & 1u) << 4) | (((rb.y >> rbit) & 1u) << 5) |
                    (((rb.z >> rbit) & 1u) << 6) | (((rb.w >> rbit) & 1u) << 7);
                chunk_step(st, krow, q0, q1, valid, vrow, L.stage, lane, p.scale_log2);
            }
        }
      }
    } else if constexpr (MODE == kModeRing) {
      {
        // ---- column-compacted path: a ring of attended columns ----
        const uint16_t* __restrict__ tile_mask = p.tile_mask;
        const int rbit = (r & 1) ? 16 + (r >> 1) : (r >> 1);   // row r in a ring row mask
        int32_t tcur = tb;
        int32_t head = 0, tail = 0;   // ring positions (monotone, wave-uniform)
        constexpr int32_t kMask = kRing - 1;
        while (true) {
            // expand tiles into attended columns until a chunk is ready
            while (tail - head < kChunk && tcur < te) {
                const int32_t t = tcur + lane;
                uint32_t u = 0;
                int32_t bc = 0;
                uint32_t wd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (t < te) {
                    bc = block_col[t];
                    if ((uint32_t)bc < (uint32_t)nbc) {
                        const int32_t left = n - bc * 16;
                        const uint32_t vmask = left >= 16 ? 0xffffu : ((1u << left) - 1u);
                        const uint4* mp = reinterpret_cast<const uint4*>(tile_mask + (int64_t)t * 16);
                        const uint4 a = mp[0], b = mp[1];
                        wd[0] = a.x; wd[1] = a.y; wd[2] = a.z; wd[3] = a.w;
                        wd[4] = b.x; wd[5] = b.y; wd[6] = b.z; wd[7] = b.w;
                        const uint32_t o = a.x | a.y | a.z | a.w | b.x | b.y | b.z | b.w;
                        u = (o | (o >> 16)) & vmask;
                    }
                }
                const int occ = __popc(u);
                const int incl = wave_scan_incl(occ);
                const int avail = kRing - kChunk - (tail - head);
                const bool accept = (t < te) && incl <= avail;
                const int nacc = __popcll(__ballot(accept));          // accepted lanes: a prefix
                const int added = __builtin_amdgcn_readlane(incl, nacc - 1);
                if (accept && occ) {
                    int32_t pos = tail + incl - occ;
                    const uint32_t base = (uint32_t)bc * 16 * ref_stride;
                    uint32_t rest = u;
                    while (rest) {
                        const int c = __ffs(rest) - 1;
                        rest &= rest - 1;
                        L.off[pos & kMask] = base + (uint32_t)c * ref_stride;
                        L.rm[pos & kMask] = column_rows(wd, c);
                        ++pos;
                    }
                }
                tail += added;
                tcur += nacc;
            }
            const int32_t pending = tail - head;
            if (pending <= 0) break;
            if (pending < kChunk && lane < kChunk - pending) {
                // last, partial chunk: pad with slots nobody attends, whose
                // loads fall outside the buffers and read as zero
                L.off[(tail + lane) & kMask] = no_ref;
                L.rm[(tail + lane) & kMask] = 0u;
            }
            F3S_WAVE_LDS_SYNC();
            // Chunks start at multiples of 32 (only the last one is partial),
            // so a chunk never wraps around the ring.
            const uint32_t* off = &L.off[head & kMask];
            const uint32_t* rmr = &L.rm[head & kMask];
            h8 krow[4], vrow[4];
            const uint32_t piece_off = head_off + 16 * (lane & 7);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ref = off[(lane >> 3) + 8 * i];
                krow[i] = load_ref<WIDE>(kres, p.K, ref, row_stride, piece_off);
                vrow[i] = load_ref<WIDE>(vres, p.V, ref, row_stride, piece_off);
            }
            const uint4 ra = *reinterpret_cast<const uint4*>(&rmr[4 * g]);
            const uint4 rb = *reinterpret_cast<const uint4*>(&rmr[16 + 4 * g]);
            const uint32_t valid =
                ((ra.x >> rbit) & 1u) | (((ra.y >> rbit) & 1u) << 1) |
                (((ra.z >> rbit) & 1u) << 2) | (((ra.w >> rbit) & 1u) << 3) |
                (((rb.x >> rbit) & 1u) << 4) | (((rb.y >> rbit) & 1u) << 5) |
                (((rb.z >> rbit) & 1u) << 6) | (((rb.w >> rbit) & 1u) << 7);
            chunk_step(st, krow, q0, q1, valid, vrow, L.stage, lane, p.scale_log2);
            head += pending < kChunk ? pending : kChunk;
        }
      }
    } else {
        // ---- tile-dense path: two whole tiles (32 contiguous columns) per chunk ----
        // Far tiles stream past the L2 when at least a quarter of the item's
        // tiles are near (kNearCols); one-wave items of the narrow path only.
        bool stream_far = false;
        if constexpr (!WIDE && TEAM == 1) {
            int64_t near = 0;
            for (int32_t t0 = tb; t0 < te; t0 += kWave) {
                const int32_t t = t0 + lane;
                bool is_near = false;
                if (t < te) {
                    const int32_t bc = block_col[t];
                    is_near = bc >= w - kNearCols && bc <= w + kNearCols;
                }
                near += __popcll(__ballot(is_near));
            }
            stream_far = 4 * near >= (int64_t)(te - tb);
        }
        for (int32_t t = tb; t < te; t += 2) {
            const int32_t bc0 = block_col[t];
            const int32_t bc1 = (t + 1 < te) ? block_col[t + 1] : -1;
            const bool ok0 = (uint32_t)bc0 < (uint32_t)nbc, ok1 = (uint32_t)bc1 < (uint32_t)nbc;
            const int32_t c0 = 16 * bc0, c1 = 16 * bc1;
            auto row_at = [&](bool ok, int32_t c, int s) -> uint32_t {
                return ok && c + s < n ? (uint32_t)(c + s) * ref_stride : no_ref;
            };
            h8 krow[4], vrow[4];
            uint32_t ref[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s = (lane >> 3) + 8 * i;   // slots 0-15: tile t, 16-31: tile t+1
                ref[i] = s < 16 ? row_at(ok0, c0, s) : row_at(ok1, c1, s - 16);
            }
            const uint32_t extra = head_off + 16 * (lane & 7);
            // wave-uniform: loads 0-1 belong to tile t, loads 2-3 to tile t+1
            const bool far0 = stream_far && (bc0 < w - kNearCols || bc0 > w + kNearCols);
            const bool far1 = stream_far && (bc1 < w - kNearCols || bc1 > w + kNearCols);
            if (!far0 && !far1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    krow[i] = load_ref<WIDE>(kres, p.K, ref[i], row_stride, extra);
                    vrow[i] = load_ref<WIDE>(vres, p.V, ref[i], row_stride, extra);
                }
            } else if (far0 && far1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    krow[i] = load_h8<kStreamLoad>(kres, ref[i] + extra);
                    vrow[i] = load_h8<kStreamLoad>(vres, ref[i] + extra);
                }
            } else if (far0) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    krow[i] = load_h8<kStreamLoad>(kres, ref[i] + extra);
                    vrow[i] = load_h8<kStreamLoad>(vres, ref[i] + extra);
                }
#pragma unroll
                for (int i = 2; i < 4; ++i) {
                    krow[i] = load_h8<0>(kres, ref[i] + extra);
                    vrow[i] = load_h8<0>(vres, ref[i] + extra);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    krow[i] = load_h8<0>(kres, ref[i] + extra);
                    vrow[i] = load_h8<0>(vres, ref[i] + extra);
                }
#pragma unroll
                for (int i = 2; i < 4; ++i) {
                    krow[i] = load_h8<kStreamLoad>(kres, ref[i] + extra);
                    vrow[i] = load_h8<kStreamLoad>(vres, ref[i] + extra);
                }
            }
            // logit j of the lane is column 4g + j of tile t (j < 4) or
            // 4g + j - 4 of tile t+1; attended iff the column exists
            uint32_t valid = 0;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                valid |= (uint32_t)(ok0 && c0 + 4 * g + v < n) << v;
                valid |= (uint32_t)(ok1 && c1 + 4 * g + v < n) << (4 + v);
            }
            chunk_step(st, krow, q0, q1, valid, vrow, L.stage, lane, p.scale_log2);
        }
    }

    if (TEAM > 1 && team_n > 1) {   // uniform over the team
        // ---- team merge: waves 1 .. team_n-1 publish (m, l, O^T) lane by
        // lane in their own LDS area, wave 0 folds them in, in wave order
        // (deterministic) ----
        F3S_WAVE_LDS_SYNC();   // this wave's last reads of its stage are done
        float* accs = reinterpret_cast<float*>(L.stage);   // [t][lane][4]: 4 KB of 4.5
        if (wave != 0 && wave < team_n) {
#pragma unroll
            for (int t = 0; t < 4; ++t) *reinterpret_cast<f4*>(&accs[(t * kWave + lane) * 4]) = st.acc[t];
            L.off[lane] = __float_as_uint(st.m);
            L.rm[lane] = __float_as_uint(st.l);
        }
        __syncthreads();
        if (wave != 0) return;
        float M = st.m;
#pragma unroll
        for (int k = 1; k < TEAM; ++k)
            if (k < team_n) M = __builtin_fmaxf(M, __uint_as_float(lds_all[k].off[lane]));
        if (M != -INFINITY) {   // else no part of the team attended row r: all zero
            const float c0 = fast_exp2(st.m - M);   // 0 when this part is empty
            st.l *= c0;
#pragma unroll
            for (int t = 0; t < 4; ++t) st.acc[t] *= c0;
#pragma unroll
            for (int k = 1; k < TEAM; ++k) {
                if (k >= team_n) break;
                const float mk = __uint_as_float(lds_all[k].off[lane]);
                const float f = fast_exp2(mk - M);   // mk = -inf: 0
                st.l += __uint_as_float(lds_all[k].rm[lane]) * f;
                const float* ak = reinterpret_cast<const float*>(lds_all[k].stage);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    st.acc[t] += *reinterpret_cast<const f4*>(&ak[(t * kWave + lane) * 4]) * f;
            }
            st.m = M;
        }
    }

    // ---- epilogue ----
    float lrow = st.l + __shfl_xor(st.l, 16, kWave);
    lrow += __shfl_xor(lrow, 32, kWave);
    if (slot < 0) {
        const float inv = lrow > 0.f ? 1.0f / lrow : 0.f;
        // O leaves in whole rows: the lane's 16 values (row r, dims
        // 16g..16g+15) pass through this wave's LDS stage so that each store
        // instruction writes four complete 256-byte rows instead of 16-byte
        // pieces of all sixteen.
        F3S_WAVE_LDS_SYNC();   // this wave's last reads of its stage are done
        float* ost = reinterpret_cast<float*>(L.stage);
#pragma unroll
        for (int v = 0; v < 4; ++v)
            *reinterpret_cast<f4*>(&ost[r * kOutStride + 16 * g + 4 * v]) =
                f4{st.acc[0][v] * inv, st.acc[1][v] * inv, st.acc[2][v] * inv, st.acc[3][v] * inv};
        F3S_WAVE_LDS_SYNC();
        const int c4 = 4 * (lane & 15);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int rr = 4 * v + (lane >> 4);
            const f4 o4 = *reinterpret_cast<const f4*>(&ost[rr * kOutStride + c4]);
            const int32_t row = w * 16 + rr;
            if (row < n) store_out(p.O + ((int64_t)row * H + h) * kD + c4, o4);
        }
        return;
    }
    // Segment of a split window: its (m, l, unnormalised O) goes through to
    // memory; once every store of the wave is done (vmcnt(0)) the segment
    // counts itself in, and the last of the window's segments to do so
    // merges all of them (its own included, from memory) and leaves the
    // count at zero for the next pass.  The count's atomics are coherent
    // across XCDs.
    const int32_t sid = p.slot_split[slot];
    const SplitInfo si = p.splits[sid];
    const __amdgpu_buffer_rsrc_t pres =
        make_rsrc(p.partials + ((int64_t)slot * H + h) * kPartialFloats,
                  sizeof(float) * kPartialFloats);
#pragma unroll
    for (int v = 0; v < 4; ++v)
        __builtin_amdgcn_raw_buffer_store_b128(
            u4{__float_as_uint(st.acc[0][v]), __float_as_uint(st.acc[1][v]),
               __float_as_uint(st.acc[2][v]), __float_as_uint(st.acc[3][v])},
            pres, (uint32_t)(sizeof(float) * (r * kD + 16 * g + 4 * v)), 0, kCoherent);
    if (g == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(st.m), pres,
                                              (uint32_t)(sizeof(float) * (16 * kD + r)), 0,
                                              kCoherent);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lrow), pres,
                                              (uint32_t)(sizeof(float) * (16 * kD + 16 + r)), 0,
                                              kCoherent);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    int32_t* cnt = p.counters + (int64_t)sid * H + h;
    int last = 0;
    if (lane == 0) {
        last = atomicAdd(cnt, 1) == si.nseg - 1;
        if (last) atomicExch(cnt, 0);
    }
    if (!__shfl(last, 0, kWave)) return;
    merge_split<2>(p, si, h, lane);
}

__global__ void warm_attention_kernel() {}

hipError_t warm_attention(hipStream_t s)
{
    hipLaunchKernelGGL(warm_attention_kernel, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Schedule of the unplanned launch on graphs of more than kHeavyMaxWindows
// windows, in natural order and, from kSchedOrderedMin window-heads on, with
// a window order too.  The order then only names the windows to compute
// (each named window once; invalid entries are skipped, unnamed windows left
// untouched); the schedule is the library's own, whatever the order:
//   * heavy windows -- more than max(kHeavyMinTiles, kHeavyMeanFactor x mean)
//     tiles -- heaviest first; the first kHeavyMaxWindows of them run as
//     16-wave teams in a launch of their own;
//   * every other window on one wave, by class of tile count (the octave;
//     heavy windows past the team list form the first classes), heaviest
//     class first, each class in index order and cut into eight contiguous
//     shares; slot i * 8 + x holds share x's i-th window, and the launch
//     deals its workgroups to the XCDs round-robin.  The longest windows
//     start first and only the smallest finish last, and each share -- a
//     contiguous range of windows -- runs on one XCD when a workgroup is one
//     window (4 heads) or on a few, which keeps a community-ordered graph's
//     neighbours in their L2s.  (Each XCD's workgroups taking its share as a
//     contiguous range of slots measured the same on config 5 but 10 %
//     slower on a plan of config 4 and 3 % with 8 heads; one sequence of the
//     classes dealt round-robin, with no shares, ran config 5 13 % slower
//     tile-dense, its communities fetched into every L2.)
// Four small kernels build it, and no memory needs clearing first (so the
// launch may be captured into a graph): sched_inverse (an order's inverse,
// scattered: window w is named iff inv[w] is a position that holds w, which
// no stale value of an unnamed entry can fake), sched_count (per-block class
// counts), sched_scan (one workgroup: class offsets, the team list's part of
// each class, the XCD tables) and sched_fill (each window's slot, and -1 in
// every slot no window takes).  Class positions q run 0 (heaviest class) to
// kSchedClasses - 1.
constexpr int kSchedClasses = 64;   // 32 octaves of the tile count, x {heavy, not}
// A window order's sequence is replaced by the schedule from this many
// window-heads on (W x H): the schedule's four small kernels cost ~30 us per
// call, 5 % of config 4's pass (62,500 window-heads, which keeps the order's
// sequence) and under 1.5 % from here on.
constexpr int64_t kSchedOrderedMin = (int64_t)1 << 18;
constexpr int kSchedBlock = 1024;   // windows per block of sched_count / sched_fill

struct SchedTables {
    int32_t size[kSchedClasses];               // windows per class outside the team list
    int32_t taken[kSchedClasses];              // windows per class in the team list
    int32_t team_base[kSchedClasses];          // team-list position of a class's first window
    int32_t xcd_base[kXcds][kSchedClasses];    // share x's windows before its part of a class
    int32_t xcd_items[kXcds];                  // share x's windows
    int32_t team_items;                        // team-list entries in use
};

// Slots per XCD share in the one-wave launch: past any share of W windows
// (each class share rounds up by at most one), a multiple of 4.
constexpr int64_t sched_xcd_slots(int64_t W)
{
    return (ceil_div(W, kXcds) + kSchedClasses + 3) / 4 * 4;
}

// Tiles of window w (-1 past the last window).
__device__ __forceinline__ int32_t window_tiles(const int32_t* __restrict__ window_offsets,
                                                int32_t W, int32_t w)
{
    if (w >= W) return -1;
    const int32_t T = window_offsets[W];
    const int32_t tb = max(0, min(window_offsets[w], T));
    const int32_t te = max(tb, min(window_offsets[w + 1], T));
    return te - tb;
}

// Class position of window w (-1: past W, or not named by the order).
__device__ __forceinline__ int sched_pos(const int32_t* __restrict__ window_offsets,
                                         const int32_t* __restrict__ order,
                                         const int32_t* __restrict__ inv, int32_t W, int32_t w,
                                         int32_t heavy)
{
    if (w >= W) return -1;
    if (order) {
        const int32_t p = inv[w];
        if (p < 0 || p >= W || order[p] != w) return -1;
    }
    const int32_t t = window_tiles(window_offsets, W, w);
    const int oct = t > 0 ? 32 - __clz(t) : 0;   // t < 2^31: 0..31
    return t > heavy ? 31 - oct : kSchedClasses - 1 - oct;
}

__global__ void __launch_bounds__(kSchedBlock)
sched_inverse(const int32_t* __restrict__ order, int32_t W, int32_t* __restrict__ inv)
{
    const int32_t p = blockIdx.x * kSchedBlock + threadIdx.x;
    if (p >= W) return;
    const int32_t w = order[p];
    if (w >= 0 && w < W) inv[w] = p;   // duplicates: any of their positions
}

__global__ void __launch_bounds__(kSchedBlock)
sched_count(const int32_t* __restrict__ window_offsets, const int32_t* __restrict__ order,
            const int32_t* __restrict__ inv, int32_t W, int32_t nb, int32_t* __restrict__ counts)
{
    __shared__ int32_t hist[kSchedClasses];
    const int t = threadIdx.x;
    if (t < kSchedClasses) hist[t] = 0;
    __syncthreads();
    const int32_t heavy = heavy_tiles(window_offsets[W], W, kHeavyMinTiles, kHeavyMeanFactor);
    const int q = sched_pos(window_offsets, order, inv, W, blockIdx.x * kSchedBlock + t, heavy);
    if (q >= 0) atomicAdd(&hist[q], 1);
    __syncthreads();
    if (t < kSchedClasses) counts[(int64_t)t * nb + blockIdx.x] = hist[t];
}

// One workgroup of 1,024 threads: counts[q][b] becomes the class-q windows in
// blocks before b; then the tables.  The counts were written by other XCDs a
// kernel earlier, so every load goes below L2: each class's row is cut into
// 16 contiguous segments, one per lane of a 16-lane row, and a lane loads its
// segment in one batch (kept in registers for the rewrite when it holds at
// most kSegRegs values: graphs of up to 524,288 windows), scans the
// 16 sums with its row and writes its segment's offsets.  The tables come
// from wave-wide scans over the classes.
constexpr int kScanSegs = 16;
constexpr int kSegRegs = 32;
static_assert(kSchedClasses * kScanSegs == 1024, "one lane per (class, segment)");
static_assert(kSchedClasses == kWave, "one lane per class in the table scans");
__global__ void __launch_bounds__(1024)
sched_scan(int32_t* __restrict__ counts, int32_t nb, int32_t team_cap, SchedTables* __restrict__ tab)
{
    __shared__ int32_t total[kSchedClasses];
    __shared__ int32_t size[kSchedClasses];
    const int q = threadIdx.x / kScanSegs, k = threadIdx.x % kScanSegs;
    const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
    const int32_t seg = (nb + kScanSegs - 1) / kScanSegs;
    const int32_t b0 = min(nb, k * seg), b1 = min(nb, b0 + seg);
    int32_t* row = counts + (int64_t)q * nb;
    int32_t sum = 0;
    int32_t v[kSegRegs];
    if (seg <= kSegRegs) {   // uniform
#pragma unroll
        for (int u = 0; u < kSegRegs; ++u) v[u] = b0 + u < b1 ? row[b0 + u] : 0;
#pragma unroll
        for (int u = 0; u < kSegRegs; ++u) sum += v[u];
    } else {
        for (int32_t b = b0; b < b1; b += kSegRegs) {
#pragma unroll
            for (int u = 0; u < kSegRegs; ++u) v[u] = b + u < b1 ? row[b + u] : 0;
#pragma unroll
            for (int u = 0; u < kSegRegs; ++u) sum += v[u];
        }
    }
    int32_t inc = sum;
#pragma unroll
    for (int off = 1; off < kScanSegs; off <<= 1) {
        const int32_t y = __shfl_up(inc, off, kScanSegs);
        if (k >= off) inc += y;
    }
    if (k == kScanSegs - 1) total[q] = inc;
    int32_t run = inc - sum;
    if (seg <= kSegRegs) {
#pragma unroll
        for (int u = 0; u < kSegRegs; ++u) {
            if (b0 + u < b1) row[b0 + u] = run;
            run += v[u];
        }
    } else {
        for (int32_t b = b0; b < b1; b += kSegRegs) {
#pragma unroll
            for (int u = 0; u < kSegRegs; ++u) v[u] = b + u < b1 ? row[b + u] : 0;
#pragma unroll
            for (int u = 0; u < kSegRegs; ++u) {
                if (b + u < b1) row[b + u] = run;
                run += v[u];
            }
        }
    }
    __syncthreads();
    if (wid == 0) {
        // lane = class: the heavy classes come first, and the team list takes
        // their first team_cap windows
        const int32_t tot = total[lane];
        const int32_t heavy = lane < kSchedClasses / 2 ? tot : 0;
        const int32_t before = wave_inclusive_scan(heavy) - heavy;
        const int32_t take = max(0, min(heavy, team_cap - before));
        const int32_t team_all = min(team_cap, __shfl(before + heavy, kWave - 1));
        tab->team_base[lane] = lane < kSchedClasses / 2 ? min(before, team_cap) : team_all;
        tab->taken[lane] = take;
        tab->size[lane] = size[lane] = tot - take;
        if (lane == 0) tab->team_items = team_all;
    }
    __syncthreads();
    if (wid < kXcds) {
        // wave x: XCD x's share of each class, scanned over the classes
        const int64_t x = wid, sc = size[lane];
        const int32_t share = (int32_t)(sc * (x + 1) / kXcds - sc * x / kXcds);
        const int32_t incl = wave_inclusive_scan(share);
        tab->xcd_base[x][lane] = incl - share;
        if (lane == kWave - 1) tab->xcd_items[x] = incl;
    }
}

// Slots: the team list (kHeavyMaxWindows entries) and 8 L one-wave slots, slot
// i * 8 + x the i-th window of share x; a class's windows keep their index
// order (stable ranks within a block from wave ballots).
__global__ void __launch_bounds__(kSchedBlock)
sched_fill(const int32_t* __restrict__ window_offsets, const int32_t* __restrict__ order,
           const int32_t* __restrict__ inv, int32_t W, int32_t nb,
           const int32_t* __restrict__ counts, const SchedTables* __restrict__ tab, int32_t L,
           int32_t* __restrict__ team, int32_t* __restrict__ sched)
{
    __shared__ int32_t wc[kSchedBlock / kWave][kSchedClasses];
    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int64_t g = (int64_t)blockIdx.x * kSchedBlock + t;
    if (g < (int64_t)kXcds * L && g / kXcds >= tab->xcd_items[g % kXcds]) sched[g] = -1;
    if (g < kHeavyMaxWindows && g >= tab->team_items) team[g] = -1;
    if ((int32_t)blockIdx.x >= nb) return;   // uniform
    const int32_t heavy = heavy_tiles(window_offsets[W], W, kHeavyMinTiles, kHeavyMeanFactor);
    const int32_t w = blockIdx.x * kSchedBlock + t;
    const int q = sched_pos(window_offsets, order, inv, W, w, heavy);
    for (int k = lane; k < kSchedClasses; k += kWave) wc[wid][k] = 0;
    int32_t rank = 0;
    const uint64_t below = (1ull << lane) - 1ull;
    uint64_t rem = __ballot(q >= 0);
    while (rem) {   // one round per class present in the wave
        const int lead = __ffsll((unsigned long long)rem) - 1;
        const int cq = __shfl(q, lead);
        const uint64_t m = __ballot(q == cq);
        if (q == cq) rank = __popcll(m & below);
        if (lane == lead) wc[wid][cq] = __popcll(m);
        rem &= ~m;
    }
    __syncthreads();
    if (q < 0) return;
    for (int v = 0; v < wid; ++v) rank += wc[v][q];
    const int32_t r = counts[(int64_t)q * nb + blockIdx.x] + rank;   // rank in its class
    const int32_t take = tab->taken[q];
    if (r < take) {
        team[tab->team_base[q] + r] = w;
        return;
    }
    const int64_t sz = tab->size[q], r2 = r - take;
    const int64_t x = (kXcds * r2 + kXcds - 1) / sz;   // its share: [sz x / 8, sz (x + 1) / 8)
    sched[(tab->xcd_base[x][q] + (r2 - sz * x / kXcds)) * kXcds + x] = w;
}

// Scratch of the scheduled launch for W windows, in 256-byte sections: the
// tables, the team list, the class counts (kSchedClasses per block of
// kSchedBlock windows), the one-wave slots and, given a window order, its
// inverse.
struct SchedScratch {
    size_t tab, team, counts, sched, inv, bytes;
};
constexpr size_t round256(size_t b) { return (b + 255) / 256 * 256; }
constexpr SchedScratch sched_scratch(int64_t W, bool ordered)
{
    auto up = round256;
    SchedScratch l{};
    l.tab = 0;
    l.team = up(sizeof(SchedTables));
    l.counts = l.team + up(sizeof(int32_t) * kHeavyMaxWindows);
    l.sched = l.counts + up(sizeof(int32_t) * kSchedClasses * (size_t)ceil_div(W, kSchedBlock));
    l.inv = l.sched + up(sizeof(int32_t) * kXcds * (size_t)sched_xcd_slots(W));
    l.bytes = l.inv + (ordered ? up(sizeof(int32_t) * (size_t)W) : 0);
    return l;
}

// Builds the schedule of W windows (those `order` names, or all) into scratch
// `sp` laid out by sched_scratch(W, order != NULL): a team list of at most
// team_cap heavy windows (kHeavyMaxWindows entries, -1 past its end) and
// kXcds * L one-wave slots (-1 where empty), L = sched_xcd_slots(W), to be
// dealt to the XCDs round-robin.
static f3s_status launch_schedule(const int32_t* d_window_offsets, const int32_t* d_window_order,
                                  int32_t W, int32_t team_cap, char* sp, hipStream_t st,
                                  int32_t** team_out, int32_t** sched_out)
{
    const bool ordered = d_window_order != nullptr;
    const SchedScratch lay = sched_scratch(W, ordered);
    SchedTables* tab = reinterpret_cast<SchedTables*>(sp + lay.tab);
    int32_t* team = reinterpret_cast<int32_t*>(sp + lay.team);
    int32_t* counts = reinterpret_cast<int32_t*>(sp + lay.counts);
    int32_t* sched = reinterpret_cast<int32_t*>(sp + lay.sched);
    int32_t* inv = ordered ? reinterpret_cast<int32_t*>(sp + lay.inv) : nullptr;
    const int32_t nb = (int32_t)ceil_div(W, kSchedBlock);
    const int64_t L = sched_xcd_slots(W);
    const int32_t fill_blocks = (int32_t)std::max<int64_t>(nb, ceil_div(kXcds * L, kSchedBlock));
    if (ordered)
        hipLaunchKernelGGL(sched_inverse, dim3((unsigned)nb), dim3(kSchedBlock), 0, st,
                           d_window_order, W, inv);
    hipLaunchKernelGGL(sched_count, dim3((unsigned)nb), dim3(kSchedBlock), 0, st,
                       d_window_offsets, d_window_order, inv, W, nb, counts);
    hipLaunchKernelGGL(sched_scan, dim3(1), dim3(1024), 0, st, counts, nb, team_cap, tab);
    hipLaunchKernelGGL(sched_fill, dim3((unsigned)fill_blocks), dim3(kSchedBlock), 0, st,
                       d_window_offsets, d_window_order, inv, W, nb, counts, tab, (int32_t)L,
                       team, sched);
    const hipError_t le = hipGetLastError();
    if (le != hipSuccess) return hip_fail(le, "window schedule", __FILE__, __LINE__);
    *team_out = team;
    *sched_out = sched;
    return F3S_OK;
}

// ----------------------------------------------------------------- planner

// Segment sizes of an automatic plan.  A window is cut into segments only
// when it is well above the mean window (4x masked, 2x tile-dense: cutting
// every window of a uniform graph just adds merge traffic) and, masked, above
// 1/3072 of the pass's tile-heads (tile-dense: 1/51200).  Forced masked sizes
// on config 4 (15.9 M tiles, one head) ran flat from 3,584 to 6,144 tiles
// (546-549 us) against 557 us at 1/8192 (1,936 tiles) and 571 us at 1,024:
// the heaviest windows, which the descending order starts first, need few
// segments.  seg[0] serves masked passes, seg[1] tile-dense ones.
__host__ __device__ __forceinline__ void auto_segments(int64_t T, int32_t W, int32_t H,
                                                       int64_t seg[2])
{
    const int64_t mean = W > 0 ? (T + W - 1) / W : 0;
    int64_t m = 256, dd = 16;
    if (4 * mean > m) m = 4 * mean;
    if ((T * H + 3071) / 3072 > m) m = (T * H + 3071) / 3072;
    if (2 * mean > dd) dd = 2 * mean;
    if ((T * H + 51199) / 51200 > dd) dd = (T * H + 51199) / 51200;
    seg[0] = m < INT32_MAX ? m : INT32_MAX;
    seg[1] = dd < INT32_MAX ? dd : INT32_MAX;
}

// Work items per position of the plan's sequence (P positions; window
// order[L], or L; invalid entries hold no window) for one or two item sets:
// counts[3 k + 0] items, [3 k + 1] partial slots, [3 k + 2] split windows of
// set k, each [P].  seg_fixed > 0 is the one set's segment size; 0 takes the
// automatic sizes from T = offs[W] (thread 0 also reports T and the sizes in
// info).
__global__ void plan_count(const int32_t* __restrict__ offs, const int32_t* __restrict__ order,
                           int32_t W, int32_t P, int32_t H, int32_t seg_fixed, int32_t nsets,
                           int32_t team0, int32_t team1, int32_t* __restrict__ counts,
                           int64_t* __restrict__ info)
{
    const int32_t L = blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t T = W > 0 ? max(0, offs[W]) : 0;
    int64_t seg[2];
    if (seg_fixed > 0) {
        seg[0] = seg[1] = seg_fixed;
    } else {
        auto_segments(T, W, H, seg);
    }
    if (L == 0) {
        info[0] = T;
        info[1] = seg[0];
        info[2] = seg[1];
    }
    if (L >= P) return;
    const int32_t w = order ? order[L] : L;
    int32_t nt = 0;
    if (w >= 0 && w < W) {
        const int32_t tb = max(0, min(offs[w], T)), te = max(tb, min(offs[w + 1], T));
        nt = te - tb;
    }
    for (int k = 0; k < nsets; ++k) {
        const int32_t team = k == 0 ? team0 : team1;
        int32_t ns = 1;
        if (team > 1) {
            ns = team;   // a team's items, merged in LDS: no partials
        } else if (nt > seg[k]) {
            ns = (int32_t)((nt + seg[k] - 1) / seg[k]);
        }
        const bool split = team == 1 && ns > 1;
        counts[(3 * k + 0) * (int64_t)P + L] = ns;
        counts[(3 * k + 1) * (int64_t)P + L] = split ? ns : 0;
        counts[(3 * k + 2) * (int64_t)P + L] = split ? 1 : 0;
    }
}

// info[3 + j] = total of scanned count array j (bases[j][P]).
__global__ void plan_totals(const int64_t* __restrict__ bases, int32_t P, int32_t arrays,
                            int64_t* __restrict__ info)
{
    const int j = threadIdx.x;
    if (j < arrays) info[3 + j] = bases[(int64_t)j * ((int64_t)P + 1) + P];
}

__global__ void plan_fill(const int32_t* __restrict__ offs, const int32_t* __restrict__ order,
                          int32_t W, int32_t P, int32_t seg, int32_t team,
                          const int64_t* __restrict__ item_base,
                          const int64_t* __restrict__ slot_base,
                          const int64_t* __restrict__ split_base, Item* __restrict__ items,
                          SplitInfo* __restrict__ splits, int32_t* __restrict__ slot_split)
{
    const int32_t L = blockIdx.x * blockDim.x + threadIdx.x;
    if (L >= P) return;
    const int32_t w = order ? order[L] : L;
    const int64_t ib = item_base[L];
    const int32_t ns = (int32_t)(item_base[L + 1] - ib);
    if (w < 0 || w >= W) {
        for (int32_t k = 0; k < ns; ++k)
            items[ib + k] = Item{-1, 0, 0, -1};   // no window: the pass skips these
        return;
    }
    const int32_t T = offs[W];
    const int32_t tb = max(0, min(offs[w], T)), te = max(tb, min(offs[w + 1], T));
    if (team > 1) {
        for (int32_t k = 0; k < team; ++k)
            items[ib + k] = Item{w, team_part(tb, te, k, team), team_part(tb, te, k + 1, team), -1};
        return;
    }
    if (ns == 1) {
        items[ib] = Item{w, tb, te, -1};
        return;
    }
    const int32_t sb = (int32_t)slot_base[L];
    const int64_t sid = split_base[L];
    splits[sid] = SplitInfo{w, sb, ns, 0};
    for (int32_t k = 0; k < ns; ++k) {
        const int32_t a = tb + k * seg;
        items[ib + k] = Item{w, a, min(te, a + seg), sb + k};
        slot_split[sb + k] = (int32_t)sid;
    }
}

__global__ void offsets_to_i32_plan(const int64_t* __restrict__ in, int32_t* __restrict__ out,
                                    int64_t count)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = (int32_t)in[i];
}

// Attended columns of each planned item (masked semantics): one wave per
// item counts them (pass 1) or lists them, in tile order, padded to whole
// chunks (pass 2) -- the expansion the ring path performs on every pass,
// done once per graph.
template <bool FILL>
__global__ void __launch_bounds__(256)
plan_columns(const Item* __restrict__ items, int64_t num_items,
             const int32_t* __restrict__ block_col, const uint16_t* __restrict__ tile_mask,
             int32_t n, uint32_t ref_stride, uint32_t no_ref, int32_t* __restrict__ nchunks,
             const int64_t* __restrict__ chunk_base, uint32_t* __restrict__ columns)
{
    const int64_t it = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (it >= num_items) return;
    const Item item = items[it];
    const int32_t nbc = (n + 15) >> 4;
    int64_t pos = 0;   // wave-uniform
    uint32_t* rec0 = FILL ? columns + chunk_base[it] * 64 : nullptr;
    for (int32_t t0 = item.tb; t0 < item.te; t0 += kWave) {
        const int32_t t = t0 + lane;
        uint32_t u = 0;
        int32_t bc = 0;
        uint32_t wd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (t < item.te) {
            bc = block_col[t];
            if ((uint32_t)bc < (uint32_t)nbc) {
                const int32_t left = n - bc * 16;
                const uint32_t vmask = left >= 16 ? 0xffffu : ((1u << left) - 1u);
                const uint4* mp = reinterpret_cast<const uint4*>(tile_mask + (int64_t)t * 16);
                const uint4 a = mp[0], b = mp[1];
                wd[0] = a.x; wd[1] = a.y; wd[2] = a.z; wd[3] = a.w;
                wd[4] = b.x; wd[5] = b.y; wd[6] = b.z; wd[7] = b.w;
                const uint32_t o = a.x | a.y | a.z | a.w | b.x | b.y | b.z | b.w;
                u = (o | (o >> 16)) & vmask;
            }
        }
        const int occ = __popc(u);
        const int incl = wave_scan_incl(occ);
        if (FILL && occ) {
            int64_t q = pos + incl - occ;
            const uint32_t base = (uint32_t)bc * 16 * ref_stride;
            uint32_t rest = u;
            while (rest) {
                const int c = __ffs(rest) - 1;
                rest &= rest - 1;
                uint32_t* rec = rec0 + (q >> 5) * 64;
                rec[q & 31] = base + (uint32_t)c * ref_stride;
                rec[32 + (q & 31)] = column_rows(wd, c);
                ++q;
            }
        }
        pos += __builtin_amdgcn_readlane(incl, kWave - 1);
    }
    const int64_t nch = (pos + kChunk - 1) / kChunk;
    if (!FILL) {
        if (lane == 0) nchunks[it] = (int32_t)nch;
        return;
    }
    // pad the last chunk with slots no row attends, read as zero
    for (int64_t q = pos + lane; q < nch * kChunk; q += kWave) {
        uint32_t* rec = rec0 + (q >> 5) * 64;
        rec[q & 31] = no_ref;
        rec[32 + (q & 31)] = 0u;
    }
}

}  // namespace f3s

namespace f3s {

// Lays out a plan's work items: counts for every item set in one pass, one
// host round trip for their totals (and, for automatic plans, T and the
// segment sizes computed on the device), then the item lists; the partial
// buffer is shared by the sets (a plan serves one pass at a time).  From
// kSchedOrderedMin window-heads on, with one wave per item (no teams), the
// items follow the drop-in launch's schedule (classes of tile count,
// heaviest first, eight interleaved XCD shares; no team list: heavy windows
// are split into segments), dealt round-robin, whatever the window order;
// otherwise they follow the order's sequence.  (On config 4, 62,500
// window-heads, the schedule measured 1-2 % slower than the descending
// order's sequence: 562 against 558 us masked, 8.96 against 8.76 ms
// tile-dense.)
static f3s_status build_plan_sets(f3s_plan* p, const int32_t* d_window_offsets,
                                  const int32_t* d_window_order, int32_t seg_tiles,
                                  hipStream_t st)
{
    const int32_t W = p->W, H = p->H;
    const bool automatic = seg_tiles == 0;
    const int32_t team_m = automatic ? team_for(W, H, true) : 1;
    const int32_t team_d = automatic ? team_for(W, H, false) : 1;
    const int32_t nsets = automatic ? 2 : 1;
    const int arrays = 3 * nsets;
    const bool scheduled = W > kHeavyMaxWindows && team_m == 1 && team_d == 1 &&
                           (int64_t)W * H >= kSchedOrderedMin;
    StreamBuffer sbuf(st);
    const int32_t* seq = d_window_order;   // the sequence of positions
    int32_t P = W;
    if (scheduled) {
        F3S_TRY(sbuf.reserve(sched_scratch(W, d_window_order != nullptr).bytes));
        int32_t* team = nullptr;
        int32_t* sched = nullptr;
        F3S_TRY(launch_schedule(d_window_offsets, d_window_order, W, 0,
                                static_cast<char*>(sbuf.ptr), st, &team, &sched));
        seq = sched;
        P = (int32_t)(kXcds * sched_xcd_slots(W));
    }
    p->xcd_contiguous = !scheduled && d_window_order == nullptr;
    const size_t cnt_bytes = sizeof(int32_t) * (size_t)arrays * (size_t)P;
    const size_t base_bytes = sizeof(int64_t) * (size_t)arrays * ((size_t)P + 1);
    const size_t tmp_bytes = sizeof(int64_t) * (size_t)scan_tmp_elems(P);
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    StreamBuffer buf(st);
    F3S_TRY(buf.reserve(256 + al(cnt_bytes) + al(base_bytes) + al(tmp_bytes)));
    char* q = static_cast<char*>(buf.ptr);
    int64_t* info = reinterpret_cast<int64_t*>(q);           // [0] T, [1..2] segs, [3..] totals
    int32_t* counts = reinterpret_cast<int32_t*>(q + 256);
    int64_t* bases = reinterpret_cast<int64_t*>(q + 256 + al(cnt_bytes));
    int64_t* tmp = reinterpret_cast<int64_t*>(q + 256 + al(cnt_bytes) + al(base_bytes));
    hipLaunchKernelGGL(plan_count, dim3((unsigned)ceil_div(P > 0 ? P : 1, 256)), dim3(256), 0, st,
                       d_window_offsets, seq, W, P, H, seg_tiles, nsets, team_m, team_d, counts,
                       info);
    F3S_HIP(hipGetLastError());
    for (int j = 0; j < arrays; ++j)
        F3S_TRY(exclusive_scan_i32_to_i64(counts + (size_t)j * P, bases + (size_t)j * (P + 1), P,
                                          tmp, st));
    hipLaunchKernelGGL(plan_totals, dim3(1), dim3(64), 0, st, bases, P, arrays, info);
    F3S_HIP(hipGetLastError());
    int64_t* h = host_staging();
    F3S_HIP(hipMemcpyAsync(h, info, sizeof(int64_t) * (3 + arrays), hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    p->T = h[0];
    const int32_t seg_m = (int32_t)h[1], seg_d = (int32_t)h[2];
    p->has_dense = automatic && (team_d != team_m || (team_d == 1 && seg_d != seg_m));
    int64_t max_slots = 0, max_split = 0;
    for (int k = 0; k < nsets; ++k) {
        f3s_item_set& set = k == 0 ? p->masked : p->dense;
        if (k == 1 && !p->has_dense) break;
        set.seg = k == 0 ? seg_m : seg_d;
        set.team = k == 0 ? team_m : team_d;
        set.num_items = h[3 + 3 * k];
        set.num_slots = h[3 + 3 * k + 1];
        set.num_split = h[3 + 3 * k + 2];
        if (set.num_slots > max_slots) max_slots = set.num_slots;
        F3S_TRY(set.items.reserve(sizeof(Item) * (size_t)(set.num_items + 1), st));
        F3S_TRY(set.splits.reserve(sizeof(SplitInfo) * (size_t)(set.num_split + 1), st));
        F3S_TRY(set.slot_split.reserve(sizeof(int32_t) * (size_t)(set.num_slots + 1), st));
        if (set.num_split > max_split) max_split = set.num_split;
    }
    F3S_TRY(p->partials.reserve(sizeof(float) * (size_t)kPartialFloats * H * (size_t)(max_slots + 1),
                                st));
    // the in-launch merge's arrival counts start at zero (each pass leaves
    // them so); both sets share them, as they share the partials
    const size_t cnt_b = sizeof(int32_t) * (size_t)H * (size_t)(max_split + 1);
    F3S_TRY(p->counters.reserve(cnt_b, st));
    F3S_HIP(hipMemsetAsync(p->counters.ptr, 0, cnt_b, st));
    for (int k = 0; k < nsets && P > 0; ++k) {
        if (k == 1 && !p->has_dense) break;
        f3s_item_set& set = k == 0 ? p->masked : p->dense;
        const int64_t* bk = bases + (size_t)3 * k * (P + 1);
        hipLaunchKernelGGL(plan_fill, dim3((unsigned)ceil_div(P, 256)), dim3(256), 0, st,
                           d_window_offsets, seq, W, P, set.seg, set.team, bk, bk + (P + 1),
                           bk + 2 * (size_t)(P + 1), reinterpret_cast<Item*>(set.items.ptr),
                           reinterpret_cast<SplitInfo*>(set.splits.ptr),
                           reinterpret_cast<int32_t*>(set.slot_split.ptr));
        F3S_HIP(hipGetLastError());
    }
    // the plan is complete (and its memory usable on any stream) on return
    F3S_HIP(hipStreamSynchronize(st));
    return F3S_OK;
}

static f3s_status check_attention_args(const void* Q, const void* K, const void* V, const void* O,
                                       int32_t n, int32_t d, int32_t H)
{
    F3S_REQUIRE(n >= 0, "attention: negative n");
    if (d != kD) {
        set_error("attention: only d == 64 is implemented (FEAT_DIM_FIXED of the reference)");
        return F3S_EUNSUPPORTED;
    }
    if (H < 1 || H > kMaxHeads) {
        set_error("attention: H must be in [1, 64]");
        return F3S_EUNSUPPORTED;
    }
    F3S_REQUIRE(n == 0 || (Q && K && V && O), "attention: NULL feature pointer");
    F3S_REQUIRE(((((uintptr_t)Q) | ((uintptr_t)K) | ((uintptr_t)V) | ((uintptr_t)O)) & 15) == 0,
                "attention: Q, K, V, O must be 16-byte aligned");
    return F3S_OK;
}

template <int MODE, bool WIDE>
static void launch_mw(const AttnParams& p, int64_t waves, hipStream_t st)
{
    if constexpr (!WIDE) {
        // teams (small graphs; never wide): one workgroup per (window, head)
        if (p.team == kTeamLarge) {
            hipLaunchKernelGGL((fused_attention_kernel<MODE, kTeamLarge, false, kTeamLarge>),
                               dim3((unsigned)(waves / kTeamLarge)), dim3(kTeamLarge * kWave), 0,
                               st, p);
            return;
        }
        if (p.team == kTeamSmall) {
            hipLaunchKernelGGL((fused_attention_kernel<MODE, kTeamSmall, false, kTeamSmall>),
                               dim3((unsigned)(waves / kTeamSmall)), dim3(kTeamSmall * kWave), 0,
                               st, p);
            return;
        }
    }
    // Small launches use one-wave workgroups so they spread over all CUs.
    if (waves < 4 * 256 * 2) {
        hipLaunchKernelGGL((fused_attention_kernel<MODE, 1, WIDE, 1>), dim3((unsigned)waves),
                           dim3(kWave), 0, st, p);
    } else {
        hipLaunchKernelGGL((fused_attention_kernel<MODE, 4, WIDE, 1>),
                           dim3((unsigned)ceil_div(waves, 4)), dim3(4 * kWave), 0, st, p);
    }
}

template <int MODE>
static void launch_m(const AttnParams& p, int64_t waves, hipStream_t st)
{
    if (wide_features(p.n, p.H))
        launch_mw<MODE, true>(p, waves, st);
    else
        launch_mw<MODE, false>(p, waves, st);
}

static f3s_status launch(AttnParams p, int32_t H, float scale, hipStream_t st)
{
    if (p.num_items <= 0) return F3S_OK;
    const int64_t waves = p.num_items * H;
    F3S_REQUIRE(waves < ((int64_t)1 << 31), "attention: too many work items");
    p.scale_log2 = scale * 1.4426950408889634f;
    p.H = H;
    // narrow launches range-check buffer loads against the tensor size;
    // wide ones never use the buffer descriptors
    p.feat_bytes = wide_features(p.n, H) ? 0u : (uint32_t)((int64_t)p.n * H * kRowBytes);
    if (p.team > 1) {
        F3S_REQUIRE((p.team == kTeamSmall || p.team == kTeamLarge) && p.num_items % p.team == 0 &&
                        p.num_split == 0 && !wide_features(p.n, H),
                    "attention: invalid team launch");
    }
    F3S_REQUIRE(p.num_split == 0 || (p.items && p.splits && p.slot_split && p.counters && p.partials),
                "attention: split windows need the plan's merge state");
    if (!p.tile_mask)
        launch_m<kModeDense>(p, waves, st);
    else if (p.chunk_base)
        launch_m<kModeList>(p, waves, st);
    else
        launch_m<kModeRing>(p, waves, st);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}

// f3s_attention_fwd; the scheduled launch takes its scratch from
// `fixed_scratch` when given (f3s_attention_fwd_noalloc, already checked to
// be large enough), else from the allocator, returned in stream order.
static f3s_status attention_fwd_impl(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                     float* O, const int32_t* d_window_offsets,
                                     const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                     const int32_t* d_window_order, int32_t W, int32_t n,
                                     int32_t d, int32_t H, float scale, void* stream,
                                     void* fixed_scratch)
{
    F3S_TRY(check_attention_args(Q, K, V, O, n, d, H));
    F3S_REQUIRE(W == (int32_t)ceil_div(n, 16), "f3s_attention_fwd: W must equal ceil(n/16)");
    F3S_REQUIRE(W == 0 || (d_window_offsets && d_block_col),
                "f3s_attention_fwd: NULL block-sparse pointer");
    F3S_REQUIRE((((uintptr_t)d_tile_mask) & 15) == 0, "f3s_attention_fwd: tile_mask alignment");
    F3S_TRY(require_device());
    clear_error();
    AttnParams p{};
    p.Q = reinterpret_cast<const _Float16*>(Q);
    p.K = reinterpret_cast<const _Float16*>(K);
    p.V = reinterpret_cast<const _Float16*>(V);
    p.O = O;
    p.window_offsets = d_window_offsets;
    p.block_col = d_block_col;
    p.tile_mask = d_tile_mask;
    p.window_order = d_window_order;
    p.team = team_for(W, H, d_tile_mask != nullptr);
    p.num_items = (int64_t)W * p.team;
    p.W = W;
    p.n = n;
    p.xcd_contiguous = d_window_order == nullptr;
    hipStream_t st = as_stream(stream);
    const bool ordered = d_window_order != nullptr;
    // The schedule's scratch: returned to the allocator in stream order when
    // this function returns, i.e. after the last launch that reads it.
    StreamBuffer scratch(st);
    // A window holds at most one tile per block column, W of them, so with
    // W <= kHeavyMinTiles no window of a valid block-sparse form is heavy:
    // then no team launch (the schedule gets an empty team list, so any
    // window still runs on one wave).
    const bool heavy_possible = W > kHeavyMinTiles;
    if (p.team == 1 && !wide_features(n, H) && W > kHeavyMaxWindows &&
        (!ordered || (int64_t)W * H >= kSchedOrderedMin)) {
        // the library's schedule (see sched_fill): heavy windows on teams of
        // 16 waves, the others on one wave each, by class, XCD by XCD
        char* sp = static_cast<char*>(fixed_scratch);
        if (!sp) {
            F3S_TRY(scratch.reserve(sched_scratch(W, ordered).bytes));
            sp = static_cast<char*>(scratch.ptr);
        }
        int32_t *team = nullptr, *sched = nullptr;
        F3S_TRY(launch_schedule(d_window_offsets, d_window_order, W,
                                heavy_possible ? kHeavyMaxWindows : 0, sp, st, &team, &sched));
        const int64_t L = sched_xcd_slots(W);
        if (heavy_possible) {
            AttnParams ph = p;
            ph.window_order = team;
            ph.xcd_contiguous = 0;
            ph.team = kTeamLarge;
            ph.num_items = (int64_t)kHeavyMaxWindows * kTeamLarge;
            F3S_TRY(launch(ph, H, scale, st));
        }
        p.window_order = sched;
        p.xcd_contiguous = 0;
        p.num_items = kXcds * L;
    } else if (p.team == 1 && ordered && !wide_features(n, H) && heavy_possible) {
        // The order's sequence: teams of 16 waves for the heavy windows among
        // its first kHeavyMaxWindows entries (the reference's descending order
        // puts the hubs there), then one wave per entry for all others; each
        // entry belongs to exactly one of the two launches.
        AttnParams ph = p;
        ph.team = kTeamLarge;
        ph.num_items = (int64_t)std::min<int32_t>(W, kHeavyMaxWindows) * kTeamLarge;
        ph.heavy_mode = 2;
        F3S_TRY(launch(ph, H, scale, st));
        p.heavy_mode = 1;
    }
    return launch(p, H, scale, st);
}


// ------------------------------------------------ allocation-free entry point
//
// f3s_attention_fwd_noalloc: the scheduled launch's scratch (tables, team
// list, class counts, one-wave slots, an order's inverse) lives in a
// file-scope device array sized for graphs of up to kNoAllocMaxWindows row
// windows; each device holds its own copy for the life of the process.  Host
// code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): its device address is looked up once per
// device with hipGetSymbolAddress and kept in g_noalloc_addr.
constexpr int32_t kNoAllocMaxWindows = 1 << 21;   // n <= 33,554,432 nodes
constexpr size_t kNoAllocScratchBytes = sched_scratch(kNoAllocMaxWindows, true).bytes;
static __device__ __align__(256) unsigned char noalloc_scratch[kNoAllocScratchBytes];

constexpr int kNoAllocDevices = 64;
static std::mutex g_noalloc_mu;
static void* g_noalloc_addr[kNoAllocDevices] = {};

// The device address of noalloc_scratch on the current device (looked up on
// the first call per device, with that device current).
static f3s_status noalloc_scratch_addr(void** out)
{
    *out = nullptr;
    int dev = 0;
    F3S_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kNoAllocDevices) {
        set_error("f3s_attention_fwd_noalloc: device index beyond the library's table");
        return F3S_EUNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_addr[dev]) {
        void* p = nullptr;
        F3S_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)));
        if (!p) {
            set_error("f3s_attention_fwd_noalloc: no device address for its scratch");
            return F3S_EHIP;
        }
        g_noalloc_addr[dev] = p;
    }
    *out = g_noalloc_addr[dev];
    return F3S_OK;
}

// f3s_init: the current device's address, looked up ahead of the first call.
f3s_status noalloc_setup()
{
    void* p = nullptr;
    return noalloc_scratch_addr(&p);
}

}  // namespace f3s

using namespace f3s;

extern "C" {

f3s_status f3s_attention_fwd(const uint16_t* Q, const uint16_t* K, const uint16_t* V, float* O,
                             const int32_t* d_window_offsets, const int32_t* d_block_col,
                             const uint16_t* d_tile_mask, const int32_t* d_window_order,
                             int32_t W, int32_t n, int32_t d, int32_t H, float scale,
                             void* stream)
{
    return attention_fwd_impl(Q, K, V, O, d_window_offsets, d_block_col, d_tile_mask,
                              d_window_order, W, n, d, H, scale, stream, nullptr);
}

f3s_status f3s_attention_fwd_noalloc(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                     float* O, const int32_t* d_window_offsets,
                                     const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                     const int32_t* d_window_order, int32_t W, int32_t n,
                                     int32_t d, int32_t H, float scale, void* stream)
{
    if (W < 0 || W > kNoAllocMaxWindows) {
        set_error("f3s_attention_fwd_noalloc: W outside [0, 2097152] (the limit of its fixed "
                  "scratch, graphs of up to 33,554,432 nodes); use f3s_attention_fwd");
        return F3S_EUNSUPPORTED;
    }
    F3S_TRY(check_attention_args(Q, K, V, O, n, d, H));
    F3S_TRY(require_device());
    void* sp = nullptr;
    F3S_TRY(noalloc_scratch_addr(&sp));
    static_assert(sched_scratch(kNoAllocMaxWindows, true).bytes >=
                      sched_scratch(kNoAllocMaxWindows, false).bytes,
                  "an order's inverse only adds to the scratch");
    return attention_fwd_impl(Q, K, V, O, d_window_offsets, d_block_col, d_tile_mask,
                              d_window_order, W, n, d, H, scale, stream, sp);
}

f3s_status f3s_plan_create(const int32_t* d_window_offsets, const int32_t* d_window_order,
                           int32_t W, int32_t H, int32_t seg_tiles, void* stream,
                           f3s_plan** plan_out)
{
    F3S_REQUIRE(plan_out != nullptr, "f3s_plan_create: NULL out pointer");
    *plan_out = nullptr;
    F3S_REQUIRE(W >= 0, "f3s_plan_create: negative W");
    F3S_REQUIRE(W == 0 || d_window_offsets, "f3s_plan_create: NULL window_offsets");
    F3S_REQUIRE(H >= 1 && H <= kMaxHeads, "f3s_plan_create: H must be in [1, 64]");
    F3S_REQUIRE(seg_tiles >= 0, "f3s_plan_create: negative seg_tiles");
    F3S_TRY(require_device());
    clear_error();
    hipStream_t st = as_stream(stream);

    f3s_plan* p = new (std::nothrow) f3s_plan();
    if (!p) {
        set_error("f3s_plan_create: out of host memory");
        return F3S_ENOMEM;
    }
    p->W = W;
    p->H = H;
    // Automatic plans give tile-dense passes their own, finer item set (a
    // tile-dense chunk costs two whole tiles, ~15x a masked chunk per tile
    // on sparse graphs); graphs whose windows leave most SIMDs idle run teams
    // instead (team_for), as the unplanned launch does.
    const f3s_status s = build_plan_sets(p, d_window_offsets, d_window_order, seg_tiles, st);
    if (s != F3S_OK) {
        delete p;
        return s;
    }
    *plan_out = p;
    return F3S_OK;
}

f3s_status f3s_plan_compile(f3s_plan* plan, const int32_t* d_block_col,
                            const uint16_t* d_tile_mask, int32_t n, void* stream)
{
    F3S_REQUIRE(plan != nullptr, "f3s_plan_compile: NULL plan");
    F3S_REQUIRE(d_tile_mask != nullptr, "f3s_plan_compile: needs the tile masks");
    F3S_REQUIRE(plan->T == 0 || d_block_col, "f3s_plan_compile: NULL block_col");
    F3S_REQUIRE((((uintptr_t)d_tile_mask) & 15) == 0, "f3s_plan_compile: tile_mask alignment");
    F3S_REQUIRE(plan->W == (int32_t)ceil_div(n, 16), "f3s_plan_compile: n does not match W");
    F3S_TRY(require_device());
    clear_error();
    hipStream_t st = as_stream(stream);
    plan->compiled_tile_mask = nullptr;
    plan->compiled_block_col = nullptr;
    plan->compiled_n = -1;
    const int64_t ni = plan->masked.num_items;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t cnt_bytes = al(sizeof(int32_t) * (size_t)(ni + 1));
    const size_t base_bytes = al(sizeof(int64_t) * (size_t)(ni + 1));
    StreamBuffer buf(st);
    F3S_TRY(buf.reserve(cnt_bytes + base_bytes + sizeof(int64_t) * (size_t)scan_tmp_elems(ni)));
    auto* counts = reinterpret_cast<int32_t*>(buf.ptr);
    auto* b64 = reinterpret_cast<int64_t*>(static_cast<char*>(buf.ptr) + cnt_bytes);
    auto* tmp = reinterpret_cast<int64_t*>(static_cast<char*>(buf.ptr) + cnt_bytes + base_bytes);
    // the records hold row references: byte offsets, or node indices when the
    // feature tensors are too large for 32-bit offsets (wide launches)
    const bool wide = wide_features(n, plan->H);
    const uint32_t ref_stride = wide ? 1u : (uint32_t)plan->H * kRowBytes;
    const uint32_t no_ref = wide ? kNoIdx : kNoRow;
    const auto* items = reinterpret_cast<const Item*>(plan->masked.items.ptr);
    const dim3 grid((unsigned)ceil_div(ni > 0 ? ni : 1, 4));
    if (ni > 0)
        hipLaunchKernelGGL(plan_columns<false>, grid, dim3(256), 0, st, items, ni, d_block_col,
                           d_tile_mask, n, ref_stride, no_ref, counts, nullptr, nullptr);
    F3S_HIP(hipGetLastError());
    F3S_TRY(exclusive_scan_i32_to_i64(counts, b64, ni, tmp, st));
    int64_t* h = host_staging();
    F3S_HIP(hipMemcpyAsync(h, b64 + ni, sizeof(int64_t), hipMemcpyDeviceToHost, st));
    F3S_HIP(hipStreamSynchronize(st));
    const int64_t total = h[0];
    if (total >= INT32_MAX) {
        set_error("f3s_plan_compile: more than 2^31-1 chunks");
        return F3S_EUNSUPPORTED;
    }
    // four records of padding: the pass reads records in blocks of four
    F3S_TRY(plan->columns.reserve(sizeof(uint32_t) * 64 * (size_t)(total + 4), st));
    F3S_TRY(plan->chunk_base.reserve(sizeof(int32_t) * (size_t)(ni + 1), st));
    if (ni > 0) {
        hipLaunchKernelGGL(plan_columns<true>, grid, dim3(256), 0, st, items, ni, d_block_col,
                           d_tile_mask, n, ref_stride, no_ref, nullptr, b64,
                           reinterpret_cast<uint32_t*>(plan->columns.ptr));
        F3S_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(offsets_to_i32_plan, dim3((unsigned)ceil_div(ni + 1, 256)), dim3(256), 0,
                       st, b64, reinterpret_cast<int32_t*>(plan->chunk_base.ptr), ni + 1);
    F3S_HIP(hipGetLastError());
    // the lists are complete (and usable on any stream) on return
    F3S_HIP(hipStreamSynchronize(st));
    plan->num_chunks = total;
    plan->compiled_tile_mask = d_tile_mask;
    plan->compiled_block_col = d_block_col;
    plan->compiled_n = n;
    return F3S_OK;
}

f3s_status f3s_plan_destroy(f3s_plan* plan)
{
    if (!plan) return F3S_OK;
    // one wait for the plan's device (its passes may run on any stream), then
    // every buffer goes back to the allocator's cache at once
    int dev = plan->masked.items.device, cur = -1;
    const bool switch_dev = dev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != dev &&
                            hipSetDevice(dev) == hipSuccess;
    (void)hipDeviceSynchronize();
    for (f3s_item_set* set : {&plan->masked, &plan->dense}) {
        set->items.release_idle();
        set->splits.release_idle();
        set->slot_split.release_idle();
    }
    plan->partials.release_idle();
    plan->counters.release_idle();
    plan->chunk_base.release_idle();
    plan->columns.release_idle();
    if (switch_dev) (void)hipSetDevice(cur);
    delete plan;
    return F3S_OK;
}

f3s_status f3s_plan_info(const f3s_plan* plan, int64_t* num_items, int64_t* num_split_windows,
                         int64_t* T, int32_t* seg_tiles)
{
    F3S_REQUIRE(plan != nullptr, "f3s_plan_info: NULL plan");
    if (num_items) *num_items = plan->masked.num_items;
    if (num_split_windows) *num_split_windows = plan->masked.num_split;
    if (T) *T = plan->T;
    if (seg_tiles) *seg_tiles = plan->masked.seg;
    return F3S_OK;
}

f3s_status f3s_plan_stats(const f3s_plan* plan, int64_t* num_chunks, int64_t* masked_items,
                          int64_t* masked_slots, int64_t* dense_items, int64_t* dense_slots)
{
    F3S_REQUIRE(plan != nullptr, "f3s_plan_stats: NULL plan");
    const f3s_item_set& dense = plan->has_dense ? plan->dense : plan->masked;
    if (num_chunks) *num_chunks = plan->compiled_n >= 0 ? plan->num_chunks : 0;
    if (masked_items) *masked_items = plan->masked.num_items;
    if (masked_slots) *masked_slots = plan->masked.num_slots;
    if (dense_items) *dense_items = dense.num_items;
    if (dense_slots) *dense_slots = dense.num_slots;
    return F3S_OK;
}

f3s_status f3s_attention_fwd_timed(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                   float* O, const int32_t* d_window_offsets,
                                   const int32_t* d_block_col, const uint16_t* d_tile_mask,
                                   const int32_t* d_window_order, int32_t W, int32_t n,
                                   int32_t d, int32_t H, float scale, void* stream,
                                   int32_t reps, float* us_out)
{
    F3S_REQUIRE(reps >= 1 && us_out, "f3s_attention_fwd_timed: reps >= 1 and us_out required");
    F3S_TRY(check_attention_args(Q, K, V, O, n, d, H));
    F3S_TRY(require_device());
    hipStream_t st = as_stream(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    F3S_HIP(hipEventCreate(&e0));
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return hip_fail(hipGetLastError(), "hipEventCreate", __FILE__, __LINE__);
    }
    f3s_status s = F3S_OK;
    hipError_t he = hipEventRecord(e0, st);
    for (int32_t i = 0; he == hipSuccess && s == F3S_OK && i < reps; ++i)
        s = f3s_attention_fwd(Q, K, V, O, d_window_offsets, d_block_col, d_tile_mask,
                              d_window_order, W, n, d, H, scale, stream);
    float ms = 0.f;
    if (he == hipSuccess && s == F3S_OK) he = hipEventRecord(e1, st);
    if (he == hipSuccess && s == F3S_OK) he = hipEventSynchronize(e1);
    if (he == hipSuccess && s == F3S_OK) he = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (s != F3S_OK) return s;
    if (he != hipSuccess) return hip_fail(he, "f3s_attention_fwd_timed", __FILE__, __LINE__);
    *us_out = ms * 1000.0f / (float)reps;
    return F3S_OK;
}

f3s_status f3s_attention_fwd_planned(const f3s_plan* plan, const uint16_t* Q, const uint16_t* K,
                                     const uint16_t* V, float* O, const int32_t* d_block_col,
                                     const uint16_t* d_tile_mask, int32_t n, int32_t d, int32_t H,
                                     float scale, void* stream)
{
    F3S_REQUIRE(plan != nullptr, "f3s_attention_fwd_planned: NULL plan");
    F3S_TRY(check_attention_args(Q, K, V, O, n, d, H));
    F3S_REQUIRE(H == plan->H, "f3s_attention_fwd_planned: H differs from the plan's");
    F3S_REQUIRE(plan->W == (int32_t)ceil_div(n, 16),
                "f3s_attention_fwd_planned: n does not match the plan's W");
    F3S_REQUIRE(plan->T == 0 || d_block_col, "f3s_attention_fwd_planned: NULL block_col");
    F3S_REQUIRE((((uintptr_t)d_tile_mask) & 15) == 0,
                "f3s_attention_fwd_planned: tile_mask alignment");
    F3S_TRY(require_device());
    clear_error();
    AttnParams p{};
    p.Q = reinterpret_cast<const _Float16*>(Q);
    p.K = reinterpret_cast<const _Float16*>(K);
    p.V = reinterpret_cast<const _Float16*>(V);
    p.O = O;
    p.block_col = d_block_col;
    p.tile_mask = d_tile_mask;
    // tile-dense passes run the finer item set when the plan has one
    const f3s_item_set& set = (!d_tile_mask && plan->has_dense) ? plan->dense : plan->masked;
    p.items = reinterpret_cast<const Item*>(set.items.ptr);
    p.num_items = set.num_items;
    p.W = plan->W;
    p.n = n;
    p.xcd_contiguous = plan->xcd_contiguous;
    p.partials = reinterpret_cast<float*>(plan->partials.ptr);
    p.splits = reinterpret_cast<const SplitInfo*>(set.splits.ptr);
    p.slot_split = reinterpret_cast<const int32_t*>(set.slot_split.ptr);
    p.counters = reinterpret_cast<int32_t*>(plan->counters.ptr);
    p.num_split = set.num_split;
    p.team = set.team;
    if (d_tile_mask && d_tile_mask == plan->compiled_tile_mask &&
        d_block_col == plan->compiled_block_col && n == plan->compiled_n) {
        p.chunk_base = reinterpret_cast<const int32_t*>(plan->chunk_base.ptr);
        p.columns = reinterpret_cast<const uint32_t*>(plan->columns.ptr);
    }
    return launch(p, H, scale, as_stream(stream));
}

}  // extern "C"
