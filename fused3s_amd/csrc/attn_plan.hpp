// attn_plan.hpp -- the plan object behind f3s_plan_create / f3s_plan_compile
// (work items, segment partials, compiled column lists).
#pragma once

#include "attn_common.hpp"

// Work items of one segment size: windows with more than `seg` tiles are cut
// into segments whose (m, l, O) partials the last segment of the window to
// finish merges, inside the same launch.
struct f3s_item_set {
    int32_t seg = 0;
    int32_t team = 1;   // > 1: every window is one team of this many items, merged in LDS
    int64_t num_items = 0, num_split = 0, num_slots = 0;
    f3s::DeviceBuffer items, splits, slot_split;   // slot_split: the split of each slot
};

struct f3s_plan {
    int32_t W = 0, H = 1;
    int32_t xcd_contiguous = 1;  // natural-order, unscheduled plans: items map to XCDs in
                                 // contiguous ranges (neighbours share an L2); scheduled
                                 // plans are dealt round-robin, their i*8+x slot
                                 // interleave already lining shares up with the XCDs
    int64_t T = 0;
    // Masked passes (compiled lists or tile expansion) run `masked`.  A
    // tile-dense chunk costs two whole tiles, about 15x a masked chunk per
    // tile on sparse graphs, so automatic plans give tile-dense passes their
    // own item set, `dense`, cut finer; without it (has_dense == false, e.g.
    // an explicit segment size) they share `masked`.
    f3s_item_set masked, dense;
    bool has_dense = false;
    // (m, l, O) partials of split-window segments, sized for the set with the
    // most slots: both sets share it, since a plan serves one pass at a time
    f3s::DeviceBuffer partials;
    // segments arrived per (split window, head), for the in-launch merge;
    // zero between passes (the last segment resets its window's count)
    f3s::DeviceBuffer counters;
    // compiled column lists (f3s_plan_compile) and the structure they describe
    f3s::DeviceBuffer chunk_base, columns;
    const int32_t* compiled_block_col = nullptr;
    const uint16_t* compiled_tile_mask = nullptr;
    int32_t compiled_n = -1;
    int64_t num_chunks = 0;
};
