// l2_model.cpp -- test-side cache model behind tests/test_l2_bound.py (CPU
// only; not part of the library).  Each function replays one XCD's L2 read
// trace -- a sequence of 128-byte line ids, -1 marking a line that is never
// read again (streamed metadata) -- and returns its misses under one policy:
//   first touch   every distinct line once: the misses of an L2 of any size
//                 (the lower bound for this trace's lines, in any order);
//   LRU           set-associative LRU (`sets` x `ways` lines), the policy the
//                 model is checked against by the measured hit rate;
//   OPT           Belady's optimal replacement for `capacity` lines, fully
//                 associative; with `bypass` a missed line is not cached when
//                 its next use lies beyond every cached line's (the optimum
//                 over policies that may also decline to cache a line);
//   pinned        a fixed set of lines resident (`pinned[id]`), every other
//                 read a miss: a policy that keeps the hub rows;
//   selective     LRU over a chosen set of lines, every other read streaming
//                 past the L2 (no allocation): what a load with a streaming
//                 cache policy for the cold rows would give.
#include <stdint.h>

#include <algorithm>
#include <queue>
#include <utility>
#include <vector>

extern "C" {

int64_t l2_first_touch(const int64_t* trace, int64_t len, int64_t id_space)
{
    std::vector<uint8_t> seen((size_t)id_space, 0);
    int64_t misses = 0;
    for (int64_t i = 0; i < len; ++i) {
        const int64_t id = trace[i];
        if (id < 0) {
            ++misses;
        } else if (!seen[(size_t)id]) {
            seen[(size_t)id] = 1;
            ++misses;
        }
    }
    return misses;
}

int64_t l2_lru(const int64_t* trace, int64_t len, int64_t sets, int32_t ways)
{
    // per set: `ways` (line, last-use stamp) entries; a streamed line gets a
    // fresh id so it occupies a way until it ages out
    std::vector<int64_t> line((size_t)(sets * ways), -1), stamp((size_t)(sets * ways), -1);
    int64_t misses = 0, fresh = -2;
    for (int64_t i = 0; i < len; ++i) {
        int64_t id = trace[i];
        if (id < 0) id = fresh--;
        const uint64_t h = (uint64_t)id * 0x9E3779B97F4A7C15ull;
        const int64_t s = (int64_t)((h >> 20) % (uint64_t)sets);
        int64_t* L = line.data() + s * ways;
        int64_t* S = stamp.data() + s * ways;
        int hit = -1, victim = 0;
        for (int k = 0; k < ways; ++k) {
            if (L[k] == id) { hit = k; break; }
            if (S[k] < S[victim]) victim = k;
        }
        if (hit >= 0) {
            S[hit] = i;
        } else {
            ++misses;
            L[victim] = id;
            S[victim] = i;
        }
    }
    return misses;
}

int64_t l2_opt(const int64_t* trace, int64_t len, int64_t id_space, int64_t capacity, int bypass)
{
    const int64_t kNever = INT64_MAX;
    // next use of the line read at each position
    std::vector<int64_t> next((size_t)len), last((size_t)id_space, kNever);
    for (int64_t i = len - 1; i >= 0; --i) {
        const int64_t id = trace[i];
        if (id < 0) {
            next[(size_t)i] = kNever;
        } else {
            next[(size_t)i] = last[(size_t)id];
            last[(size_t)id] = i;
        }
    }
    std::vector<int64_t> cur((size_t)id_space, -1);   // cached line's next use; -1: not cached
    std::priority_queue<std::pair<int64_t, int64_t>> heap;   // (next use, id), lazily updated
    int64_t size = 0, misses = 0;
    for (int64_t i = 0; i < len; ++i) {
        const int64_t id = trace[i];
        const int64_t nu = next[(size_t)i];
        if (id >= 0 && cur[(size_t)id] >= 0) {   // hit
            cur[(size_t)id] = nu;
            heap.push({nu, id});
            continue;
        }
        ++misses;
        if (id < 0 || nu == kNever) continue;    // never read again: caching it gains nothing
        if (size == capacity) {
            // the cached line used furthest in the future (skip stale entries)
            while (!heap.empty()) {
                const auto top = heap.top();
                if (cur[(size_t)top.second] == top.first) break;
                heap.pop();
            }
            if (heap.empty()) continue;
            if (bypass && heap.top().first <= nu) continue;   // the new line is used last
            cur[(size_t)heap.top().second] = -1;
            heap.pop();
            --size;
        }
        cur[(size_t)id] = nu;
        heap.push({nu, id});
        ++size;
    }
    return misses;
}

// LRU over the lines with cacheable[id] set; every other read is a miss that
// allocates nothing (a load that streams past the L2).
int64_t l2_lru_selective(const int64_t* trace, int64_t len, int64_t sets, int32_t ways,
                         const uint8_t* cacheable)
{
    std::vector<int64_t> line((size_t)(sets * ways), -1), stamp((size_t)(sets * ways), -1);
    int64_t misses = 0;
    for (int64_t i = 0; i < len; ++i) {
        const int64_t id = trace[i];
        if (id < 0 || !cacheable[(size_t)id]) {
            ++misses;
            continue;
        }
        const uint64_t h = (uint64_t)id * 0x9E3779B97F4A7C15ull;
        const int64_t s = (int64_t)((h >> 20) % (uint64_t)sets);
        int64_t* L = line.data() + s * ways;
        int64_t* S = stamp.data() + s * ways;
        int hit = -1, victim = 0;
        for (int k = 0; k < ways; ++k) {
            if (L[k] == id) { hit = k; break; }
            if (S[k] < S[victim]) victim = k;
        }
        if (hit >= 0) {
            S[hit] = i;
        } else {
            ++misses;
            L[victim] = id;
            S[victim] = i;
        }
    }
    return misses;
}

int64_t l2_pinned(const int64_t* trace, int64_t len, const uint8_t* pinned, int64_t id_space)
{
    std::vector<uint8_t> seen((size_t)id_space, 0);
    int64_t misses = 0;
    for (int64_t i = 0; i < len; ++i) {
        const int64_t id = trace[i];
        if (id < 0 || !pinned[(size_t)id]) {
            ++misses;
        } else if (!seen[(size_t)id]) {
            seen[(size_t)id] = 1;
            ++misses;
        }
    }
    return misses;
}

}  // extern "C"
