// graph_file.cpp -- binary on-disk form of a graph: the CSR and, optionally,
// its block-sparse form (tile lists and row masks), written and read back
// with a few large sequential transfers.  The reference keeps graphs only as
// whitespace-separated text (include/utils.cuh:26-40), which is parsed one
// integer at a time; at 10^8 edges that parse dominates the host side.
//
// Layout (little-endian, every array starts at a multiple of 64 bytes and the
// gaps are zero):
//   0   char[8] "F3SGRAPH"
//   8   u32     version (1)
//   12  u32     flags: bit 0 = block-sparse section, bit 1 = tile masks
//   16  i64     n          24  i64  nnz
//   32  i64     W          40  i64  T        (both 0 without the section)
//   48  u64     payload checksum             56  u64  header checksum (bytes 0-55)
//   64  row_ptr i32[n+1], col_idx i32[nnz],
//       window_offsets i32[W+1], block_col i32[T], tile_mask u16[16 T]
// The payload checksum is the XOR over the arrays' 8-byte words w_i (i
// counted from the payload start; an array's last word is zero-filled, the
// padding after it is not covered) of mix(w_i + (i + 1) * 0x9E3779B97F4A7C15),
// mix being the splitmix64 finaliser (Steele, Lea, Flood, "Fast splittable
// pseudorandom number generators", OOPSLA 2014): position-dependent, so moved
// words are caught, and an XOR reduction, so it is computed in parallel.  The
// header checksum applies the same to header words 0-6 with i = -7 .. -1.
// Arrays are streamed to and from their own buffers: no second copy of the
// graph is held.
//
// Loading validates everything a consumer relies on: the header, sizes
// against the file length, the checksum, a monotone row_ptr from 0 to nnz,
// columns in [0, n), and for the block-sparse section W = ceil(n/16),
// window_offsets from 0 to T and monotone, and block columns in [0, W) and
// strictly ascending within each window.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <stdexcept>
#include <string>

#include "../../../include/f3s_host.h"

namespace f3s_host {
void set_error(const std::string& s);
}
using f3s_host::set_error;

namespace {

constexpr char kMagic[8] = {'F', '3', 'S', 'G', 'R', 'A', 'P', 'H'};
constexpr uint32_t kVersion = 1;
constexpr uint32_t kFlagBsf = 1u, kFlagMasks = 2u;
constexpr int64_t kHeaderBytes = 64;
constexpr int64_t kAlign = 64;

struct Header {
    char magic[8];
    uint32_t version, flags;
    int64_t n, nnz, W, T;
    uint64_t payload_sum, header_sum;
};
static_assert(sizeof(Header) == kHeaderBytes, "header layout");

uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Checksum of `bytes` bytes at `p` whose first 8-byte word has index `w0`
// in the payload; a partial last word is zero-filled.
uint64_t checksum(const unsigned char* p, int64_t bytes, int64_t w0)
{
    const int64_t words = bytes / 8;
    uint64_t h = 0;
#pragma omp parallel for reduction(^ : h) schedule(static)
    for (int64_t i = 0; i < words; ++i) {
        uint64_t w;
        memcpy(&w, p + 8 * i, 8);
        h ^= mix64(w + (uint64_t)(w0 + i + 1) * 0x9E3779B97F4A7C15ull);
    }
    if (bytes % 8) {
        uint64_t w = 0;
        memcpy(&w, p + 8 * words, (size_t)(bytes % 8));
        h ^= mix64(w + (uint64_t)(w0 + words + 1) * 0x9E3779B97F4A7C15ull);
    }
    return h;
}

int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Section {
    int64_t offset, bytes;   // offset from the payload start
};

struct Layout {
    Section rp, ci, wo, bc, tm;
    int64_t payload;
};

Layout layout_of(int64_t n, int64_t nnz, int64_t W, int64_t T, bool bsf, bool masks)
{
    Layout L{};
    int64_t at = 0;
    auto put = [&](Section& s, int64_t bytes) {
        s.offset = at;
        s.bytes = bytes;
        at = round_up(at + bytes);
    };
    put(L.rp, 4 * (n + 1));
    put(L.ci, 4 * nnz);
    put(L.wo, bsf ? 4 * (W + 1) : 0);
    put(L.bc, bsf ? 4 * T : 0);
    put(L.tm, masks ? 32 * T : 0);
    L.payload = at;
    return L;
}

struct File {
    FILE* f = nullptr;
    ~File()
    {
        if (f) fclose(f);
    }
};

}  // namespace

// The entry points below catch what the C++ library may throw (allocation
// failures in std::string) so that nothing crosses the C ABI.
static int32_t save_impl(const char* path, int32_t n, int64_t nnz, const int32_t* row_ptr,
                         const int32_t* col_idx, int32_t W, int64_t T,
                         const int32_t* window_offsets, const int32_t* block_col,
                         const uint16_t* tile_mask);
static int32_t load_impl(const char* path, int32_t* n_out, int64_t* nnz_out, int32_t** row_ptr,
                         int32_t** col_idx, int32_t* W_out, int64_t* T_out,
                         int32_t** window_offsets, int32_t** block_col, uint16_t** tile_mask);

extern "C" {

int32_t f3s_host_save_graph(const char* path, int32_t n, int64_t nnz, const int32_t* row_ptr,
                            const int32_t* col_idx, int32_t W, int64_t T,
                            const int32_t* window_offsets, const int32_t* block_col,
                            const uint16_t* tile_mask)
{
    try {
        return save_impl(path, n, nnz, row_ptr, col_idx, W, T, window_offsets, block_col,
                         tile_mask);
    } catch (const std::exception& e) {
        set_error(std::string("f3s_host_save_graph: ") + e.what());
        return 1;
    }
}

int32_t f3s_host_load_graph(const char* path, int32_t* n_out, int64_t* nnz_out,
                            int32_t** row_ptr, int32_t** col_idx, int32_t* W_out, int64_t* T_out,
                            int32_t** window_offsets, int32_t** block_col, uint16_t** tile_mask)
{
    try {
        return load_impl(path, n_out, nnz_out, row_ptr, col_idx, W_out, T_out, window_offsets,
                         block_col, tile_mask);
    } catch (const std::exception& e) {
        set_error(std::string("f3s_host_load_graph: ") + e.what());
        return 1;
    }
}

}  // extern "C"

static int32_t save_impl(const char* path, int32_t n, int64_t nnz, const int32_t* row_ptr,
                         const int32_t* col_idx, int32_t W, int64_t T,
                         const int32_t* window_offsets, const int32_t* block_col,
                         const uint16_t* tile_mask)
{
    if (!path || n < 0 || nnz < 0 || !row_ptr || (nnz > 0 && !col_idx)) {
        set_error("f3s_host_save_graph: bad CSR arguments");
        return 1;
    }
    const bool bsf = window_offsets != nullptr;
    const bool masks = bsf && tile_mask != nullptr;
    if (bsf && (W != (n + 15) / 16 || T < 0 || (T > 0 && !block_col))) {
        set_error("f3s_host_save_graph: bad block-sparse arguments (W must be ceil(n/16))");
        return 1;
    }
    if (!bsf && tile_mask) {
        set_error("f3s_host_save_graph: tile_mask requires window_offsets and block_col");
        return 1;
    }
    const Layout L = layout_of(n, nnz, bsf ? W : 0, bsf ? T : 0, bsf, masks);
    const void* src[5] = {row_ptr, col_idx, window_offsets, block_col, tile_mask};
    const Section* sec[5] = {&L.rp, &L.ci, &L.wo, &L.bc, &L.tm};

    Header h{};
    memcpy(h.magic, kMagic, 8);
    h.version = kVersion;
    h.flags = (bsf ? kFlagBsf : 0u) | (masks ? kFlagMasks : 0u);
    h.n = n;
    h.nnz = nnz;
    h.W = bsf ? W : 0;
    h.T = bsf ? T : 0;
    for (int k = 0; k < 5; ++k)
        if (sec[k]->bytes)
            h.payload_sum ^= checksum((const unsigned char*)src[k], sec[k]->bytes,
                                      sec[k]->offset / 8);
    h.header_sum = checksum(reinterpret_cast<const unsigned char*>(&h), 56, -7);

    const std::string tmp = std::string(path) + ".tmp";
    bool ok = false;
    {
        File f;
        f.f = fopen(tmp.c_str(), "wb");
        if (f.f) {
            static const unsigned char zeros[kAlign] = {};
            ok = fwrite(&h, sizeof h, 1, f.f) == 1;
            int64_t at = 0;
            for (int k = 0; ok && k < 5; ++k) {
                if (!sec[k]->bytes) continue;
                ok = fwrite(zeros, 1, (size_t)(sec[k]->offset - at), f.f) ==
                         (size_t)(sec[k]->offset - at) &&
                     fwrite(src[k], (size_t)sec[k]->bytes, 1, f.f) == 1;
                at = sec[k]->offset + sec[k]->bytes;
            }
            ok = ok && fwrite(zeros, 1, (size_t)(L.payload - at), f.f) == (size_t)(L.payload - at);
            ok = (fclose(f.f) == 0) && ok;
            f.f = nullptr;
        }
    }
    if (!ok || rename(tmp.c_str(), path) != 0) {
        remove(tmp.c_str());
        set_error(std::string("f3s_host_save_graph: cannot write ") + path);
        return 1;
    }
    return 0;
}

static int32_t load_impl(const char* path, int32_t* n_out, int64_t* nnz_out,
                         int32_t** row_ptr, int32_t** col_idx, int32_t* W_out, int64_t* T_out,
                         int32_t** window_offsets, int32_t** block_col, uint16_t** tile_mask)
{
    if (!path || !n_out || !nnz_out || !row_ptr || !col_idx || !W_out || !T_out ||
        !window_offsets || !block_col || !tile_mask) {
        set_error("f3s_host_load_graph: NULL argument");
        return 1;
    }
    *row_ptr = *col_idx = *window_offsets = *block_col = nullptr;
    *tile_mask = nullptr;
    const std::string where = std::string("f3s_host_load_graph: ") + path + ": ";
    File f;
    f.f = fopen(path, "rb");
    if (!f.f) {
        set_error(where + "cannot open");
        return 1;
    }
    Header h;
    if (fread(&h, sizeof h, 1, f.f) != 1 || memcmp(h.magic, kMagic, 8) != 0) {
        set_error(where + "not a graph file");
        return 1;
    }
    if (h.version != kVersion) {
        set_error(where + "unsupported version " + std::to_string(h.version));
        return 1;
    }
    if (checksum(reinterpret_cast<const unsigned char*>(&h), 56, -7) != h.header_sum) {
        set_error(where + "header checksum mismatch");
        return 1;
    }
    const bool bsf = h.flags & kFlagBsf, masks = h.flags & kFlagMasks;
    if ((h.flags & ~(kFlagBsf | kFlagMasks)) || (masks && !bsf) || h.n < 0 ||
        h.n > INT32_MAX || h.nnz < 0 || h.nnz > INT32_MAX ||
        (bsf && (h.W != (h.n + 15) / 16 || h.T < 0 || h.T > INT32_MAX)) ||
        (!bsf && (h.W != 0 || h.T != 0))) {
        set_error(where + "inconsistent header");
        return 1;
    }
    const Layout L = layout_of(h.n, h.nnz, h.W, h.T, bsf, masks);
    if (fseek(f.f, 0, SEEK_END) != 0) {
        set_error(where + "cannot seek");
        return 1;
    }
    const long long size = ftell(f.f);
    if (size != kHeaderBytes + L.payload) {
        set_error(where + "file size " + std::to_string(size) + " does not match the header (" +
                  std::to_string(kHeaderBytes + L.payload) + ")");
        return 1;
    }
    // one buffer per array, read in place (these are the returned arrays)
    const Section* sec[5] = {&L.rp, &L.ci, &L.wo, &L.bc, &L.tm};
    void* arr[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    auto release = [&]() {
        for (void*& p : arr) {
            free(p);
            p = nullptr;
        }
    };
    uint64_t sum = 0;
    for (int k = 0; k < 5; ++k) {
        const bool present = k < 2 || (k < 4 && bsf) || (k == 4 && masks);
        if (!present) continue;
        arr[k] = malloc(sec[k]->bytes ? (size_t)sec[k]->bytes : 8);
        if (!arr[k]) {
            release();
            set_error(where + "out of host memory");
            return 1;
        }
        if (!sec[k]->bytes) continue;
        if (fseek(f.f, kHeaderBytes + sec[k]->offset, SEEK_SET) != 0 ||
            fread(arr[k], (size_t)sec[k]->bytes, 1, f.f) != 1) {
            release();
            set_error(where + "short read");
            return 1;
        }
        sum ^= checksum((const unsigned char*)arr[k], sec[k]->bytes, sec[k]->offset / 8);
    }
    if (sum != h.payload_sum) {
        release();
        set_error(where + "payload checksum mismatch");
        return 1;
    }
    const int32_t n = (int32_t)h.n;
    const int64_t nnz = h.nnz, W = h.W, T = h.T;
    const int32_t* rp = (const int32_t*)arr[0];
    const int32_t* ci = (const int32_t*)arr[1];
    std::string bad;
    if (rp[0] != 0 || rp[n] != nnz) bad = "row_ptr must run from 0 to nnz";
    for (int64_t i = 0; bad.empty() && i < n; ++i)
        if (rp[i + 1] < rp[i]) bad = "row_ptr is not monotone";
    for (int64_t e = 0; bad.empty() && e < nnz; ++e)
        if (ci[e] < 0 || ci[e] >= n) bad = "a column index is outside [0, n)";
    if (bsf && bad.empty()) {
        const int32_t* wo = (const int32_t*)arr[2];
        const int32_t* bc = (const int32_t*)arr[3];
        if (wo[0] != 0 || wo[W] != T) bad = "window_offsets must run from 0 to T";
        // The whole offset array first: monotone from 0 to T puts every entry
        // in [0, T], so the block-column walk below stays inside block_col.
        for (int64_t w = 0; bad.empty() && w < W; ++w)
            if (wo[w + 1] < wo[w]) bad = "window_offsets is not monotone";
        for (int64_t w = 0; bad.empty() && w < W; ++w) {
            for (int64_t t = wo[w]; t < wo[w + 1]; ++t)
                if (bc[t] < 0 || bc[t] >= W || (t > wo[w] && bc[t] <= bc[t - 1])) {
                    bad = "block columns must ascend within [0, W) in each window";
                    break;
                }
        }
    }
    if (!bad.empty()) {
        release();
        set_error(where + bad);
        return 1;
    }
    *n_out = n;
    *nnz_out = nnz;
    *row_ptr = (int32_t*)arr[0];
    *col_idx = (int32_t*)arr[1];
    *W_out = bsf ? (int32_t)W : 0;
    *T_out = bsf ? T : 0;
    *window_offsets = (int32_t*)arr[2];
    *block_col = (int32_t*)arr[3];
    *tile_mask = (uint16_t*)arr[4];
    return 0;
}


