/*
 * f3s_oracle.c -- CPU restatement of the fused3S hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path (see the header).
 * Nothing in the product links this file.
 *
 * Built by oracle/Makefile with gcc -O3 -fopenmp (no -ffast-math, no FMA
 * contraction on the default x86-64 target), the flags the reference uses
 * for its host code (CMakeLists.txt:9).
 */
#include "f3s_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

uint16_t orc_f32_to_f16(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ex = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (ex == 0xffu)                              /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    if (ex == 0u)                                 /* f32 zero / subnormal: < 2^-126 */
        return (uint16_t)sign;
    int ue = (int)ex - 127;
    uint32_t sig = man | 0x800000u;               /* 24-bit significand */
    if (ue >= -14) {                              /* normal half (or overflow) */
        if (ue > 15) return (uint16_t)(sign | 0x7c00u);
        uint32_t h = ((uint32_t)(ue + 15) << 10) | ((sig >> 13) & 0x3ffu);
        uint32_t rem = sig & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;   /* carry may reach inf */
        return (uint16_t)(sign | h);
    }
    /* subnormal half: value in units of 2^-24 is sig * 2^(ue+1) */
    int shift = -ue - 1;                          /* >= 14 */
    if (shift > 24) return (uint16_t)sign;
    uint32_t h = sig >> shift;
    uint32_t rem = sig & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (ex == 0x1fu) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (ex == 0u) {
        if (man == 0u) {
            u = sign;
        } else {                                  /* subnormal: man * 2^-24, exact in f32 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&u, &v, 4);
            u |= sign;
        }
    } else {
        u = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_cast_f32_to_f16(const float* in, uint16_t* out, int64_t count)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_cast_f16_to_f32(const uint16_t* in, float* out, int64_t count)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* ---------------------------------------------------------------- loader */

static int read_ints(const char* path, int64_t count, int32_t* dst)
{
    FILE* f = fopen(path, "r");
    if (!f) return -1;
    for (int64_t i = 0; i < count; ++i) {
        long v;
        if (fscanf(f, "%ld", &v) != 1) { fclose(f); return -2; }
        dst[i] = (int32_t)v;
    }
    fclose(f);
    return 0;
}

/* include/utils.cuh:26-40 (meta -> n, nnz; row_ptr n+1; col nnz) */
int orc_load_csr(const char* dir, int32_t* n_out, int64_t* nnz_out,
                 int32_t** row_ptr_out, int32_t** col_out)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/meta.txt", dir);
    FILE* f = fopen(path, "r");
    if (!f) return 1;
    long n = -1, nnz = -1;
    int ok = fscanf(f, "%ld %ld", &n, &nnz);
    fclose(f);
    if (ok != 2 || n < 0 || nnz < 0 || n > 0x7fffffffL) return 1;
    int32_t* rp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n + 1));
    int32_t* ci = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nnz > 0 ? nnz : 1));
    snprintf(path, sizeof path, "%s/row_ptr.txt", dir);
    if (read_ints(path, n + 1, rp) != 0) { free(rp); free(ci); return 2; }
    snprintf(path, sizeof path, "%s/col_idx.txt", dir);
    int rc = read_ints(path, nnz, ci);
    if (rc == -1) {                               /* the name the reference loader opens */
        snprintf(path, sizeof path, "%s/col_ind.txt", dir);
        rc = read_ints(path, nnz, ci);
    }
    if (rc != 0) { free(rp); free(ci); return 3; }
    if (rp[0] != 0 || rp[n] != nnz) { free(rp); free(ci); return 4; }
    for (long i = 0; i < n; ++i)
        if (rp[i + 1] < rp[i]) { free(rp); free(ci); return 4; }
    for (long e = 0; e < nnz; ++e)
        if (ci[e] < 0 || ci[e] >= n) { free(rp); free(ci); return 4; }
    *n_out = (int32_t)n;
    *nnz_out = nnz;
    *row_ptr_out = rp;
    *col_out = ci;
    return 0;
}

void orc_free(void* p) { free(p); }

/* ------------------------------------------------------------- converter */

static int cmp_i32(const void* a, const void* b)
{
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

static int cmp_u64(const void* a, const void* b)
{
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x > y) - (x < y);
}

/* src/converter.cu:15 (W), :19-36 (set of v/16 per window), :39 (offsets) */
int64_t orc_convert_count(int32_t n, const int32_t* row_ptr, const int32_t* col_idx,
                          int32_t* window_offsets)
{
    int32_t W = (int32_t)(((int64_t)n + 15) / 16);
    int32_t* cnt = (int32_t*)malloc(sizeof(int32_t) * (size_t)(W > 0 ? W : 1));
#pragma omp parallel for schedule(dynamic, 64)
    for (int32_t w = 0; w < W; ++w) {
        int32_t u0 = w * 16, u1 = (w * 16 + 16 < n) ? w * 16 + 16 : n;
        int64_t e0 = row_ptr[u0], e1 = row_ptr[u1];
        int64_t E = e1 - e0;
        if (E == 0) { cnt[w] = 0; continue; }
        int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
        for (int64_t e = 0; e < E; ++e) tmp[e] = col_idx[e0 + e] / 16;
        qsort(tmp, (size_t)E, sizeof(int32_t), cmp_i32);
        int32_t u = 1;
        for (int64_t e = 1; e < E; ++e) u += (tmp[e] != tmp[e - 1]);
        cnt[w] = u;
        free(tmp);
    }
    int64_t acc = 0;
    window_offsets[0] = 0;
    for (int32_t w = 0; w < W; ++w) {
        acc += cnt[w];
        window_offsets[w + 1] = (int32_t)acc;
    }
    free(cnt);
    return acc;
}

/* src/converter.cu:34-36 (ascending append); masks: bit c of row r <=> edge */
void orc_convert_fill(int32_t n, const int32_t* row_ptr, const int32_t* col_idx,
                      const int32_t* window_offsets, int32_t* block_col,
                      uint16_t* tile_mask)
{
    int32_t W = (int32_t)(((int64_t)n + 15) / 16);
#pragma omp parallel for schedule(dynamic, 64)
    for (int32_t w = 0; w < W; ++w) {
        int32_t u0 = w * 16, u1 = (w * 16 + 16 < n) ? w * 16 + 16 : n;
        int64_t e0 = row_ptr[u0], e1 = row_ptr[u1];
        int64_t E = e1 - e0;
        if (E == 0) continue;
        uint64_t* key = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)E);
        int64_t k = 0;
        for (int32_t u = u0; u < u1; ++u)
            for (int64_t e = row_ptr[u]; e < row_ptr[u + 1]; ++e) {
                int32_t c = col_idx[e];
                key[k++] = ((uint64_t)(uint32_t)(c / 16) << 8) |
                           ((uint64_t)(u - u0) << 4) | (uint64_t)(c % 16);
            }
        qsort(key, (size_t)E, sizeof(uint64_t), cmp_u64);
        int64_t t = window_offsets[w] - 1;
        uint64_t prev_bc = ~(uint64_t)0;
        for (int64_t i = 0; i < E; ++i) {
            uint64_t bc = key[i] >> 8;
            if (bc != prev_bc) {
                ++t;
                block_col[t] = (int32_t)bc;
                if (tile_mask) memset(tile_mask + 16 * t, 0, 32);
                prev_bc = bc;
            }
            if (tile_mask) {
                int r = (int)((key[i] >> 4) & 15u), c = (int)(key[i] & 15u);
                tile_mask[16 * t + r] |= (uint16_t)(1u << c);
            }
        }
        free(key);
    }
}

/* ----------------------------------------------------------- window order */

/* include/utils.cuh:48-59 with a stable tie rule (merge sort). */
void orc_window_order(const int32_t* window_offsets, int32_t W, int32_t* order)
{
    if (W <= 0) return;
    int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)W);
    for (int32_t i = 0; i < W; ++i) order[i] = i;
    for (int32_t width = 1; width < W; width *= 2) {
        for (int32_t lo = 0; lo < W; lo += 2 * width) {
            int32_t mid = lo + width < W ? lo + width : W;
            int32_t hi = lo + 2 * width < W ? lo + 2 * width : W;
            int32_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) {
                int32_t wa = order[a], wb = order[b];
                int32_t ca = window_offsets[wa + 1] - window_offsets[wa];
                int32_t cb = window_offsets[wb + 1] - window_offsets[wb];
                tmp[o++] = (cb > ca) ? order[b++] : order[a++];   /* take b only if strictly heavier */
            }
            while (a < mid) tmp[o++] = order[a++];
            while (b < hi) tmp[o++] = order[b++];
        }
        memcpy(order, tmp, sizeof(int32_t) * (size_t)W);
    }
    free(tmp);
}

/* ------------------------------------------------------------ attention */

/* baselines/cpu_baseline.cpp:16-91: per node, dots over neighbours (:38-50),
 * max from -1e9 (:56-59), exp and sum (:62-66), normalise (:69-71), weighted
 * V sum in neighbour order (:78-90); degree 0 -> zero row (:26-32). */
void orc_masked_attention(int32_t n, int32_t d, int32_t H,
                          const float* Q, const float* K, const float* V,
                          const int32_t* row_ptr, const int32_t* col_idx,
                          float scale, int32_t r0, int32_t r1, float* O,
                          int32_t threads)
{
    (void)n;
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        int32_t cap = 0;
        float* sc = NULL;
#pragma omp for schedule(dynamic, 256)
        for (int32_t i = r0; i < r1; ++i) {
            int32_t s = row_ptr[i], e = row_ptr[i + 1], deg = e - s;
            if (deg > cap) { free(sc); cap = deg; sc = (float*)malloc(sizeof(float) * (size_t)cap); }
            for (int32_t h = 0; h < H; ++h) {
                float* o = O + ((int64_t)i * H + h) * d;
                const float* q = Q + ((int64_t)i * H + h) * d;
                if (deg == 0) { for (int32_t f = 0; f < d; ++f) o[f] = 0.0f; continue; }
                for (int32_t x = 0; x < deg; ++x) {
                    const float* k = K + ((int64_t)col_idx[s + x] * H + h) * d;
                    float dot = 0.0f;
                    for (int32_t f = 0; f < d; ++f) dot += q[f] * k[f];
                    sc[x] = dot * scale;
                }
                float mx = -1e9f;
                for (int32_t x = 0; x < deg; ++x) mx = sc[x] > mx ? sc[x] : mx;
                float sum = 0.0f;
                for (int32_t x = 0; x < deg; ++x) { sc[x] = expf(sc[x] - mx); sum += sc[x]; }
                for (int32_t x = 0; x < deg; ++x) sc[x] /= sum;
                for (int32_t f = 0; f < d; ++f) o[f] = 0.0f;
                for (int32_t x = 0; x < deg; ++x) {
                    const float* v = V + ((int64_t)col_idx[s + x] * H + h) * d;
                    float wgt = sc[x];
                    for (int32_t f = 0; f < d; ++f) o[f] += wgt * v[f];
                }
            }
        }
        free(sc);
    }
}

/* tests/test_fused_3s_v2.cu:17-59: per real row, logits over all 16 columns
 * of each active tile of its window (:27-41; column >= n -> -1e9, :36),
 * max from -1e9 (:44-45), exp/sum (:47-48), normalise (:49), then for each
 * feature a sum over in-range columns in tile order (:50-58). */
void orc_tile_dense_attention(int32_t n, int32_t d, int32_t H,
                              const float* Q, const float* K, const float* V,
                              const int32_t* window_offsets, const int32_t* block_col,
                              float scale, int32_t r0, int32_t r1, float* O,
                              int32_t threads)
{
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        int64_t cap = 0;
        float* S = NULL;
        int32_t* gcs = NULL;
#pragma omp for schedule(dynamic, 16)
        for (int32_t row = r0; row < r1; ++row) {
            int32_t w = row / 16;
            int32_t b0 = window_offsets[w], b1 = window_offsets[w + 1];
            int64_t len = (int64_t)(b1 - b0) * 16;
            if (len > cap) {
                free(S); free(gcs);
                cap = len;
                S = (float*)malloc(sizeof(float) * (size_t)cap);
                gcs = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
            }
            for (int32_t h = 0; h < H; ++h) {
                float* o = O + ((int64_t)row * H + h) * d;
                if (len == 0) continue;           /* empty window: O untouched (:42) */
                const float* q = Q + ((int64_t)row * H + h) * d;
                int64_t x = 0;
                for (int32_t b = b0; b < b1; ++b)
                    for (int32_t c = 0; c < 16; ++c) {
                        int32_t gc = block_col[b] * 16 + c;
                        float s = -1e9f;
                        if (gc < n) {
                            const float* k = K + ((int64_t)gc * H + h) * d;
                            float dot = 0.0f;
                            for (int32_t f = 0; f < d; ++f) dot += q[f] * k[f];
                            s = dot * scale;
                        }
                        S[x] = s;
                        gcs[x] = gc;
                        ++x;
                    }
                float mx = -1e9f;
                for (int64_t i = 0; i < len; ++i) mx = S[i] > mx ? S[i] : mx;
                float sum = 0.0f;
                for (int64_t i = 0; i < len; ++i) { S[i] = expf(S[i] - mx); sum += S[i]; }
                for (int64_t i = 0; i < len; ++i) S[i] /= sum;
                for (int32_t f = 0; f < d; ++f) {
                    float acc = 0.0f;
                    for (int64_t i = 0; i < len; ++i)
                        if (gcs[i] < n) acc += S[i] * V[((int64_t)gcs[i] * H + h) * d + f];
                    o[f] = acc;
                }
            }
        }
        free(S);
        free(gcs);
    }
}

/* The same TILE_DENSE truth, one window at a time with its 16 rows as SIMD
 * lanes (a window's rows attend the same columns).  Every lane performs the
 * scalar restatement's operations in the scalar restatement's order -- each
 * dot product over f = 0..63 (multiply, then add: no contraction), the max
 * from -1e9 in column order (MAXPS(a, b) is a > b ? a : b, the scalar
 * form's comparison), expf per element, the sum in column order, the
 * division, and per feature the weighted sum in column order -- so the
 * result is bit-identical to orc_tile_dense_attention (tests/test_oracle.py
 * checks it); only the arithmetic runs in AVX2 vectors.  Hosts without AVX2,
 * and head sizes other than 64, run the scalar form. */
#pragma GCC push_options
#pragma GCC target("avx2")
#include <immintrin.h>

#define TD_D 64       /* the fast form's head size (the only one the path supports) */
#define TD_COLS 4     /* columns whose dot products run interleaved */
#define TD_BLOCK 64   /* columns per block of the weighted V sum */

static const float td_zero_row[TD_D] __attribute__((aligned(32)));

static void td_window(int32_t n, int32_t H, const float* Q, const float* K, const float* V,
                      int32_t b0, int32_t b1, const int32_t* block_col, float scale, int32_t lo,
                      int32_t hi, int32_t h, float* O, __m256* S, int32_t* gcs, __m256* qT,
                      __m256* acc)
{
    const int32_t row0 = lo & ~15;
    const int64_t len = (int64_t)(b1 - b0) * 16;
    /* qT[2f], qT[2f+1] = {Q[row0 + r][h][f] : r = 0..15} (rows outside [lo, hi) zero) */
    for (int32_t f = 0; f < TD_D; ++f) {
        float t[16];
        for (int r = 0; r < 16; ++r) {
            const int32_t row = row0 + r;
            t[r] = (row >= lo && row < hi) ? Q[((int64_t)row * H + h) * TD_D + f] : 0.0f;
        }
        qT[2 * f] = _mm256_loadu_ps(t);
        qT[2 * f + 1] = _mm256_loadu_ps(t + 8);
    }
    for (int64_t x = 0; x < len; ++x) gcs[x] = block_col[b0 + x / 16] * 16 + (int32_t)(x % 16);
    /* logits, TD_COLS columns at a time (independent dot products) */
    const __m256 vscale = _mm256_set1_ps(scale), vlow = _mm256_set1_ps(-1e9f);
    for (int64_t x = 0; x < len; x += TD_COLS) {
        const float* kp[TD_COLS];
        __m256 a0[TD_COLS], a1[TD_COLS];
        for (int j = 0; j < TD_COLS; ++j) {
            const int32_t gc = gcs[x + j];
            kp[j] = gc < n ? K + ((int64_t)gc * H + h) * TD_D : td_zero_row;
            a0[j] = _mm256_setzero_ps();
            a1[j] = _mm256_setzero_ps();
        }
        for (int32_t f = 0; f < TD_D; ++f) {
            const __m256 q0 = qT[2 * f], q1 = qT[2 * f + 1];
            for (int j = 0; j < TD_COLS; ++j) {
                const __m256 kb = _mm256_broadcast_ss(kp[j] + f);
                a0[j] = _mm256_add_ps(a0[j], _mm256_mul_ps(q0, kb));
                a1[j] = _mm256_add_ps(a1[j], _mm256_mul_ps(q1, kb));
            }
        }
        for (int j = 0; j < TD_COLS; ++j) {
            const int valid = gcs[x + j] < n;
            S[2 * (x + j)] = valid ? _mm256_mul_ps(a0[j], vscale) : vlow;
            S[2 * (x + j) + 1] = valid ? _mm256_mul_ps(a1[j], vscale) : vlow;
        }
    }
    __m256 mx0 = vlow, mx1 = vlow;
    for (int64_t x = 0; x < len; ++x) {
        mx0 = _mm256_max_ps(S[2 * x], mx0);
        mx1 = _mm256_max_ps(S[2 * x + 1], mx1);
    }
    float mx[16];
    _mm256_storeu_ps(mx, mx0);
    _mm256_storeu_ps(mx + 8, mx1);
    __m256 sum0 = _mm256_setzero_ps(), sum1 = sum0;
    for (int64_t x = 0; x < len; ++x) {
        float* e = (float*)&S[2 * x];
        for (int r = 0; r < 16; ++r) e[r] = expf(e[r] - mx[r]);
        sum0 = _mm256_add_ps(sum0, S[2 * x]);
        sum1 = _mm256_add_ps(sum1, S[2 * x + 1]);
    }
    for (int64_t x = 0; x < len; ++x) {
        S[2 * x] = _mm256_div_ps(S[2 * x], sum0);
        S[2 * x + 1] = _mm256_div_ps(S[2 * x + 1], sum1);
    }
    /* O[row][f] = sum over columns < n, in column order, of P * V[col][f];
     * acc holds the 16 rows' 64 running sums (8 vectors a row), blocks of
     * TD_BLOCK columns */
    for (int32_t i = 0; i < 16 * 8; ++i) acc[i] = _mm256_setzero_ps();
    for (int64_t x0 = 0; x0 < len; x0 += TD_BLOCK) {
        const int64_t x1 = x0 + TD_BLOCK < len ? x0 + TD_BLOCK : len;
        for (int32_t r = lo - row0; r < hi - row0; ++r) {
            __m256 a[8];
            for (int k = 0; k < 8; ++k) a[k] = acc[8 * r + k];
            for (int64_t x = x0; x < x1; ++x) {
                if (gcs[x] >= n) continue;
                const float* vrow = V + ((int64_t)gcs[x] * H + h) * TD_D;
                const __m256 p = _mm256_broadcast_ss((const float*)&S[2 * x] + r);
                for (int k = 0; k < 8; ++k)
                    a[k] = _mm256_add_ps(a[k], _mm256_mul_ps(p, _mm256_loadu_ps(vrow + 8 * k)));
            }
            for (int k = 0; k < 8; ++k) acc[8 * r + k] = a[k];
        }
    }
    for (int32_t row = lo; row < hi; ++row)
        for (int k = 0; k < 8; ++k)
            _mm256_storeu_ps(O + ((int64_t)row * H + h) * TD_D + 8 * k, acc[8 * (row - row0) + k]);
}

static void td_all(int32_t n, int32_t H, const float* Q, const float* K, const float* V,
                   const int32_t* window_offsets, const int32_t* block_col, float scale,
                   int32_t r0, int32_t r1, float* O, int32_t threads)
{
    const int32_t w0 = r0 / 16, w1 = (r1 - 1) / 16 + 1;
#pragma omp parallel num_threads(threads)
    {
        int64_t cap = 0;
        __m256* S = NULL;
        int32_t* gcs = NULL;
        __m256* qT = (__m256*)aligned_alloc(32, sizeof(__m256) * 2 * TD_D);
        __m256* acc = (__m256*)aligned_alloc(32, sizeof(__m256) * 16 * 8);
#pragma omp for schedule(dynamic, 1)
        for (int32_t w = w0; w < w1; ++w) {
            const int32_t b0 = window_offsets[w], b1 = window_offsets[w + 1];
            const int64_t len = (int64_t)(b1 - b0) * 16;
            if (len == 0) continue;               /* empty window: O untouched (:42) */
            if (len > cap) {
                free(S); free(gcs);
                cap = len;
                S = (__m256*)aligned_alloc(32, sizeof(__m256) * 2 * (size_t)cap);
                gcs = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
            }
            const int32_t lo = w * 16 > r0 ? w * 16 : r0;
            const int32_t hi = w * 16 + 16 < r1 ? w * 16 + 16 : r1;
            for (int32_t h = 0; h < H; ++h)
                td_window(n, H, Q, K, V, b0, b1, block_col, scale, lo, hi, h, O, S, gcs, qT, acc);
        }
        free(S);
        free(gcs);
        free(qT);
        free(acc);
    }
}
#pragma GCC pop_options

void orc_tile_dense_attention_fast(int32_t n, int32_t d, int32_t H,
                                   const float* Q, const float* K, const float* V,
                                   const int32_t* window_offsets, const int32_t* block_col,
                                   float scale, int32_t r0, int32_t r1, float* O,
                                   int32_t threads)
{
    if (d != TD_D || !__builtin_cpu_supports("avx2")) {
        orc_tile_dense_attention(n, d, H, Q, K, V, window_offsets, block_col, scale, r0, r1, O,
                                 threads);
        return;
    }
    if (threads < 1) threads = 1;
    if (r1 > n) r1 = n;
    if (r0 < 0) r0 = 0;
    if (r0 >= r1) return;
    td_all(n, H, Q, K, V, window_offsets, block_col, scale, r0, r1, O, threads);
}

/* ------------------------------------------------------------- occupancy */

void orc_bsf_occupancy(int32_t n, int64_t T, const int32_t* block_col,
                       const uint16_t* tile_mask, int masked,
                       int64_t* occ_sum, int64_t* mask_bits)
{
    int64_t occ = 0, bits = 0;
#pragma omp parallel for reduction(+ : occ, bits) schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        int64_t first = (int64_t)block_col[t] * 16;
        int64_t valid = n - first;
        if (valid > 16) valid = 16;
        if (valid < 0) valid = 0;
        if (masked && tile_mask) {
            uint32_t u = 0;
            for (int r = 0; r < 16; ++r) {
                u |= tile_mask[16 * t + r];
                bits += __builtin_popcount(tile_mask[16 * t + r]);
            }
            occ += __builtin_popcount(u);
        } else {
            occ += valid;
            if (tile_mask)
                for (int r = 0; r < 16; ++r) bits += __builtin_popcount(tile_mask[16 * t + r]);
        }
    }
    *occ_sum = occ;
    *mask_bits = bits;
}
