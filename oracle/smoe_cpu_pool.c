/* oracle/smoe_cpu_pool.c - TEST INFRASTRUCTURE: the timed CPU baseline of bench.py (and nothing else).
 *
 * The decode contract of the MoE block (q8_1 activations, integer Q2_0 / IQ2_S dots, the device's f32 orders),
 * organised as the reference's CPU path organises it: every stage is one flat batch of (expert, row-range) jobs
 * spread over one worker per core, and every weight row is decoded once per call for all of the tokens routed
 * to its expert (include/strata/kernels/cpu/pool.hpp:1-12,85-91; the grouped-expert contract
 * include/strata/kernels/iq_kernels.hpp:53-65: "decode each weight part once for all entries").
 *
 * The results are bitwise those of or_moe_decode_dev (tests/test_oracle.py checks it): the integer sums are exact
 * whatever their order, and every f32 sum is formed in the order or_moe_decode_dev restates.  The product never
 * links or runs this file. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "smoe_oracle.h"

#if defined(__AVX2__) || defined(__F16C__)
#include <immintrin.h>
#endif

/* sum_k a[k] * b[k] over 32 unsigned codes and 32 signed values (exact) */
static inline int32_t dot32_u8s8(const uint8_t* a, const int8_t* b) {
#if defined(__AVX2__)
    const __m256i va = _mm256_loadu_si256((const __m256i*)a), vb = _mm256_loadu_si256((const __m256i*)b);
#if defined(__AVX512VNNI__) && defined(__AVX512VL__)
    const __m256i s = _mm256_dpbusd_epi32(_mm256_setzero_si256(), va, vb);
#else
    /* pairs of u8 * s8 products fit int16 (codes are at most 3) */
    const __m256i s = _mm256_madd_epi16(_mm256_maddubs_epi16(va, vb), _mm256_set1_epi16(1));
#endif
    __m128i h = _mm_add_epi32(_mm256_castsi256_si128(s), _mm256_extracti128_si256(s, 1));
    h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0x4e));
    h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0xb1));
    return _mm_cvtsi128_si32(h);
#else
    int32_t s = 0;
    for (int k = 0; k < 32; ++k) s += (int32_t)a[k] * (int32_t)b[k];
    return s;
#endif
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* fp16 -> f32 (exact): the F16C instruction where the host has it, else the oracle's conversion */
static inline float f16(uint16_t h) {
#if defined(__F16C__)
    return _cvtsh_ss(h);
#else
    return or_f32_from_f16(h);
#endif
}

static int lanes_per_row(int units) {
    int l = units & -units;
    return l > 16 ? 16 : l;
}

/* Per q8_1 block: the f32 of its scale, the int sum of its 32 values, and the values in "plane order", the order in
 * which q2_row_cols unpacks a Q2_0 half block's codes: position 8i + j holds value 4j + i (i < 4, j < 8), so that
 * a half block's code-times-value sum is one contiguous 32-byte dot. */
static void q8_meta(const uint8_t* xq, int n_blocks, float* dx, int32_t* qsum, int8_t* qp) {
    for (int b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = xq + (size_t)b * 36;
        dx[b] = f16(rd16(blk));
        int32_t s = 0;
        for (int k = 0; k < 32; ++k) s += (int8_t)blk[4 + k];
        qsum[b] = s;
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 8; ++j) qp[(size_t)b * 32 + 8 * i + j] = (int8_t)blk[4 + 4 * j + i];
    }
}

/* One Q2_0 row (n_in values) against ncol q8_1 columns: the row's codes are unpacked once (plane order), then per
 * column the half-block sums sum(code * q) - sum(q) (exact), the partials (f32(d_w) * f32(d_x)) * sumi, and the
 * device order's row sum: units of four half blocks ((P0 + P1) + P2) + P3, lanes_per_row lanes adding their units
 * g = l, l + lpr, ... in order, then the xor butterfly (lpr / 2 first).  `codes` holds n_in bytes, `P` n_in / 32. */
static void q2_row_cols(const uint8_t* row, int n_in, const int8_t* const* qp, const float* const* dx,
                        const int32_t* const* qsum, int ncol, float* out, uint8_t* codes, float* P) {
    const int nblk = n_in / 64, nhb = n_in / 32, units = n_in / 128, lpr = lanes_per_row(units);
    float dw[64];
    for (int b = 0; b < nblk; ++b) {
        const uint8_t* blk = row + (size_t)b * 18;
        dw[b] = f16(rd16(blk));
        uint8_t* cb = codes + 64 * b;
        for (int h = 0; h < 2; ++h) {  /* plane i of eight code bytes: (byte >> 2i) & 3, eight at a time */
            uint64_t v;
            memcpy(&v, blk + 2 + 8 * h, 8);
            for (int i = 0; i < 4; ++i) {
                const uint64_t plane = (v >> (2 * i)) & 0x0303030303030303ull;
                memcpy(cb + 32 * h + 8 * i, &plane, 8);
            }
        }
    }
    for (int c = 0; c < ncol; ++c) {
        const int8_t* q = qp[c];
        for (int hb = 0; hb < nhb; ++hb) {
            const int32_t s = dot32_u8s8(codes + 32 * hb, q + 32 * hb) - qsum[c][hb];
            const float d = dw[hb >> 1] * dx[c][hb];
            P[hb] = d * (float)s;
        }
        float lane[16];
        for (int l = 0; l < lpr; ++l) {
            float A = 0.0f;
            for (int g = l, m = 0; g < units; g += lpr, ++m) {
                const float L = ((P[4 * g] + P[4 * g + 1]) + P[4 * g + 2]) + P[4 * g + 3];
                A = m == 0 ? L : A + L;
            }
            lane[l] = A;
        }
        for (int o = lpr / 2; o > 0; o >>= 1) {
            float nxt[16];
            for (int l = 0; l < lpr; ++l) nxt[l] = lane[l] + lane[l ^ o];
            memcpy(lane, nxt, sizeof(float) * (size_t)lpr);
        }
        out[c] = lane[0];
    }
}

/* One row of either type against ncol columns (IQ2_S through the oracle's own row, per column). */
static void row_cols(int type, const uint8_t* row, int n_in, const uint8_t* const* xq, const int8_t* const* qp,
                     const float* const* dx, const int32_t* const* qsum, int ncol, float* out, uint8_t* codes,
                     float* P) {
    if (type == 42) {
        q2_row_cols(row, n_in, qp, dx, qsum, ncol, out, codes, P);
    } else {
        for (int c = 0; c < ncol; ++c) or_iq2_s_gemv_dev(row, xq[c], n_in, 1, out + c);
    }
}

/* A work item: a touched expert with its pairs (dispatch positions first .. first + n), or the shared expert with
 * every token (positions P .. P + T). */
typedef struct {
    int e; /* expert id, -1 = the shared expert */
    int first, n;
} pool_item;

enum { kGuRows = 32, kDownRows = 64, kRouterRows = 16 };

int or_moe_decode_pool(const or_geom* g, const or_weights* w, const float* x, int T, float* y, int add_shared,
                       int n_threads) {
    if (!g || !w || T < 0 || g->n_embd <= 0 || g->n_ff <= 0 || g->n_expert <= 0 || g->top_k <= 0 ||
        g->top_k > g->n_expert)
        return -1;
    if (T == 0) return 0;
    const int H = g->n_embd, F = g->n_ff, E = g->n_expert, K = g->top_k, P = T * K;
    const int has_sh = g->sh_type >= 0;
    const int Fs = has_sh ? g->n_ff_shared : 0;
    const int Fmax = Fs > F ? Fs : F;
    const int64_t grow = or_row_bytes(g->w_type, H), drow = or_row_bytes(g->w_type, F);
    const int64_t sgrow = has_sh ? or_row_bytes(g->sh_type, H) : 0, sdrow = has_sh ? or_row_bytes(g->sh_type, Fs) : 0;
    if (grow <= 0 || drow <= 0 || (has_sh && (sgrow <= 0 || sdrow <= 0))) return -1;
    if (g->router_dtype != 0 && (g->router_dtype != 1 || H % 4)) return -1;
    if ((g->w_type == 42 && (H % 128 || F % 128)) || (has_sh && g->sh_type == 42 && Fs % 128)) return -1;
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
    const int R = P + (has_sh ? T : 0); /* pair rows, then the shared rows */
    const size_t xqb = (size_t)H / 32 * 36, hqb = (size_t)Fmax / 32 * 36;
    uint8_t* xq = (uint8_t*)malloc((size_t)T * xqb);
    uint16_t* xb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    float* xdx = (float*)malloc(sizeof(float) * (size_t)T * (H / 32));
    int32_t* xqs = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * (H / 32));
    int8_t* xqp = (int8_t*)malloc((size_t)T * H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    float* sg = (float*)calloc((size_t)T, sizeof(float));
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)P);
    float* wts = (float*)malloc(sizeof(float) * (size_t)P);
    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)P);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)P);
    float* gate = (float*)malloc(sizeof(float) * (size_t)R * Fmax);
    float* up = (float*)malloc(sizeof(float) * (size_t)R * Fmax);
    uint8_t* hq = (uint8_t*)malloc((size_t)R * hqb);
    float* hdx = (float*)malloc(sizeof(float) * (size_t)R * (Fmax / 32));
    int32_t* hqs = (int32_t*)malloc(sizeof(int32_t) * (size_t)R * (Fmax / 32));
    int8_t* hqp = (int8_t*)malloc((size_t)R * Fmax);
    float* Y = (float*)malloc(sizeof(float) * (size_t)R * H);
    pool_item* items = (pool_item*)malloc(sizeof(pool_item) * (size_t)(E + 1));

    /* stage 0: q8_1 and bf16 of x */
    for (int t = 0; t < T; ++t) {
        or_quant_q8_1(x + (size_t)t * H, H, xq + t * xqb);
        or_bf16_from_f32_n(x + (size_t)t * H, H, xb + (size_t)t * H);
        q8_meta(xq + t * xqb, H / 32, xdx + (size_t)t * (H / 32), xqs + (size_t)t * (H / 32), xqp + (size_t)t * H);
    }
    /* stage 1: router rows (and the shared gate row) in row ranges, every token per range */
    const int n_rjobs = (E + kRouterRows - 1) / kRouterRows + (has_sh ? 1 : 0);
#pragma omp parallel for schedule(dynamic, 1)
    for (int j = 0; j < n_rjobs; ++j) {
        const int r0 = j * kRouterRows;
        if (r0 >= E) {
            for (int t = 0; t < T; ++t) or_bf16_gemv_dev(xb + (size_t)t * H, w->gate_inp_sh, H, 1, sg + t);
            continue;
        }
        const int nr = E - r0 < kRouterRows ? E - r0 : kRouterRows;
        for (int t = 0; t < T; ++t) {
            float* lo = logits + (size_t)t * E + r0;
            if (g->router_dtype == 1)
                or_f32_gemv_dev(x + (size_t)t * H, (const float*)(const void*)w->router + (size_t)r0 * H, H, nr, lo);
            else
                or_bf16_gemv_dev(xb + (size_t)t * H, w->router + (size_t)r0 * H, H, nr, lo);
            if (w->logit_bias)
                for (int r = 0; r < nr; ++r) lo[r] = lo[r] + w->logit_bias[r0 + r];
        }
    }
    /* stage 2: top-k and the dispatch (serial: microseconds) */
    or_route_dev(logits, T, E, K, ids, wts);
    or_dispatch(ids, T, K, E, counts, offsets, perm, slot);
    int n_items = 0;
    if (has_sh) items[n_items++] = (pool_item){-1, P, T};
    for (int e = 0; e < E; ++e)
        if (counts[e] > 0) items[n_items++] = (pool_item){e, offsets[e], counts[e]};

    /* the column pointers of every pair / shared row: the token's x image and its metadata */
    const uint8_t** cx = (const uint8_t**)malloc(sizeof(void*) * (size_t)R);
    const float** cdx = (const float**)malloc(sizeof(void*) * (size_t)R);
    const int32_t** cqs = (const int32_t**)malloc(sizeof(void*) * (size_t)R);
    const int8_t** cqp = (const int8_t**)malloc(sizeof(void*) * (size_t)R);
    for (int pos = 0; pos < R; ++pos) {
        const int t = pos < P ? perm[pos] / K : pos - P;
        cx[pos] = xq + t * xqb;
        cdx[pos] = xdx + (size_t)t * (H / 32);
        cqs[pos] = xqs + (size_t)t * (H / 32);
        cqp[pos] = xqp + (size_t)t * H;
    }
    /* stage 3: gate and up rows, jobs (item, 32-row range) */
    int n_gjobs = 0;
    int* gjob_item = (int*)malloc(sizeof(int) * (size_t)n_items * (Fmax / kGuRows + 1));
    int* gjob_r0 = (int*)malloc(sizeof(int) * (size_t)n_items * (Fmax / kGuRows + 1));
    for (int i = 0; i < n_items; ++i) {
        const int Fi = items[i].e < 0 ? Fs : F;
        for (int r0 = 0; r0 < Fi; r0 += kGuRows) {
            gjob_item[n_gjobs] = i;
            gjob_r0[n_gjobs++] = r0;
        }
    }
#pragma omp parallel
    {
        uint8_t* codes = (uint8_t*)malloc((size_t)(H > Fmax ? H : Fmax));
        float* Pp = (float*)malloc(sizeof(float) * (size_t)((H > Fmax ? H : Fmax) / 32));
        float* col = (float*)malloc(sizeof(float) * (size_t)R);
#pragma omp for schedule(dynamic, 1)
        for (int j = 0; j < n_gjobs; ++j) {
            const pool_item it = items[gjob_item[j]];
            const int sh = it.e < 0, type = sh ? g->sh_type : g->w_type, Fi = sh ? Fs : F;
            const int64_t rb = sh ? sgrow : grow;
            const uint8_t* gbase = sh ? w->gate_sh : w->gate_exps + (int64_t)it.e * Fi * rb;
            const uint8_t* ubase = sh ? w->up_sh : w->up_exps + (int64_t)it.e * Fi * rb;
            const int r1 = gjob_r0[j] + kGuRows < Fi ? gjob_r0[j] + kGuRows : Fi;
            for (int r = gjob_r0[j]; r < r1; ++r) {
                row_cols(type, gbase + (int64_t)r * rb, H, cx + it.first, cqp + it.first, cdx + it.first, cqs + it.first, it.n, col,
                         codes, Pp);
                for (int c = 0; c < it.n; ++c) gate[(size_t)(it.first + c) * Fmax + r] = col[c];
                row_cols(type, ubase + (int64_t)r * rb, H, cx + it.first, cqp + it.first, cdx + it.first, cqs + it.first, it.n, col,
                         codes, Pp);
                for (int c = 0; c < it.n; ++c) up[(size_t)(it.first + c) * Fmax + r] = col[c];
            }
        }
        free(codes);
        free(Pp);
        free(col);
    }
    /* stage 4: SwiGLU and q8_1 of h, per row */
#pragma omp parallel for schedule(static)
    for (int pos = 0; pos < R; ++pos) {
        const int Fi = pos < P ? F : Fs;
        or_swiglu_q8(gate + (size_t)pos * Fmax, up + (size_t)pos * Fmax, Fi, hq + pos * hqb);
        q8_meta(hq + pos * hqb, Fi / 32, hdx + (size_t)pos * (Fmax / 32), hqs + (size_t)pos * (Fmax / 32),
                hqp + (size_t)pos * Fmax);
    }
    for (int pos = 0; pos < R; ++pos) {
        cx[pos] = hq + pos * hqb;
        cdx[pos] = hdx + (size_t)pos * (Fmax / 32);
        cqs[pos] = hqs + (size_t)pos * (Fmax / 32);
        cqp[pos] = hqp + (size_t)pos * Fmax;
    }
    /* stage 5: down rows, jobs (item, 64-row range); the shared rows times sigmoid of the shared gate */
    const int dranges = (H + kDownRows - 1) / kDownRows;
    const int n_djobs = n_items * dranges;
#pragma omp parallel
    {
        uint8_t* codes = (uint8_t*)malloc((size_t)Fmax);
        float* Pp = (float*)malloc(sizeof(float) * (size_t)(Fmax / 32));
        float* col = (float*)malloc(sizeof(float) * (size_t)R);
#pragma omp for schedule(dynamic, 1)
        for (int j = 0; j < n_djobs; ++j) {
            const pool_item it = items[j / dranges];
            const int sh = it.e < 0, type = sh ? g->sh_type : g->w_type, Fi = sh ? Fs : F;
            const int64_t rb = sh ? sdrow : drow;
            const uint8_t* base = sh ? w->down_sh : w->down_exps + (int64_t)it.e * H * rb;
            const int r0 = (j % dranges) * kDownRows, r1 = r0 + kDownRows < H ? r0 + kDownRows : H;
            for (int r = r0; r < r1; ++r) {
                row_cols(type, base + (int64_t)r * rb, Fi, cx + it.first, cqp + it.first, cdx + it.first, cqs + it.first, it.n, col,
                         codes, Pp);
                for (int c = 0; c < it.n; ++c) {
                    float v = col[c];
                    if (sh) v = v * or_sigmoid(sg[c]);
                    Y[(size_t)(it.first + c) * H + r] = v;
                }
            }
        }
        free(codes);
        free(Pp);
        free(col);
    }
    /* stage 6: the combine in selection order, per token */
#pragma omp parallel
    {
        float* rows = (float*)malloc(sizeof(float) * (size_t)K * H);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            for (int s = 0; s < K; ++s)
                memcpy(rows + (size_t)s * H, Y + (size_t)slot[t * K + s] * H, sizeof(float) * (size_t)H);
            const float* shp = (has_sh && add_shared) ? Y + (size_t)(P + t) * H : NULL;
            or_combine_dev(rows, wts + (size_t)t * K, shp, H, K, y + (size_t)t * H);
        }
        free(rows);
    }
    free(xq); free(xb); free(xdx); free(xqs); free(xqp); free(hqp); free(cqp); free(logits); free(sg); free(ids); free(wts); free(counts);
    free(offsets); free(perm); free(slot); free(gate); free(up); free(hq); free(hdx); free(hqs); free(Y);
    free(items); free(cx); free(cdx); free(cqs); free(gjob_item); free(gjob_r0);
    return 0;
}
