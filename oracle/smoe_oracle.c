/* oracle/smoe_oracle.c - CPU restatement of StrataMetal's quantized MoE block.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the timed CPU baseline.  The product
 * (stratametal_amd/libsmoe.so) never links, loads or calls this file's library.
 *
 * Build: oracle/Makefile (gcc -O3 -march=native -ffp-contract=off -fopenmp).  -ffp-contract=off matters:
 * every multiply-add below is either written as fmaf() on purpose or must round twice, exactly as the
 * device kernels do, for the *_dev functions to agree with the device bit for bit.
 *
 * Spec: the bit-level contracts restated from the reference (file:line at each function).
 */
#include "smoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ */
/* A1. fp16 / bf16, as bits.  Restates include/strata/kernels/f16_bits.hpp:37-101 and
 *     include/strata/kernels/bf16_bits.hpp:37-59 (RNE, subnormals with a moving rounding point,
 *     finite overflow -> inf, NaN quieted). */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_f16_from_f32(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e8 = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (e8 == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    const int e = (int)e8 - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        const uint32_t rest = man & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (h & 1u))) h += 1u;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)h;
}

float or_f32_from_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (e == 0) {
        if (man == 0) return u2f(sign);
        int s = 0;
        while (!(man & 0x400u)) { man <<= 1; ++s; }
        return u2f(sign | ((uint32_t)(113 - s) << 23) | ((man & 0x3FFu) << 13));
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((e + 112u) << 23) | (man << 13));
}

uint16_t or_bf16_from_f32(float f) {
    uint32_t i = f2u(f);
    if ((i & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((i >> 16) | 64u);
    i += ((i >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)(i >> 16);
}

float or_f32_from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

void or_f16_from_f32_n(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_f16_from_f32(x[i]);
}
void or_f32_from_f16_n(const uint16_t* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_f32_from_f16(x[i]);
}
void or_bf16_from_f32_n(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_bf16_from_f32(x[i]);
}

/* ------------------------------------------------------------------------------------------------ */
/* Elementary functions.  The device kernels use the same algorithms (Cody-Waite reduction + Taylor
 * polynomial in Horner form with fused multiply-adds), so SiLU, the router softmax and the synthetic
 * generators agree bit for bit between host and device.  Accuracy is checked against libm in tests. */

static const float kLn2Hi = 0.693359375f;         /* 355/512: n * kLn2Hi is exact for |n| <= 2^15 */
static const float kLn2Lo = -2.12194440e-4f;      /* ln 2 - kLn2Hi */
static const float kLog2e = 1.44269504088896341f;

float or_expf(float x) {
    if (x != x) return x;
    if (x > 89.0f) return INFINITY;
    if (x < -87.0f) return 0.0f; /* below FLT_MIN: flushed on both sides */
    const float n = rintf(x * kLog2e);
    float r = fmaf(n, -kLn2Hi, x);
    r = fmaf(n, -kLn2Lo, r);
    /* e^r on |r| <= 0.35: Taylor to degree 7, truncation < 6e-9 relative */
    float p = 1.98412698e-4f;          /* 1/5040 */
    p = fmaf(p, r, 1.38888889e-3f);    /* 1/720 */
    p = fmaf(p, r, 8.33333333e-3f);    /* 1/120 */
    p = fmaf(p, r, 4.16666667e-2f);    /* 1/24 */
    p = fmaf(p, r, 1.66666667e-1f);    /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

float or_logf(float x) {
    /* x > 0, normal.  x = m * 2^e with m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(s), s = (m-1)/(m+1). */
    const uint32_t b = f2u(x);
    int e = (int)((b >> 23) & 0xFFu) - 127;
    float m = u2f((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 9.09090909e-2f;          /* 1/11 */
    p = fmaf(p, s2, 1.11111111e-1f);   /* 1/9 */
    p = fmaf(p, s2, 1.42857143e-1f);   /* 1/7 */
    p = fmaf(p, s2, 2.0e-1f);          /* 1/5 */
    p = fmaf(p, s2, 3.33333333e-1f);   /* 1/3 */
    const float r = fmaf(s * s2, p, s);
    const float lnm = 2.0f * r;
    const float fe = (float)e;
    return fmaf(fe, kLn2Hi, fmaf(fe, kLn2Lo, lnm));
}

float or_cos2pi(float v) {
    float t = v - rintf(v);           /* [-1/2, 1/2], exact */
    float a = fabsf(t);
    float sign = 1.0f;
    if (a > 0.25f) { a = 0.5f - a; sign = -1.0f; }   /* exact (Sterbenz) */
    const int use_sin = a > 0.125f;
    if (use_sin) a = 0.25f - a;                      /* exact */
    const float th = 6.28318531f * a;                /* [0, pi/4] */
    const float z = th * th;
    float r;
    if (use_sin) {
        float p = -2.50521084e-8f;          /* -1/11! */
        p = fmaf(p, z, 2.75573192e-6f);     /* 1/9! */
        p = fmaf(p, z, -1.98412698e-4f);    /* -1/7! */
        p = fmaf(p, z, 8.33333333e-3f);     /* 1/5! */
        p = fmaf(p, z, -1.66666667e-1f);    /* -1/3! */
        r = fmaf(th * z, p, th);
    } else {
        float p = -2.75573192e-7f;          /* -1/10! */
        p = fmaf(p, z, 2.48015873e-5f);     /* 1/8! */
        p = fmaf(p, z, -1.38888889e-3f);    /* -1/6! */
        p = fmaf(p, z, 4.16666667e-2f);     /* 1/4! */
        p = fmaf(p, z, -0.5f);
        r = fmaf(z, p, 1.0f);
    }
    return sign * r;
}

/* ------------------------------------------------------------------------------------------------ */
/* Synthetic inputs: a counter-based SplitMix64 (the SplitMix64 finaliser applied to a Weyl sequence
 * keyed by seed and stream), so host and device fill any slice identically and in parallel. */

uint64_t or_hash(uint64_t seed, uint64_t stream, uint64_t i) {
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull + (i + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float or_uniform(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint32_t top = (uint32_t)(or_hash(seed, stream, i) >> 40);
    return ((float)top + 0.5f) * 5.9604644775390625e-8f; /* 2^-24 */
}

float or_normal(uint64_t seed, uint64_t stream, uint64_t i) {
    const float u1 = or_uniform(seed, stream, 2ull * i);
    const float u2 = or_uniform(seed, stream, 2ull * i + 1ull);
    const float r = sqrtf(-2.0f * or_logf(u1));
    return r * or_cos2pi(u2);
}

void or_gen_normal(uint64_t seed, uint64_t stream, int64_t n, float sigma, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = sigma * or_normal(seed, stream, (uint64_t)i);
}

void or_gen_bf16(uint64_t seed, uint64_t stream, int64_t n, float sigma, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_from_f32(sigma * or_normal(seed, stream, (uint64_t)i));
}

/* Q2_0 block i: d = fp16(|sigma * N|) from stream 2s, the 16 code bytes from two hashes of stream 2s+1. */
void or_gen_q2_0(uint64_t seed, uint64_t stream, int64_t n_blocks, float sigma, uint8_t* out) {
    for (int64_t i = 0; i < n_blocks; ++i) {
        uint8_t* b = out + i * 18;
        const uint16_t d = or_f16_from_f32(fabsf(sigma * or_normal(seed, 2ull * stream, (uint64_t)i)));
        b[0] = (uint8_t)d;
        b[1] = (uint8_t)(d >> 8);
        for (int h = 0; h < 2; ++h) {
            const uint64_t v = or_hash(seed, 2ull * stream + 1ull, 2ull * (uint64_t)i + (uint64_t)h);
            for (int j = 0; j < 8; ++j) b[2 + 8 * h + j] = (uint8_t)(v >> (8 * j));
        }
    }
}

/* IQ2_S block i: d = fp16(|sigma * N|); the other 80 bytes (grid low bytes, signs, high bits, 4-bit
 * sub-scales) are uniform, from ten hashes of stream 2s+1. */
void or_gen_iq2_s(uint64_t seed, uint64_t stream, int64_t n_blocks, float sigma, uint8_t* out) {
    for (int64_t i = 0; i < n_blocks; ++i) {
        uint8_t* b = out + i * 82;
        const uint16_t d = or_f16_from_f32(fabsf(sigma * or_normal(seed, 2ull * stream, (uint64_t)i)));
        b[0] = (uint8_t)d;
        b[1] = (uint8_t)(d >> 8);
        for (int h = 0; h < 10; ++h) {
            const uint64_t v = or_hash(seed, 2ull * stream + 1ull, 10ull * (uint64_t)i + (uint64_t)h);
            for (int j = 0; j < 8; ++j) b[2 + 8 * h + j] = (uint8_t)(v >> (8 * j));
        }
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* A2. Q2_0: 18 bytes = {fp16 d; 16 code bytes}, 64 weights, code (qs[j/4] >> 2(j%4)) & 3, value
 *     (code - 1) * d.  include/strata/artifact/dequant.hpp:69-78. */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void or_dequant_q2_0(const uint8_t* blocks, int64_t n_blocks, float* out) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 18;
        const float d = or_f32_from_f16(rd16(blk));
        for (int j = 0; j < 64; ++j) {
            const int code = (blk[2 + j / 4] >> (2 * (j % 4))) & 3;
            out[b * 64 + j] = (float)(code - 1) * d;
        }
    }
}

int64_t or_row_bytes(int type, int64_t n) {
    if (type == 42) return n % 64 ? -1 : n / 64 * 18;
    if (type == 22) return n % 256 ? -1 : n / 256 * 82;
    return -1;
}

/* ------------------------------------------------------------------------------------------------ */
/* A3. q8_1 block (36 bytes: fp16 d, fp16 s, 32 int8).  metal/shaders/iq.metal:597-627 and its host
 *     restatement metal/src/iq_parity.cpp:350-382: amax and the sum by an xor butterfly 16..1 over the
 *     32 values, d = amax / 127 (an f32 DIVISION), |d| clamped to 65504, q = clamp(round(x / d)) with
 *     half-away rounding, s clamped to +-65504, both stored as fp16 RNE.  A NaN x stores q = 0. */

static void quant_block(const float* x, uint8_t* y) {
    float a[32], s[32];
    for (int i = 0; i < 32; ++i) { a[i] = fabsf(x[i]); s[i] = x[i]; }
    for (int o = 16; o > 0; o >>= 1) {
        float na[32], ns[32];
        for (int i = 0; i < 32; ++i) { na[i] = fmaxf(a[i], a[i ^ o]); ns[i] = s[i] + s[i ^ o]; }
        memcpy(a, na, sizeof a);
        memcpy(s, ns, sizeof s);
    }
    const float amax = a[0];
    const float sum = s[0];
    float d = amax / 127.0f;
    if (fabsf(d) > 65504.0f) d = copysignf(65504.0f, d);
    for (int i = 0; i < 32; ++i) {
        int q = 0;
        if (amax != 0.0f) {
            float r = roundf(x[i] / d);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q = (r == r) ? (int)r : 0;
        }
        y[4 + i] = (uint8_t)(int8_t)q;
    }
    const float sc = fabsf(sum) > 65504.0f ? copysignf(65504.0f, sum) : sum;
    const uint16_t dh = or_f16_from_f32(d), sh = or_f16_from_f32(sc);
    y[0] = (uint8_t)dh;
    y[1] = (uint8_t)(dh >> 8);
    y[2] = (uint8_t)sh;
    y[3] = (uint8_t)(sh >> 8);
}

void or_quant_q8_1(const float* x, int64_t n, uint8_t* y) {
    for (int64_t b = 0; b < n / 32; ++b) quant_block(x + b * 32, y + b * 36);
}

/* ------------------------------------------------------------------------------------------------ */
/* A4. Q2_0 x q8_1.  Per 32-weight half block h of block b (metal/shaders/iq.metal:444-456):
 *       sumi = sum_i (code_i - 1) * q_i               (exact int)
 *       P    = (f32(d_w[b]) * f32(d_x[2b+h])) * (float) sumi   (the first product is exact) */

static inline float q2_partial(const uint8_t* blk, const uint8_t* xblk, int half, int minus_one) {
    const uint8_t* qs = blk + 2 + 8 * half;
    const int8_t* q = (const int8_t*)(xblk + 4);
    int32_t sumi = 0;
    for (int i = 0; i < 32; ++i) {
        const int code = (qs[i >> 2] >> (2 * (i & 3))) & 3;
        sumi += (code - (minus_one ? 1 : 0)) * (int32_t)q[i];
    }
    const float d = or_f32_from_f16(rd16(blk)) * or_f32_from_f16(rd16(xblk));
    return d * (float)sumi;
}

/* Device order (stratametal_amd/csrc/smoe_decode.hip, q2_unit_dot / row_butterfly): a row of n_in values
 * is dpr = n_in / 128 "units" of 36 bytes (blocks 2g, 2g+1; half blocks 4g..4g+3), unit part
 * L_g = ((P_4g + P_4g+1) + P_4g+2) + P_4g+3.  LPR = the largest power of two dividing dpr, at most 16, lanes
 * share a row; lane l adds its units g = l, l + LPR, l + 2 LPR, ... in that order (the first assigned, not
 * added to 0); then an xor butterfly over the LPR lanes (distance LPR/2 first).  Requires n_in % 128 == 0. */
static int lanes_per_row(int dpr) {
    int l = dpr & -dpr;
    return l > 16 ? 16 : l;
}

static float q2_row_dev(const uint8_t* row, const uint8_t* xq, int n_in) {
    const int dpr = n_in / 128;
    const int lpr = lanes_per_row(dpr);
    float lane[16];
    for (int l = 0; l < lpr; ++l) {
        float A = 0.0f;
        for (int g = l, m = 0; g < dpr; g += lpr, ++m) {
            float L = 0.0f;
            for (int h = 0; h < 4; ++h) {
                const int hb = 4 * g + h;
                const float P = q2_partial(row + (size_t)(hb >> 1) * 18, xq + (size_t)hb * 36, hb & 1, 1);
                L = h == 0 ? P : L + P;
            }
            A = m == 0 ? L : A + L;
        }
        lane[l] = A;
    }
    for (int o = lpr / 2; o > 0; o >>= 1) {
        float nxt[16];
        for (int l = 0; l < lpr; ++l) nxt[l] = lane[l] + lane[l ^ o];
        memcpy(lane, nxt, sizeof(float) * (size_t)lpr);
    }
    return lane[0];
}

void or_q2_0_gemv_dev(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    const size_t rb = (size_t)(n_in / 64) * 18;
    for (int r = 0; r < n_out; ++r) y[r] = q2_row_dev(w + (size_t)r * rb, xq, n_in);
}

/* Reference order, metal/src/iq_parity.cpp:275-291 with Q2_0's iq_row<64,2,1,18>: partial k (block
 * k/2, half k%2) is added into lane k%32 (lanes start at 0), then an xor butterfly 16..1; lane 0. */
static float q2_row_ref(const uint8_t* row, const uint8_t* xq, int n_in, int minus_one) {
    float lane[32] = {0};
    const int npart = (n_in / 64) * 2;
    for (int k = 0; k < npart; ++k)
        lane[k & 31] += q2_partial(row + (size_t)(k / 2) * 18, xq + (size_t)(k / 2) * 72 + (size_t)(k % 2) * 36,
                                   k % 2, minus_one);
    for (int o = 16; o > 0; o >>= 1) {
        float nxt[32];
        for (int i = 0; i < 32; ++i) nxt[i] = lane[i] + lane[i ^ o];
        memcpy(lane, nxt, sizeof lane);
    }
    return lane[0];
}

void or_q2_0_gemv_ref(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    const size_t rb = (size_t)(n_in / 64) * 18;
    for (int r = 0; r < n_out; ++r) y[r] = q2_row_ref(w + (size_t)r * rb, xq, n_in, 1);
}

void or_q2_0_gemv_no_minus_one(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    const size_t rb = (size_t)(n_in / 64) * 18;
    for (int r = 0; r < n_out; ++r) y[r] = q2_row_ref(w + (size_t)r * rb, xq, n_in, 0);
}

/* Brute force: dequantize every weight, multiply by q in int64, one double sum per half block scaled
 * by the exact d_w * d_x. */
void or_q2_0_gemv_exact(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, double* y) {
    const size_t rb = (size_t)(n_in / 64) * 18;
    for (int r = 0; r < n_out; ++r) {
        const uint8_t* row = w + (size_t)r * rb;
        double acc = 0.0;
        for (int b = 0; b < n_in / 64; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            for (int h = 0; h < 2; ++h) {
                const uint8_t* xb = xq + (size_t)(2 * b + h) * 36;
                int64_t s = 0;
                for (int i = 0; i < 32; ++i) {
                    const int j = 32 * h + i;
                    const int code = (blk[2 + j / 4] >> (2 * (j % 4))) & 3;
                    s += (int64_t)(code - 1) * (int64_t)(int8_t)xb[4 + i];
                }
                acc += (double)or_f32_from_f16(rd16(blk)) * (double)or_f32_from_f16(rd16(xb)) * (double)s;
            }
        }
        y[r] = acc;
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* A8. IQ2_S (82 bytes / 256 weights: d @0, qs @2, signs @34, qh @66, scales @74).  The integer dot of
 *     metal/shaders/iq.metal:152-180 (host restatement metal/src/iq_parity.cpp:125-151).  The codebook
 *     is ggml's iq2s_grid (metal/include/strata/metal/iq_grids.hpp:5-262); it is stored here as 2 bits
 *     per magnitude (0 -> 8, 1 -> 25, 2 -> 43), byte j of an entry at bits 2j..2j+1. */

static const uint16_t kGridCodes[1024] = {
#include "iq2s_grid_codes.inc"
};

void or_iq2s_grid(uint64_t* grid) {
    static const uint8_t mag[3] = {8, 25, 43};
    for (int i = 0; i < 1024; ++i) {
        uint64_t v = 0;
        for (int j = 0; j < 8; ++j) v |= (uint64_t)mag[(kGridCodes[i] >> (2 * j)) & 3] << (8 * j);
        grid[i] = v;
    }
}

static uint64_t g_grid[1024];
static int g_grid_ready = 0;
static const uint64_t* grid_table(void) {
    if (!g_grid_ready) { or_iq2s_grid(g_grid); g_grid_ready = 1; }
    return g_grid;
}

/* sub block ib of an IQ2_S block against q8_1 block xblk */
static float iq2s_partial(const uint8_t* blk, const uint8_t* xblk, int ib) {
    const uint64_t* grid = grid_table();
    const uint8_t* qs = blk + 2;
    const uint8_t* signs = blk + 34;
    const uint8_t qh = blk[66 + ib];
    const uint8_t sc = blk[74 + ib];
    const int ls0 = sc & 15, ls1 = sc >> 4;
    const int8_t* q = (const int8_t*)(xblk + 4);
    int32_t sum0 = 0, sum1 = 0;
    for (int grp = 0; grp < 4; ++grp) {
        const int idx = qs[4 * ib + grp] | (((qh >> (2 * grp)) & 3) << 8);
        const uint64_t gv = grid[idx];
        const uint8_t sb = signs[4 * ib + grp];
        int32_t s = 0;
        for (int j = 0; j < 8; ++j) {
            int m = (int)((gv >> (8 * j)) & 0xFF);
            if (sb & (1u << j)) m = -m;
            s += m * (int32_t)q[8 * grp + j];
        }
        if (grp < 2) sum0 += s; else sum1 += s;
    }
    const int32_t sumi = (sum0 * ls0 + sum1 * ls1 + (sum0 + sum1) / 2) / 4;
    const float d = or_f32_from_f16(rd16(blk)) * or_f32_from_f16(rd16(xblk));
    return d * (float)sumi;
}

/* Device order (stratametal_amd/csrc/smoe_iq2.hip): nb = n_in / 256 blocks per row, one lane per block
 * (lanes_per_row(nb) lanes, each summing blocks l, l + lpr, ... in order); a block's lane value is
 * ((P_0 + P_1) + ...) + P_7 over its sub-blocks; the row is the xor butterfly over the lanes, distance
 * lpr / 2 first. */
void or_iq2_s_gemv_dev(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    const int nb = n_in / 256;
    const int lpr = lanes_per_row(nb);
    const size_t rb = (size_t)nb * 82;
    for (int r = 0; r < n_out; ++r) {
        const uint8_t* row = w + (size_t)r * rb;
        float lane[16];
        for (int l = 0; l < lpr; ++l) {
            float A = 0.0f;
            for (int b = l, m = 0; b < nb; b += lpr, ++m) {
                float L = 0.0f;
                for (int ib = 0; ib < 8; ++ib) {
                    const float P = iq2s_partial(row + (size_t)b * 82, xq + (size_t)(8 * b + ib) * 36, ib);
                    L = ib == 0 ? P : L + P;
                }
                A = m == 0 ? L : A + L;
            }
            lane[l] = A;
        }
        for (int o = lpr / 2; o > 0; o >>= 1) {
            float nxt[16];
            for (int l = 0; l < lpr; ++l) nxt[l] = lane[l] + lane[l ^ o];
            memcpy(lane, nxt, sizeof(float) * (size_t)lpr);
        }
        y[r] = lane[0];
    }
}

/* Reference order: iq_row<256,8,2,82> (metal/shaders/iq.metal:459-488,498): part k = (block k/8,
 * sub block k%8) into lane k%32, xor butterfly 16..1. */
void or_iq2_s_gemv_ref(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    const int nb = n_in / 256;
    const size_t rb = (size_t)nb * 82;
    for (int r = 0; r < n_out; ++r) {
        const uint8_t* row = w + (size_t)r * rb;
        float lane[32] = {0};
        for (int k = 0; k < nb * 8; ++k)
            lane[k & 31] += iq2s_partial(row + (size_t)(k / 8) * 82, xq + (size_t)k * 36, k % 8);
        for (int o = 16; o > 0; o >>= 1) {
            float nxt[32];
            for (int i = 0; i < 32; ++i) nxt[i] = lane[i] + lane[i ^ o];
            memcpy(lane, nxt, sizeof lane);
        }
        y[r] = lane[0];
    }
}

static void gemv_dev(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    if (or_native_type(type)) or_native_gemv(type, w, xq, n_in, n_out, 1, y);
    else if (type == 22) or_iq2_s_gemv_dev(w, xq, n_in, n_out, y);
    else or_q2_0_gemv_dev(w, xq, n_in, n_out, y);
}
static void gemv_ref(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y) {
    if (or_native_type(type)) or_native_gemv(type, w, xq, n_in, n_out, 1, y);
    else if (type == 22) or_iq2_s_gemv_ref(w, xq, n_in, n_out, y);
    else or_q2_0_gemv_ref(w, xq, n_in, n_out, y);
}

/* ------------------------------------------------------------------------------------------------ */
/* A5. Router.  logits[e] = sum_i f32(bf16 x_i) * f32(W[e][i]); every product is exact in f32.
 *
 * Device order (smoe_router.hip): eight consecutive elements form a chunk; lane l (of 64) owns chunks
 * l, l+64, l+128, ... and adds their products in element order into an accumulator that starts at 0;
 * then an xor butterfly 32,16,8,4,2,1; every lane ends with the same sum. */
void or_bf16_gemv_dev(const uint16_t* xb, const uint16_t* w, int n_in, int n_out, float* y) {
    const int chunks = n_in / 8;
    for (int r = 0; r < n_out; ++r) {
        const uint16_t* row = w + (size_t)r * n_in;
        float lane[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int c = l; c < chunks; c += 64)
                for (int i = 0; i < 8; ++i) {
                    const int k = 8 * c + i;
                    acc = acc + or_f32_from_bf16(xb[k]) * or_f32_from_bf16(row[k]);
                }
            lane[l] = acc;
        }
        for (int o = 32; o > 0; o >>= 1) {
            float nxt[64];
            for (int i = 0; i < 64; ++i) nxt[i] = lane[i] + lane[i ^ o];
            memcpy(lane, nxt, sizeof lane);
        }
        y[r] = lane[0];
    }
}

/* The f32 router of the literal benchmark configuration (router_dtype 1: "Router weight fp32", BASELINE configs[0];
 * no counterpart in the reference, whose router is bf16, include/strata/core/layer.hpp:128-137):
 * logits[e] = sum_i x_i * W[e][i] with x and W in f32.  Device order (k_router<MAXC, true>): four consecutive
 * elements form a chunk; lane l owns chunks l, l+64, ... and fuses each product into its accumulator in element
 * order (fmaf: one rounding per step), then the xor butterfly 32..1. */
void or_f32_gemv_dev(const float* x, const float* w, int n_in, int n_out, float* y) {
    const int chunks = n_in / 4;
    for (int r = 0; r < n_out; ++r) {
        const float* row = w + (size_t)r * n_in;
        float lane[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int c = l; c < chunks; c += 64)
                for (int i = 0; i < 4; ++i) acc = fmaf(x[4 * c + i], row[4 * c + i], acc);
            lane[l] = acc;
        }
        for (int o = 32; o > 0; o >>= 1) {
            float nxt[64];
            for (int i = 0; i < 64; ++i) nxt[i] = lane[i] + lane[i ^ o];
            memcpy(lane, nxt, sizeof lane);
        }
        y[r] = lane[0];
    }
}

/* The f32 router as the reference's host computes its router: a double sum cast to f32. */
void or_f32_gemv_double(const float* x, const float* w, int n_in, int n_out, float* y) {
    for (int r = 0; r < n_out; ++r) {
        double acc = 0.0;
        for (int i = 0; i < n_in; ++i) acc += (double)x[i] * (double)w[(size_t)r * n_in + i];
        y[r] = (float)acc;
    }
}

/* The reference's host router product: a double sum cast to f32 (metal/src/pack_parity.cpp:3795-3799). */
void or_bf16_gemv_double(const uint16_t* xb, const uint16_t* w, int n_in, int n_out, float* y) {
    for (int r = 0; r < n_out; ++r) {
        double acc = 0.0;
        for (int i = 0; i < n_in; ++i)
            acc += (double)or_f32_from_bf16(xb[i]) * (double)or_f32_from_bf16(w[(size_t)r * n_in + i]);
        y[r] = (float)acc;
    }
}

/* Device routing (smoe_router.hip, one wave per token): selection by (logit desc, id asc), a NaN logit
 * ranks as -inf; ex_e = expf(l_e - max); S = lane-sequential sums (lane l owns e = l, l+64, ...) then
 * an xor butterfly 32..1; p_i = ex_i / S; w_i = p_i / max(sum of the k p_i in selection order, 2^-14).
 * metal/shaders/router.metal:30-132 (same selection rule; its sums are double-float, within 1e-5). */
static inline int better(float av, int ai, float bv, int bi) { return av > bv || (av == bv && ai < bi); }

void or_route_dev(const float* logits, int n_tok, int n_expert, int k, int32_t* ids, float* w) {
    float* key = (float*)malloc(sizeof(float) * (size_t)n_expert);
    float* ex = (float*)malloc(sizeof(float) * (size_t)n_expert);
    unsigned char* taken = (unsigned char*)malloc((size_t)n_expert);
    for (int t = 0; t < n_tok; ++t) {
        const float* l = logits + (size_t)t * n_expert;
        float mx = -INFINITY;
        for (int e = 0; e < n_expert; ++e) {
            key[e] = (l[e] != l[e]) ? -INFINITY : l[e];
            mx = fmaxf(mx, key[e]);
            taken[e] = 0;
        }
        float lane[64];
        for (int j = 0; j < 64; ++j) {
            float acc = 0.0f;
            for (int e = j; e < n_expert; e += 64) {
                ex[e] = or_expf(key[e] - mx);
                acc = acc + ex[e];
            }
            lane[j] = acc;
        }
        for (int o = 32; o > 0; o >>= 1) {
            float nxt[64];
            for (int i = 0; i < 64; ++i) nxt[i] = lane[i] + lane[i ^ o];
            memcpy(lane, nxt, sizeof lane);
        }
        const float S = lane[0];
        float ssel = 0.0f;
        float* wt = w + (size_t)t * k;
        int32_t* it = ids + (size_t)t * k;
        for (int i = 0; i < k; ++i) {
            int bi = -1;
            float bv = -INFINITY;
            for (int e = 0; e < n_expert; ++e) {
                if (taken[e]) continue;
                if (bi < 0 || better(key[e], e, bv, bi)) { bv = key[e]; bi = e; }
            }
            taken[bi] = 1;
            it[i] = bi;
            wt[i] = ex[bi] / S;
            ssel = ssel + wt[i];
        }
        const float den = fmaxf(ssel, 6.103515625e-05f);
        for (int i = 0; i < k; ++i) wt[i] = wt[i] / den;
    }
    free(key);
    free(ex);
    free(taken);
}

/* The router-margin diagnostic (metal/src/forward.cpp:441-513): per token, the k-th and (k+1)-th experts ranked
 * by softmax probability (strict greater-than, so a tie keeps the lower id), p_k - p_k1 before renormalisation,
 * and their logit gap.  Device order (k_router_margin): ex and S as or_route_dev forms them, p_e = ex_e / S.
 * stats [T][4] = {p_k - p_k1, l_k - l_k1, p_k, p_k1} (a NaN logit counts as -inf); ids [T][2] = {id_k, id_k1}. */
int or_router_margin_dev(const float* logits, int n_tok, int n_expert, int k, float* stats, int32_t* ids) {
    if (k < 1 || n_expert < k + 1) return -1;
    float* key = (float*)malloc(sizeof(float) * (size_t)n_expert);
    float* p = (float*)malloc(sizeof(float) * (size_t)n_expert);
    char* taken = (char*)malloc((size_t)n_expert);
    for (int t = 0; t < n_tok; ++t) {
        const float* l = logits + (size_t)t * n_expert;
        float mx = -INFINITY;
        for (int e = 0; e < n_expert; ++e) {
            key[e] = (l[e] != l[e]) ? -INFINITY : l[e];
            mx = fmaxf(mx, key[e]);
            taken[e] = 0;
        }
        float lane[64];
        for (int j = 0; j < 64; ++j) {
            float acc = 0.0f;
            for (int e = j; e < n_expert; e += 64) {
                p[e] = or_expf(key[e] - mx);
                acc = acc + p[e];
            }
            lane[j] = acc;
        }
        for (int o = 32; o > 0; o >>= 1) {
            float nxt[64];
            for (int i = 0; i < 64; ++i) nxt[i] = lane[i] + lane[i ^ o];
            memcpy(lane, nxt, sizeof lane);
        }
        for (int e = 0; e < n_expert; ++e) p[e] = p[e] / lane[0];
        int pick[2] = {0, 0};
        for (int i = 0; i <= k; ++i) {
            int bi = -1;
            for (int e = 0; e < n_expert; ++e)
                if (!taken[e] && (bi < 0 || p[e] > p[bi])) bi = e;
            taken[bi] = 1;
            if (i >= k - 1) pick[i - (k - 1)] = bi;
        }
        float* st = stats + (size_t)t * 4;
        st[0] = p[pick[0]] - p[pick[1]];
        st[1] = key[pick[0]] - key[pick[1]];
        st[2] = p[pick[0]];
        st[3] = p[pick[1]];
        ids[(size_t)t * 2] = pick[0];
        ids[(size_t)t * 2 + 1] = pick[1];
    }
    free(key);
    free(p);
    free(taken);
    return 0;
}

/* The reference's host routing, metal/src/router_parity.cpp:48-72 and metal/src/pack_parity.cpp:5144-5166:
 * double softmax over every expert, a stable descending sort (ties keep the lower id), the first k,
 * renormalised by max(sum, 2^-14) in double. */
static const double* g_sort_p;
static int cmp_desc(const void* a, const void* b) {
    const int ia = *(const int*)a, ib = *(const int*)b;
    const double pa = g_sort_p[ia], pb = g_sort_p[ib];
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    return ia - ib; /* stable: lower id first */
}

void or_route_ref(const float* logits, int n_tok, int n_expert, int k, int32_t* ids, float* w) {
    double* p = (double*)malloc(sizeof(double) * (size_t)n_expert);
    int* idx = (int*)malloc(sizeof(int) * (size_t)n_expert);
    for (int t = 0; t < n_tok; ++t) {
        const float* l = logits + (size_t)t * n_expert;
        double mx = l[0];
        for (int e = 1; e < n_expert; ++e) mx = fmax(mx, (double)l[e]);
        double sum = 0.0;
        for (int e = 0; e < n_expert; ++e) { p[e] = exp((double)l[e] - mx); sum += p[e]; }
        for (int e = 0; e < n_expert; ++e) { p[e] /= sum; idx[e] = e; }
        g_sort_p = p;
        qsort(idx, (size_t)n_expert, sizeof(int), cmp_desc);
        double chosen = 0.0;
        for (int i = 0; i < k; ++i) {
            ids[(size_t)t * k + i] = idx[i];
            w[(size_t)t * k + i] = (float)p[idx[i]];
            chosen += p[idx[i]];
        }
        chosen = fmax(chosen, 6.103515625e-05);
        for (int i = 0; i < k; ++i) w[(size_t)t * k + i] = (float)((double)w[(size_t)t * k + i] / chosen);
    }
    free(p);
    free(idx);
}

/* ------------------------------------------------------------------------------------------------ */
/* A6. SwiGLU then q8_1: h = (g / (1 + exp(-g))) * u (metal/shaders/iq.metal:630-663), SiLU on the gate. */
float or_silu_mul(float g, float u) { return (g / (1.0f + or_expf(-g))) * u; }
float or_sigmoid(float z) { return 1.0f / (1.0f + or_expf(-z)); }

void or_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y) {
    float h[32];
    for (int64_t b = 0; b < n / 32; ++b) {
        for (int i = 0; i < 32; ++i) h[i] = or_silu_mul(gate[b * 32 + i], up[b * 32 + i]);
        quant_block(h, y + b * 36);
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* A9. Combine.  Device order = the upstream CUDA contract (include/strata/kernels/native_moe.hpp:10-15):
 * the first product rounds to f32, the others accumulate with fma in selection order, shared added last. */
void or_combine_dev(const float* parts, const float* w, const float* shared, int n_embd, int k, float* y) {
    for (int j = 0; j < n_embd; ++j) {
        float acc = w[0] * parts[j];
        for (int s = 1; s < k; ++s) acc = fmaf(w[s], parts[(size_t)s * n_embd + j], acc);
        if (shared) acc = acc + shared[j];
        y[j] = acc;
    }
}

/* The reference's host combine: a double sum (metal/src/moe_combine_parity.cpp:55-71). */
void or_combine_double(const float* parts, const float* w, const float* shared, int n_embd, int k, float* y) {
    for (int j = 0; j < n_embd; ++j) {
        double a = 0.0;
        for (int s = 0; s < k; ++s) a += (double)w[s] * (double)parts[(size_t)s * n_embd + j];
        if (shared) a += (double)shared[j];
        y[j] = (float)a;
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* The stacked benchmark configuration's layer junction, x_{l+1} = RMSNorm(x_l + MoE_l(x_l)) with unit weight
 * (the configuration's definition; the reference's MoE block has no such call).  Device order
 * (stratametal_amd/csrc/smoe_decode.hip, k_residual_rmsnorm): s_j = x_j + r_j (s_j = x_j when r is NULL);
 * thread i of 256 accumulates fmaf(s_j, s_j, acc) over j = i, i + 256, ... from 0; the 64 threads of each
 * wave combine by the xor butterfly 32..1; the four wave sums add as ((w0 + w1) + w2) + w3;
 * out_j = s_j * (1 / sqrtf(ss / n + eps)), IEEE division and square root. */
void or_residual_rmsnorm_dev(const float* x, const float* r, int n_rows, int n, float eps, float* out) {
    for (int t = 0; t < n_rows; ++t) {
        const float* xr = x + (size_t)t * n;
        const float* rr = r ? r + (size_t)t * n : NULL;
        float th[256];
        for (int i = 0; i < 256; ++i) {
            float acc = 0.0f;
            for (int j = i; j < n; j += 256) {
                const float sj = rr ? xr[j] + rr[j] : xr[j];
                acc = fmaf(sj, sj, acc);
            }
            th[i] = acc;
        }
        float ws[4];
        for (int w = 0; w < 4; ++w) {
            float* lane = th + 64 * w;
            for (int o = 32; o > 0; o >>= 1) {
                float nxt[64];
                for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ o];
                memcpy(lane, nxt, sizeof nxt);
            }
            ws[w] = lane[0];
        }
        const float ss = ((ws[0] + ws[1]) + ws[2]) + ws[3];
        const float inv = 1.0f / sqrtf(ss / (float)n + eps);
        for (int j = 0; j < n; ++j) out[(size_t)t * n + j] = (rr ? xr[j] + rr[j] : xr[j]) * inv;
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* A10. Canonical dispatch: pair i = t*k + s; counts by expert; offsets = exclusive scan in ascending
 * expert; perm = stable counting sort (ascending i within an expert); slot[i] = position of i in perm.
 * The reference leaves the order open (include/strata/prefill/moe_fused.hpp:46-48); this fixes it. */
void or_dispatch(const int32_t* ids, int n_tok, int k, int n_expert, int32_t* counts, int32_t* offsets,
                 int32_t* perm, int32_t* slot) {
    const int n = n_tok * k;
    for (int e = 0; e < n_expert; ++e) counts[e] = 0;
    for (int i = 0; i < n; ++i) counts[ids[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < n_expert; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_expert > 0 ? n_expert : 1));
    for (int e = 0; e < n_expert; ++e) fill[e] = offsets[e];
    for (int i = 0; i < n; ++i) {
        const int p = fill[ids[i]]++;
        perm[p] = i;
        slot[i] = p;
    }
    free(fill);
}

/* ------------------------------------------------------------------------------------------------ */
/* The whole block.  FfnExec::run's MoE interior (metal/src/layer_exec.cpp:470-530), mixed -> combined:
 * bf16 router product, top-k, q8_1 of x, for each selected expert gate/up, SwiGLU + q8_1, down; the
 * shared expert (gate/up/SwiGLU/down, times sigmoid of the bf16 gate_inp_shexp dot); the combine. */

/* the shared expert's projection types (0 in the geometry: sh_type); `native` when any differs from the routed type */
static int sh_gate_t(const or_geom* g) { return g->sh_gate_type ? g->sh_gate_type : g->sh_type; }
static int sh_up_t(const or_geom* g) { return g->sh_up_type ? g->sh_up_type : g->sh_type; }
static int sh_down_t(const or_geom* g) { return g->sh_down_type ? g->sh_down_type : g->sh_type; }
static int sh_native(const or_geom* g) {
    return g->sh_type >= 0 && (sh_gate_t(g) != g->w_type || sh_up_t(g) != g->w_type || sh_down_t(g) != g->w_type);
}
static int64_t any_row_bytes(int type, int64_t n) {
    return or_native_type(type) ? or_native_row_bytes(type, n) : or_row_bytes(type, n);
}

static int geom_ok(const or_geom* g) {
    if (g->n_embd <= 0 || g->n_ff <= 0 || g->n_expert <= 0 || g->top_k <= 0 || g->top_k > g->n_expert) return 0;
    if (g->router_dtype != 0 && g->router_dtype != 1) return 0;
    if (g->router_dtype == 1 && g->n_embd % 4) return 0;
    if (or_row_bytes(g->w_type, g->n_embd) <= 0 || or_row_bytes(g->w_type, g->n_ff) <= 0) return 0;
    if (g->sh_type >= 0 && (any_row_bytes(sh_gate_t(g), g->n_embd) <= 0 || any_row_bytes(sh_up_t(g), g->n_embd) <= 0 ||
                            any_row_bytes(sh_down_t(g), g->n_ff_shared) <= 0 || g->n_ff_shared % 32))
        return 0;
    return 1;
}

/* The shared expert on the q8_1 contract with each projection in its own type: gate, up, SwiGLU + q8_1, down. */
static void shared_chain(const or_geom* g, const or_weights* w, const uint8_t* xq, float* out, int dev) {
    const int H = g->n_embd, F = g->n_ff_shared;
    float* gate = (float*)malloc(sizeof(float) * (size_t)F);
    float* up = (float*)malloc(sizeof(float) * (size_t)F);
    uint8_t* hq = (uint8_t*)malloc((size_t)F / 32 * 36);
    if (dev) {
        gemv_dev(sh_gate_t(g), w->gate_sh, xq, H, F, gate);
        gemv_dev(sh_up_t(g), w->up_sh, xq, H, F, up);
        or_swiglu_q8(gate, up, F, hq);
        gemv_dev(sh_down_t(g), w->down_sh, hq, F, H, out);
    } else {
        gemv_ref(sh_gate_t(g), w->gate_sh, xq, H, F, gate);
        gemv_ref(sh_up_t(g), w->up_sh, xq, H, F, up);
        float h[32];
        for (int b = 0; b < F / 32; ++b) {
            for (int i = 0; i < 32; ++i) {
                const float gv = gate[b * 32 + i];
                h[i] = (gv / (1.0f + expf(-gv))) * up[b * 32 + i];
            }
            quant_block(h, hq + (size_t)b * 36);
        }
        gemv_ref(sh_down_t(g), w->down_sh, hq, F, H, out);
    }
    free(gate);
    free(up);
    free(hq);
}

static void expert_chain(int type, const uint8_t* gw, const uint8_t* uw, const uint8_t* dw, int H, int F,
                         const uint8_t* xq, float* out, uint8_t* hq_out, int dev) {
    float* gate = (float*)malloc(sizeof(float) * (size_t)F);
    float* up = (float*)malloc(sizeof(float) * (size_t)F);
    uint8_t* hq = (uint8_t*)malloc((size_t)F / 32 * 36);
    if (dev) {
        gemv_dev(type, gw, xq, H, F, gate);
        gemv_dev(type, uw, xq, H, F, up);
        or_swiglu_q8(gate, up, F, hq);
        gemv_dev(type, dw, hq, F, H, out);
    } else {
        gemv_ref(type, gw, xq, H, F, gate);
        gemv_ref(type, uw, xq, H, F, up);
        /* metal/src/iq_parity.cpp:384: silu with libm exp */
        float h[32];
        for (int b = 0; b < F / 32; ++b) {
            for (int i = 0; i < 32; ++i) {
                const float g = gate[b * 32 + i];
                h[i] = (g / (1.0f + expf(-g))) * up[b * 32 + i];
            }
            quant_block(h, hq + (size_t)b * 36);
        }
        gemv_ref(type, dw, hq, F, H, out);
    }
    if (hq_out) memcpy(hq_out, hq, (size_t)F / 32 * 36);
    free(gate);
    free(up);
    free(hq);
}

/* One routed expert on a blob [gate rows | up rows | down rows] of `type`, one token's q8_1 row xq. */
int or_expert_dev(int type, const uint8_t* blob, int H, int F, const uint8_t* xq, float* out) {
    if (type != 42 && type != 22) return -1;
    const int64_t gu = or_row_bytes(type, H) * F;
    expert_chain(type, blob, blob + gu, blob + 2 * gu, H, F, xq, out, NULL, 1);
    return 0;
}

/* Router logits of one token: bf16 x and W (router_dtype 0, the repo's contract) or f32 x and W (1). */
static void router_logits(const or_geom* g, const or_weights* w, const float* x, const uint16_t* xb, int dev,
                          float* out) {
    const int H = g->n_embd, E = g->n_expert;
    if (g->router_dtype == 1) {
        const float* W = (const float*)(const void*)w->router;
        if (dev) or_f32_gemv_dev(x, W, H, E, out);
        else or_f32_gemv_double(x, W, H, E, out);
    } else if (dev) {
        or_bf16_gemv_dev(xb, w->router, H, E, out);
    } else {
        or_bf16_gemv_double(xb, w->router, H, E, out);
    }
}

static int moe_decode(const or_geom* g, const or_weights* w, const float* x, int T, float* y, int add_shared,
                      const or_trace* tr, int n_threads, int dev) {
    if (!geom_ok(g) || T < 0) return -1;
    if (T == 0) return 0;
    const int H = g->n_embd, F = g->n_ff, Fs = g->n_ff_shared, E = g->n_expert, K = g->top_k;
    const int64_t xqb = (int64_t)H / 32 * 36, hqb = (int64_t)F / 32 * 36;
    const int64_t grow = or_row_bytes(g->w_type, H), drow = or_row_bytes(g->w_type, F);
    const int64_t ebytes_gu = grow * F, ebytes_d = drow * H;
    const int has_sh = g->sh_type >= 0;

    uint8_t* xq = (uint8_t*)malloc((size_t)(T * xqb));
    uint16_t* xb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    float* wts = (float*)malloc(sizeof(float) * (size_t)T * K);
    float* sg = (float*)calloc((size_t)T, sizeof(float));
    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    float* parts = (float*)malloc(sizeof(float) * (size_t)T * K * H);
    uint8_t* hq = (uint8_t*)malloc((size_t)(T * K * hqb));
    float* shared = (float*)calloc((size_t)T * H, sizeof(float));

    for (int t = 0; t < T; ++t) {
        or_quant_q8_1(x + (size_t)t * H, H, xq + t * xqb);
        or_bf16_from_f32_n(x + (size_t)t * H, H, xb + (size_t)t * H);
    }
    for (int t = 0; t < T; ++t) {
        router_logits(g, w, x + (size_t)t * H, xb + (size_t)t * H, dev, logits + (size_t)t * E);
        if (w->logit_bias)
            for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] = logits[(size_t)t * E + e] + w->logit_bias[e];
        if (has_sh) {
            if (dev) or_bf16_gemv_dev(xb + (size_t)t * H, w->gate_inp_sh, H, 1, sg + t);
            else or_bf16_gemv_double(xb + (size_t)t * H, w->gate_inp_sh, H, 1, sg + t);
        }
    }
    if (dev) or_route_dev(logits, T, E, K, ids, wts);
    else or_route_ref(logits, T, E, K, ids, wts);
    or_dispatch(ids, T, K, E, counts, offsets, perm, slot);

    const int n_jobs = T * K + (has_sh ? T : 0);
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel for schedule(dynamic, 1) if (n_threads > 1)
#endif
    for (int job = 0; job < n_jobs; ++job) {
        if (job < T * K) {
            const int i = job, t = i / K, e = ids[i];
            expert_chain(g->w_type, w->gate_exps + (int64_t)e * ebytes_gu, w->up_exps + (int64_t)e * ebytes_gu,
                         w->down_exps + (int64_t)e * ebytes_d, H, F, xq + t * xqb,
                         parts + (size_t)slot[i] * H, hq + (int64_t)slot[i] * hqb, dev);
        } else {
            const int t = job - T * K;
            float* sh = shared + (size_t)t * H;
            if (sh_native(g)) shared_chain(g, w, xq + t * xqb, sh, dev);
            else expert_chain(g->sh_type, w->gate_sh, w->up_sh, w->down_sh, H, Fs, xq + t * xqb, sh, NULL, dev);
            const float sig = dev ? or_sigmoid(sg[t]) : 1.0f / (1.0f + expf(-sg[t]));
            for (int j = 0; j < H; ++j) sh[j] = sh[j] * sig;
        }
    }
    float* rows = (float*)malloc(sizeof(float) * (size_t)K * H);
    for (int t = 0; t < T; ++t) {
        for (int s = 0; s < K; ++s)
            memcpy(rows + (size_t)s * H, parts + (size_t)slot[t * K + s] * H, sizeof(float) * (size_t)H);
        const float* shp = (has_sh && add_shared) ? shared + (size_t)t * H : NULL;
        if (dev) or_combine_dev(rows, wts + (size_t)t * K, shp, H, K, y + (size_t)t * H);
        else or_combine_double(rows, wts + (size_t)t * K, shp, H, K, y + (size_t)t * H);
    }
    free(rows);

    if (tr) {
        if (tr->logits) memcpy(tr->logits, logits, sizeof(float) * (size_t)T * E);
        if (tr->ids) memcpy(tr->ids, ids, sizeof(int32_t) * (size_t)T * K);
        if (tr->weights) memcpy(tr->weights, wts, sizeof(float) * (size_t)T * K);
        if (tr->counts) memcpy(tr->counts, counts, sizeof(int32_t) * (size_t)E);
        if (tr->offsets) memcpy(tr->offsets, offsets, sizeof(int32_t) * (size_t)(E + 1));
        if (tr->perm) memcpy(tr->perm, perm, sizeof(int32_t) * (size_t)T * K);
        if (tr->slot) memcpy(tr->slot, slot, sizeof(int32_t) * (size_t)T * K);
        if (tr->xq) memcpy(tr->xq, xq, (size_t)(T * xqb));
        if (tr->hq) memcpy(tr->hq, hq, (size_t)(T * K * hqb));
        if (tr->parts) memcpy(tr->parts, parts, sizeof(float) * (size_t)T * K * H);
        if (tr->shared) memcpy(tr->shared, shared, sizeof(float) * (size_t)T * H);
        if (tr->sgate) memcpy(tr->sgate, sg, sizeof(float) * (size_t)T);
    }
    free(xq); free(xb); free(logits); free(ids); free(wts); free(sg); free(counts); free(offsets);
    free(perm); free(slot); free(parts); free(hq); free(shared);
    return 0;
}

int or_moe_decode_dev(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                      const or_trace* tr, int n_threads) {
    return moe_decode(g, w, x, n_tok, y, add_shared, tr, n_threads, 1);
}

int or_moe_decode_ref(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                      int n_threads) {
    return moe_decode(g, w, x, n_tok, y, add_shared, NULL, n_threads, 0);
}

/* ------------------------------------------------------------------------------------------------ */
/* A11 (as built).  Prefill contract: activations rounded to bf16; weights used EXACTLY as
 * (code - 1) * f32(d) -- the bf16 tile holds the symbol (code - 1), and d scales each 64-block's
 * partial sum; SwiGLU in f32 (or_silu_mul), h rounded to bf16 for the down product.  Here every
 * block sum is exact and the row is a double sum of the scaled block sums, cast to f32 once.  The
 * reference's float prompt path is the FP16/BF16-dequant GEMM (include/strata/prefill/gemm.hpp:3-6,
 * include/strata/prefill/kernels.hpp:54-57,97-98).  Routing is A5 per token, as in decode. */

static void q2_rows_bf16act(const uint8_t* w, const float* a /* bf16-valued */, int n_in, int n_out, float* y) {
    const size_t rb = (size_t)(n_in / 64) * 18;
    for (int r = 0; r < n_out; ++r) {
        const uint8_t* row = w + (size_t)r * rb;
        double acc = 0.0;
        for (int b = 0; b < n_in / 64; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            double s = 0.0;
            for (int j = 0; j < 64; ++j) {
                const int code = (blk[2 + j / 4] >> (2 * (j % 4))) & 3;
                s += (double)(code - 1) * (double)a[b * 64 + j];
            }
            acc += (double)or_f32_from_f16(rd16(blk)) * s;
        }
        y[r] = (float)acc;
    }
}

int or_moe_prefill(const or_geom* g, const or_weights* w, const float* x, int T, float* y, int add_shared,
                   const or_trace* tr, int n_threads) {
    return or_moe_prefill_logits(g, w, x, T, NULL, NULL, y, add_shared, tr, n_threads);
}

/* The prefill contract with the router's logits (bias included) and the shared gate dots given: the device's own, for
 * the device path whose router runs on the matrix cores (their f32 sums are in the hardware's order).  The routing of
 * the given logits is the device order's (or_route_dev).  NULL: the oracle's own router (router_logits). */
int or_moe_prefill_logits(const or_geom* g, const or_weights* w, const float* x, int T, const float* logits_in,
                          const float* sg_in, float* y, int add_shared, const or_trace* tr, int n_threads) {
    if (!geom_ok(g) || T < 0) return -1;
    if (g->w_type != 42 || (g->sh_type >= 0 && g->sh_type != 42 && !sh_native(g))) return -2;
    if (T == 0) return 0;
    const int H = g->n_embd, F = g->n_ff, Fs = g->n_ff_shared, E = g->n_expert, K = g->top_k;
    const int64_t grow = or_row_bytes(42, H), drow = or_row_bytes(42, F);
    const int has_sh = g->sh_type >= 0;
    uint16_t* xb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    float* xa = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    float* wts = (float*)malloc(sizeof(float) * (size_t)T * K);
    float* sg = (float*)calloc((size_t)T, sizeof(float));
    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
    float* parts = (float*)malloc(sizeof(float) * (size_t)T * K * H);
    float* shared = (float*)calloc((size_t)T * H, sizeof(float));
    for (int64_t i = 0; i < (int64_t)T * H; ++i) {
        xb[i] = or_bf16_from_f32(x[i]);
        xa[i] = or_f32_from_bf16(xb[i]);
    }
    for (int t = 0; t < T; ++t) {
        if (logits_in) {
            memcpy(logits + (size_t)t * E, logits_in + (size_t)t * E, sizeof(float) * (size_t)E);
            if (has_sh) sg[t] = sg_in ? sg_in[t] : 0.0f;
            continue;
        }
        router_logits(g, w, x + (size_t)t * H, xb + (size_t)t * H, 1, logits + (size_t)t * E);
        if (w->logit_bias)
            for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] = logits[(size_t)t * E + e] + w->logit_bias[e];
        if (has_sh) or_bf16_gemv_dev(xb + (size_t)t * H, w->gate_inp_sh, H, 1, sg + t);
    }
    or_route_dev(logits, T, E, K, ids, wts);
    or_dispatch(ids, T, K, E, counts, offsets, perm, slot);
    const int n_jobs = T * K + (has_sh ? T : 0);
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel for schedule(dynamic, 1) if (n_threads > 1)
#endif
    for (int job = 0; job < n_jobs; ++job) {
        const int is_sh = job >= T * K;
        const int t = is_sh ? job - T * K : job / K;
        const int Fj = is_sh ? Fs : F;
        const uint8_t *gw, *uw, *dw;
        if (is_sh && sh_native(g)) {
            uint8_t* xq = (uint8_t*)malloc((size_t)H / 32 * 36);
            or_quant_q8_1(x + (size_t)t * H, H, xq);
            float* out = shared + (size_t)t * H;
            shared_chain(g, w, xq, out, 1);
            const float sig = or_sigmoid(sg[t]);
            for (int j = 0; j < H; ++j) out[j] = out[j] * sig;
            free(xq);
            continue;
        }
        if (is_sh) {
            gw = w->gate_sh; uw = w->up_sh; dw = w->down_sh;
        } else {
            const int e = ids[job];
            gw = w->gate_exps + (int64_t)e * grow * F;
            uw = w->up_exps + (int64_t)e * grow * F;
            dw = w->down_exps + (int64_t)e * drow * H;
        }
        float* gate = (float*)malloc(sizeof(float) * (size_t)Fj);
        float* up = (float*)malloc(sizeof(float) * (size_t)Fj);
        float* h = (float*)malloc(sizeof(float) * (size_t)Fj);
        q2_rows_bf16act(gw, xa + (size_t)t * H, H, Fj, gate);
        q2_rows_bf16act(uw, xa + (size_t)t * H, H, Fj, up);
        for (int r = 0; r < Fj; ++r) h[r] = or_f32_from_bf16(or_bf16_from_f32(or_silu_mul(gate[r], up[r])));
        float* out = is_sh ? shared + (size_t)t * H : parts + (size_t)slot[job] * H;
        q2_rows_bf16act(dw, h, Fj, H, out);
        if (is_sh) {
            const float sig = or_sigmoid(sg[t]);
            for (int j = 0; j < H; ++j) out[j] = out[j] * sig;
        }
        free(gate); free(up); free(h);
    }
    float* rows = (float*)malloc(sizeof(float) * (size_t)K * H);
    for (int t = 0; t < T; ++t) {
        for (int s = 0; s < K; ++s)
            memcpy(rows + (size_t)s * H, parts + (size_t)slot[t * K + s] * H, sizeof(float) * (size_t)H);
        or_combine_dev(rows, wts + (size_t)t * K, (has_sh && add_shared) ? shared + (size_t)t * H : NULL, H, K,
                       y + (size_t)t * H);
    }
    free(rows);
    if (tr) {
        if (tr->logits) memcpy(tr->logits, logits, sizeof(float) * (size_t)T * E);
        if (tr->ids) memcpy(tr->ids, ids, sizeof(int32_t) * (size_t)T * K);
        if (tr->weights) memcpy(tr->weights, wts, sizeof(float) * (size_t)T * K);
        if (tr->counts) memcpy(tr->counts, counts, sizeof(int32_t) * (size_t)E);
        if (tr->offsets) memcpy(tr->offsets, offsets, sizeof(int32_t) * (size_t)(E + 1));
        if (tr->perm) memcpy(tr->perm, perm, sizeof(int32_t) * (size_t)T * K);
        if (tr->slot) memcpy(tr->slot, slot, sizeof(int32_t) * (size_t)T * K);
        if (tr->parts) memcpy(tr->parts, parts, sizeof(float) * (size_t)T * K * H);
        if (tr->shared) memcpy(tr->shared, shared, sizeof(float) * (size_t)T * H);
        if (tr->sgate) memcpy(tr->sgate, sg, sizeof(float) * (size_t)T);
    }
    free(xb); free(xa); free(logits); free(ids); free(wts); free(sg); free(counts); free(offsets);
    free(perm); free(slot); free(parts); free(shared);
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* The hyper-connection ends of FfnExec::run (metal/src/layer_exec.cpp:469,531): gr_read before the block and
 * gr_write after it (metal/include/strata/metal/gr.hpp:1-48, metal/shaders/gr.metal, metal/src/gr.mm:85-155), one
 * token at a time; R is [hc][n] (stream c at c * n).
 *   xn = R * rs_c * w_norm (rs_c = 1 / sqrt(mean(R_c^2) + eps), the stored (1 + w) weight), act = bf16(xn);
 *   proj_r = act . down_r (r < hc_lr), lo = silu(proj / hc), lq = bf16(lo);
 *   gate_i = lq . up_i (i < hc * n), mixed_d = (sum_c xn_cd * sigmoid(gate_cd)) / hc;
 *   inject_c = act . inj_c;  out_cd = R_cd + y_d * 2 sigmoid(inject_c / hc).
 *
 * Device order (stratametal_amd/csrc/smoe_hc.hip): per stream, thread i of 256 adds fmaf(v, v, acc) over
 * d = i, i + 256, ... from 0, the xor butterfly 32..1 over each wave, the four wave sums ((w0 + w1) + w2) + w3;
 * rs = 1 / sqrtf(ss / n + eps); xn = (R * rs) * w_norm.  The products with down and inj in the router's order
 * (or_bf16_gemv_dev); the products with up with 8 lanes per row: lane l adds the 8-element chunks l, l + 8, ...
 * (fma in element order from 0), then the xor butterfly 4, 2, 1.  silu(z) = z / (1 + exp(-z)) and sigmoid with
 * or_expf; mixed = (((0 + g_0) + g_1) + ...) / hc in stream order. */

static float stream_rs_dev(const float* r, int n, float eps) {
    float th[256];
    for (int i = 0; i < 256; ++i) {
        float acc = 0.0f;
        for (int d = i; d < n; d += 256) acc = fmaf(r[d], r[d], acc);
        th[i] = acc;
    }
    float ws[4];
    for (int w = 0; w < 4; ++w) {
        float* lane = th + 64 * w;
        for (int o = 32; o > 0; o >>= 1) {
            float nxt[64];
            for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ o];
            memcpy(lane, nxt, sizeof nxt);
        }
        ws[w] = lane[0];
    }
    const float ss = ((ws[0] + ws[1]) + ws[2]) + ws[3];
    return 1.0f / sqrtf(ss / (float)n + eps);
}

/* y[r] = x . w_r over n_in bf16 values with `lanes` lanes per row (lanes a power of two, at most 64). */
static void bf16_gemv_lanes(const uint16_t* xb, const uint16_t* w, int n_in, int n_out, int lanes, float* y) {
    const int chunks = n_in / 8;
    for (int r = 0; r < n_out; ++r) {
        const uint16_t* row = w + (size_t)r * n_in;
        float lane[64];
        for (int l = 0; l < lanes; ++l) {
            float acc = 0.0f;
            for (int c = l; c < chunks; c += lanes)
                for (int i = 0; i < 8; ++i) acc = acc + or_f32_from_bf16(xb[8 * c + i]) * or_f32_from_bf16(row[8 * c + i]);
            lane[l] = acc;
        }
        for (int o = lanes / 2; o > 0; o >>= 1) {
            float nxt[64];
            for (int l = 0; l < lanes; ++l) nxt[l] = lane[l] + lane[l ^ o];
            memcpy(lane, nxt, sizeof(float) * (size_t)lanes);
        }
        y[r] = lane[0];
    }
}

int or_hc_read_dev(const float* R, int n_tok, int n, int hc, int hc_lr, float eps, const float* norm,
                   const uint16_t* down, const uint16_t* up, const uint16_t* inj, float* mixed, float* inject) {
    if (n_tok < 0 || n <= 0 || hc <= 0 || hc_lr <= 0 || n % 8 || hc_lr % 8) return -1;
    const int hd = hc * n;
    float* xn = (float*)malloc(sizeof(float) * (size_t)hd);
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hd);
    float* proj = (float*)malloc(sizeof(float) * (size_t)hc_lr);
    uint16_t* lq = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hc_lr);
    float* gate = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int t = 0; t < n_tok; ++t) {
        const float* Rt = R + (size_t)t * hd;
        for (int c = 0; c < hc; ++c) {
            const float rs = stream_rs_dev(Rt + (size_t)c * n, n, eps);
            for (int d = 0; d < n; ++d) {
                const int i = c * n + d;
                xn[i] = (Rt[i] * rs) * norm[i];
                act[i] = or_bf16_from_f32(xn[i]);
            }
        }
        or_bf16_gemv_dev(act, down, hd, hc_lr, proj);
        if (inject) or_bf16_gemv_dev(act, inj, hd, hc, inject + (size_t)t * hc);
        for (int r = 0; r < hc_lr; ++r) {
            const float z = proj[r] / (float)hc;
            lq[r] = or_bf16_from_f32(z / (1.0f + or_expf(-z)));
        }
        bf16_gemv_lanes(lq, up, hc_lr, hd, 8, gate);
        for (int d = 0; d < n; ++d) {
            float m = 0.0f;
            for (int c = 0; c < hc; ++c) m = m + xn[c * n + d] * or_sigmoid(gate[c * n + d]);
            mixed[(size_t)t * n + d] = m / (float)hc;
        }
    }
    free(xn); free(act); free(proj); free(lq); free(gate);
    return 0;
}

/* The reference's host gr_read (metal/src/pack_parity.cpp:7929-7969, metal/src/gr_parity.cpp:95-168): the norm
 * and every product in double, libm exp; `round_act` false keeps xn and lo in f32 (the fp32_act contract). */
int or_hc_read_ref(const float* R, int n_tok, int n, int hc, int hc_lr, float eps, const float* norm,
                   const uint16_t* down, const uint16_t* up, const uint16_t* inj, int round_act, float* mixed,
                   float* inject) {
    if (n_tok < 0 || n <= 0 || hc <= 0 || hc_lr <= 0) return -1;
    const int hd = hc * n;
    float* xn = (float*)malloc(sizeof(float) * (size_t)hd);
    float* act = (float*)malloc(sizeof(float) * (size_t)hd);
    float* lq = (float*)malloc(sizeof(float) * (size_t)hc_lr);
    for (int t = 0; t < n_tok; ++t) {
        const float* Rt = R + (size_t)t * hd;
        for (int c = 0; c < hc; ++c) {
            double ms = 0.0;
            for (int d = 0; d < n; ++d) ms += (double)Rt[c * n + d] * (double)Rt[c * n + d];
            ms /= (double)n;
            const float rs = (float)(1.0 / sqrt(ms + (double)eps));
            for (int d = 0; d < n; ++d) {
                const int i = c * n + d;
                xn[i] = Rt[i] * rs * norm[i];
                act[i] = round_act ? or_f32_from_bf16(or_bf16_from_f32(xn[i])) : xn[i];
            }
        }
        for (int r = 0; r < hc_lr; ++r) {
            double a = 0.0;
            for (int i = 0; i < hd; ++i) a += (double)act[i] * (double)or_f32_from_bf16(down[(size_t)r * hd + i]);
            const float z = (float)a / (float)hc;
            const float lo = z / (1.0f + expf(-z));
            lq[r] = round_act ? or_f32_from_bf16(or_bf16_from_f32(lo)) : lo;
        }
        for (int d = 0; d < n; ++d) {
            float m = 0.0f;
            for (int c = 0; c < hc; ++c) {
                const int i = c * n + d;
                double a = 0.0;
                for (int r = 0; r < hc_lr; ++r) a += (double)lq[r] * (double)or_f32_from_bf16(up[(size_t)i * hc_lr + r]);
                m += xn[i] * (1.0f / (1.0f + expf(-(float)a)));
            }
            mixed[(size_t)t * n + d] = m / (float)hc;
        }
        if (inject)
            for (int c = 0; c < hc; ++c) {
                double a = 0.0;
                for (int i = 0; i < hd; ++i) a += (double)act[i] * (double)or_f32_from_bf16(inj[(size_t)c * hd + i]);
                inject[(size_t)t * hc + c] = (float)a;
            }
    }
    free(xn); free(act); free(lq);
    return 0;
}

/* gr_write (metal/shaders/gr.metal:106-117): out_cd = R_cd + y_d * (2 * s_c), s_c = 1 / (1 + exp(-inject_c / hc)). */
void or_hc_write_dev(const float* R, const float* y, const float* inject, int n_tok, int n, int hc, float* out) {
    for (int t = 0; t < n_tok; ++t)
        for (int c = 0; c < hc; ++c) {
            const float s = or_sigmoid(inject[(size_t)t * hc + c] / (float)hc);
            for (int d = 0; d < n; ++d) {
                const size_t i = ((size_t)t * hc + c) * n + d;
                out[i] = R[i] + y[(size_t)t * n + d] * (2.0f * s);
            }
        }
}
