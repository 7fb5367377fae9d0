/* oracle/smoe_native.c - TEST INFRASTRUCTURE ONLY (the CPU checker; never linked into the product).
 *
 * The other native GGUF types of real layers (the shared expert's projections and the down quants:
 * include/strata/kernels/shared_expert.hpp:54-58): Q8_0 (8), Q4_0 (2), Q5_0 (6), IQ4_NL (20), IQ4_XS (23),
 * Q3_K (11), Q4_K (12), Q5_K (13), Q6_K (14).
 *
 *   - or_native_dequant: the blocks' values, following the reference's own dequantisers
 *     (include/strata/artifact/dequant.hpp:81-280).  Pinned bitwise against them (oracle/_ref, live, and the
 *     committed vectors in tests/golden/native_ref.npz).
 *   - or_native_part: one q8_1 integer partial of a row, the reference's MMVQ contract per type
 *     (metal/shaders/iq.metal:224-442; its host restatements metal/src/pack_parity.cpp:2785-3475).
 *   - or_native_gemv: a row is the sum of its partials k = 0 .. npart - 1 taken by 32 lanes (lane k & 31 adds
 *     them in k order from 0), then the xor butterfly 16, 8, 4, 2, 1 (iq_row / iq_mmvq_body,
 *     metal/shaders/iq.metal:458-513; the host refs' lane[32] loops).  The device kernel
 *     (stratametal_amd/csrc/smoe_native.hip) runs this order, so the two agree bit for bit, and it is also the
 *     reference's own host order.
 *   - or_native_gemv_double: dequantised weights times dequantised q8_1 values, summed in double (the
 *     reference's scalar refs, e.g. q40_scalar, metal/src/pack_parity.cpp:3300-3312): the independent check.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "smoe_oracle.h"

/* values per block, bytes per block, partials per block, iqs step (iq_row<QK, IPB, STEP, BLOCK>) */
typedef struct {
    int qk, bytes, ipb, step;
} native_info;

static int native_info_of(int type, native_info* o) {
    switch (type) {
        case 8: *o = (native_info){32, 34, 1, 1}; return 1;     /* Q8_0 */
        case 2: *o = (native_info){32, 18, 2, 2}; return 1;     /* Q4_0 */
        case 6: *o = (native_info){32, 22, 2, 2}; return 1;     /* Q5_0 */
        case 20: *o = (native_info){32, 18, 2, 2}; return 1;    /* IQ4_NL */
        case 23: *o = (native_info){256, 136, 8, 4}; return 1;  /* IQ4_XS */
        case 11: *o = (native_info){256, 110, 16, 1}; return 1; /* Q3_K */
        case 12: *o = (native_info){256, 144, 16, 2}; return 1; /* Q4_K */
        case 13: *o = (native_info){256, 176, 16, 2}; return 1; /* Q5_K */
        case 14: *o = (native_info){256, 210, 32, 1}; return 1; /* Q6_K */
        default: return 0;
    }
}

int or_native_type(int type) {
    native_info i;
    return native_info_of(type, &i);
}

int64_t or_native_row_bytes(int type, int64_t n) {
    native_info i;
    if (!native_info_of(type, &i) || n <= 0 || n % i.qk) return -1;
    return n / i.qk * i.bytes;
}

static uint32_t u16le(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
static int32_t u32le(const uint8_t* p) {
    return (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}
static float h2f(const uint8_t* p) { return or_f32_from_f16((uint16_t)u16le(p)); }

/* four signed bytes times four signed bytes, added to c */
static int32_t dot4(int32_t a, int32_t b, int32_t c) {
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
}
static int32_t sub4(int32_t a, int32_t b) {
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) r |= (uint32_t)(((a >> (8 * i)) - (b >> (8 * i))) & 0xFF) << (8 * i);
    return (int32_t)r;
}
static const int8_t kNl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
/* the codebook bytes of the low (lo) and high (hi) nibbles of four code bytes */
static void nl_bytes(int32_t codes, int32_t* lo, int32_t* hi) {
    uint32_t a = 0, b = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t c = ((uint32_t)codes >> (8 * i)) & 0xFF;
        a |= (uint32_t)(uint8_t)kNl[c & 15] << (8 * i);
        b |= (uint32_t)(uint8_t)kNl[c >> 4] << (8 * i);
    }
    *lo = (int32_t)a;
    *hi = (int32_t)b;
}
/* the q8_1 block's int8 word w (values 4w .. 4w + 3) and its scale */
static int32_t qw(const uint8_t* b, int w) { return u32le(b + 4 + 4 * w); }

/* Q4_K / Q5_K: the 6-bit scale and min pair of 32-value groups 2 j' and 2 j' + 1, j' = bq8_offset / 2
 * (iq_k_scale_min, metal/shaders/iq.metal:254-262) */
static void k_scale_min(const uint8_t* s, int bq8_offset, int sc[2], int mn[2]) {
    const int j = bq8_offset / 2, jm = j & 1;
    const uint32_t s0 = u16le(s + 2 * (jm + 0)), s2 = u16le(s + 2 * (jm + 2)), s4 = u16le(s + 2 * (jm + 4));
    uint32_t a0, a1;
    if (j >= 2) {
        a0 = ((s4 >> 0) & 0x0F0Fu) | ((s0 & 0xC0C0u) >> 2);
        a1 = ((s4 >> 4) & 0x0F0Fu) | ((s2 & 0xC0C0u) >> 2);
    } else {
        a0 = s0 & 0x3F3Fu;
        a1 = s2 & 0x3F3Fu;
    }
    sc[0] = (int)(a0 & 0xFF);
    sc[1] = (int)((a0 >> 8) & 0xFF);
    mn[0] = (int)(a1 & 0xFF);
    mn[1] = (int)((a1 >> 8) & 0xFF);
}

float or_native_part(int type, const uint8_t* blk, const uint8_t* x0, int iqs) {
    switch (type) {
        case 8: { /* Q8_0: d * sum(q_w q_x) over the block's 32 values */
            int32_t s = 0;
            for (int j = 0; j < 8; ++j) s = dot4(u32le(blk + 2 + 4 * (iqs + j)), qw(x0, iqs + j), s);
            return (h2f(blk) * h2f(x0)) * (float)s;
        }
        case 2:   /* Q4_0: nibble - 8 */
        case 6: { /* Q5_0: (nibble | high bit << 4) - 16 */
            const uint8_t* qs = blk + (type == 2 ? 2 : 6);
            int32_t s = 0, a = 0;
            for (int i = 0; i < 2; ++i) {
                const int32_t v = u32le(qs + 4 * (iqs + i));
                int32_t lo = v & 0x0F0F0F0F, hi = (v >> 4) & 0x0F0F0F0F;
                if (type == 6) {  /* element 4(iqs+i)+b takes bit 4(iqs+i)+b of qh, element +16 bit 16+... */
                    const uint32_t h = (uint32_t)u32le(blk + 2) >> (4 * (iqs + i));
                    for (int b = 0; b < 4; ++b) {
                        lo |= (int32_t)(((h >> b) & 1u) << (8 * b + 4));
                        hi |= (int32_t)(((h >> (16 + b)) & 1u) << (8 * b + 4));
                    }
                }
                const int32_t u0 = qw(x0, iqs + i), u1 = qw(x0, iqs + i + 4);
                s = dot4(lo, u0, s);
                s = dot4(hi, u1, s);
                a = dot4(0x01010101, u0, a);
                a = dot4(0x01010101, u1, a);
            }
            return (h2f(blk) * h2f(x0)) * (float)(s - (type == 2 ? 8 : 16) * a);
        }
        case 20: { /* IQ4_NL: codebook values of the nibbles */
            int32_t s = 0;
            for (int l = 0; l < 2; ++l) {
                int32_t lo, hi;
                nl_bytes(u32le(blk + 2 + 4 * (iqs + l)), &lo, &hi);
                s = dot4(lo, qw(x0, iqs + l), s);
                s = dot4(hi, qw(x0, iqs + l + 4), s);
            }
            return (h2f(blk) * h2f(x0)) * (float)s;
        }
        case 23: { /* IQ4_XS: 32-value group iqs / 4 with its 6-bit scale - 32 */
            const uint8_t* x = x0 + (size_t)(iqs / 4) * 36;
            int32_t s = 0;
            for (int j = 0; j < 4; ++j) {
                int32_t lo, hi;
                nl_bytes(u32le(blk + 8 + 4 * (iqs + j)), &lo, &hi);
                s = dot4(lo, qw(x, j), s);
                s = dot4(hi, qw(x, j + 4), s);
            }
            const int ls = ((blk[4 + iqs / 8] >> (iqs & 4)) & 15) | (int)(((u16le(blk + 2) >> (iqs / 2)) & 3) << 4);
            s *= ls - 32;
            return (h2f(blk) * h2f(x)) * (float)s;
        }
        case 12:   /* Q4_K */
        case 13: { /* Q5_K: d * sum(scale * q * a) - dmin * sum(min * a) over two 32-value groups */
            const int q5 = type == 13;
            const int bq8_offset = 2 * ((iqs / 2) / 4), qoff = (iqs / 2) % 4;
            const uint8_t* ql = blk + (q5 ? 48 : 16);
            const int byte = 16 * bq8_offset + 4 * qoff;
            const int32_t v0 = u32le(ql + byte), v1 = u32le(ql + byte + 16);
            uint32_t vh0 = 0, vh1 = 0;  // (unsigned: the high-bit shifts below are defined)
            if (q5) {
                vh0 = u32le(blk + 16 + 4 * qoff) >> bq8_offset;
                vh1 = u32le(blk + 32 + 4 * qoff) >> bq8_offset;
            }
            int sc[2], mn[2];
            k_scale_min(blk + 4, bq8_offset, sc, mn);
            float sum_d = 0.0f, sum_m = 0.0f;
            for (int i = 0; i < 2; ++i) {
                const uint8_t* b8 = x0 + (size_t)(bq8_offset + i) * 36;
                const float d8 = h2f(b8);
                const int32_t u0 = qw(b8, qoff), u1 = qw(b8, qoff + 4);
                int32_t p0 = (v0 >> (4 * i)) & 0x0F0F0F0F, p1 = (v1 >> (4 * i)) & 0x0F0F0F0F;
                if (q5) {
                    p0 |= ((vh0 >> i) << 4) & 0x10101010;
                    p1 |= ((vh1 >> i) << 4) & 0x10101010;
                }
                const int32_t dq = dot4(p1, u1, dot4(p0, u0, 0));
                const int32_t da = dot4(0x01010101, u1, dot4(0x01010101, u0, 0));
                sum_d = sum_d + d8 * (float)(dq * sc[i]);
                sum_m = sum_m + d8 * (float)(da * mn[i]);
            }
            return h2f(blk) * sum_d - h2f(blk + 2) * sum_m;
        }
        case 11: { /* Q3_K: (2 low bits - 4 when the high bit is clear) * (6-bit scale - 32), four q8_1 blocks */
            const int bq8_offset = 4 * (iqs / 8), scale_offset = iqs - (iqs % 8) + (iqs % 8) / 4;
            const uint8_t* sc8 = blk + 96;
            const int32_t vl = u32le(blk + 32 + 4 * iqs);
            const uint32_t vh = (~(uint32_t)u32le(blk + 4 * (iqs % 8))) >> bq8_offset;
            float sumf = 0.0f;
            for (int i = 0; i < 4; ++i) {
                const int isc = scale_offset + 2 * i;
                const int sc = (((sc8[isc % 8] >> (4 * (isc / 8))) & 15) | (((sc8[8 + (isc % 4)] >> (2 * (isc / 4))) & 3) << 4)) - 32;
                const int32_t v = sub4((vl >> (2 * i)) & 0x03030303, (int32_t)(((vh >> i) << 2) & 0x04040404u));
                const uint8_t* b8 = x0 + (size_t)(bq8_offset + i) * 36;
                sumf = sumf + h2f(b8) * (float)(dot4(v, qw(b8, iqs % 8), 0) * sc);
            }
            return h2f(blk + 108) * sumf;
        }
        case 14: { /* Q6_K: (low nibble | 2 high bits << 4) - 32 times an int8 scale, two q8_1 blocks */
            const int bq8_offset = 4 * (iqs / 16) + (iqs % 16) / 8, scale_offset = 8 * (iqs / 16) + (iqs % 16) / 4;
            const int vh_shift = 2 * ((iqs % 16) / 8);
            const int32_t vl = u32le(blk + 4 * iqs);
            const uint32_t vh = (uint32_t)u32le(blk + 128 + 4 * (8 * (iqs / 16) + (iqs % 8))) >> vh_shift;
            float sumf = 0.0f;
            for (int i = 0; i < 2; ++i) {
                const int sc = (int)(int8_t)blk[192 + scale_offset + 4 * i];
                const int32_t v = sub4(((vl >> (4 * i)) & 0x0F0F0F0F) | (int32_t)(((vh >> (4 * i)) << 4) & 0x30303030u),
                                       0x20202020);
                const uint8_t* b8 = x0 + (size_t)(bq8_offset + 2 * i) * 36;
                sumf = sumf + h2f(b8) * (float)(dot4(v, qw(b8, iqs % 8), 0) * sc);
            }
            return h2f(blk + 208) * sumf;
        }
        default: return NAN;
    }
}

/* y[c * n_out + r] for n_col q8_1 columns: the 32-lane order of the reference's MMVQ rows */
int or_native_gemv(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y) {
    native_info I;
    if (!native_info_of(type, &I) || n_in <= 0 || n_in % I.qk) return -1;
    const int nb = n_in / I.qk, npart = nb * I.ipb;
    const size_t rb = (size_t)nb * I.bytes, xb = (size_t)(n_in / 32) * 36;
    for (int c = 0; c < n_col; ++c) {
        const uint8_t* col = xq + (size_t)c * xb;
        for (int r = 0; r < n_out; ++r) {
            const uint8_t* row = w + (size_t)r * rb;
            float lane[32];
            for (int l = 0; l < 32; ++l) lane[l] = 0.0f;
            for (int k = 0; k < npart; ++k) {
                const int kb = k / I.ipb;
                lane[k & 31] = lane[k & 31] +
                               or_native_part(type, row + (size_t)kb * I.bytes, col + (size_t)kb * (I.qk / 32) * 36,
                                              I.step * (k % I.ipb));
            }
            for (int o = 16; o > 0; o >>= 1) {
                float nxt[32];
                for (int l = 0; l < 32; ++l) nxt[l] = lane[l] + lane[l ^ o];
                memcpy(lane, nxt, sizeof nxt);
            }
            y[(size_t)c * n_out + r] = lane[0];
        }
    }
    return 0;
}

/* ---- the blocks' values (include/strata/artifact/dequant.hpp:81-280) */
static void k_group(int j, const uint8_t* s, int* sc, int* mn) {  /* 6-bit scale and min of 32-value group j */
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void dequant_block(int type, const uint8_t* b, float* o) {
    switch (type) {
        case 8: {
            const float d = h2f(b);
            for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)b[2 + j] * d;
            break;
        }
        case 2:
        case 6: {
            const float d = h2f(b);
            const uint8_t* qs = b + (type == 2 ? 2 : 6);
            const uint32_t h = type == 6 ? (uint32_t)u32le(b + 2) : 0u;
            const int bias = type == 2 ? 8 : 16;
            for (int j = 0; j < 16; ++j) {
                const int a0 = (qs[j] & 15) | (int)(((h >> j) & 1u) << 4);
                const int a1 = (qs[j] >> 4) | (int)(((h >> (j + 16)) & 1u) << 4);
                o[j] = (float)(a0 - bias) * d;
                o[j + 16] = (float)(a1 - bias) * d;
            }
            break;
        }
        case 20: {
            const float d = h2f(b);
            for (int j = 0; j < 16; ++j) {
                o[j] = d * (float)kNl[b[2 + j] & 15];
                o[j + 16] = d * (float)kNl[b[2 + j] >> 4];
            }
            break;
        }
        case 23: {
            const float d = h2f(b);
            const uint32_t sh = u16le(b + 2);
            for (int g = 0; g < 8; ++g) {
                const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 15) | (int)(((sh >> (2 * g)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                const uint8_t* qs = b + 8 + 16 * g;
                for (int j = 0; j < 16; ++j) {
                    o[32 * g + j] = dl * (float)kNl[qs[j] & 15];
                    o[32 * g + 16 + j] = dl * (float)kNl[qs[j] >> 4];
                }
            }
            break;
        }
        case 12:
        case 13: {
            const int q5 = type == 13;
            const float d = h2f(b), dm = h2f(b + 2);
            const uint8_t* ql = b + (q5 ? 48 : 16);
            for (int g = 0; g < 4; ++g) {  /* 64 values: low nibbles (group 2g), high nibbles (group 2g + 1) */
                int sc, mn;
                k_group(2 * g, b + 4, &sc, &mn);
                const float d1 = d * (float)sc, m1 = dm * (float)mn;
                k_group(2 * g + 1, b + 4, &sc, &mn);
                const float d2 = d * (float)sc, m2 = dm * (float)mn;
                for (int l = 0; l < 32; ++l) {
                    const int hb1 = q5 ? ((b[16 + l] >> (2 * g)) & 1) << 4 : 0;
                    const int hb2 = q5 ? ((b[16 + l] >> (2 * g + 1)) & 1) << 4 : 0;
                    o[64 * g + l] = d1 * (float)((ql[32 * g + l] & 15) + hb1) - m1;
                    o[64 * g + 32 + l] = d2 * (float)((ql[32 * g + l] >> 4) + hb2) - m2;
                }
            }
            break;
        }
        case 11: {
            const float d = h2f(b + 108);
            int8_t sc[16];  /* the 12 scale bytes as 16 6-bit values (low 4 bits, then 2 high bits) */
            for (int i = 0; i < 16; ++i) {
                const int lo = (b[96 + (i % 8)] >> (4 * (i / 8))) & 15;
                const int hi = (b[104 + (i % 4)] >> (2 * (i / 4))) & 3;
                sc[i] = (int8_t)(lo | (hi << 4));
            }
            for (int half = 0; half < 2; ++half)
                for (int j = 0; j < 4; ++j)
                    for (int part = 0; part < 2; ++part) {
                        const int is = 8 * half + 2 * j + part;
                        const float dl = d * (float)(sc[is] - 32);
                        for (int l = 0; l < 16; ++l) {
                            const int idx = 16 * part + l;
                            const int q = (b[32 + 32 * half + idx] >> (2 * j)) & 3;
                            const int m = (b[idx] >> (4 * half + j)) & 1;
                            o[128 * half + 32 * j + idx] = dl * (float)(q - (m ? 0 : 4));
                        }
                    }
            break;
        }
        case 14: {
            const float d = h2f(b + 208);
            for (int half = 0; half < 2; ++half) {
                const uint8_t* ql = b + 64 * half;
                const uint8_t* qh = b + 128 + 32 * half;
                const int8_t* sc = (const int8_t*)(b + 192 + 8 * half);
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    o[128 * half + l] = d * (float)sc[is] * (float)q1;
                    o[128 * half + l + 32] = d * (float)sc[is + 2] * (float)q2;
                    o[128 * half + l + 64] = d * (float)sc[is + 4] * (float)q3;
                    o[128 * half + l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
            break;
        }
        default: break;
    }
}

int or_native_dequant(int type, const uint8_t* blocks, int64_t n_values, float* out) {
    native_info I;
    if (!native_info_of(type, &I) || n_values % I.qk) return -1;
    for (int64_t b = 0; b < n_values / I.qk; ++b) dequant_block(type, blocks + b * I.bytes, out + b * I.qk);
    return 0;
}

/* the independent check: double sums of dequantised weights times the q8_1 values d * q */
int or_native_gemv_double(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y) {
    const int64_t rb = or_native_row_bytes(type, n_in);
    if (rb < 0) return -1;
    float* row = (float*)malloc(sizeof(float) * (size_t)n_in);
    double* a = (double*)malloc(sizeof(double) * (size_t)n_in);
    for (int c = 0; c < n_col; ++c) {
        const uint8_t* col = xq + (size_t)c * (n_in / 32) * 36;
        for (int i = 0; i < n_in; ++i) a[i] = (double)h2f(col + (size_t)(i / 32) * 36) * (double)(int8_t)col[(size_t)(i / 32) * 36 + 4 + i % 32];
        for (int r = 0; r < n_out; ++r) {
            or_native_dequant(type, w + (size_t)r * rb, n_in, row);
            double acc = 0.0;
            for (int i = 0; i < n_in; ++i) acc += (double)row[i] * a[i];
            y[(size_t)c * n_out + r] = (float)acc;
        }
    }
    free(row);
    free(a);
    return 0;
}
