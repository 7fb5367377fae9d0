// stratametal_amd/csrc/smoe_device.hpp - device helpers shared by the MoE kernels (gfx950, wave64).
//
// The library is compiled with -ffp-contract=off: a multiply-add is fused only where __builtin_fmaf is
// written, so every reduction order stated in the kernels is the order that executes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smoe {

constexpr int kWave = 64;

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// fp16 bits -> f32, exact including subnormals (include/strata/kernels/f16_bits.hpp:73-101).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (e == 0) {
        if (man == 0) return u2f(sign);
        const int s = __builtin_clz(man) - 21;  // shifts that bring the leading one to bit 10
        man = (man << s) & 0x3FFu;
        return u2f(sign | ((uint32_t)(113 - s) << 23) | (man << 13));
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((e + 112u) << 23) | (man << 13));
}

// f32 -> fp16 bits, round to nearest even (include/strata/kernels/f16_bits.hpp:37-66).
__device__ inline uint32_t f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e8 = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (e8 == 0xFFu) return sign | 0x7C00u | (man ? 0x200u : 0u);
    const int e = (int)e8 - 112;
    if (e >= 31) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -10) return sign;
        man |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        const uint32_t rest = man & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (h & 1u))) h += 1u;
        return sign | h;
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return h;
}

// f32 -> bf16 bits, RNE with NaN quieted (include/strata/kernels/bf16_bits.hpp:37-47).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    const uint32_t i = f2u(f);
    const uint32_t rounded = (i + ((i >> 16) & 1u) + 0x7FFFu) >> 16;
    const uint32_t quiet = ((i >> 16) | 64u) & 0xFFFFu;
    return (i & 0x7FFFFFFFu) > 0x7F800000u ? quiet : rounded;  // a select, no branch
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return u2f(h << 16); }

// e^x: Cody-Waite reduction by ln 2 (split 355/512 + remainder), Taylor polynomial of degree 7 in Horner
// form with fused multiply-adds, scaled by 2^n.  Inputs below -87 return 0, above 89 return +inf.
__device__ inline float expf_smoe(float x) {
    // branch-free: the polynomial runs on a clamped argument and the out-of-range cases are selected after
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -87.0f), 89.0f);
    const float n = __builtin_rintf(xc * 1.44269504088896341f);
    float r = __builtin_fmaf(n, -0.693359375f, xc);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float e = __builtin_ldexpf(p, (int)n);
    e = x < -87.0f ? 0.0f : e;
    e = x > 89.0f ? __builtin_inff() : e;
    return x != x ? x : e;
}

// ln x for normal x > 0: x = m 2^e, m in [1/sqrt 2, sqrt 2), ln m = 2 atanh((m-1)/(m+1)) to s^11.
__device__ inline float logf_smoe(float x) {
    const uint32_t b = f2u(x);
    int e = (int)((b >> 23) & 0xFFu) - 127;
    float m = u2f((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 9.09090909e-2f;
    p = __builtin_fmaf(p, s2, 1.11111111e-1f);
    p = __builtin_fmaf(p, s2, 1.42857143e-1f);
    p = __builtin_fmaf(p, s2, 2.0e-1f);
    p = __builtin_fmaf(p, s2, 3.33333333e-1f);
    const float r = __builtin_fmaf(s * s2, p, s);
    const float lnm = 2.0f * r;
    const float fe = (float)e;
    return __builtin_fmaf(fe, 0.693359375f, __builtin_fmaf(fe, -2.12194440e-4f, lnm));
}

// cos(2 pi v): fold to [0, 1/8] of a turn, Taylor cos to degree 10 or sin to degree 11.
__device__ inline float cos2pi_smoe(float v) {
    const float t = v - __builtin_rintf(v);
    float a = __builtin_fabsf(t);
    float sign = 1.0f;
    if (a > 0.25f) { a = 0.5f - a; sign = -1.0f; }
    const bool use_sin = a > 0.125f;
    if (use_sin) a = 0.25f - a;
    const float th = 6.28318531f * a;
    const float z = th * th;
    float r;
    if (use_sin) {
        float p = -2.50521084e-8f;
        p = __builtin_fmaf(p, z, 2.75573192e-6f);
        p = __builtin_fmaf(p, z, -1.98412698e-4f);
        p = __builtin_fmaf(p, z, 8.33333333e-3f);
        p = __builtin_fmaf(p, z, -1.66666667e-1f);
        r = __builtin_fmaf(th * z, p, th);
    } else {
        float p = -2.75573192e-7f;
        p = __builtin_fmaf(p, z, 2.48015873e-5f);
        p = __builtin_fmaf(p, z, -1.38888889e-3f);
        p = __builtin_fmaf(p, z, 4.16666667e-2f);
        p = __builtin_fmaf(p, z, -0.5f);
        r = __builtin_fmaf(z, p, 1.0f);
    }
    return sign * r;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf_smoe(-g))) * u; }
__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + expf_smoe(-z)); }

// Counter-based SplitMix64: the finaliser over a Weyl sequence keyed by (seed, stream).
__device__ __forceinline__ uint64_t hash64(uint64_t seed, uint64_t stream, uint64_t i) {
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull + (i + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float uniform24(uint64_t seed, uint64_t stream, uint64_t i) {
    return ((float)(uint32_t)(hash64(seed, stream, i) >> 40) + 0.5f) * 5.9604644775390625e-8f;
}
__device__ inline float normal_bm(uint64_t seed, uint64_t stream, uint64_t i) {
    const float u1 = uniform24(seed, stream, 2ull * i);
    const float u2 = uniform24(seed, stream, 2ull * i + 1ull);
    return __builtin_sqrtf(-2.0f * logf_smoe(u1)) * cos2pi_smoe(u2);
}

// xor butterfly over the whole wave (distance 32 first); every lane ends with the same sum.
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// q8_1 of one 32-value block held one value per lane of a 32-lane half wave (lane & 31 = position):
// amax and sum by the xor butterfly 16..1, d = amax / 127 clamped to 65504, q = clamp(round(x / d)),
// s clamped to 65504, d and s stored as fp16 (metal/shaders/iq.metal:597-627).  A NaN value stores 0.
// Every lane returns its int8; lane 0 of the half returns the packed {d, s} dword in *ds.
__device__ __forceinline__ int q8_1_value(float v, uint32_t* ds) {
    float a = __builtin_fabsf(v), s = v;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        a = __builtin_fmaxf(a, __shfl_xor(a, o, kWave));
        s = s + __shfl_xor(s, o, kWave);
    }
    float d = a / 127.0f;
    if (__builtin_fabsf(d) > 65504.0f) d = __builtin_copysignf(65504.0f, d);
    int q = 0;
    if (a != 0.0f) {
        float r = __builtin_roundf(v / d);
        r = r > 127.0f ? 127.0f : r;
        r = r < -127.0f ? -127.0f : r;
        q = (r == r) ? (int)r : 0;
    }
    const float sc = __builtin_fabsf(s) > 65504.0f ? __builtin_copysignf(65504.0f, s) : s;
    *ds = f32_to_f16(d) | (f32_to_f16(sc) << 16);
    return q;
}

// Packs the 32 int8 of a half wave into a q8_1 block in global memory: lanes 0..7 of the half write
// one dword each of q, lane 0 also the {d, s} dword.  Every lane of the half must call it; `store` false (the same
// for the whole half) writes nothing.
__device__ __forceinline__ void q8_1_store(int q, uint32_t ds, uint8_t* blk, bool store = true) {
    const int l32 = threadIdx.x & 31;
    const int base = threadIdx.x & 32;
    // gather bytes 4j..4j+3 into lane j
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int src = base + ((4 * l32 + b) & 31);
        const uint32_t v = (uint32_t)__shfl(q, src, kWave) & 0xFFu;
        word |= v << (8 * b);
    }
    uint32_t* p = reinterpret_cast<uint32_t*>(blk);
    if (store && l32 < 8) p[1 + l32] = word;
    if (store && l32 == 0) p[0] = ds;
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP: row shifts by 1, 2, 4 and 8 (zero fill at the
// start of each 16-lane row), then lane 15 of each row added into the next row (rows 1 and 3) and lane 31
// into rows 2 and 3.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return x;
}

// N exclusive scans over the 1024 threads of the block at once: a DPP scan inside each wave, the 16 wave
// totals through LDS (scratch: N x 17 ints), then every wave scans the totals itself (one barrier).
template <int N>
__device__ __forceinline__ void block_exclusive_scan_1024(const int (&v)[N], int* scratch, int (&r)[N],
                                                          int (&total)[N]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl[N];
#pragma unroll
    for (int j = 0; j < N; ++j) incl[j] = wave_inclusive_scan(v[j]);
    if (lane == 63) {
#pragma unroll
        for (int j = 0; j < N; ++j) scratch[17 * j + wave] = incl[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const int x = wave_inclusive_scan(lane < 16 ? scratch[17 * j + lane] : 0);
        const int before = wave > 0 ? __builtin_amdgcn_readlane(x, (wave - 1) & 15) : 0;
        r[j] = before + incl[j] - v[j];
        total[j] = __builtin_amdgcn_readlane(x, 15);
    }
}

}  // namespace smoe
