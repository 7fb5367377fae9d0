// stratametal_amd/csrc/smoe_gemv.hpp - wave helpers and the q8_1 activation images shared by the decode-path
// GEMV kernels (Q2_0 and IQ2_S).
#pragma once

#include "smoe_device.hpp"
#include "smoe_items.hpp"
#include "smoe_launch.hpp"

namespace smoe {

// ------------------------------------------------------------------------------------------------ lane exchange
// xor exchange inside groups of up to 32 lanes without LDS traffic: DPP quad permutes for distance 1 and 2,
// ds_swizzle (bit mode, xor mask) for 4, 8 and 16.
template <int O>
__device__ __forceinline__ int xor_swap_i(int i) {
    if constexpr (O == 1) return __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false);       // quad_perm [1,0,3,2]
    else if constexpr (O == 2) return __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else return __builtin_amdgcn_ds_swizzle(i, 0x1F | (O << 10));                          // lane ^ O within 32
}
template <int O>
__device__ __forceinline__ float xor_swap(float v) {
    return __int_as_float(xor_swap_i<O>(__float_as_int(v)));
}

// The value of lane ^ D (D a power of two below 64), by VALU lane moves only: quad permutes (1, 2), the half-row
// mirror (lane ^ 7) then the quad reversal (lane ^ 3) for 4, the row rotation by 8 (within 16 lanes it is lane ^ 8),
// and for 16 and 32 a permlane swap of the value with itself (the partner is the half the lane did not keep).
template <int D>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    const int i = (int)v;
    if constexpr (D == 1) return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false);
    else if constexpr (D == 2) return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false);
    else if constexpr (D == 4)
        return (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(i, 0x141, 0xF, 0xF, false), 0x1B, 0xF, 0xF,
                                                  false);
    else if constexpr (D == 8) return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0x128, 0xF, 0xF, false);
    else if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
        return (uint32_t)((threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        static_assert(D == 32, "xor_lane: D is a power of two below 64");
        const auto r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
        return (uint32_t)((threadIdx.x & 32) ? r[0] : r[1]);
    }
}
__device__ __forceinline__ uint32_t xor_lane_d(uint32_t v, int d) {  // d constant after unrolling
    switch (d) {
        case 1: return xor_lane<1>(v);
        case 2: return xor_lane<2>(v);
        case 4: return xor_lane<4>(v);
        case 8: return xor_lane<8>(v);
        case 16: return xor_lane<16>(v);
        default: return xor_lane<32>(v);
    }
}

// Bitonic sort of one value per lane over the wave, descending (lane 0 the largest): 21 compare-exchange stages on
// the VALU, no scalar round trip.
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int d = size >> 1; d > 0; d >>= 1) {
            const uint32_t p = xor_lane_d(v, d);
            const bool take_max = ((lane & d) == 0) != ((lane & size) != 0);
            v = take_max ? max(v, p) : min(v, p);
        }
    }
    return v;
}

// Sum over groups of `lpr` consecutive lanes, distance lpr/2 first; every lane of a group ends with the sum.
__device__ __forceinline__ float group_sum(float v, int lpr) {
    if (lpr >= 16) v = v + xor_swap<8>(v);
    if (lpr >= 8) v = v + xor_swap<4>(v);
    if (lpr >= 4) v = v + xor_swap<2>(v);
    if (lpr >= 2) v = v + xor_swap<1>(v);
    return v;
}

// group_sum with the lanes per row as data: every distance is exchanged and each addition kept or not by a
// select (the same additions as group_sum), so that the sums of several rows interleave with no branch between.
__device__ __forceinline__ float group_sum_sel(float v, int lpr) {
    float t = xor_swap<8>(v);
    v = lpr >= 16 ? v + t : v;
    t = xor_swap<4>(v);
    v = lpr >= 8 ? v + t : v;
    t = xor_swap<2>(v);
    v = lpr >= 4 ? v + t : v;
    t = xor_swap<1>(v);
    v = lpr >= 2 ? v + t : v;
    return v;
}

// v + v[lane ^ 32] by one v_permlane32_swap: with both operands v, the two results hold the lower and the upper
// half of v in both halves, and their sum is that addition (commutative, so bit for bit).
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// The xor butterfly 32, 16, ..., 1 over the whole wave (the same sums as wave_sum_xor): distance 32 by
// add_xor32, the rest as in xor_swap.
__device__ __forceinline__ float wave_sum_xor_fast(float v) {
    v = add_xor32(v);
    v = v + xor_swap<16>(v);
    v = v + xor_swap<8>(v);
    v = v + xor_swap<4>(v);
    v = v + xor_swap<2>(v);
    v = v + xor_swap<1>(v);
    return v;
}

// wave_sum_xor_fast of N independent values, stage by stage, so that the N exchanges of a stage are in
// flight together.
template <int N>
__device__ __forceinline__ void wave_sum_xor_fast_n(float (&v)[N]) {
    float t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = add_xor32(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = xor_swap<16>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = xor_swap<8>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = xor_swap<4>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = xor_swap<2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = xor_swap<1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
}

// Wave maxima for order-free reductions: row rotations by DPP (8, 4, 2, 1), then the four row results read
// into scalars.  The result is uniform.
__device__ __forceinline__ uint32_t wave_max_u32_fast(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));  // row_ror:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));  // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xF, 0xF, false));  // row_ror:2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xF, 0xF, false));  // row_ror:1
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}
__device__ __forceinline__ float wave_max_fast(float v) {
    v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));
    v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));
    v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xF, 0xF, false)));
    v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return __builtin_fmaxf(__builtin_fmaxf(a, b), __builtin_fmaxf(c, d));
}
__device__ __forceinline__ int wave_min_i32_fast(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false));
    const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return min(min(a, b), min(c, d));
}

__device__ __forceinline__ int lanes_per_row(int dpr) {
    const int l = dpr & -dpr;
    return l > 16 ? 16 : l;
}

// ------------------------------------------------------------------------------------------------ q8_1 images
// A q8_1 block (32 activations) as the GEMV kernels read it: 12 dwords, 16-byte aligned:
//   dwords 0..7  the 32 int8 values q, in one of two layouts:
//     split (the Q2_0 kernels): each q as q = 16 qh + ql, qh = q >> 4 (signed 4-bit), ql = q & 15 (unsigned
//       4-bit); for each 16-group g, dword 4g holds qh of positions 16g + 2i in nibble i, dword 4g + 1 their ql,
//       dwords 4g + 2 and 4g + 3 the same for positions 16g + 2i + 1 -- the nibble order in which
//       (codes >> 2s) & 0x33333333 delivers a 2-bit code dword (s = 0: even positions, s = 1: odd), so that
//       sum(code * q) = 16 sdot8(codes, qh) + udot8(codes, ql) exactly;
//     natural (the IQ2_S kernels): dword c holds q[4c .. 4c + 3];
//   dword 8      f32 of the stored fp16 scale d; dword 9 the int sum of q; dwords 10..11 unused.
// Built by the same quantiser as the q8_1 block (metal/shaders/iq.metal:597-627); the fp16 sum field of the
// q8_1 block is not needed by the Q2_0 / IQ2_S dots (metal/shaders/iq.metal:152-180,444-456) and is not kept.
constexpr int kImgDw = 12;

// Images staged in LDS: every unit of four images (192 bytes) is followed by 16 bytes of padding, so that the
// lanes of a row group, which read consecutive units, start on different LDS banks (unpadded, the 192-byte
// stride put 4 or 8 of them on the same banks).  Image B of a staged region (column-major, a column a whole
// number of units) starts at dword lds_blk(B); a column of qb images spans qb * kImgLdsDw dwords; unit u of a
// column starts at dword u * kUnitLdsDw; the 16-byte pieces of the unpadded order land at lds_piece(p).
constexpr int kImgLdsDw = 13;
constexpr int kUnitLdsDw = 4 * kImgDw + 4;
__host__ __device__ __forceinline__ int lds_blk(int b) { return kImgDw * b + 4 * (b >> 2); }
__host__ __device__ __forceinline__ int lds_piece(int p) { return p + p / 12; }

// Maximum and sum over each 32-lane half of the wave, every lane receiving its half's result: DPP rotations
// inside the 16-lane rows, then the other row of the half by swizzle.  Both are independent of the order of
// combination (max of finite values, integer sum), so these equal any other reduction of the same values.
__device__ __forceinline__ float half_max(float a) {
    a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x128, 0xF, 0xF, false)));
    a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x124, 0xF, 0xF, false)));
    a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x122, 0xF, 0xF, false)));
    a = __builtin_fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x121, 0xF, 0xF, false)));
    return __builtin_fmaxf(a, __int_as_float(xor_swap_i<16>(__float_as_int(a))));
}
__device__ __forceinline__ int half_sum_i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);  // row_ror:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false);  // row_ror:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false);  // row_ror:1
    return v + xor_swap_i<16>(v);
}

// The h image exchange of the fused small-batch layer (k_q2_moe_small): image dwords 0..9 of a block, each in a
// 64-bit word {dword, tag} written and read as one agent-scope atomic, tag 1 once written (the router kernel of the
// same call clears the words first), so that every word is checked by itself and needs no fence.
constexpr int kXchgSlots = 10;
__device__ __forceinline__ void xchg_put(uint64_t* w, uint32_t v) {
    __hip_atomic_store(w, (uint64_t)v | (1ull << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t xchg_get(const uint64_t* w) {
    return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A 32-lane half wave quantises one block (lane & 31 = position) and writes its image, split or `natural`;
// `sc` is 32 bytes of LDS scratch owned by the half (natural layout only).  Every lane of the half must call
// it; `store` false skips the global store.  With `xchg` (split layout only) the image goes to kXchgSlots
// tagged exchange words instead of `img`.
__device__ __forceinline__ void q8_image_store(float v, bool store, uint8_t* sc, uint32_t* img, bool natural = false,
                                               uint64_t* xchg = nullptr) {
    const int l32 = threadIdx.x & 31;
    const float a = half_max(__builtin_fabsf(v));
    float d = a / 127.0f;
    if (__builtin_fabsf(d) > 65504.0f) d = __builtin_copysignf(65504.0f, d);
    int q = 0;
    if (a != 0.0f) {
        float r = __builtin_roundf(v / d);
        r = r > 127.0f ? 127.0f : r;
        r = r < -127.0f ? -127.0f : r;
        q = (r == r) ? (int)r : 0;
    }
    const int sq = half_sum_i(q);
    if (natural) {
        sc[l32] = (uint8_t)(int8_t)q;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (store && l32 < 8) img[l32] = reinterpret_cast<const uint32_t*>(sc)[l32];
    } else {
        // nibble (l32 & 15) >> 1 of dword 4 (l32 >> 4) + 2 (l32 & 1) (qh) and of the next one (ql): OR over
        // the eight lanes that share the dwords (xor 2, 4, 8), then lanes 0, 1, 16 and 17 hold them
        const int sh = 4 * ((l32 & 15) >> 1);
        int vh = ((q >> 4) & 15) << sh, vl = (q & 15) << sh;
        vh |= xor_swap_i<2>(vh);
        vl |= xor_swap_i<2>(vl);
        vh |= xor_swap_i<4>(vh);
        vl |= xor_swap_i<4>(vl);
        vh |= xor_swap_i<8>(vh);
        vl |= xor_swap_i<8>(vl);
        if (store && (l32 & 14) == 0) {
            const int i0 = 4 * (l32 >> 4) + 2 * (l32 & 1);
            if (xchg) {
                xchg_put(xchg + i0, (uint32_t)vh);
                xchg_put(xchg + i0 + 1, (uint32_t)vl);
            } else {
                *reinterpret_cast<uint2*>(img + i0) = make_uint2((uint32_t)vh, (uint32_t)vl);
            }
        }
    }
    if (store && (l32 == 8 || l32 == 9)) {
        const uint32_t w = l32 == 8 ? f2u(f16_to_f32(f32_to_f16(d))) : (uint32_t)sq;
        if (xchg) xchg_put(xchg + l32, w);
        else img[l32] = w;
    }
}

// Activation registers for the four q8_1 blocks of one 36-byte weight unit.
struct Act4 {
    uint32_t q[4][8];
    float d[4];
    int sq[4];
};

// Two consecutive q8_1 images (half a Q2_0 unit's activations).
struct Act2 {
    uint32_t q[2][8];
    float d[2];
    int sq[2];
};
__device__ __forceinline__ void load_act_img2(const uint32_t* __restrict__ img, Act2& a) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const uint4* p = reinterpret_cast<const uint4*>(img + b * kImgDw);
        const uint4 lo = p[0], hi = p[1], ds = p[2];
        a.q[b][0] = lo.x; a.q[b][1] = lo.y; a.q[b][2] = lo.z; a.q[b][3] = lo.w;
        a.q[b][4] = hi.x; a.q[b][5] = hi.y; a.q[b][6] = hi.z; a.q[b][7] = hi.w;
        a.d[b] = u2f(ds.x);
        a.sq[b] = (int)ds.y;
    }
}

__device__ __forceinline__ void load_act_img(const uint32_t* __restrict__ img, Act4& a) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint4* p = reinterpret_cast<const uint4*>(img + b * kImgDw);
        const uint4 lo = p[0], hi = p[1], ds = p[2];
        a.q[b][0] = lo.x; a.q[b][1] = lo.y; a.q[b][2] = lo.z; a.q[b][3] = lo.w;
        a.q[b][4] = hi.x; a.q[b][5] = hi.y; a.q[b][6] = hi.z; a.q[b][7] = hi.w;
        a.d[b] = u2f(ds.x);
        a.sq[b] = (int)ds.y;
    }
}

__device__ __forceinline__ void transpose4x4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t* o) {
    const uint32_t t0 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
    const uint32_t u0 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
    const uint32_t u1 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(u0, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(u0, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(u1, t1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(u1, t1, 0x07060302u);
}

// From four standard 36-byte q8_1 blocks (the stage API's input): permuted in registers.
__device__ __forceinline__ void load_act_std(const uint8_t* __restrict__ blk, Act4& a) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        uint32_t w[9];
        __builtin_memcpy(w, __builtin_assume_aligned(blk + b * 36, 4), 36);
        transpose4x4(w[1], w[2], w[3], w[4], a.q[b]);
        transpose4x4(w[5], w[6], w[7], w[8], a.q[b] + 4);
        int sq = 0;
#pragma unroll
        for (int i = 1; i < 9; ++i) sq = __builtin_amdgcn_sdot4((int)w[i], 0x01010101, sq, false);
        a.d[b] = f16_to_f32(w[0] & 0xFFFFu);
        a.sq[b] = sq;
    }
}

// Copying the images of columns c0 .. c0 + nc of the item (x rows by token, or h rows first + c) into LDS,
// column-major, in rounds of four 16-byte pieces per thread (pieces base + j * NT + tid; NT the work-group's threads,
// a constant, so that no kernel reads its group size, a scalar load, before these loads).  A round is
// issued into registers (stage_issue) and stored (stage_commit) separately, so that a kernel can issue its
// weight loads in between and the stores wait for the image loads only.  Within a round every load and store
// is unconditional (a piece past the end reloads the last one and lands in slot cap_cols * per-column pieces,
// which the caller's LDS holds beyond its cap_cols columns), so the loads are not serialised behind branches;
// a j with no live piece in the whole work-group is skipped.
typedef __attribute__((ext_vector_type(4))) uint32_t img_u32x4;  // a native vector: stays in registers
struct StagePieces {
    img_u32x4 v[4];
    int dst[4];
};
template <int NT>
__device__ __forceinline__ void stage_issue(StagePieces& sp, const uint32_t* __restrict__ img, int qb, int c0, int nc,
                                            int cap_cols, int base, const Item& it, const int32_t* perm, int k,
                                            bool by_token) {
    const int per_col = qb * (kImgDw / 4);  // uint4 per column
    const int total = nc * per_col, dead = cap_cols * per_col;
    constexpr int nt = NT;
    // rows without memory reads (h rows, shared tokens, or a routed item's first four columns), so that the
    // image loads of all rounds go out together; otherwise item_token reads perm
    const bool direct = !by_token || it.shared || c0 + nc <= 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (base + j * nt < total) {
            const int raw = base + j * nt + (int)threadIdx.x;
            const int idx = min(raw, total - 1);
            const int c = idx / per_col;
            int row;
            if (direct) row = !by_token ? it.first + c0 + c : it.shared ? it.tok0 + c0 + c : item_token_head(it, c0 + c);
            else row = item_token(it, perm, k, c0 + c);
            sp.v[j] = reinterpret_cast<const img_u32x4*>(img)[(size_t)row * per_col + (idx - c * per_col)];
            sp.dst[j] = raw < total ? raw : dead;
        }
    }
}
template <int NT>
__device__ __forceinline__ void stage_commit(const StagePieces& sp, uint32_t* act, int qb, int nc, int base) {
    const int total = nc * qb * (kImgDw / 4);
    constexpr int nt = NT;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (base + j * nt < total) reinterpret_cast<img_u32x4*>(act)[lds_piece(sp.dst[j])] = sp.v[j];
}
// Round `base` with rows that need no memory read (see stage_issue) as straight-line code: all four loads
// unconditional (a piece past the end, or a whole j past the end, reloads the last piece and is stored to the
// dead slot), so that the compiler counts the loads in flight exactly and a later store waits for its own load
// alone.
template <int NT>
__device__ __forceinline__ void stage_issue_direct(StagePieces& sp, const uint32_t* __restrict__ img, int qb, int c0,
                                                   int nc, int cap_cols, int base, const Item& it, bool by_token) {
    const int per_col = qb * (kImgDw / 4);
    const int total = nc * per_col, dead = cap_cols * per_col;
    constexpr int nt = NT;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int raw = base + j * nt + (int)threadIdx.x;
        const int idx = min(raw, total - 1);
        const int c = idx / per_col;
        const int row = !by_token ? it.first + c0 + c : it.shared ? it.tok0 + c0 + c : item_token_head(it, c0 + c);
        sp.v[j] = reinterpret_cast<const img_u32x4*>(img)[(size_t)row * per_col + (idx - c * per_col)];
        sp.dst[j] = raw < total ? raw : dead;
    }
}
__device__ __forceinline__ void stage_commit_direct(const StagePieces& sp, uint32_t* act) {
#pragma unroll
    for (int j = 0; j < 4; ++j) reinterpret_cast<img_u32x4*>(act)[lds_piece(sp.dst[j])] = sp.v[j];
}
// True when stage_issue_direct can serve columns c0 .. c0 + nc.
__device__ __forceinline__ bool stage_direct(const Item& it, int c0, int nc, bool by_token) {
    return !by_token || it.shared || c0 + nc <= 4;
}

// The rounds from `from` on, each issued and stored in turn.
template <int NT>
__device__ __forceinline__ void stage_images(uint32_t* act, const uint32_t* __restrict__ img, int qb, int c0, int nc,
                                             int cap_cols, const Item& it, const int32_t* perm, int k, bool by_token,
                                             int from = 0, int to = 1 << 30) {
    const int total = min(nc * qb * (kImgDw / 4), to);
    for (int base = from; base < total; base += 4 * NT) {
        StagePieces sp;
        stage_issue<NT>(sp, img, qb, c0, nc, cap_cols, base, it, perm, k, by_token);
        stage_commit<NT>(sp, act, qb, nc, base);
    }
}

// out[j] = RMSNorm(x + r)[j] of one row with unit weight (r may be NULL), by a 256-thread work-group: s = x + r in
// f32; ss = sum of s^2 with thread i accumulating fmaf(s_j, s_j, acc) over j = i, i + 256, ... in order, then the
// wave butterfly 32..1, then the wave sums ((w0 + w1) + w2) + w3; out = s * (1 / sqrt(ss / n + eps)) with IEEE
// division and square root (oracle: or_residual_rmsnorm_dev).  n <= 4096.  VEC (x, r, out 16-byte aligned,
// n % 4 == 0): the row is read with 16-byte loads into `row` (LDS, n floats), summed from there in the same
// order, and written from there with 16-byte stores; `row` then holds the outputs.  Otherwise each thread reads
// and writes its own elements (`row`, if given, receives the outputs).  Every load precedes every store, so out
// may alias x.
constexpr int kNormPer = 16;  // elements per thread: rows up to 4096
template <bool VEC>
__device__ __forceinline__ void residual_rmsnorm_row(const float* xr, const float* rr, int n, float eps, float* o,
                                                     float* wsum, float* row) {
    float v[kNormPer];
    float acc = 0.0f;
    if constexpr (VEC) {
        for (int c = (int)threadIdx.x; c < (n >> 2); c += 256) {
            float4 a = reinterpret_cast<const float4*>(xr)[c];
            if (rr) {
                const float4 b = reinterpret_cast<const float4*>(rr)[c];
                a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
            }
            reinterpret_cast<float4*>(row)[c] = a;
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < kNormPer; ++m) {
        const int j = (int)threadIdx.x + 256 * m;
        const int jc = j < n ? j : n - 1;  // clamped, so that every load issues
        float sj;
        if constexpr (VEC) {
            sj = row[jc];
        } else {
            sj = xr[jc];
            if (rr) sj = sj + rr[jc];
        }
        v[m] = sj;
        if (j < n) acc = __builtin_fmaf(sj, sj, acc);
    }
    acc = wave_sum_xor_fast(acc);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int m = 0; m < kNormPer; ++m) {
        const int j = (int)threadIdx.x + 256 * m;
        if (j < n) {
            if constexpr (VEC) {
                row[j] = v[m] * inv;
            } else {
                o[j] = v[m] * inv;
                if (row) row[j] = v[m] * inv;
            }
        }
    }
    if constexpr (VEC) {
        __syncthreads();
        for (int c = (int)threadIdx.x; c < (n >> 2); c += 256)
            reinterpret_cast<float4*>(o)[c] = reinterpret_cast<const float4*>(row)[c];
    }
}

// The expert stages of a traced call for one column's 32 values of h (half wave = column, lane & 31 = value i of
// rows block hb): the gate and up dots g, u and the q8_1 block of h, at pair row `row` (dispatch position; rows from
// so.P are the shared expert's tokens).  Every lane of the half must call it (the quantiser exchanges lanes); `live`
// is the same for the whole half.
__device__ __forceinline__ void stage_store(const StageOut& so, int row, int hb, float g, float u, float h, bool live,
                                            int F, int Fs) {
    const int i = threadIdx.x & 31;
    uint32_t ds;
    const int q = q8_1_value(h, &ds);
    const bool routed = row < so.P;
    const int t = row - so.P;
    const bool ok = live && (routed || t < so.T);
    const int width = routed ? F : Fs;
    uint8_t* hqb = routed ? so.hq : so.shq;
    const size_t r = routed ? (size_t)row : (size_t)t;
    if (hqb) q8_1_store(q, ds, hqb + (r * (size_t)(width >> 5) + hb) * 36, ok);
    const size_t e = r * (size_t)width + (size_t)hb * 32 + i;
    if (ok && routed) {
        if (so.egate) so.egate[e] = g;
        if (so.eup) so.eup[e] = u;
    }
    if (ok && !routed && so.sgu) {
        so.sgu[e] = g;
        so.sgu[(size_t)so.T * Fs + e] = u;
    }
}

}  // namespace smoe
