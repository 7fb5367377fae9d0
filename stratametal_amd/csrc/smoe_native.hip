// stratametal_amd/csrc/smoe_native.hip - GEMV of the other native GGUF types of real layers (gfx950, wave64).
//
// The shared expert's projections and the down quants of real layers come in Q8_0, Q4_0, Q5_0, IQ4_NL, IQ4_XS,
// Q3_K, Q4_K, Q5_K and Q6_K (include/strata/kernels/shared_expert.hpp:54-58, metal/src/pack_parity.cpp:7782-7799).
// Each runs the reference's q8_1 MMVQ contract: a row is a sum of per-block integer partials against q8_1
// activations (metal/shaders/iq.metal:224-442), taken by 32 lanes -- lane l adds partials l, l + 32, ... in order
// from 0 -- then an xor butterfly 16, 8, 4, 2, 1 (iq_row / iq_mmvq_body, metal/shaders/iq.metal:458-513).  Here a
// 32-lane half wave owns one row, so that order runs unchanged (oracle: or_native_gemv, which is also the
// reference's own host order, metal/src/pack_parity.cpp:2785-3475).  Bandwidth is not the aim: these are the shared
// expert's few rows per layer.
#include "smoe_device.hpp"
#include "smoe_gemv.hpp"
#include "smoe_launch.hpp"

namespace smoe {

namespace {

// values, bytes, partials per block and the iqs step of each type (iq_row<QK, IPB, STEP, BLOCK>)
template <int TYPE>
struct NativeType;
template <> struct NativeType<8> { static constexpr int qk = 32, bytes = 34, ipb = 1, step = 1; };
template <> struct NativeType<2> { static constexpr int qk = 32, bytes = 18, ipb = 2, step = 2; };
template <> struct NativeType<6> { static constexpr int qk = 32, bytes = 22, ipb = 2, step = 2; };
template <> struct NativeType<20> { static constexpr int qk = 32, bytes = 18, ipb = 2, step = 2; };
template <> struct NativeType<23> { static constexpr int qk = 256, bytes = 136, ipb = 8, step = 4; };
template <> struct NativeType<11> { static constexpr int qk = 256, bytes = 110, ipb = 16, step = 1; };
template <> struct NativeType<12> { static constexpr int qk = 256, bytes = 144, ipb = 16, step = 2; };
template <> struct NativeType<13> { static constexpr int qk = 256, bytes = 176, ipb = 16, step = 2; };
template <> struct NativeType<14> { static constexpr int qk = 256, bytes = 210, ipb = 32, step = 1; };

// Block fields are 2-byte aligned (every block size is even); a 32-bit field is read as two halves.
__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ int32_t rd32(const uint8_t* p) { return (int32_t)(rd16(p) | (rd16(p + 2) << 16)); }
__device__ __forceinline__ float rdh(const uint8_t* p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)rd16(p));  // exact fp16 -> f32
}
// the q8_1 block's int8 word w (4-byte aligned: blocks are 36 bytes)
__device__ __forceinline__ int32_t qword(const uint8_t* b, int w) {
    return *reinterpret_cast<const int32_t*>(b + 4 + 4 * w);
}
__device__ __forceinline__ int32_t dot4(int32_t a, int32_t b, int32_t c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__constant__ int8_t kNl4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
// the codebook bytes of the low and high nibbles of four code bytes
__device__ __forceinline__ void nl_bytes(int32_t codes, int32_t& lo, int32_t& hi) {
    uint32_t a = 0, b = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t c = ((uint32_t)codes >> (8 * i)) & 0xFFu;
        a |= (uint32_t)(uint8_t)kNl4[c & 15u] << (8 * i);
        b |= (uint32_t)(uint8_t)kNl4[c >> 4] << (8 * i);
    }
    lo = (int32_t)a;
    hi = (int32_t)b;
}

// Q4_K / Q5_K: the 6-bit scale and min pair of two 32-value groups (iq_k_scale_min, metal/shaders/iq.metal:254-262)
__device__ __forceinline__ void k_scale_min(const uint8_t* s, int bq8_offset, int (&sc)[2], int (&mn)[2]) {
    const int j = bq8_offset / 2, jm = j & 1;
    const uint32_t s0 = rd16(s + 2 * (jm + 0)), s2 = rd16(s + 2 * (jm + 2)), s4 = rd16(s + 2 * (jm + 4));
    const uint32_t a0 = j >= 2 ? (((s4 >> 0) & 0x0F0Fu) | ((s0 & 0xC0C0u) >> 2)) : (s0 & 0x3F3Fu);
    const uint32_t a1 = j >= 2 ? (((s4 >> 4) & 0x0F0Fu) | ((s2 & 0xC0C0u) >> 2)) : (s2 & 0x3F3Fu);
    sc[0] = (int)(a0 & 0xFFu);
    sc[1] = (int)((a0 >> 8) & 0xFFu);
    mn[0] = (int)(a1 & 0xFFu);
    mn[1] = (int)((a1 >> 8) & 0xFFu);
}

// One partial of a row: block `blk`, its q8_1 blocks from x0, part iqs.  Integer sums are exact; the float steps
// are the reference's, one rounding each (no contraction).
template <int TYPE>
__device__ __forceinline__ float native_part(const uint8_t* __restrict__ blk, const uint8_t* __restrict__ x0, int iqs) {
    if constexpr (TYPE == 8) {  // Q8_0
        int32_t s = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) s = dot4(rd32(blk + 2 + 4 * (iqs + j)), qword(x0, iqs + j), s);
        return (rdh(blk) * rdh(x0)) * (float)s;
    } else if constexpr (TYPE == 2 || TYPE == 6) {  // Q4_0: nibble - 8; Q5_0: (nibble | high bit << 4) - 16
        const uint8_t* qs = blk + (TYPE == 2 ? 2 : 6);
        int32_t s = 0, a = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int32_t v = rd32(qs + 4 * (iqs + i));
            int32_t lo = v & 0x0F0F0F0F, hi = (v >> 4) & 0x0F0F0F0F;
            if constexpr (TYPE == 6) {
                const uint32_t h = (uint32_t)rd32(blk + 2) >> (4 * (iqs + i));
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    lo |= (int32_t)(((h >> b) & 1u) << (8 * b + 4));
                    hi |= (int32_t)(((h >> (16 + b)) & 1u) << (8 * b + 4));
                }
            }
            const int32_t u0 = qword(x0, iqs + i), u1 = qword(x0, iqs + i + 4);
            s = dot4(lo, u0, s);
            s = dot4(hi, u1, s);
            a = dot4(0x01010101, u0, a);
            a = dot4(0x01010101, u1, a);
        }
        return (rdh(blk) * rdh(x0)) * (float)(s - (TYPE == 2 ? 8 : 16) * a);
    } else if constexpr (TYPE == 20) {  // IQ4_NL
        int32_t s = 0;
#pragma unroll
        for (int l = 0; l < 2; ++l) {
            int32_t lo, hi;
            nl_bytes(rd32(blk + 2 + 4 * (iqs + l)), lo, hi);
            s = dot4(lo, qword(x0, iqs + l), s);
            s = dot4(hi, qword(x0, iqs + l + 4), s);
        }
        return (rdh(blk) * rdh(x0)) * (float)s;
    } else if constexpr (TYPE == 23) {  // IQ4_XS: 32-value group iqs / 4, its 6-bit scale - 32
        const uint8_t* x = x0 + (size_t)(iqs / 4) * 36;
        int32_t s = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int32_t lo, hi;
            nl_bytes(rd32(blk + 8 + 4 * (iqs + j)), lo, hi);
            s = dot4(lo, qword(x, j), s);
            s = dot4(hi, qword(x, j + 4), s);
        }
        const int ls = ((blk[4 + iqs / 8] >> (iqs & 4)) & 15) | (int)(((rd16(blk + 2) >> (iqs / 2)) & 3u) << 4);
        s *= ls - 32;
        return (rdh(blk) * rdh(x)) * (float)s;
    } else if constexpr (TYPE == 12 || TYPE == 13) {  // Q4_K, Q5_K
        constexpr bool q5 = TYPE == 13;
        const int bq8_offset = 2 * ((iqs / 2) / 4), qoff = (iqs / 2) % 4;
        const uint8_t* ql = blk + (q5 ? 48 : 16);
        const int byte = 16 * bq8_offset + 4 * qoff;
        const int32_t v0 = rd32(ql + byte), v1 = rd32(ql + byte + 16);
        int32_t vh0 = 0, vh1 = 0;
        if constexpr (q5) {
            vh0 = rd32(blk + 16 + 4 * qoff) >> bq8_offset;
            vh1 = rd32(blk + 32 + 4 * qoff) >> bq8_offset;
        }
        int sc[2], mn[2];
        k_scale_min(blk + 4, bq8_offset, sc, mn);
        float sum_d = 0.0f, sum_m = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint8_t* b8 = x0 + (size_t)(bq8_offset + i) * 36;
            const float d8 = rdh(b8);
            const int32_t u0 = qword(b8, qoff), u1 = qword(b8, qoff + 4);
            int32_t p0 = (v0 >> (4 * i)) & 0x0F0F0F0F, p1 = (v1 >> (4 * i)) & 0x0F0F0F0F;
            if constexpr (q5) {
                p0 |= ((vh0 >> i) << 4) & 0x10101010;
                p1 |= ((vh1 >> i) << 4) & 0x10101010;
            }
            const int32_t dq = dot4(p1, u1, dot4(p0, u0, 0));
            const int32_t da = dot4(0x01010101, u1, dot4(0x01010101, u0, 0));
            sum_d = sum_d + d8 * (float)(dq * sc[i]);
            sum_m = sum_m + d8 * (float)(da * mn[i]);
        }
        return rdh(blk) * sum_d - rdh(blk + 2) * sum_m;
    } else if constexpr (TYPE == 11) {  // Q3_K: 2 low bits, - 4 where the high bit is clear; scale - 32
        const int bq8_offset = 4 * (iqs / 8), scale_offset = iqs - (iqs % 8) + (iqs % 8) / 4;
        const uint8_t* sc8 = blk + 96;
        const int32_t vl = rd32(blk + 32 + 4 * iqs);
        const uint32_t vh = (~(uint32_t)rd32(blk + 4 * (iqs % 8))) >> bq8_offset;
        float sumf = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int isc = scale_offset + 2 * i;
            const int sc = (((sc8[isc % 8] >> (4 * (isc / 8))) & 15) | (((sc8[8 + (isc % 4)] >> (2 * (isc / 4))) & 3) << 4)) -
                           32;
            const uint8_t* b8 = x0 + (size_t)(bq8_offset + i) * 36;
            const int32_t u = qword(b8, iqs % 8);
            // the byte-wise difference (low - 4 * clear) dotted with u, as two exact dots
            const int32_t dl = dot4((vl >> (2 * i)) & 0x03030303, u, 0);
            const int32_t dh = dot4((int32_t)(((vh >> i) << 2) & 0x04040404u), u, 0);
            sumf = sumf + rdh(b8) * (float)((dl - dh) * sc);
        }
        return rdh(blk + 108) * sumf;
    } else {  // Q6_K (14): (low nibble | 2 high bits << 4) - 32 times an int8 scale
        static_assert(TYPE == 14, "native_part: unknown type");
        const int bq8_offset = 4 * (iqs / 16) + (iqs % 16) / 8, scale_offset = 8 * (iqs / 16) + (iqs % 16) / 4;
        const int vh_shift = 2 * ((iqs % 16) / 8);
        const int32_t vl = rd32(blk + 4 * iqs);
        const uint32_t vh = (uint32_t)rd32(blk + 128 + 4 * (8 * (iqs / 16) + (iqs % 8))) >> vh_shift;
        float sumf = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int sc = (int)(int8_t)blk[192 + scale_offset + 4 * i];
            const int32_t v = ((vl >> (4 * i)) & 0x0F0F0F0F) | (int32_t)(((vh >> (4 * i)) << 4) & 0x30303030u);
            const uint8_t* b8 = x0 + (size_t)(bq8_offset + 2 * i) * 36;
            const int32_t u = qword(b8, iqs % 8);
            const int32_t d = dot4(v, u, 0) - dot4(0x20202020, u, 0);
            sumf = sumf + rdh(b8) * (float)(d * sc);
        }
        return rdh(blk + 208) * sumf;
    }
}

// y[c * ldy + r] = row r . column c (times sigmoid(sg[c]) when sg is given).  Grid (ceil(n_out / 8), column
// groups); a 32-lane half wave per row; a work-group takes columns blockIdx.y, + gridDim.y, ...
template <int TYPE>
__global__ __launch_bounds__(256) void k_mmvq_native(const uint8_t* __restrict__ w, int n_in, int n_out, int n_col,
                                                     const uint8_t* __restrict__ xq, float* __restrict__ y, int ldy,
                                                     const float* __restrict__ sg) {
    using NT = NativeType<TYPE>;
    const int hw = threadIdx.x >> 5, l = threadIdx.x & 31;
    const int r = blockIdx.x * 8 + hw;
    const size_t rb = (size_t)(n_in / NT::qk) * NT::bytes, xb = (size_t)(n_in / 32) * 36;
    const uint8_t* row = w + (size_t)(r < n_out ? r : n_out - 1) * rb;  // a dead half wave reads the last row
    const int npart = (n_in / NT::qk) * NT::ipb;
    for (int c = blockIdx.y; c < n_col; c += gridDim.y) {
        const uint8_t* col = xq + (size_t)c * xb;
        float acc = 0.0f;
        for (int k = l; k < npart; k += 32) {
            const int kb = k / NT::ipb;
            acc = acc + native_part<TYPE>(row + (size_t)kb * NT::bytes, col + (size_t)kb * (NT::qk / 32) * 36,
                                          NT::step * (k % NT::ipb));
        }
        acc = acc + xor_swap<16>(acc);
        acc = acc + xor_swap<8>(acc);
        acc = acc + xor_swap<4>(acc);
        acc = acc + xor_swap<2>(acc);
        acc = acc + xor_swap<1>(acc);
        if (r < n_out && l == 0) y[(size_t)c * ldy + r] = sg ? acc * sigmoid(sg[c]) : acc;
    }
}

// y[t][j] *= sigmoid(sg[t]) for the shared rows a Q2_0 / IQ2_S down projection wrote
__global__ __launch_bounds__(256) void k_sigmoid_rows(float* __restrict__ y, int n, const float* __restrict__ sg) {
    const int t = blockIdx.y;
    const float s = sigmoid(sg[t]);
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) y[(size_t)t * n + j] = y[(size_t)t * n + j] * s;
}

// y[t][j] = y[t][j] + r[t][j]: a native shared expert's rows added after a combine that left them out (the same last
// addition the combine makes)
__global__ __launch_bounds__(256) void k_add_rows(float* __restrict__ y, const float* __restrict__ r, int n) {
    const size_t o = (size_t)blockIdx.y * n;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) y[o + j] = y[o + j] + r[o + j];
}

}  // namespace

bool native_type(int type) {
    switch (type) {
        case 8: case 2: case 6: case 20: case 23: case 11: case 12: case 13: case 14: return true;
        default: return false;
    }
}

int native_block_values(int type) {
    switch (type) {
        case 8: case 2: case 6: case 20: return 32;
        case 23: case 11: case 12: case 13: case 14: return 256;
        default: return 0;
    }
}

int64_t native_row_bytes(int type, int64_t n) {
    int bytes = 0;
    switch (type) {
        case 8: bytes = 34; break;
        case 2: case 20: bytes = 18; break;
        case 6: bytes = 22; break;
        case 23: bytes = 136; break;
        case 11: bytes = 110; break;
        case 12: bytes = 144; break;
        case 13: bytes = 176; break;
        case 14: bytes = 210; break;
        default: return -1;
    }
    const int qk = native_block_values(type);
    return (n <= 0 || n % qk) ? -1 : n / qk * bytes;
}

hipError_t launch_mmvq_native(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y,
                              int ldy, const float* sg, hipStream_t s) {
    if (!native_type(type) || n_in % native_block_values(type)) return hipErrorInvalidValue;
    const int cg = n_col < 64 ? n_col : 64;
    dim3 grid((unsigned)((n_out + 7) / 8), (unsigned)cg);
#define SMOE_NAT(T) hipLaunchKernelGGL(k_mmvq_native<T>, grid, dim3(256), 0, s, w, n_in, n_out, n_col, xq, y, ldy, sg)
    switch (type) {
        case 8: SMOE_NAT(8); break;
        case 2: SMOE_NAT(2); break;
        case 6: SMOE_NAT(6); break;
        case 20: SMOE_NAT(20); break;
        case 23: SMOE_NAT(23); break;
        case 11: SMOE_NAT(11); break;
        case 12: SMOE_NAT(12); break;
        case 13: SMOE_NAT(13); break;
        default: SMOE_NAT(14); break;
    }
#undef SMOE_NAT
    return hipGetLastError();
}

hipError_t launch_sigmoid_rows(float* y, int T, int n, const float* sg, hipStream_t s) {
    const int bx = (n + 255) / 256;
    hipLaunchKernelGGL(k_sigmoid_rows, dim3((unsigned)(bx < 16 ? bx : 16), (unsigned)T), dim3(256), 0, s, y, n, sg);
    return hipGetLastError();
}

hipError_t launch_add_rows(float* y, const float* r, int T, int n, hipStream_t s) {
    const int bx = (n + 255) / 256;
    hipLaunchKernelGGL(k_add_rows, dim3((unsigned)(bx < 16 ? bx : 16), (unsigned)T), dim3(256), 0, s, y, r, n);
    return hipGetLastError();
}

}  // namespace smoe
