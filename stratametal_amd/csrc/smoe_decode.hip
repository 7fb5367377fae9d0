// stratametal_amd/csrc/smoe_decode.hip - the decode-contract kernels of the MoE block (gfx950, wave64).
//
// Decode is a bandwidth-bound dequant-GEMV: each touched expert's 2-bit rows are streamed once with
// coalesced dwordx4 loads, unpacked in registers and multiplied with v_dot4_i32_i8 against q8_1 activations
// held in registers.  No MFMA.  The forward call is five or six launches:
//   k_router   bf16(x) staged in LDS; router logits and the shared expert's gate dot, one wave per weight row;
//              also the q8_1 images of x
//   k_topk_dispatch (up to 4 tokens) or k_topk + k_dispatch: softmax / top-k, one wave per token, then the
//              canonical stable dispatch in one work-group
//   k_q2_gu    per (touched expert | shared, 32 rows of h): gate and up rows, SwiGLU, q8_1 image of h
//   k_q2_down  per (touched expert | shared, a chunk of output rows): down rows (times the shared gate)
//   k_combine  y = routing-weighted sum of the pair rows + the shared row
// Reduction orders are fixed and restated on the host by the test oracle (oracle/smoe_oracle.c).
#include <atomic>
#include <utility>

#include "smoe_device.hpp"
#include "smoe_items.hpp"
#include "smoe_gemv.hpp"
#include "smoe_launch.hpp"

namespace smoe {

// ------------------------------------------------------------------------------------------------ phase stamps
// The decode timeline (python -m stratametal_amd.timeline): built with SMOE_STAMPS defined (lib/libsmoe_stamps.so,
// never the product library), thread 0 of a work-group writes the 100 MHz clock (s_memrealtime) into slot i of its
// 32-slot row of the stamp buffer (rows [kernel][work-group]: kernel 0 the router, 1 the fused decode launch);
// SMOE_STAMP_AFTER first waits for a value (so that the stamp marks its arrival).  Without SMOE_STAMPS every stamp
// compiles to nothing.
#if defined(SMOE_STAMPS)
__constant__ uint64_t* g_stamp;  // (constant memory: a scalar load, no wait on the vector loads in flight)
#define SMOE_STAMP_VAL(k, i, v)                                                                      \
    do {                                                                                             \
        if (threadIdx.x == 0 && g_stamp) g_stamp[((size_t)(k) * 4096 + blockIdx.x) * 32 + (i)] = (v); \
    } while (0)
#define SMOE_STAMP(k, i) SMOE_STAMP_VAL(k, i, __builtin_amdgcn_s_memrealtime())
#define SMOE_STAMP_AFTER(k, i, x)                                                 \
    do {                                                                          \
        const int stamp_v_ = __builtin_amdgcn_readfirstlane((int)(x));            \
        asm volatile("" ::"s"(stamp_v_));                                         \
        SMOE_STAMP(k, i);                                                         \
    } while (0)
#else
#define SMOE_STAMP_VAL(k, i, v) ((void)0)
#define SMOE_STAMP(k, i) ((void)0)
#define SMOE_STAMP_AFTER(k, i, x) ((void)0)
#endif

// ------------------------------------------------------------------------------------------------ Q2_0 unit
// Unit = one 36-byte double block (two Q2_0 blocks, 128 weights, dword aligned), 9 dwords:
//   w0 = {d0, codes0[0..1]}, w1..w3 = codes0[2..13], w4 = {codes0[14..15], d1}, w5..w8 = codes1[0..15].
// L = ((P0 + P1) + P2) + P3, P_h = (f32(d_w) * f32(d_x)) * (float) sumi_h, sumi_h = sum(code * q) - sum(q)
// = sum((code - 1) * q) exactly (metal/shaders/iq.metal:444-456).
__device__ __forceinline__ void load_unit(const uint8_t* p, uint32_t (&w)[9]) {
    __builtin_memcpy(w, __builtin_assume_aligned(p, 4), 36);
}

// sum(code * q) of one q8_1 block against its two code dwords a (positions 0..15) and b (16..31), with the
// block's image in the split layout: per code dword, the even codes (& 0x33333333) and the odd codes
// (>> 2, & 0x33333333) as 4-bit lanes, 16 * sdot8(codes, qh) + udot8(codes, ql).  Exact: the sums are
// integers well inside int32.
__device__ __forceinline__ int half_dot_split(uint32_t a, uint32_t b, const uint32_t* X) {
    const uint32_t M = 0x33333333u;
    const uint32_t a0 = a & M, a1 = (a >> 2) & M, b0 = b & M, b1 = (b >> 2) & M;
    int h = __builtin_amdgcn_sdot8((int)a0, (int)X[0], 0, false);
    uint32_t l = __builtin_amdgcn_udot8(a0, X[1], 0u, false);
    h = __builtin_amdgcn_sdot8((int)a1, (int)X[2], h, false);
    l = __builtin_amdgcn_udot8(a1, X[3], l, false);
    h = __builtin_amdgcn_sdot8((int)b0, (int)X[4], h, false);
    l = __builtin_amdgcn_udot8(b0, X[5], l, false);
    h = __builtin_amdgcn_sdot8((int)b1, (int)X[6], h, false);
    l = __builtin_amdgcn_udot8(b1, X[7], l, false);
    return h * 16 + (int)l;
}

// The same sum against 8 dwords of int8 q in the (codes >> 2c) & 0x03030303 byte order (the standard q8_1
// activations of the stage-API GEMV, permuted on load).
__device__ __forceinline__ int half_dot(uint32_t a, uint32_t b, const uint32_t* X) {
    const uint32_t M = 0x03030303u;
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)(a & M), (int)X[0], s, false);
    s = __builtin_amdgcn_sdot4((int)((a >> 2) & M), (int)X[1], s, false);
    s = __builtin_amdgcn_sdot4((int)((a >> 4) & M), (int)X[2], s, false);
    s = __builtin_amdgcn_sdot4((int)((a >> 6) & M), (int)X[3], s, false);
    s = __builtin_amdgcn_sdot4((int)(b & M), (int)X[4], s, false);
    s = __builtin_amdgcn_sdot4((int)((b >> 2) & M), (int)X[5], s, false);
    s = __builtin_amdgcn_sdot4((int)((b >> 4) & M), (int)X[6], s, false);
    s = __builtin_amdgcn_sdot4((int)((b >> 6) & M), (int)X[7], s, false);
    return s;
}

// Marks the weight registers as rewritten, so the compiler keeps the per-column unpacking inside the column
// loop instead of hoisting every unit's unpacked codes (4 words per code dword) and running out of registers.
template <int NIT, int MAXUPL>
__device__ __forceinline__ void pin_units(uint32_t (&w)[NIT][MAXUPL][9]) {
#pragma unroll
    for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m)
#pragma unroll
            for (int i = 0; i < 9; ++i) asm volatile("" : "+v"(w[it][m][i]));
}

// The unit's two block scales (exact hardware fp16 -> f32, subnormals included), computed once per work item.
__device__ __forceinline__ float unit_d0(const uint32_t (&w)[9]) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[0] & 0xFFFFu));
}
__device__ __forceinline__ float unit_d1(const uint32_t (&w)[9]) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[4] >> 16));
}

// Every unit's two block scales; the asm barrier keeps the conversions (and so the wait for the weight loads)
// where the call stands.
template <int NIT, int MAXUPL>
__device__ __forceinline__ void unit_scales(uint32_t (&w)[NIT][MAXUPL][9], float (&dw)[NIT][MAXUPL][2]) {
    pin_units(w);
#pragma unroll
    for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m) {
            dw[it][m][0] = unit_d0(w[it][m]);
            dw[it][m][1] = unit_d1(w[it][m]);
        }
}

// A unit's first block (P0 + P1, activation images 0 and 1) and second block (P2, P3, images 2 and 3), so that
// only two images are live at a time; q2_unit_dot's order is L = ((P0 + P1) + P2) + P3.
__device__ __forceinline__ float q2_unit_first(const uint32_t (&w)[9], float d0, const Act2& a) {
    const uint32_t c0 = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
    const uint32_t c1 = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
    const uint32_t c2 = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
    const uint32_t c3 = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
    const float P0 = (d0 * a.d[0]) * (float)(half_dot_split(c0, c1, a.q[0]) - a.sq[0]);
    const float P1 = (d0 * a.d[1]) * (float)(half_dot_split(c2, c3, a.q[1]) - a.sq[1]);
    return P0 + P1;
}
__device__ __forceinline__ float q2_unit_second(const uint32_t (&w)[9], float d1, float p01, const Act2& a) {
    const float P2 = (d1 * a.d[0]) * (float)(half_dot_split(w[5], w[6], a.q[0]) - a.sq[0]);
    const float P3 = (d1 * a.d[1]) * (float)(half_dot_split(w[7], w[8], a.q[1]) - a.sq[1]);
    return (p01 + P2) + P3;
}

__device__ __forceinline__ float q2_unit_dot(const uint32_t (&w)[9], float d0, float d1, const Act4& a) {
    const uint32_t c0 = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
    const uint32_t c1 = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
    const uint32_t c2 = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
    const uint32_t c3 = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
    const float P0 = (d0 * a.d[0]) * (float)(half_dot(c0, c1, a.q[0]) - a.sq[0]);
    const float P1 = (d0 * a.d[1]) * (float)(half_dot(c2, c3, a.q[1]) - a.sq[1]);
    const float P2 = (d1 * a.d[2]) * (float)(half_dot(w[5], w[6], a.q[2]) - a.sq[2]);
    const float P3 = (d1 * a.d[3]) * (float)(half_dot(w[7], w[8], a.q[3]) - a.sq[3]);
    return ((P0 + P1) + P2) + P3;
}

// ------------------------------------------------------------------------------------------------ router
// logits[t][row] = sum_i f32(bf16 x[t][i]) * f32(bf16 W[row][i]); row == E is the shared gate row (w_inp),
// written to sg[t].  The block stages its token tile of x as bf16 in LDS (RNE, NaN quieted), then each wave
// takes one weight row: lane l owns the 8-element chunks l, l+64, ...; accumulates them in element order from
// 0, then an xor butterfly 32..1 (oracle: or_bf16_gemv_dev).  Every bf16 product is exact in f32, so
// fmaf(x, w, acc) == acc + x * w.  `xf` (f32) or `xb` (bf16 bits) supplies x.  With `ximg`, extra blocks
// past the row blocks write the q8_1 images of the tile's x (the decode path's activations), eight q8_1 blocks
// each, beside the logits instead of before them.
// With `rprev` (the layer junction of a stack, fused; rows up to 4096): x = RMSNorm(xf + rprev) with unit
// weight, formed as k_residual_rmsnorm forms it -- every work-group takes the scale of each token of its tile in
// that order (per thread an fma chain over elements tid + 256 m, the wave butterfly, the wave sums in order)
// while its weight row (or its image values) is in flight; a row block then stages x = (xf + rprev) * scale
// from the same registers, an image block quantises its own (xf + rprev) * scale; row block 0 of each token
// tile writes x to `xout`.
// F32 (router_dtype 1, the literal benchmark configuration's f32 router): x is staged in LDS as f32 and an expert
// row is f32: lane l owns the 4-element chunks l, l+64, ... and fuses each product into its accumulator in element
// order (fmaf, one rounding per step; oracle: or_f32_gemv_dev), then the same butterfly.  The shared gate row
// stays bf16: its x values are rounded to bf16 from the f32 tile, so that sg equals the bf16 kernel's bit for bit.
// The pieces of a router work-group (k_router).
// One wave's weight row (row block rb, wave w: row 4 rb + w, clamped), loaded with every load issued.
template <int MAXC, bool F32>
struct RouterRow {
    uint4 wv[MAXC];
    float bv;
    int row;       // rows_total or more: a dead wave (stores nothing)
    bool frow;     // an f32 weight row (wave-uniform)
    int wchunks;   // 16-byte chunks of the row
};
template <int MAXC, bool F32>
__device__ __forceinline__ void router_row_load(const void* __restrict__ W, const uint16_t* __restrict__ w_inp,
                                                const float* __restrict__ bias, int H, int E, int rows_total, int rb,
                                                RouterRow<MAXC, F32>& R) {
    const int lane = threadIdx.x & 63;
    R.row = rb * 4 + (int)(threadIdx.x >> 6);
    const int rowc = min(R.row, rows_total - 1);
    R.frow = F32 && rowc < E;
    const uint8_t* wr = rowc < E ? static_cast<const uint8_t*>(W) + (size_t)rowc * H * (F32 ? 4 : 2)
                                 : reinterpret_cast<const uint8_t*>(w_inp);
    R.wchunks = R.frow ? H >> 2 : H >> 3;
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        R.wv[j] = c < R.wchunks ? *reinterpret_cast<const uint4*>(wr + 16 * c) : make_uint4(0, 0, 0, 0);
    }
    R.bv = (bias && rowc < E) ? bias[rowc] : 0.0f;  // loaded once, outside the token loop
}

// The fused junction for tokens t0 .. t0 + nt - 1, four at a time: every thread holds xf + rprev of elements
// tid + 256 m; the sums of squares in k_residual_rmsnorm's order give inv_s[t - t0]; with `stage` the scaled rows go
// to the LDS tile (bf16, or f32 with F32), and with `xout` to xout.  Every thread of the work-group calls it.
template <int NMJ, bool F32>
__device__ __forceinline__ void router_junction(const float* __restrict__ xf, const float* __restrict__ rprev, int t0,
                                                int nt, int H, float eps, bool stage, float* __restrict__ xout,
                                                uint32_t* smem, float* inv_s, float (&wsum_s)[4][4]) {
    const int tid = threadIdx.x;
    uint16_t* xs16 = reinterpret_cast<uint16_t*>(smem);
    float* xs32 = reinterpret_cast<float*>(smem);
    for (int tb = 0; tb < nt; tb += 4) {
        constexpr int NM = NMJ <= 16 ? NMJ : 1;
        float sv[4][NM];
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (tb + g < nt) {
                const float* xr = xf + (size_t)(t0 + tb + g) * H;
                const float* rr = rprev + (size_t)(t0 + tb + g) * H;
#pragma unroll
                for (int m = 0; m < NM; ++m) {  // 256 NM >= H
                    const int j = tid + 256 * m;
                    const int jc = j < H ? j : H - 1;
                    sv[g][m] = xr[jc] + rr[jc];
                    if (j < H) acc[g] = __builtin_fmaf(sv[g][m], sv[g][m], acc[g]);
                }
            }
        }
        wave_sum_xor_fast_n<4>(acc);
        if ((tid & 63) == 0) {
#pragma unroll
            for (int g = 0; g < 4; ++g) wsum_s[g][tid >> 6] = acc[g];
        }
        __syncthreads();
        if (tid < 4 && tb + tid < nt) {
            const float ss = ((wsum_s[tid][0] + wsum_s[tid][1]) + wsum_s[tid][2]) + wsum_s[tid][3];
            inv_s[tb + tid] = 1.0f / __builtin_sqrtf(ss / (float)H + eps);
        }
        __syncthreads();
        if (stage) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (tb + g < nt) {
                    const float sc = inv_s[tb + g];
                    float* xo = xout ? xout + (size_t)(t0 + tb + g) * H : nullptr;
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        const int j = tid + 256 * m;
                        if (j < H) {
                            const float v = sv[g][m] * sc;
                            if constexpr (F32) xs32[(size_t)(tb + g) * H + j] = v;
                            else xs16[(size_t)(tb + g) * H + j] = (uint16_t)f32_to_bf16(v);
                            if (xo) xo[j] = v;
                        }
                    }
                }
            }
        }
    }
}

// The token tile of x into LDS (no junction): f32 as it is with F32, else bf16 (from xf, or the bf16 bits xb),
// 8 vector loads in flight per thread.  The caller synchronises after.
template <bool F32>
__device__ __forceinline__ void router_stage(const float* __restrict__ xf, const uint16_t* __restrict__ xb, int t0,
                                             int nt, int H, uint32_t* smem) {
    if constexpr (F32) {
        const int n4 = nt * H / 4;
        for (int base = 0; base < n4; base += 256 * 8) {
            float4 f[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int g = min(base + u * 256 + (int)threadIdx.x, n4 - 1);
                f[u] = reinterpret_cast<const float4*>(xf + (size_t)t0 * H)[g];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int g = base + u * 256 + threadIdx.x;
                if (g < n4) reinterpret_cast<float4*>(smem)[g] = f[u];
            }
        }
    } else {
        const int n8 = nt * H / 8;  // groups of 8 values = one uint4 of bf16
        for (int base = 0; base < n8; base += 256 * 4) {
            uint4 v[4];
            if (xf) {
                float4 f[8];
#pragma unroll
                for (int u = 0; u < 4; ++u) {  // clamped, so that every load issues back to back
                    const int g = min(base + u * 256 + (int)threadIdx.x, n8 - 1);
                    const float4* src = reinterpret_cast<const float4*>(xf + (size_t)t0 * H) + 2 * (size_t)g;
                    f[2 * u] = src[0];
                    f[2 * u + 1] = src[1];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 a = f[2 * u], b = f[2 * u + 1];
                    v[u] = make_uint4(f32_to_bf16(a.x) | (f32_to_bf16(a.y) << 16),
                                      f32_to_bf16(a.z) | (f32_to_bf16(a.w) << 16),
                                      f32_to_bf16(b.x) | (f32_to_bf16(b.y) << 16),
                                      f32_to_bf16(b.z) | (f32_to_bf16(b.w) << 16));
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int g = base + u * 256 + threadIdx.x;
                    if (g < n8) v[u] = reinterpret_cast<const uint4*>(xb + (size_t)t0 * H)[g];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int g = base + u * 256 + threadIdx.x;
                if (g < n8) reinterpret_cast<uint4*>(smem)[g] = v[u];
            }
        }
    }
}

// The wave's row against every token of the staged tile, NG tokens at a time (NG independent chains; each token's
// chain is the same for any NG); lane 0 calls store(row, t, value) with the bias added to an expert row (row < E; row
// E is the shared gate).
template <int MAXC, bool F32, int NG = 4, class Store>
__device__ __forceinline__ void router_row_dots(const RouterRow<MAXC, F32>& R, const uint32_t* smem, int H, int E,
                                                int rows_total, int nt, bool has_bias, Store store) {
    const int lane = threadIdx.x & 63;
    const uint16_t* xs = reinterpret_cast<const uint16_t*>(smem);
    const float* xs32 = reinterpret_cast<const float*>(smem);
    const int chunks = H >> 3;
    if (R.row >= rows_total) return;
    for (int t = 0; t < nt; t += NG) {
        const int ng = min(NG, nt - t);
        float acc[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) acc[g] = 0.0f;
        if constexpr (F32) {
            if (R.frow) {
#pragma unroll
                for (int j = 0; j < MAXC; ++j) {
                    const int c = lane + 64 * j;
                    if (c < R.wchunks) {
                        const float w4[4] = {u2f(R.wv[j].x), u2f(R.wv[j].y), u2f(R.wv[j].z), u2f(R.wv[j].w)};
#pragma unroll
                        for (int g = 0; g < NG; ++g) {
                            if (g < ng) {
                                const float4 xv = *reinterpret_cast<const float4*>(xs32 + (size_t)(t + g) * H + 4 * c);
                                acc[g] = __builtin_fmaf(xv.x, w4[0], acc[g]);
                                acc[g] = __builtin_fmaf(xv.y, w4[1], acc[g]);
                                acc[g] = __builtin_fmaf(xv.z, w4[2], acc[g]);
                                acc[g] = __builtin_fmaf(xv.w, w4[3], acc[g]);
                            }
                        }
                    }
                }
            } else {  // the shared gate row: bf16(x) * bf16 w_inp, exact products in the bf16 kernel's order
#pragma unroll
                for (int j = 0; j < MAXC; ++j) {
                    const int c = lane + 64 * j;
                    if (c < chunks) {
                        const uint32_t wq[4] = {R.wv[j].x, R.wv[j].y, R.wv[j].z, R.wv[j].w};
#pragma unroll
                        for (int g = 0; g < NG; ++g) {
                            if (g < ng) {
                                const float* xr = xs32 + (size_t)(t + g) * H + 8 * c;
                                const float4 a = reinterpret_cast<const float4*>(xr)[0];
                                const float4 b = reinterpret_cast<const float4*>(xr)[1];
                                const float xv8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                                for (int q = 0; q < 4; ++q) {
                                    const float x0 = u2f(f32_to_bf16(xv8[2 * q]) << 16);
                                    const float x1 = u2f(f32_to_bf16(xv8[2 * q + 1]) << 16);
                                    acc[g] = __builtin_fmaf(x0, u2f(wq[q] << 16), acc[g]);
                                    acc[g] = __builtin_fmaf(x1, u2f(wq[q] & 0xFFFF0000u), acc[g]);
                                }
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < MAXC && !F32; ++j) {
            const int c = lane + 64 * j;
            if (c < chunks) {
                const uint32_t wq[4] = {R.wv[j].x, R.wv[j].y, R.wv[j].z, R.wv[j].w};
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    if (g < ng) {
                        const uint4 xv = *reinterpret_cast<const uint4*>(xs + (size_t)(t + g) * H + 8 * c);
                        const uint32_t xq[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            acc[g] = __builtin_fmaf(u2f(xq[q] << 16), u2f(wq[q] << 16), acc[g]);
                            acc[g] = __builtin_fmaf(u2f(xq[q] & 0xFFFF0000u), u2f(wq[q] & 0xFFFF0000u), acc[g]);
                        }
                    }
                }
            }
        }
        wave_sum_xor_fast_n<NG>(acc);
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < NG; ++g)
                if (g < ng) store(R.row, t + g, (has_bias && R.row < E) ? acc[g] + R.bv : acc[g]);
        }
    }
}

// One token against the wave's bf16 row with x read straight into registers (no LDS tile, no barrier): lane l loads
// the f32 values of its chunks l + 64 j right behind its weight loads, rounds them to bf16 as router_stage does, and
// forms the same chain and butterfly as router_row_dots for that token, so the logit is the same bits.
template <int MAXC>
struct RouterX1 {
    float4 x[MAXC][2];
};
template <int MAXC>
__device__ __forceinline__ void router_x1_load(const float* __restrict__ xr, int H, RouterX1<MAXC>& X) {
    const int lane = threadIdx.x & 63, chunks = H >> 3;
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {  // clamped: every load issues back to back
        const int c = min(lane + 64 * j, chunks - 1);
        X.x[j][0] = reinterpret_cast<const float4*>(xr)[2 * c];
        X.x[j][1] = reinterpret_cast<const float4*>(xr)[2 * c + 1];
    }
}
template <int MAXC, class Store>
__device__ __forceinline__ void router_row_dot1(const RouterRow<MAXC, false>& R, const RouterX1<MAXC>& X, int H, int E,
                                                int rows_total, bool has_bias, Store store) {
    const int lane = threadIdx.x & 63;
    const int chunks = H >> 3;
    if (R.row >= rows_total) return;
    float acc[1] = {0.0f};
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
            const uint32_t wq[4] = {R.wv[j].x, R.wv[j].y, R.wv[j].z, R.wv[j].w};
            const float4 a = X.x[j][0], b = X.x[j][1];
            const uint32_t xq[4] = {f32_to_bf16(a.x) | (f32_to_bf16(a.y) << 16), f32_to_bf16(a.z) | (f32_to_bf16(a.w) << 16),
                                    f32_to_bf16(b.x) | (f32_to_bf16(b.y) << 16), f32_to_bf16(b.z) | (f32_to_bf16(b.w) << 16)};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[0] = __builtin_fmaf(u2f(xq[q] << 16), u2f(wq[q] << 16), acc[0]);
                acc[0] = __builtin_fmaf(u2f(xq[q] & 0xFFFF0000u), u2f(wq[q] & 0xFFFF0000u), acc[0]);
            }
        }
    }
    wave_sum_xor_fast_n<1>(acc);
    if (lane == 0) store(R.row, 0, (has_bias && R.row < E) ? acc[0] + R.bv : acc[0]);
}

// The same for the f32 router (RouterRow<MAXC, true>): an f32 row's lane takes the 4-value chunks l + 64 j (x[j]), the
// shared gate row (bf16) the 8-value chunks l + 64 j (x[2 j], x[2 j + 1], rounded to bf16), as router_row_dots
// forms them for one token.
template <int MAXC>
struct RouterX1F {
    float4 x[MAXC];
};
template <int MAXC>
__device__ __forceinline__ void router_x1f_load(const float* __restrict__ xr, int H, bool frow, RouterX1F<MAXC>& X) {
    const int lane = threadIdx.x & 63;
    if (frow) {  // wave-uniform
        const int chunks = H >> 2;
#pragma unroll
        for (int j = 0; j < MAXC; ++j) X.x[j] = reinterpret_cast<const float4*>(xr)[min(lane + 64 * j, chunks - 1)];
    } else {
        const int chunks = H >> 3;
#pragma unroll
        for (int j = 0; j < MAXC / 2; ++j) {
            const int c = min(lane + 64 * j, chunks - 1);
            X.x[2 * j] = reinterpret_cast<const float4*>(xr)[2 * c];
            X.x[2 * j + 1] = reinterpret_cast<const float4*>(xr)[2 * c + 1];
        }
    }
}
template <int MAXC, class Store>
__device__ __forceinline__ void router_row_dot1f(const RouterRow<MAXC, true>& R, const RouterX1F<MAXC>& X, int H, int E,
                                                 int rows_total, bool has_bias, Store store) {
    const int lane = threadIdx.x & 63;
    if (R.row >= rows_total) return;
    float acc[1] = {0.0f};
    if (R.frow) {
#pragma unroll
        for (int j = 0; j < MAXC; ++j) {
            if (lane + 64 * j < R.wchunks) {
                const float4 xv = X.x[j];
                acc[0] = __builtin_fmaf(xv.x, u2f(R.wv[j].x), acc[0]);
                acc[0] = __builtin_fmaf(xv.y, u2f(R.wv[j].y), acc[0]);
                acc[0] = __builtin_fmaf(xv.z, u2f(R.wv[j].z), acc[0]);
                acc[0] = __builtin_fmaf(xv.w, u2f(R.wv[j].w), acc[0]);
            }
        }
    } else {
        const int chunks = H >> 3;
#pragma unroll
        for (int j = 0; j < MAXC / 2; ++j) {
            if (lane + 64 * j < chunks) {
                const uint32_t wq[4] = {R.wv[j].x, R.wv[j].y, R.wv[j].z, R.wv[j].w};
                const float4 a = X.x[2 * j], b = X.x[2 * j + 1];
                const float xv8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float x0 = u2f(f32_to_bf16(xv8[2 * q]) << 16);
                    const float x1 = u2f(f32_to_bf16(xv8[2 * q + 1]) << 16);
                    acc[0] = __builtin_fmaf(x0, u2f(wq[q] << 16), acc[0]);
                    acc[0] = __builtin_fmaf(x1, u2f(wq[q] & 0xFFFF0000u), acc[0]);
                }
            }
        }
    }
    wave_sum_xor_fast_n<1>(acc);
    if (lane == 0) store(R.row, 0, (has_bias && R.row < E) ? acc[0] + R.bv : acc[0]);
}

template <int MAXC, bool F32>
// (Every argument a row block reads before its first loads is among the first 14 dwords: the library is built with
// kernel-argument preloading, so those arrive in SGPRs with the wave, and a scalar load of a later argument, a round
// trip to memory, is waited for only after the loads are out.  The rows are E, and one more, the shared gate's, when
// w_inp is given.)
__global__ __launch_bounds__(256) void k_router(int H, int E, int T, int tok_tile, const void* __restrict__ W,
                                                 const uint16_t* __restrict__ w_inp, const float* __restrict__ bias,
                                                 const float* __restrict__ xf, const float* __restrict__ rprev,
                                                 int clear_n16, const uint16_t* __restrict__ xb,
                                                 float* __restrict__ logits, int ld_logits, float* __restrict__ sg,
                                                 uint32_t* __restrict__ ximg, int img_natural, float eps,
                                                 float* __restrict__ xout, uint4* __restrict__ clear) {
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ uint8_t qsc[8][32];
    __shared__ float inv_s[16];
    __shared__ float wsum_s[4][4];
    SMOE_STAMP(0, 2);
    const int rows_total = E + (w_inp ? 1 : 0);
    const int t0 = blockIdx.y * tok_tile;
    const int nt = min(tok_tile, T - t0);
    const int row_blocks = (rows_total + 3) / 4;
    const bool img_block = (int)blockIdx.x >= row_blocks;  // uniform
    const int tid = threadIdx.x;
    // a row block: the wave's weight row (clamped, every load issued), in flight during the staging below
    RouterRow<MAXC, F32> R;
    if (!img_block) router_row_load<MAXC, F32>(W, w_inp, bias, H, E, rows_total, blockIdx.x, R);
    // one token of f32 x without the junction (decode at batch 1): x straight into registers, no LDS tile
    const bool x1 = nt == 1 && xf != nullptr && rprev == nullptr;  // uniform
    RouterX1<MAXC> X1;
    RouterX1F<MAXC> X1F;
    if constexpr (F32) {
        if (x1 && !img_block) router_x1f_load<MAXC>(xf + (size_t)t0 * H, H, R.frow, X1F);
    } else {
        if (x1 && !img_block) router_x1_load<MAXC>(xf + (size_t)t0 * H, H, X1);
    }
    // an image block: eight q8_1 blocks of the tile's x, one per half wave (blocks past the tile, where the grid pads,
    // load block 0 and store nothing; without f32 x there are no images, and padding blocks load nothing)
    const int hw = tid >> 5;
    const int bb = ((int)blockIdx.x - row_blocks) * 8 + hw;
    const bool in_tile = bb < nt * (H >> 5);
    const size_t blk = (size_t)t0 * (H >> 5) + (in_tile ? bb : 0);
    float iv = 0.0f, ir = 0.0f;
    if (img_block && xf) {
        iv = xf[blk * 32 + (tid & 31)];
        if (rprev) ir = rprev[blk * 32 + (tid & 31)];
    }
    const bool live = img_block && ximg != nullptr && in_tile;
    // the exchange words of the kernel after this one (k_q2_moe_small), cleared: no launch reads them before it.
    // This kernel's outputs are read by work-groups on other XCDs: they are written with streaming stores, which
    // leave no dirty lines in this XCD's L2 for the end of the kernel to write back (measured: b=1 0.1 us per layer)
    typedef uint32_t zu4 __attribute__((ext_vector_type(4)));
    for (int i = ((int)blockIdx.y * (int)gridDim.x + (int)blockIdx.x) * 256 + (int)threadIdx.x; i < clear_n16;
         i += (int)(gridDim.x * gridDim.y) * 256)
        __builtin_nontemporal_store(zu4{0u, 0u, 0u, 0u}, reinterpret_cast<zu4*>(clear + i));
    // values of a row per thread of the junction: 256 NM >= H (8 values per bf16 chunk, 4 per f32 chunk)
    constexpr int NMJ = F32 ? MAXC : 2 * MAXC;
    if (NMJ <= 16 && rprev)  // the fused junction; a row block stages s * scale from registers
        router_junction<NMJ, F32>(xf, rprev, t0, nt, H, eps, !img_block, blockIdx.x == 0 ? xout : nullptr, smem, inv_s,
                                  wsum_s);
    if (img_block) {
        float v = iv;
        if (rprev && live) v = (iv + ir) * inv_s[bb / (H >> 5)];
        q8_image_store(v, live, qsc[hw], ximg + blk * kImgDw, img_natural != 0);
        return;
    }
    auto store = [&](int row, int t, float v) {
        if (row < E) __builtin_nontemporal_store(v, &logits[(size_t)(t0 + t) * ld_logits + row]);
        else __builtin_nontemporal_store(v, &sg[t0 + t]);
    };
    if (x1) {
        SMOE_STAMP(0, 3);
        if constexpr (F32) router_row_dot1f<MAXC>(R, X1F, H, E, rows_total, bias != nullptr, store);
        else router_row_dot1<MAXC>(R, X1, H, E, rows_total, bias != nullptr, store);
        SMOE_STAMP(0, 10);
        return;
    }
    if (!rprev) router_stage<F32>(xf, xb, t0, nt, H, smem);  // (F32: xf is given)
    __syncthreads();
    SMOE_STAMP(0, 3);
    router_row_dots<MAXC, F32>(R, smem, H, E, rows_total, nt, bias != nullptr, store);
    SMOE_STAMP(0, 10);
}


// One stage of a reduce-scatter over per-lane values v[0 .. N): at distance D a lane keeps the half of its items
// selected by its bit D and adds the partner's copy of them, so every item's sum is formed by exactly the additions
// of the xor butterfly (own value plus the partner's at every stage, in that stage order).
template <int D, int N>
__device__ __forceinline__ void rs_stage(float* v, int lane) {
    const bool upper = (lane & D) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float send = upper ? v[i] : v[i + N / 2];
        float recv;
        if constexpr (D == 32) recv = __shfl_xor(send, 32, kWave);
        else recv = xor_swap<D>(send);
        v[i] = (upper ? v[i + N / 2] : v[i]) + recv;
    }
}

// group_sum of NIT values at once when lpr = 4 NIT (NIT = 2 or 4): a reduce-scatter over the group's upper
// lane bits leaves lane l with the sum of value (l >> 2) & (NIT - 1), formed by exactly the butterfly's
// additions (distance lpr / 2 first), then the last two stages as in group_sum.  NIT = 1: group_sum.
template <int NIT>
__device__ __forceinline__ float group_sum_rs(float (&v)[NIT], int lpr, int lane, int& item) {
    if constexpr (NIT == 1) {
        item = 0;
        return group_sum(v[0], lpr);
    } else {
        static_assert(NIT == 2 || NIT == 4, "lpr = 4 NIT");
        if constexpr (NIT == 4) {
            rs_stage<8, 4>(v, lane);
            rs_stage<4, 2>(v, lane);
        } else {
            rs_stage<4, 2>(v, lane);
        }
        float r = v[0];
        r = r + xor_swap<2>(r);
        r = r + xor_swap<1>(r);
        item = (lane >> 2) & (NIT - 1);
        return r;
    }
}

// ------------------------------------------------------------------------------------------------ top-k
// Orderable 32-bit key of a logit: NaN ranks as -inf, -0 as +0, then the sign-flip map, so that
// key(a) > key(b) <=> a > b and key(a) == key(b) <=> a == b.
__device__ __forceinline__ uint32_t order_key(float v) {
    if (v != v) v = -__builtin_inff();
    if (v == 0.0f) v = 0.0f;
    const uint32_t b = f2u(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, kWave));
    return v;
}

// Sorting networks that order a lane's slots (checked exhaustively by the 0-1 principle): the optimal
// 19-comparator network for 8 inputs and Batcher's odd-even merge sort for 16.
struct Cmp {
    int a, b;
};
constexpr Cmp kNet8[19] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6}, {3, 7}, {0, 1}, {2, 3}, {4, 5}, {6, 7}, {2, 4}, {3, 5}, {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
constexpr Cmp kNet16[63] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {8, 9}, {10, 11}, {12, 13}, {14, 15}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {8, 10}, {9, 11}, {12, 14}, {13, 15}, {1, 2}, {5, 6}, {9, 10}, {13, 14}, {0, 4}, {1, 5}, {2, 6}, {3, 7}, {8, 12}, {9, 13}, {10, 14}, {11, 15}, {2, 4}, {3, 5}, {10, 12}, {11, 13}, {1, 2}, {3, 4}, {5, 6}, {9, 10}, {11, 12}, {13, 14}, {0, 8}, {1, 9}, {2, 10}, {3, 11}, {4, 12}, {5, 13}, {6, 14}, {7, 15}, {4, 8}, {5, 9}, {6, 10}, {7, 11}, {2, 4}, {3, 5}, {6, 8}, {7, 9}, {10, 12}, {11, 13}, {1, 2}, {3, 4}, {5, 6}, {7, 8}, {9, 10}, {11, 12}, {13, 14}};

// One wave routes one token, E <= 64 J (lane l holds e = l + 64 j, j < J).  Selection by (logit desc, id
// asc): each lane sorts its slots once by (key desc, slot asc); a round takes the wave maximum of the lanes'
// head keys, the single lane holding it wins (or, on an exact tie across lanes, the lowest candidate id) and
// pops its head.  ex_e = exp(l_e - max); S = per-lane sums in j order, then the xor butterfly 32..1;
// p_i = ex_i / S; w_i = p_i / max(sum of the k p_i in selection order, 2^-14)
// (metal/shaders/router.metal:30-132; oracle: or_route_dev).  With WTS false only the ids are formed (the
// selection never reads the probabilities).
template <int J, bool WTS = true>
__device__ __forceinline__ void route_token_t(const float* __restrict__ l, int E, int k, int32_t* __restrict__ ids,
                              float* __restrict__ wts, int32_t* ids_lds = nullptr, float* wts_lds = nullptr) {
    const int lane = threadIdx.x & 63;
    uint32_t key[J];
    float ex[J];
    int jj[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {  // all loads first, unconditional (clamped index), so they overlap
        const int e = lane + 64 * j;
        ex[j] = l[e < E ? e : E - 1];
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool valid = lane + 64 * j < E;
        float v = ex[j];
        v = (v != v || !valid) ? -__builtin_inff() : v;
        key[j] = valid ? order_key(v) : 0u;  // 0 is below every real key (order_key(-inf) = 0x007FFFFF)
        ex[j] = v;
        jj[j] = j;
        mx = __builtin_fmaxf(mx, v);
    }
    float S = 0.0f;
    if constexpr (WTS) {
        mx = wave_max_fast(mx);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool valid = lane + 64 * j < E;
            const float x = expf_smoe(ex[j] - mx);
            ex[j] = valid ? x : 0.0f;
            acc = valid ? acc + x : acc;
        }
        S = wave_sum_xor_fast(acc);
    }
    const Cmp* net = J == 8 ? kNet8 : kNet16;
    constexpr int NC = J == 8 ? 19 : 63;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int a = net[c].a, b = net[c].b;
        const bool sw = key[b] > key[a] || (key[b] == key[a] && jj[b] < jj[a]);
        const uint32_t ka = key[a], kb = key[b];
        const float xa = ex[a], xb = ex[b];
        const int ja = jj[a], jb = jj[b];
        key[a] = sw ? kb : ka;
        key[b] = sw ? ka : kb;
        if constexpr (WTS) {
            ex[a] = sw ? xb : xa;
            ex[b] = sw ? xa : xb;
        }
        jj[a] = sw ? jb : ja;
        jj[b] = sw ? ja : jb;
    }
    float my_x = 0.0f;
    int my_id = 0;
    for (int i = 0; i < k; ++i) {
        const uint32_t gk = wave_max_u32_fast(key[0]);
        const bool mine = key[0] == gk;
        const unsigned long long tied = __ballot(mine);
        int wid;
        if (__popcll(tied) == 1) {
            wid = __builtin_amdgcn_readlane(lane + 64 * jj[0], __ffsll((long long)tied) - 1);
        } else {  // an exact tie across lanes: the lowest id among the tied heads
            wid = wave_min_i32_fast(mine ? lane + 64 * jj[0] : 0x7FFFFFFF);
        }
        const int wl = wid & 63;
        if constexpr (WTS) {
            const float xw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex[0]), wl));
            if (lane == i) my_x = xw;
        }
        if (lane == i) my_id = wid;
        if (lane == wl) {  // pop the head
#pragma unroll
            for (int j = 0; j + 1 < J; ++j) {
                key[j] = key[j + 1];
                if constexpr (WTS) ex[j] = ex[j + 1];
                jj[j] = jj[j + 1];
            }
            key[J - 1] = 0u;
        }
    }
    if constexpr (WTS) {
        const float p = my_x / S;
        float ssel = 0.0f;
        for (int i = 0; i < k; ++i) ssel = ssel + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), i));
        const float den = __builtin_fmaxf(ssel, 6.103515625e-05f);
        if (lane < k && ids) {  // NULL: the ids go to LDS only
            ids[lane] = my_id;
            wts[lane] = p / den;
        }
        if (lane < k && wts_lds) wts_lds[lane] = p / den;
    }
    if (lane < k && ids_lds) ids_lds[lane] = my_id;
}

// The same selection with few instructions in the wave's serial path (route_token_t's rounds each pop a sorted head
// in every lane): theta = the k-th largest lane maximum (a bitwise search over ballot counts), so that at least k
// keys are >= theta; those candidates (C of them, usually a few more than k) are compacted into lanes c < C in
// ascending id order through `cand` (64 LDS entries of this wave); each candidate's rank is the number of
// candidates with a larger key or an equal key at a lower id, which is its selection round.  ok is false (nothing
// formed; the caller runs route_token_t) when more than 64 keys reach theta (ties across many experts).
// Lane i < k ends with the i-th selection (sel_id, and with WTS its weight, formed as route_token_t forms it:
// ex = expf(v - max) of the selected logit over S, the same lane sums and butterfly); lane c < C holds candidate c
// (cid) and its rank (crank; >= k: not selected; 64 for lanes past C).
// One step of route_fast_t's rank: the candidate in lane ^ S (within 32 lanes) counts when its (key, position) is
// ahead of this lane's.
template <int S>
__device__ __forceinline__ void rank_xor_step(uint32_t ck, uint64_t self, int lane, int& r) {
    const uint32_t pk = (uint32_t)__builtin_amdgcn_ds_swizzle((int)ck, 0x1F | (S << 10));
    r += (((uint64_t)pk << 32) | (uint32_t)(63 - (lane ^ S))) > self ? 1 : 0;
}
template <int... S>
__device__ __forceinline__ void rank_xor_steps(uint32_t ck, uint64_t self, int lane, int& r,
                                               std::integer_sequence<int, S...>) {
    (rank_xor_step<S + 1>(ck, self, lane, r), ...);
}

struct FastRoute {
    bool ok;
    int sel_id, cid, crank;
    float sel_w;
};
template <int J, bool WTS>
__device__ __forceinline__ FastRoute route_fast_t(const float* __restrict__ l, int E, int k, uint2* cand) {
    const int lane = threadIdx.x & 63;
    FastRoute R;
    float x[J];
    uint32_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        x[j] = l[e < E ? e : E - 1];
    }
    uint32_t m = 0u;
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool valid = lane + 64 * j < E;
        float v = x[j];
        v = (v != v || !valid) ? -__builtin_inff() : v;
        key[j] = valid ? order_key(v) : 0u;
        x[j] = v;
        m = max(m, key[j]);
        mx = __builtin_fmaxf(mx, v);
    }
    SMOE_STAMP_AFTER(1, 13, m);  // the logits are in registers
    // theta = the k-th largest lane maximum: at least k keys reach it, and every key above the k-th largest does
    const uint32_t th = (uint32_t)__builtin_amdgcn_readlane((int)wave_sort_desc_u32(m), k - 1);
    unsigned long long bj[J];
    int C = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        bj[j] = __ballot(key[j] >= th);
        C += __popcll(bj[j]);
    }
    R.ok = C >= k && C <= 64;
    if (!R.ok) return R;  // uniform
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (key[j] >= th) {
            const int pos = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bj[j] >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bj[j], 0u));
            cand[pos] = make_uint2(key[j], (uint32_t)(lane + 64 * j));
        }
        base += __popcll(bj[j]);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const uint2 c = cand[lane < C ? lane : 0];
    const uint32_t ck = lane < C ? c.x : 0u;
    // rank: (key, position) pairs ordered by key, then the lower position (lower id) first; up to 32 candidates by
    // independent xor exchanges (lanes past C hold key 0, below every key), beyond that one candidate per step
    int r = 0;
    const uint64_t self = ((uint64_t)ck << 32) | (uint32_t)(63 - lane);
    if (C <= 16) {
        rank_xor_steps(ck, self, lane, r, std::make_integer_sequence<int, 15>{});
    } else if (C <= 32) {
        rank_xor_steps(ck, self, lane, r, std::make_integer_sequence<int, 31>{});
    } else {
        for (int q = 0; q < C; ++q) {
            const uint32_t sk = (uint32_t)__builtin_amdgcn_readlane((int)ck, q);
            r += (sk > ck || (sk == ck && q < lane)) ? 1 : 0;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    R.cid = (int)c.y;
    R.crank = lane < C ? r : 64;
    const int to = lane < C ? r : lane;  // candidate ranks and the lanes past C: a permutation of 0..63
    R.sel_id = __builtin_amdgcn_ds_permute(4 * to, (int)c.y);
    R.sel_w = 0.0f;
    if constexpr (WTS) {
        const uint32_t skey = (uint32_t)__builtin_amdgcn_ds_permute(4 * to, (int)ck);
        mx = wave_max_fast(mx);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool valid = lane + 64 * j < E;
            const float ex = expf_smoe(x[j] - mx);
            acc = valid ? acc + ex : acc;
        }
        const float S = wave_sum_xor_fast(acc);
        const float v = u2f((skey & 0x80000000u) ? (skey & 0x7FFFFFFFu) : ~skey);  // order_key inverted
        const float p = lane < k ? expf_smoe(v - mx) / S : 0.0f;
        float ssel = 0.0f;
        for (int i = 0; i < k; ++i) ssel = ssel + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), i));
        R.sel_w = p / __builtin_fmaxf(ssel, 6.103515625e-05f);
    }
    return R;
}

// route_token_t's outputs by route_fast_t, or by route_token_t itself when the fast selection declines.
template <int J, bool WTS>
__device__ __forceinline__ void route_token_any(const float* __restrict__ l, int E, int k, int32_t* __restrict__ ids,
                                                float* __restrict__ wts, int32_t* ids_lds, float* wts_lds) {
    __shared__ uint2 s_cand[4][64];
    const int lane = threadIdx.x & 63;
    const FastRoute R = route_fast_t<J, WTS>(l, E, k, s_cand[(threadIdx.x >> 6) & 3]);
    if (!R.ok) {
        route_token_t<J, WTS>(l, E, k, ids, wts, ids_lds, wts_lds);
        return;
    }
    if (lane < k) {
        if (ids) ids[lane] = R.sel_id;
        if (WTS && wts) wts[lane] = R.sel_w;
        if (ids_lds) ids_lds[lane] = R.sel_id;
        if (WTS && wts_lds) wts_lds[lane] = R.sel_w;
    }
}

__device__ __forceinline__ void route_token(const float* __restrict__ l, int E, int k, int32_t* __restrict__ ids,
                                            float* __restrict__ wts, int32_t* ids_lds = nullptr,
                                            float* wts_lds = nullptr) {
    if (E <= 512) route_token_any<8, true>(l, E, k, ids, wts, ids_lds, wts_lds);
    else route_token_any<16, true>(l, E, k, ids, wts, ids_lds, wts_lds);
}
// The ids alone, into LDS.
__device__ __forceinline__ void route_token_ids(const float* __restrict__ l, int E, int k, int32_t* ids_lds) {
    if (E <= 512) route_token_any<8, false>(l, E, k, nullptr, nullptr, ids_lds, nullptr);
    else route_token_any<16, false>(l, E, k, nullptr, nullptr, ids_lds, nullptr);
}

// The router-margin diagnostic (metal/src/forward.cpp:441-513), one wave per token: ex and S as route_token_t forms
// them, p = ex / S, then k + 1 rounds of a wave argmax over the untaken (p desc, id asc); rounds k - 1 and k give
// stats[t] = {p_k - p_k1, l_k - l_k1, p_k, p_k1} and ids[t] = {id_k, id_k1} (oracle: or_router_margin_dev).
template <int J>
__global__ __launch_bounds__(64) void k_router_margin(const float* __restrict__ logits, int E, int k,
                                                       float* __restrict__ stats, int32_t* __restrict__ ids) {
    const int lane = threadIdx.x;
    const float* l = logits + (size_t)blockIdx.x * E;
    float key[J], p[J];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        const float v = e < E ? l[e] : -__builtin_inff();
        key[j] = v != v ? -__builtin_inff() : v;
        mx = __builtin_fmaxf(mx, key[j]);
    }
    mx = wave_max_fast(mx);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool valid = lane + 64 * j < E;
        const float x = expf_smoe(key[j] - mx);
        p[j] = valid ? x : 0.0f;
        acc = valid ? acc + x : acc;
    }
    const float S = wave_sum_xor_fast(acc);
#pragma unroll
    for (int j = 0; j < J; ++j) p[j] = lane + 64 * j < E ? p[j] / S : -__builtin_inff();  // -inf: never picked
    int pick[2] = {0, 0};
    float pk[2] = {0.0f, 0.0f}, lk[2] = {0.0f, 0.0f};
    for (int i = 0; i <= k; ++i) {
        int bj = 0;  // the lane's best untaken slot: (p desc, id asc)
#pragma unroll
        for (int j = 1; j < J; ++j) bj = p[j] > p[bj] ? j : bj;
        float bp = p[0], bk = key[0];
#pragma unroll
        for (int j = 1; j < J; ++j) {
            bp = j == bj ? p[j] : bp;
            bk = j == bj ? key[j] : bk;
        }
        const float gp = wave_max_fast(bp);
        const int wid = wave_min_i32_fast(bp == gp ? lane + 64 * bj : 0x7FFFFFFF);
        if (i >= k - 1) {
            const int at = i - (k - 1);
            pick[at] = wid;
            pk[at] = gp;
            lk[at] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bk), wid & 63));
        }
        if (lane == (wid & 63)) {
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (j == (wid >> 6)) p[j] = -__builtin_inff();
        }
    }
    if (lane == 0) {
        float* st = stats + (size_t)blockIdx.x * 4;
        st[0] = pk[0] - pk[1];
        st[1] = lk[0] - lk[1];
        st[2] = pk[0];
        st[3] = pk[1];
        ids[(size_t)blockIdx.x * 2] = pick[0];
        ids[(size_t)blockIdx.x * 2 + 1] = pick[1];
    }
}

hipError_t launch_router_margin(const float* logits, int T, int E, int k, float* stats, int32_t* ids, hipStream_t s) {
    if (E > 1024 || k < 1 || k >= E || T <= 0) return hipErrorInvalidValue;
    if (E <= 64) hipLaunchKernelGGL((k_router_margin<1>), dim3((unsigned)T), dim3(64), 0, s, logits, E, k, stats, ids);
    else if (E <= 512) hipLaunchKernelGGL((k_router_margin<8>), dim3((unsigned)T), dim3(64), 0, s, logits, E, k, stats, ids);
    else hipLaunchKernelGGL((k_router_margin<16>), dim3((unsigned)T), dim3(64), 0, s, logits, E, k, stats, ids);
    return hipGetLastError();
}

__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ logits, int ld_logits, int T, int E, int k,
                                              int32_t* __restrict__ ids, float* __restrict__ wts) {
    const int t = blockIdx.x;
    if (t >= T) return;
    route_token(logits + (size_t)t * ld_logits, E, k, ids + (size_t)t * k, wts + (size_t)t * k);
}

// ------------------------------------------------------------------------------------------------ dispatch
// Stable counting sort of the pairs i = t*k + s by expert, in one work-group of 1024 threads: counts by LDS
// atomics (order-free), offsets by an exclusive scan, ranks by a ballot match inside each wave plus per-wave
// counts in LDS, 1024 pairs per pass: position = offsets[e] + (number of earlier pairs with expert e) (oracle:
// or_dispatch).  Also the ascending list of touched experts.  An out-of-range id gets slot -1.
// Per expert (thread tid < E of a 1024-thread block, c its pair count): the exclusive offsets, the position in
// the touched list and the work-item classes of its pairs in chunks of at most `chunk` columns, longest first:
// every expert's full chunks, then the remainders of more than chunk / 2 columns, then those of more than
// chunk / 8, then the rest (each class in ascending expert order).  The longest work-groups start first, and
// the short streaming ones fill in last.  (16-bit fields: E <= 1024.)
struct ItemClasses {
    int off, fpos, fbase, rbase, total, n_touched, n_full, n_rc;
};
__device__ __forceinline__ ItemClasses item_classes(int c, int chunk, int* scratch) {
    const int flag = c > 0 ? 1 : 0;
    const int nfull = c / chunk, rem = c - nfull * chunk;
    const int wide = rem > (chunk >> 1) ? 1 : 0, mid = !wide && rem > (chunk >> 3) ? 1 : 0,
              thin = rem > 0 && !wide && !mid ? 1 : 0;
    int sc[4], tot[4];
    block_exclusive_scan_1024<4>({c, flag | (wide << 16), mid | (thin << 16), nfull}, scratch, sc, tot);
    ItemClasses ic;
    ic.off = sc[0];
    ic.fpos = sc[1] & 0xFFFF;
    ic.fbase = sc[3];
    ic.total = tot[0];
    ic.n_touched = tot[1] & 0xFFFF;
    ic.n_full = tot[3];
    const int n_wide = tot[1] >> 16, n_mid = tot[2] & 0xFFFF, n_thin = tot[2] >> 16;
    ic.n_rc = ic.n_full + n_wide + n_mid + n_thin;
    ic.rbase = wide  ? ic.n_full + (sc[1] >> 16)
               : mid ? ic.n_full + n_wide + (sc[2] & 0xFFFF)
                     : ic.n_full + n_wide + n_mid + (sc[2] >> 16);
    return ic;
}

constexpr int kDispatchIdRegs = 4;                      // passes of 1024 pairs whose ids stay in registers
constexpr int kDispatchLdsPairs = 1024 * kDispatchIdRegs;  // pairs whose perm entry is also kept in LDS
struct DispatchLds {
    int cnt[1024];
    int run[1024];
    int el[1024];
    uint8_t wcnt[16][1024];
    int scan[4 * 17];
    int perm[kDispatchLdsPairs];  // the first pairs' dispatch order, for the work items
};

// With `items`, also the work-item table: the shared expert's tokens in chunks of `sh_chunk`, then the routed
// experts' pairs in the classes of item_classes, then empty items up to max_items.
__device__ __forceinline__ void dispatch_block(const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ counts,
                               int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ slot,
                               int32_t* __restrict__ elist, int32_t* __restrict__ n_list, DispatchLds& s,
                               int4* __restrict__ items = nullptr, int max_items = 0, int T = 0, int k = 1,
                               int has_shared = 0, int chunk = 1 << 30, int sh_chunk = kShCols) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    s.cnt[tid] = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) reinterpret_cast<uint32_t*>(&s.wcnt[0][0])[w * 1024 + tid] = 0u;
    __syncthreads();
    int idr[kDispatchIdRegs];  // ids of this thread's pairs tid + 1024 j, loaded once
#pragma unroll
    for (int j = 0; j < kDispatchIdRegs; ++j) idr[j] = tid + 1024 * j < P ? ids[tid + 1024 * j] : -1;
#pragma unroll
    for (int j = 0; j < kDispatchIdRegs; ++j)
        if (idr[j] >= 0 && idr[j] < E) atomicAdd(&s.cnt[idr[j]], 1);
    for (int i = tid + kDispatchLdsPairs; i < P; i += 1024) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&s.cnt[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? s.cnt[tid] : 0;
    const int flag = c > 0 ? 1 : 0;
    const int nfull = c / chunk;
    const ItemClasses ic = item_classes(c, chunk, s.scan);
    const int off = ic.off, fpos = ic.fpos, fbase = ic.fbase, rbase = ic.rbase;
    const int total = ic.total, n_touched = ic.n_touched, n_rc = ic.n_rc;
    if (tid < E) {
        if (counts) counts[tid] = c;
        offsets[tid] = off;
        s.run[tid] = off;
        if (flag) s.el[fpos] = tid;
        if (flag && elist) elist[fpos] = tid;
    }
    if (tid == 0) {
        offsets[E] = total;
        if (n_list) *n_list = n_touched;
    }
    __syncthreads();
    const unsigned long long lt = (1ull << lane) - 1ull;
    // one pass over pairs base .. base + 1023: rank inside the wave by ballot match, then across waves
    auto rank_pass = [&](int base, int id) {
        const int i = base + tid;
        const bool valid = id >= 0 && id < E;
        const int key = valid ? id : 0;
        if (i < P && !valid) slot[i] = -1;
        unsigned long long m = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 10; ++b) {
            const bool bit = (key >> b) & 1;
            const unsigned long long bal = __ballot(bit);
            m &= bit ? bal : ~bal;
        }
        const int rank_w = __popcll(m & lt);
        const int cnt_w = __popcll(m);
        const bool leader = (m & lt) == 0ull;
        if (valid && leader) s.wcnt[wave][key] = (uint8_t)cnt_w;
        __syncthreads();
        if (valid) {
            int pos = s.run[key] + rank_w;
            for (int w = 0; w < wave; ++w) pos += s.wcnt[w][key];
            perm[pos] = i;
            slot[i] = pos;
            if (pos < kDispatchLdsPairs) s.perm[pos] = i;
        }
        __syncthreads();
        if (valid && leader) {
            atomicAdd(&s.run[key], cnt_w);
            s.wcnt[wave][key] = 0;
        }
        __syncthreads();
    };
#pragma unroll
    for (int j = 0; j < kDispatchIdRegs; ++j)
        if (1024 * j < P) rank_pass(1024 * j, idr[j]);
    for (int base = kDispatchLdsPairs; base < P; base += 1024) rank_pass(base, base + tid < P ? ids[base + tid] : -1);
    if (!items) return;
    // the shared expert's chunks first (they carry the most columns, so their work-groups start first), then the
    // routed chunks in expert order, then empty items
    const int n_sh = has_shared ? (T + sh_chunk - 1) / sh_chunk : 0;
    if (tid < E && c > 0) {
        for (int ch = 0; ch <= nfull; ++ch) {
            const int first = off + ch * chunk, n = min(chunk, c - ch * chunk);
            if (n == 0) break;
            int tk[4] = {0, 0, 0, 0};
            if (first + 4 <= kDispatchLdsPairs) {  // two loops, so that the LDS and global loads stay apart
                for (int j = 0; j < 4 && j < n; ++j) tk[j] = s.perm[first + j] / k;
            } else {
                for (int j = 0; j < 4 && j < n; ++j) tk[j] = perm[first + j] / k;
            }
            const int wi = n_sh + (ch < nfull ? fbase + ch : rbase);
            items[2 * wi] = make_int4(tid, first, n, tk[0]);
            items[2 * wi + 1] = make_int4(tk[1], tk[2], tk[3], 0);
        }
    }
    for (int wi = tid; wi < max_items; wi += 1024) {
        if (wi >= n_sh && wi < n_sh + n_rc) continue;  // a routed chunk
        int4 a = make_int4(kItemEmpty, 0, 0, 0), b = make_int4(0, 0, 0, 0);
        if (wi < n_sh) {
            const int t0 = wi * sh_chunk;
            a = make_int4(kItemShared, P + t0, min(sh_chunk, T - t0), t0);
            b = make_int4(t0 + 1, t0 + 2, t0 + 3, 0);
        }
        items[2 * wi] = a;
        items[2 * wi + 1] = b;
    }
}

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t* __restrict__ ids, int P, int E,
                                                    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                    int32_t* __restrict__ perm, int32_t* __restrict__ slot,
                                                    int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
                                                    int4* __restrict__ items, int max_items, int T, int k,
                                                    int has_shared, int chunk, int sh_chunk) {
    __shared__ DispatchLds s;
    dispatch_block(ids, P, E, counts, offsets, perm, slot, elist, n_list, s, items, max_items, T, k, has_shared, chunk,
                   sh_chunk);
}

// ------------------------------------------------------------------------------------------------ dispatch (many pairs)
// The same stable counting sort in three launches (two for at most kScanLdsChunks chunks), for many pairs: chunk c
// holds pairs 1024 c .. 1024 c + 1023.
//   k_dispatch_hist:  per chunk, the expert histogram (LDS atomics) -> hist[c][e] (for few chunks, k_dispatch_scan
//                     forms the same counts in its own LDS instead);
//   k_dispatch_scan:  one work-group: per expert the total, the offsets, the touched list and the work-item table
//                     (dispatch_block's classes and order), then hist[c][e] <- the position of chunk c's first pair
//                     of expert e (offset + the counts of the chunks before), and each expert's first full item and
//                     remainder item;
//   k_dispatch_rank:  per chunk, dispatch_block's rank pass from those positions: perm, slot, and the first four
//                     tokens of every work item.
// Within an expert the pairs stay in ascending pair order: chunks in order, and inside a chunk by ballot ranks.
constexpr int kDispatchChunk = 1024;
// k_dispatch_scan counts the pairs itself, in LDS, for at most this many chunks (at 512 tokens x top-10: 5 chunks,
// one launch fewer; at 40 chunks the one work-group's 40 id loads and LDS atomics per thread cost more than the
// separate k_dispatch_hist launch)
constexpr int kScanLdsChunks = 8;
constexpr int kScanLdsCounts = kScanLdsChunks * 1024;

__global__ __launch_bounds__(1024) void k_dispatch_hist(const int32_t* __restrict__ ids, int P, int E,
                                                         int32_t* __restrict__ hist) {
    __shared__ int cnt[1024];
    const int tid = threadIdx.x, c = blockIdx.x;
    cnt[tid] = 0;
    const int i = c * kDispatchChunk + tid;
    const int e = i < P ? ids[i] : -1;
    __syncthreads();
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    __syncthreads();
    if (tid < E) hist[(size_t)c * E + tid] = cnt[tid];
}

__global__ __launch_bounds__(1024) void k_dispatch_scan(int32_t* __restrict__ hist, int n_chunks, int P, int E,
                                                         int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
                                                         int4* __restrict__ items, int32_t* __restrict__ item_of,
                                                         int max_items, int T, int has_shared, int chunk, int sh_chunk,
                                                         const int32_t* __restrict__ ids) {
    __shared__ int scan[4 * 17];
    __shared__ int lh[kScanLdsCounts];
    const int tid = threadIdx.x;
    // with `ids`: the chunks' expert counts formed here in LDS (n_chunks * E <= kScanLdsCounts; LDS atomics, whose
    // order does not change a count), instead of read from hist as k_dispatch_hist left them
    const bool in_lds = ids != nullptr;
    if (in_lds) {
        for (int i = tid; i < n_chunks * E; i += 1024) lh[i] = 0;
        __syncthreads();
        for (int i0 = 0; i0 < P; i0 += 8 * 1024) {  // eight loads in flight per thread
            int e[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + 1024 * u + tid;
                e[u] = i < P ? ids[i] : -1;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + 1024 * u + tid;
                if (e[u] >= 0 && e[u] < E) atomicAdd(&lh[(i / kDispatchChunk) * E + e[u]], 1);
            }
        }
        __syncthreads();
    }
    int c = 0;
    if (tid < E && in_lds) {
        for (int ch = 0; ch < n_chunks; ++ch) c += lh[ch * E + tid];
    } else if (tid < E) {  // the chunks' counts, eight loads in flight at a time
        int ch = 0;
        for (; ch + 8 <= n_chunks; ch += 8) {
            int h[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) h[u] = hist[(size_t)(ch + u) * E + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u) c += h[u];
        }
        for (; ch < n_chunks; ++ch) c += hist[(size_t)ch * E + tid];
    }
    const int flag = c > 0 ? 1 : 0;
    const int nfull = c / chunk;
    const ItemClasses ic = item_classes(c, chunk, scan);
    const int off = ic.off, fpos = ic.fpos, fbase = ic.fbase, rbase = ic.rbase;
    const int total = ic.total, n_touched = ic.n_touched, n_rc = ic.n_rc;
    const int n_sh = has_shared ? (T + sh_chunk - 1) / sh_chunk : 0;
    if (tid < E) {
        if (counts) counts[tid] = c;
        offsets[tid] = off;
        if (flag && elist) elist[fpos] = tid;
        item_of[tid] = n_sh + fbase;      // the expert's first full item
        item_of[E + tid] = n_sh + rbase;  // its remainder item
        int run = off;
        int ch = 0;
        if (in_lds) {
            for (; ch < n_chunks; ++ch) {
                hist[(size_t)ch * E + tid] = run;
                run += lh[ch * E + tid];
            }
        }
        for (; ch + 8 <= n_chunks; ch += 8) {
            int h[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) h[u] = hist[(size_t)(ch + u) * E + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                hist[(size_t)(ch + u) * E + tid] = run;
                run += h[u];
            }
        }
        for (; ch < n_chunks; ++ch) {
            const int h = hist[(size_t)ch * E + tid];
            hist[(size_t)ch * E + tid] = run;
            run += h;
        }
        if (c > 0 && items) {  // the tokens are filled in by k_dispatch_rank
            for (int q = 0; q <= nfull; ++q) {
                const int first = off + q * chunk, n = min(chunk, c - q * chunk);
                if (n == 0) break;
                const int wi = n_sh + (q < nfull ? fbase + q : rbase);
                items[2 * wi] = make_int4(tid, first, n, 0);
                items[2 * wi + 1] = make_int4(0, 0, 0, 0);
            }
        }
    }
    if (tid == 0) {
        offsets[E] = total;
        if (n_list) *n_list = n_touched;
    }
    if (!items) return;
    for (int wi = tid; wi < max_items; wi += 1024) {
        if (wi >= n_sh && wi < n_sh + n_rc) continue;  // a routed chunk
        int4 a = make_int4(kItemEmpty, 0, 0, 0), b = make_int4(0, 0, 0, 0);
        if (wi < n_sh) {
            const int t0 = wi * sh_chunk;
            a = make_int4(kItemShared, P + t0, min(sh_chunk, T - t0), t0);
            b = make_int4(t0 + 1, t0 + 2, t0 + 3, 0);
        }
        items[2 * wi] = a;
        items[2 * wi + 1] = b;
    }
}

struct RankLds {
    int run[1024];
    uint8_t wcnt[16][1024];
};
__global__ __launch_bounds__(1024) void k_dispatch_rank(const int32_t* __restrict__ ids, int P, int E,
                                                         const int32_t* __restrict__ base, const int32_t* __restrict__ counts,
                                                         const int32_t* __restrict__ offsets,
                                                         const int32_t* __restrict__ item_of, int32_t* __restrict__ perm,
                                                         int32_t* __restrict__ slot, int4* __restrict__ items, int k,
                                                         int chunk) {
    __shared__ RankLds s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
    const int i = c * kDispatchChunk + tid;
    const int id = i < P ? ids[i] : -1;
    s.run[tid] = tid < E ? base[(size_t)c * E + tid] : 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) reinterpret_cast<uint32_t*>(&s.wcnt[0][0])[w * 1024 + tid] = 0u;
    const bool valid = id >= 0 && id < E;
    const int key = valid ? id : 0;
    if (i < P && !valid) slot[i] = -1;
    __syncthreads();
    // rank inside the wave by ballot match on the 10 id bits, then the counts of the earlier waves
    unsigned long long m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
        const bool bit = (key >> b) & 1;
        const unsigned long long bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    const unsigned long long lt = (1ull << lane) - 1ull;
    const int rank_w = __popcll(m & lt);
    if (valid && (m & lt) == 0ull) s.wcnt[wave][key] = (uint8_t)__popcll(m);
    __syncthreads();
    if (!valid) return;
    int pos = s.run[key] + rank_w;
    for (int w = 0; w < wave; ++w) pos += s.wcnt[w][key];
    perm[pos] = i;
    slot[i] = pos;
    if (!items) return;
    const int j = pos - offsets[key];  // position inside the expert
    const int q = j / chunk, jj = j - q * chunk;
    if (jj < 4) {  // one of the first four pairs of its work item: the item's token field
        const int wi = q < counts[key] / chunk ? item_of[key] + q : item_of[E + key];
        reinterpret_cast<int32_t*>(items)[8 * wi + 3 + jj] = i / k;
    }
}

// ------------------------------------------------------------------------------------------------ route (fused)
// The decode call's middle for up to 4 tokens, one work-group of 256 threads: wave t routes token t
// (route_token, its ids also into LDS), then the dispatch of the T * k <= 256 pairs with the results of
// dispatch_block: thread i owns experts 4i .. 4i + 3 for the counts, offsets and touched list (one block
// scan), thread p owns pair p, whose rank within its expert is the number of earlier pairs with the same
// expert; the work-item table as dispatch_block's (shared chunks first).
constexpr int kSmallPairs = 256;
struct SmallDispatchLds {
    int ids[kSmallPairs];
    float wts[kSmallPairs];
    int perm[kSmallPairs];
    int cnt[1024];
    int off[1024];
    int el[1024];  // touched experts, ascending
    int scan[3 * 4];
    int n_touched;
};

// Every thread of a 256-thread work-group calls it.  With `store` false nothing is written to global memory and
// the work-item table is not built: the work-group keeps the routing in LDS (s.ids, s.wts, s.cnt, s.off, s.el,
// s.n_touched, s.perm = pair of each dispatch position) for its own use.  Ends with a barrier.
__device__ __forceinline__ void small_route_dispatch(const float* __restrict__ logits, int T, int E, int k, bool store,
                                                     int32_t* __restrict__ ids, float* __restrict__ wts,
                                                     int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                     int32_t* __restrict__ perm, int32_t* __restrict__ slot,
                                                     int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
                                                     int4* __restrict__ items, int max_items, int has_shared, int chunk,
                                                     int sh_chunk, SmallDispatchLds& s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int P = T * k;
#pragma unroll
    for (int j = 0; j < 4; ++j) s.cnt[tid + 256 * j] = 0;
    if (wave < T) route_token(logits + (size_t)wave * E, E, k, store ? ids + (size_t)wave * k : nullptr,
                              store ? wts + (size_t)wave * k : nullptr, s.ids + wave * k, s.wts + wave * k);
    __syncthreads();
    const int id = tid < P ? s.ids[tid] : -1;
    const bool valid = id >= 0 && id < E;
    if (valid) atomicAdd(&s.cnt[id], 1);
    if (store && tid < P && !valid) slot[tid] = -1;
    __syncthreads();
    // experts 4 tid .. 4 tid + 3: counts, touched flags and item chunks, then one scan of the three sums
    int c[4], nch[4];
    int v[3] = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        c[j] = e < E ? s.cnt[e] : 0;
        nch[j] = c[j] > 0 ? (c[j] - 1) / chunk + 1 : 0;
        v[0] += c[j];
        v[1] += c[j] > 0 ? 1 : 0;
        v[2] += nch[j];
    }
    int excl[3], total[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const int incl = wave_inclusive_scan(v[q]);
        if (lane == 63) s.scan[4 * q + wave] = incl;
        excl[q] = incl - v[q];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const int w0 = s.scan[4 * q], w1 = s.scan[4 * q + 1], w2 = s.scan[4 * q + 2], w3 = s.scan[4 * q + 3];
        excl[q] += (wave > 0 ? w0 : 0) + (wave > 1 ? w1 : 0) + (wave > 2 ? w2 : 0);
        total[q] = w0 + w1 + w2 + w3;
    }
    const int n_sh = has_shared ? (T + sh_chunk - 1) / sh_chunk : 0;
    const int n_rc = total[2];
    int run_off = excl[0], run_flag = excl[1], run_item = excl[2];
    int first_of[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        first_of[j] = run_off;
        if (e < E) {
            s.off[e] = run_off;
            if (c[j] > 0) s.el[run_flag] = e;
            if (store) {
                if (counts) counts[e] = c[j];
                offsets[e] = run_off;
                if (c[j] > 0 && elist) elist[run_flag] = e;
            }
        }
        run_off += c[j];
        run_flag += c[j] > 0 ? 1 : 0;
    }
    if (tid == 0) {
        s.n_touched = total[1];
        if (store) {
            offsets[E] = total[0];
            if (n_list) *n_list = total[1];
        }
    }
    __syncthreads();
    if (valid) {  // rank = earlier pairs with the same expert (ascending pair order within an expert)
        int rank = 0;
        for (int q = 0; q < tid; ++q) rank += s.ids[q] == id ? 1 : 0;
        const int pos = s.off[id] + rank;
        s.perm[pos] = tid;
        if (store) {
            perm[pos] = tid;
            slot[tid] = pos;
        }
    }
    __syncthreads();
    if (!store || !items) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        for (int ch = 0; ch < nch[j]; ++ch) {
            const int first = first_of[j] + ch * chunk, n = min(chunk, c[j] - ch * chunk);
            int tk[4] = {0, 0, 0, 0};
            for (int q = 0; q < 4 && q < n; ++q) tk[q] = s.perm[first + q] / k;
            items[2 * (n_sh + run_item + ch)] = make_int4(4 * tid + j, first, n, tk[0]);
            items[2 * (n_sh + run_item + ch) + 1] = make_int4(tk[1], tk[2], tk[3], 0);
        }
        run_item += nch[j];
    }
    for (int wi = tid; wi < max_items; wi += 256) {
        if (wi >= n_sh && wi < n_sh + n_rc) continue;  // a routed chunk
        int4 a = make_int4(kItemEmpty, 0, 0, 0), b = make_int4(0, 0, 0, 0);
        if (wi < n_sh) {
            const int t0 = wi * sh_chunk;
            a = make_int4(kItemShared, P + t0, min(sh_chunk, T - t0), t0);
            b = make_int4(t0 + 1, t0 + 2, t0 + 3, 0);
        }
        items[2 * wi] = a;
        items[2 * wi + 1] = b;
    }
}

__global__ __launch_bounds__(256) void k_topk_dispatch(const float* __restrict__ logits, int T, int E, int k,
                                                        int32_t* __restrict__ ids, float* __restrict__ wts,
                                                        int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                        int32_t* __restrict__ perm, int32_t* __restrict__ slot,
                                                        int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
                                                        int4* __restrict__ items, int max_items, int has_shared,
                                                        int chunk, int sh_chunk) {
    __shared__ SmallDispatchLds s;
    small_route_dispatch(logits, T, E, k, true, ids, wts, counts, offsets, perm, slot, elist, n_list, items, max_items,
                         has_shared, chunk, sh_chunk, s);
}

// ------------------------------------------------------------------------------------------------ expert GEMV
// Row geometry: dpr = n_in / 128 units; lpr = lanes per row; upl = units per lane; rpi = 64 / lpr rows per
// wave pass.  Lane (group, l) handles units g = l + lpr * m (m < upl) of its row.
struct RowGeo {
    int dpr, lpr, upl, rpi;
};
__device__ __forceinline__ RowGeo row_geo(int n_in) {
    RowGeo r;
    r.dpr = n_in >> 7;
    r.lpr = lanes_per_row(r.dpr);
    r.upl = r.dpr / r.lpr;
    r.rpi = 64 / r.lpr;
    return r;
}

constexpr int kGuCols = 8;

// Gate/up + SwiGLU + q8_1 image of h.  Grid (Fmax / 32, max work items), 4 waves.  Wave w computes gate rows
// [32 hb + 8 w, +8) (rows rho 0..7) and the same up rows (rho 8..15); the item's columns are processed in
// stages of kGuCols: their x images are copied to LDS, every column's row values parked in LDS by the group
// leaders, then each half wave quantises one column's 32 h values into image block hb.
// Pieces of a gate/up work unit (work item `item`, rows 32 hb .. + 31 of gate and of up), shared by the one-shot
// kernels and the pipelined one.  Weight units: every load unconditional (a dead slot reloads the row's first
// unit), so that the loads in flight are counted exactly.
template <int NIT, int MAXUPL>
__device__ __forceinline__ void gu_load_weights(const Item& item, int hb, const uint8_t* __restrict__ gate_exps,
                                                const uint8_t* __restrict__ up_exps, const uint8_t* __restrict__ gate_sh,
                                                const uint8_t* __restrict__ up_sh, int H, int F,
                                                uint32_t (&w)[NIT][MAXUPL][9]) {
    const RowGeo G = row_geo(H);
    const size_t rb = (size_t)G.dpr * 36;
    const uint8_t* g0 = item.shared ? gate_sh : gate_exps + (size_t)item.e * F * rb;
    const uint8_t* u0 = item.shared ? up_sh : up_exps + (size_t)item.e * F * rb;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / G.lpr, l = lane - grp * G.lpr;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int rho = min(it * G.rpi + grp, 15);  // 0..15 within the wave (a dead pass repeats row 15)
        const int r = 32 * hb + 8 * wave + (rho & 7);
        const uint8_t* rowp = (rho < 8 ? g0 : u0) + (size_t)r * rb;
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m) load_unit(rowp + (size_t)(m < G.upl ? l + G.lpr * m : l) * 36, w[it][m]);
    }
}

// The unit's loads: the first column batch's image loads (L2) into registers when their rows need no memory read,
// then the weight loads (HBM), so that committing the images waits for the image loads alone.  Returns whether
// the images were issued (else gu_commit stages them itself).
template <int NIT, int MAXUPL>
__device__ __forceinline__ bool gu_issue(const Item& item, int hb, const uint8_t* __restrict__ gate_exps,
                                         const uint8_t* __restrict__ up_exps, const uint8_t* __restrict__ gate_sh,
                                         const uint8_t* __restrict__ up_sh, const uint32_t* __restrict__ ximg, int H,
                                         int F, StagePieces& sp, uint32_t (&w)[NIT][MAXUPL][9]) {
    const int nc0 = min(kGuCols, item.ncol);
    const bool direct = stage_direct(item, 0, nc0, true);
    if (direct) stage_issue_direct<256>(sp, ximg, H >> 5, 0, nc0, kGuCols, 0, item, true);
    __builtin_amdgcn_sched_barrier(0);
    gu_load_weights<NIT, MAXUPL>(item, hb, gate_exps, up_exps, gate_sh, up_sh, H, F, w);
    __builtin_amdgcn_sched_barrier(0);
    return direct;
}

// The first column batch's images into `smem` (the caller synchronises after).
__device__ __forceinline__ void gu_commit(const Item& item, bool direct, const StagePieces& sp, uint32_t* smem,
                                          const uint32_t* __restrict__ ximg, const int32_t* __restrict__ perm, int k,
                                          int H) {
    const int qb = H >> 5, nc0 = min(kGuCols, item.ncol);
    if (direct) stage_commit_direct(sp, smem);
    else stage_images<256>(smem, ximg, qb, 0, nc0, kGuCols, item, perm, k, true, 0, 4 * 256);
    stage_images<256>(smem, ximg, qb, 0, nc0, kGuCols, item, perm, k, true, 4 * 256);  // rounds beyond the first
}

// Dots of every column of the unit (the first batch already in `smem`, later batches staged here), SwiGLU, q8_1
// image of h.  PRESTAGED: the images of every token are in LDS, token t in column slot t (batches of at most 4
// tokens).
template <int NIT, int MAXUPL, bool PRESTAGED, bool HQ = false>
__device__ __forceinline__ void gu_compute(const Item& item, int hb, uint32_t* smem, uint32_t (&w)[NIT][MAXUPL][9],
                                           const uint32_t* __restrict__ ximg, const int32_t* __restrict__ perm, int k,
                                           int H, uint32_t* __restrict__ himg, int h_blocks, float (&rowv)[kGuCols][64],
                                           uint8_t (&qsc)[8][32], uint64_t* __restrict__ xchg, const StageOut& so,
                                           int F, int Fs) {
    const RowGeo G = row_geo(H);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / G.lpr, l = lane - grp * G.lpr;
    const int qb = H >> 5;
    float dw[NIT][MAXUPL][2];
    unit_scales(w, dw);
    SMOE_STAMP(1, 7);  // the weights are in registers

    for (int c0 = 0; c0 < item.ncol; c0 += kGuCols) {
        const int nc = min(kGuCols, item.ncol - c0);
        if (!PRESTAGED && c0 > 0) {
            stage_images<256>(smem, ximg, qb, c0, nc, kGuCols, item, perm, k, true);
            __syncthreads();
        }
        for (int c = 0; c < nc; ++c) {
            const uint32_t* xt = smem + (size_t)(PRESTAGED ? item_token_head(item, c) : c) * qb * kImgLdsDw;
            pin_units(w);
            float acc[NIT];
#pragma unroll
            for (int m = 0; m < MAXUPL; ++m) {
                if (m < G.upl) {
                    const uint32_t* img = xt + (size_t)(l + G.lpr * m) * kUnitLdsDw;
                    float p01[NIT];
                    // both image halves before the dots (one LDS round trip)
                    Act2 a, b;
                    load_act_img2(img, a);
                    load_act_img2(img + 2 * kImgDw, b);
#pragma unroll
                    for (int it = 0; it < NIT; ++it) p01[it] = q2_unit_first(w[it][m], dw[it][m][0], a);
#pragma unroll
                    for (int it = 0; it < NIT; ++it) {
                        const float L = q2_unit_second(w[it][m], dw[it][m][1], p01[it], b);
                        acc[it] = m == 0 ? L : acc[it] + L;
                    }
                }
            }
            int it;
            const float v = group_sum_rs<NIT>(acc, G.lpr, lane, it);
            const int rho = it * G.rpi + grp;
            if (rho < 16 && (l & 3) == 0 && (NIT > 1 || l == 0))
                rowv[c][(rho < 8 ? 0 : 32) + 8 * wave + (rho & 7)] = v;
        }
        __syncthreads();
        if (2 * wave < nc) {  // the waves whose half waves own live columns
            const int hw = threadIdx.x >> 5;  // half wave = column
            const bool live_c = hw < nc;
            const int i = lane & 31;
            const float h = live_c ? silu_mul(rowv[hw][i], rowv[hw][32 + i]) : 0.0f;
            const int row = item.first + c0 + (live_c ? hw : 0);
            if (xchg)
                q8_image_store(h, live_c, qsc[hw], nullptr, false, xchg + ((size_t)row * h_blocks + hb) * kXchgSlots);
            else
                q8_image_store(h, live_c, qsc[hw], himg + ((size_t)row * h_blocks + hb) * kImgDw);
            if constexpr (HQ)  // the trace's stages: gate and up dots, the standard q8_1 block of h (k_prep's quantiser)
                stage_store(so, row, hb, live_c ? rowv[hw][i] : 0.0f, live_c ? rowv[hw][32 + i] : 0.0f, h, live_c, F, Fs);
        }
        if (c0 + kGuCols < item.ncol) __syncthreads();
    }
}

// The work-group's item, one unit (rows block hb): `smem` is the kernel's dynamic LDS (the image staging area).
// With `xchg` the h images go to the tagged exchange words instead of himg.  `sync_after_loads` (PRESTAGED): the
// staged images are published by a barrier here, after the weight loads were issued.
template <int NIT, int MAXUPL, bool PRESTAGED = false, bool HQ = false>
__device__ __forceinline__ void q2_gu_item(const Item& item, int hb, uint32_t* smem, const uint8_t* __restrict__ gate_exps,
                                           const uint8_t* __restrict__ up_exps, const uint8_t* __restrict__ gate_sh,
                                           const uint8_t* __restrict__ up_sh, const uint32_t* __restrict__ ximg,
                                           const int32_t* __restrict__ perm, int k, int H, int F,
                                           uint32_t* __restrict__ himg, int h_blocks, uint64_t* __restrict__ xchg = nullptr,
                                           StageOut so = {}, int Fs = 0, bool sync_after_loads = false) {
    __shared__ float rowv[kGuCols][64];
    __shared__ uint8_t qsc[8][32];
    uint32_t w[NIT][MAXUPL][9];
    if constexpr (PRESTAGED) {
        gu_load_weights<NIT, MAXUPL>(item, hb, gate_exps, up_exps, gate_sh, up_sh, H, F, w);
        if (sync_after_loads) __syncthreads();  // uniform
    } else {
        StagePieces sp;
        const bool direct = gu_issue<NIT, MAXUPL>(item, hb, gate_exps, up_exps, gate_sh, up_sh, ximg, H, F, sp, w);
        gu_commit(item, direct, sp, smem, ximg, perm, k, H);
        __syncthreads();
    }
    gu_compute<NIT, MAXUPL, PRESTAGED, HQ>(item, hb, smem, w, ximg, perm, k, H, himg, h_blocks, rowv, qsc, xchg, so, F,
                                           Fs);
}

template <int NIT, int MAXUPL, bool HQ>
// (What a routed item's work-group reads before its image and weight loads is in the first 14 dwords, which arrive
// preloaded in SGPRs: the item's entry is the one scalar round trip before those loads; the shared expert's weights
// and the later arguments are scalar loads waited for where they are used.)
__global__ __launch_bounds__(256) void k_q2_gu(const int4* __restrict__ items, const uint32_t* __restrict__ ximg,
                                                const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps,
                                                const uint64_t* __restrict__ eptr, int H, int F, int Fs, int k,
                                                const uint8_t* __restrict__ gate_sh, const uint8_t* __restrict__ up_sh,
                                                const int32_t* __restrict__ perm, uint32_t* __restrict__ himg,
                                                int h_blocks, const StageOut so) {
    extern __shared__ __align__(16) uint32_t smem[];
    Item item;
    if (!work_item_uniform(items, blockIdx.y, item)) return;
    if ((int)blockIdx.x * 32 >= (item.shared ? Fs : F)) return;
    if (eptr && !item.shared) {  // a pointer per routed item: its blob holds the gate rows, then the up rows
        gate_exps = reinterpret_cast<const uint8_t*>(eptr[item.e]);
        up_exps = gate_exps + (size_t)F * ((size_t)(H >> 7) * 36);
        item.e = 0;
    }
    q2_gu_item<NIT, MAXUPL, false, HQ>(item, blockIdx.x, smem, gate_exps, up_exps, gate_sh, up_sh, ximg, perm, k, H, F,
                                       himg, h_blocks, nullptr, so, Fs);
}

// Gate/up of a batch of at most kShCols tokens straight from the logits, with no route kernel before it.  Grid
// (Fmax / 32, max work items + 1).  Every work-group first loads the images of all T tokens (they reach LDS while
// the routing runs).  The shared expert's work-groups (item 0 with a shared expert) start the expert at once;
// every other work-group routes the batch itself (ids only, one wave per token) and takes as its item the
// (y - n_sh)-th touched expert in ascending order, with its pairs in ascending pair order -- the item
// dispatch_block writes there.  The last row of work-groups (y = max_items) only routes, dispatches and writes
// the routing, the dispatch and the work-item table for the kernels after it.
struct GuRouteLds {
    int ids[kSmallPairs];
    int lt[kSmallPairs];     // pairs with a smaller expert id
    int first[kSmallPairs];  // 1 for the first pair of its expert
    int item[8];             // e (-1: none), first, ncol, tk[0..3]
};
// One work-group of k_q2_gu_route / k_q2_moe_small: work item y (shared first, then the touched experts in
// ascending order; y = max_items is the writer), rows block hb of h.  Returns whether it computed a unit (false:
// no expert for this item, or rows past the expert's width); with `xchg` the h images go to the exchange words.
// The routing and the work item of a gate/up work-group of the small-batch launches (item y: the shared expert
// first, then the touched experts in ascending order, with their pairs in ascending pair order -- the item
// dispatch_block writes there), from the logits `lg` ([T][E], global memory or LDS; wave t routes token t).
// `commit` runs after the routing and before the barrier that publishes it (the caller's staging of the x images).
// Returns whether the work-group has an expert (uniform; false after the barrier when its item has none).  `synced`
// false: the one-token fast path returned without that barrier (every wave routed the token itself), and the caller
// synchronises before it reads what `commit` wrote.
template <class Commit>
__device__ __forceinline__ bool gu_route_item(int y, GuRouteLds& L, const float* lg, int T, int E, int k,
                                              int has_shared, Item& item, Commit commit, bool& synced) {
    const int n_sh = has_shared ? 1 : 0;
    const int tid = threadIdx.x, wave = tid >> 6;
    const bool shared_wg = y < n_sh;
    const int P = T * k;
    synced = true;
    // one token: every wave routes it (the same selection in each, from the same logits) and takes the item from
    // the candidates (the y-th selected id in ascending order, its one pair at dispatch position y), so that no
    // barrier stands between the routing and the item's weight loads; when the fast selection declines (in every
    // wave alike), wave 0 writes the ids to L.ids and the general path below finds the item
    const bool one = !shared_wg && T == 1 && k <= 64;
    if (one) {
        __shared__ uint2 s_cand1[4][64];
        const FastRoute R = E <= 512 ? route_fast_t<8, false>(lg, E, k, s_cand1[wave])
                                     : route_fast_t<16, false>(lg, E, k, s_cand1[wave]);
        SMOE_STAMP(1, 14);
        if (R.ok) {  // uniform over the work-group
            const bool sel = R.crank < k;
            const unsigned long long sm = __ballot(sel);
            const int yc = __builtin_amdgcn_mbcnt_hi((uint32_t)(sm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)sm, 0u));
            const unsigned long long own = __ballot(sel && yc == y - n_sh);
            commit();
            synced = false;
            if (own == 0ull) return false;  // uniform: no expert for this item
            item.shared = false;
            item.e = __builtin_amdgcn_readlane(R.cid, __builtin_ctzll(own));
            item.first = y - n_sh;
            item.ncol = 1;
            item.tok0 = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) item.tk[c] = 0;
            return true;
        }
        if (wave == 0) {
            if (E <= 512) route_token_t<8, false>(lg, E, k, nullptr, nullptr, L.ids);
            else route_token_t<16, false>(lg, E, k, nullptr, nullptr, L.ids);
        }
    } else if (!shared_wg && wave < T) {
        route_token_ids(lg + (size_t)wave * E, E, k, L.ids + wave * k);
    }
    commit();
    __syncthreads();
    if (shared_wg) {
        item.shared = true;
        item.e = kItemShared;
        item.first = P;
        item.ncol = T;
        item.tok0 = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) item.tk[c] = c;
    } else if (P <= 64) {
        // every wave on its own, lane p holding pair p: counts by broadcasting each pair's id (no LDS loop)
        const int lane = tid & 63;
        const int id = lane < P ? L.ids[lane] : 0x7FFFFFFF;
        int lt = 0, cnt = 0, fst = 1;
        for (int q = 0; q < P; ++q) {
            const int o = __builtin_amdgcn_readlane(id, q);
            lt += o < id ? 1 : 0;
            cnt += o == id ? 1 : 0;
            fst = (q < lane && o == id) ? 0 : fst;
        }
        const unsigned long long firsts = __ballot(lane < P && fst);
        int rank = 0;  // touched experts below id
        for (unsigned long long m = firsts; m; m &= m - 1) {
            const int q = __builtin_ctzll(m);
            rank += __builtin_amdgcn_readlane(id, q) < id ? 1 : 0;
        }
        const unsigned long long own = __ballot(lane < P && fst && rank == y - n_sh);
        if (own == 0ull) return false;  // uniform: no expert for this item
        const int ol = __builtin_ctzll(own);
        item.shared = false;
        item.e = __builtin_amdgcn_readlane(id, ol);
        item.first = __builtin_amdgcn_readlane(lt, ol);
        item.ncol = __builtin_amdgcn_readlane(cnt, ol);  // at most T <= 4: a token picks an expert once
        unsigned long long pm = __ballot(lane < P && id == item.e);  // its pairs, ascending
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            item.tk[c] = pm ? __builtin_ctzll(pm) / k : 0;
            pm &= pm - 1;
        }
        item.tok0 = item.tk[0];
    } else {
        const int id = tid < P ? L.ids[tid] : 0;
        if (tid < P) {
            int lt = 0, fst = 1;
            for (int q = 0; q < P; ++q) {
                const int o = L.ids[q];
                lt += o < id ? 1 : 0;
                fst = (q < tid && o == id) ? 0 : fst;
            }
            L.lt[tid] = lt;
            L.first[tid] = fst;
        }
        if (tid == 0) L.item[0] = -1;
        __syncthreads();
        const int yr = y - n_sh;
        if (tid < P && L.first[tid]) {
            int rank = 0;  // touched experts below id
            for (int q = 0; q < P; ++q) rank += (L.first[q] && L.ids[q] < id) ? 1 : 0;
            if (rank == yr) {
                int n = 0, tk[4] = {0, 0, 0, 0};
                for (int q = 0; q < P; ++q) {
                    if (L.ids[q] == id) {
                        if (n < 4) tk[n] = q / k;
                        ++n;
                    }
                }
                L.item[0] = id;
                L.item[1] = L.lt[tid];
                L.item[2] = n;
#pragma unroll
                for (int c = 0; c < 4; ++c) L.item[3 + c] = tk[c];
            }
        }
        __syncthreads();
        if (L.item[0] < 0) return false;  // uniform: no expert for this item
        item.shared = false;
        item.e = L.item[0];
        item.first = L.item[1];
        item.ncol = L.item[2];  // at most T <= 4: a token picks an expert once
#pragma unroll
        for (int c = 0; c < 4; ++c) item.tk[c] = L.item[3 + c];
        item.tok0 = item.tk[0];
    }
    return true;
}

template <int NIT, int MAXUPL>
__device__ __forceinline__ bool gu_route_wg(
    int y, int hb, uint32_t* smem, const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps,
    const uint8_t* __restrict__ gate_sh, const uint8_t* __restrict__ up_sh, const uint32_t* __restrict__ ximg,
    const float* __restrict__ logits, int T, int E, int k, int H, int F, int Fs, int has_shared,
    int32_t* __restrict__ ids, float* __restrict__ wts, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm, int32_t* __restrict__ slot, int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
    int4* __restrict__ items, int max_items, uint32_t* __restrict__ himg, int h_blocks, uint64_t* __restrict__ xchg) {
    typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
    const int n_sh = has_shared ? 1 : 0;
    const int tid = threadIdx.x;
    if (y == max_items) {
        if (hb == 0)
            small_route_dispatch(logits, T, E, k, true, ids, wts, counts, offsets, perm, slot, elist, n_list, items,
                                 max_items, has_shared, 1 << 30, kShCols, *reinterpret_cast<SmallDispatchLds*>(smem));
        return false;
    }
    const bool shared_wg = y < n_sh;
    if (hb * 32 >= (shared_wg ? Fs : F)) return false;
    SMOE_STAMP_VAL(1, 0, shared_wg ? 1 : 2);  // role: gate/up of the shared expert (1) or of a routed one (2)
    const int qb = H >> 5;
    const int pieces = T * qb * (kImgDw / 4);  // at most 4 * 128 * 3
    const int npre = (pieces + 255) >> 8;      // uniform
    // unconditional loads (clamped index; a branch around a load makes the compiler wait for it), so that the
    // logits loads of the routing go out behind them without waiting
    u32x4 pre[6];
#pragma unroll
    for (int j = 0; j < 6; ++j)
        pre[j] = reinterpret_cast<const u32x4*>(ximg)[min(min(j, npre - 1) * 256 + tid, pieces - 1)];
    SMOE_STAMP(1, 15);  // the image loads are issued
    GuRouteLds& L = *reinterpret_cast<GuRouteLds*>(smem + kGuCols * qb * kImgLdsDw + 4);
    Item item;
    bool synced;
    const bool has = gu_route_item(
        y, L, logits, T, E, k, has_shared, item,
        [&] {
#pragma unroll
            for (int j = 0; j < 6; ++j)
                if (j * 256 + tid < pieces) reinterpret_cast<u32x4*>(smem)[lds_piece(j * 256 + tid)] = pre[j];
        },
        synced);
    SMOE_STAMP(1, 6);  // the item is known
    if (!has) {
        SMOE_STAMP_VAL(1, 0, 9);  // role: no expert for this item
        return false;
    }
    // (unsynchronised routing: the weight loads go out first, then the barrier that publishes the images)
    q2_gu_item<NIT, MAXUPL, true>(item, hb, smem, gate_exps, up_exps, gate_sh, up_sh, ximg, nullptr, k, H, F, himg,
                                  h_blocks, xchg, {}, 0, !synced);
    SMOE_STAMP(1, 10);
    return true;
}

template <int NIT, int MAXUPL>
__global__ __launch_bounds__(256) void k_q2_gu_route(
    const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps, const uint8_t* __restrict__ gate_sh,
    const uint8_t* __restrict__ up_sh, const uint32_t* __restrict__ ximg, const float* __restrict__ logits, int T,
    int E, int k, int H, int F, int Fs, int has_shared, int32_t* __restrict__ ids, float* __restrict__ wts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ slot, int32_t* __restrict__ elist, int32_t* __restrict__ n_list, int4* __restrict__ items,
    int max_items, uint32_t* __restrict__ himg, int h_blocks) {
    extern __shared__ __align__(16) uint32_t smem[];
    gu_route_wg<NIT, MAXUPL>(blockIdx.y, blockIdx.x, smem, gate_exps, up_exps, gate_sh, up_sh, ximg, logits, T, E, k, H,
                             F, Fs, has_shared, ids, wts, counts, offsets, perm, slot, elist, n_list, items, max_items,
                             himg, h_blocks, nullptr);
}

// Down rows.  Grid (ceil(H / rows per block), max work items), 4 waves; a wave owns NIT passes of rpi rows.
// The item's h images are copied to LDS `cps` columns at a time; each group leader writes its row's value to
// Y[first + c][row] (the shared rows times sigmoid(sg[t])).
template <int NIT, int MAXUPL>
// (As k_q2_gu: what a routed item's work-group reads before its image and weight loads is in the first 14 dwords.)
__global__ __launch_bounds__(256) void k_q2_down(const int4* __restrict__ items, const uint32_t* __restrict__ himg,
                                                  const uint8_t* __restrict__ down_exps,
                                                  const uint64_t* __restrict__ eptr, int H, int F, int Fs, int h_blocks,
                                                  int cps, const uint8_t* __restrict__ down_sh,
                                                  const float* __restrict__ sg, float* __restrict__ Y,
                                                  const int32_t* __restrict__ dmap) {
    extern __shared__ __align__(16) uint32_t smem[];
    Item item;
    if (!work_item_uniform(items, blockIdx.y, item)) return;
    const int Fe = item.shared ? Fs : F;
    const RowGeo G = row_geo(Fe);
    const int rpw = NIT * G.rpi;  // rows per wave
    const size_t rb = (size_t)G.dpr * 36;
    const uint8_t* base =
        item.shared ? down_sh
        : eptr      ? reinterpret_cast<const uint8_t*>(eptr[item.e]) + (size_t)2 * F * ((size_t)(H >> 7) * 36)
                    : down_exps + (size_t)item.e * H * ((size_t)(F >> 7) * 36);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / G.lpr, l = lane - grp * G.lpr;
    const int row0 = blockIdx.x * 4 * rpw + wave * rpw;

    // first column batch: its image loads go out before the weight loads, which are all unconditional (a row
    // past H reloads row H - 1; see k_q2_gu)
    const int nc0 = min(cps, item.ncol);
    StagePieces sp;
    stage_issue_direct<256>(sp, himg, h_blocks, 0, nc0, cps, 0, item, false);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t w[NIT][MAXUPL][9];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int r = min(row0 + it * G.rpi + grp, H - 1);
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m)
            load_unit(base + (size_t)r * rb + (size_t)(m < G.upl ? l + G.lpr * m : l) * 36, w[it][m]);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_commit_direct(sp, smem);
    stage_images<256>(smem, himg, h_blocks, 0, nc0, cps, item, nullptr, 1, false, 4 * 256);  // rounds beyond the first
    __syncthreads();
    float dw[NIT][MAXUPL][2];
    unit_scales(w, dw);
    for (int c0 = 0; c0 < item.ncol; c0 += cps) {
        const int nc = min(cps, item.ncol - c0);
        if (c0 > 0) {
            stage_images<256>(smem, himg, h_blocks, c0, nc, cps, item, nullptr, 1, false);
            __syncthreads();
        }
        for (int c = 0; c < nc; ++c) {
            const uint32_t* ht = smem + (size_t)c * h_blocks * kImgLdsDw;
            pin_units(w);
            float acc[NIT];
#pragma unroll
            for (int m = 0; m < MAXUPL; ++m) {
                if (m < G.upl) {
                    const uint32_t* img = ht + (size_t)(l + G.lpr * m) * kUnitLdsDw;
                    float p01[NIT];
                    Act2 a;
                    load_act_img2(img, a);
#pragma unroll
                    for (int it = 0; it < NIT; ++it) p01[it] = q2_unit_first(w[it][m], dw[it][m][0], a);
                    load_act_img2(img + 2 * kImgDw, a);
#pragma unroll
                    for (int it = 0; it < NIT; ++it) {
                        const float L = q2_unit_second(w[it][m], dw[it][m][1], p01[it], a);
                        acc[it] = m == 0 ? L : acc[it] + L;
                    }
                }
            }
            const float sig = item.shared ? sigmoid(sg[item.tok0 + c0 + c]) : 1.0f;
            const int orow = (dmap && !item.shared) ? dmap[item.first + c0 + c] : item.first + c0 + c;
            float* yc = Y + (size_t)orow * H;
            if (NIT == 1 || G.lpr == 4 * NIT) {  // one reduce-scatter: lane l ends with pass (l >> 2) & (NIT - 1)
                int it;
                float v = group_sum_rs<NIT>(acc, G.lpr, lane, it);
                if (item.shared) v = v * sig;
                const int r = row0 + it * G.rpi + grp;
                if (orow >= 0 && r < H && (l & 3) == 0 && (NIT > 1 || l == 0)) yc[r] = v;
            } else {  // each pass on its own: the same butterfly per row
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    float v = group_sum(acc[it], G.lpr);
                    if (item.shared) v = v * sig;
                    const int r = row0 + it * G.rpi + grp;
                    if (orow >= 0 && r < H && l == 0) yc[r] = v;
                }
            }
        }
        if (c0 + cps < item.ncol) __syncthreads();
    }
}

// Down rows and the combine of a batch of at most kShCols tokens in one kernel.  Grid (ceil(H / kDcRows)), 4
// waves.  Work-group b owns output rows [kDcRows b, + kDcRows) of every item: the h images of all P + T pair rows
// go to LDS; the tasks (item i, pass p: rows p rpi .. + rpi - 1 of the block's rows, rpi = 64 / lpr of the
// item's row length) are dealt to the waves round robin, a wave holding the weight units of NT tasks (at most
// MAXUPL units per lane each, NT * MAXUPL <= 8) at once.  Each row value is formed as k_q2_down forms it (the
// lane's units in order, the butterfly over its lpr lanes, shared rows times sigmoid(sg)) and parked in LDS;
// then y[t][row] as k_combine forms it: w0 * Y[slot0], fma in selection order, + the shared row.
constexpr int kDcRows = 16;
constexpr size_t kDownCombineLds = 96 * 1024;  // images + rows of the batch
constexpr int kDcItems = 384;                  // work items whose table entries fit in LDS
// The task loop and the combine of the small-batch down kernels: the h images of every pair row in `img` (LDS),
// the row values parked in Ys, the item table, routing slots and weights, and the shared gate dots `sg` in LDS.  `before_compute` runs once, after
// the first batch's weight loads were issued and before any weight or image is read (k_q2_moe_small waits for its
// h images there); it must end with a barrier when it writes LDS.
template <int MAXUPL, int NT, class Prep>
__device__ __forceinline__ void down_combine_tasks(const uint8_t* __restrict__ down_exps,
                                                   const uint8_t* __restrict__ down_sh, const uint32_t* img, float* Ys,
                                                   const int4* s_items, const int* s_slot, const float* s_wts,
                                                   int n_items, int npass, int r0, int H, int F, int Fs,
                                                   const float* sg, int T, int k, int add_shared,
                                                   int h_blocks, float* __restrict__ y, Prep before_compute) {
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_tasks = n_items * npass, P = T * k;
    for (int tb = 0; tb < n_tasks; tb += 4 * NT) {
        Item it[NT];
        bool live[NT];
        int lpr[NT], upl[NT], rloc[NT];
        uint32_t w[NT][MAXUPL][9];
#pragma unroll
        for (int q = 0; q < NT; ++q) {
            const int j = tb + 4 * q + wave;  // wave-uniform task
            const int i = j < n_tasks ? j / npass : 0, p = j < n_tasks ? j - i * npass : 0;
            const int4 ia = s_items[2 * i];
            live[q] = j < n_tasks && ia.x != kItemEmpty;
            it[q].shared = ia.x == kItemShared;
            it[q].e = ia.x;
            it[q].first = ia.y;
            it[q].ncol = ia.z;
            it[q].tok0 = ia.w;
            const bool sh = live[q] && it[q].shared;
            const RowGeo G = row_geo(sh ? Fs : F);
            lpr[q] = G.lpr;
            upl[q] = G.upl;
            live[q] = live[q] && p * G.rpi < kDcRows;
            const int grp = lane / G.lpr, l = lane - grp * G.lpr;
            rloc[q] = p * G.rpi + grp;
            const size_t rb = (size_t)G.dpr * 36;
            const uint8_t* base = sh ? down_sh : down_exps + (size_t)(live[q] ? it[q].e : 0) * H * ((size_t)(F >> 7) * 36);
            const int r = min(r0 + min(rloc[q], kDcRows - 1), H - 1);  // every load in bounds
#pragma unroll
            for (int m = 0; m < MAXUPL; ++m)
                load_unit(base + (size_t)r * rb + (size_t)(m < G.upl ? l + G.lpr * m : l) * 36, w[q][m]);
        }
        if (tb == 0) before_compute();  // work-group uniform: every wave runs the first batch
        float dw[NT][MAXUPL][2];
        unit_scales(w, dw);
        // a row value of one column of one task: the lane's units in order, then the butterfly over its lpr lanes
        // (a unit per lane always exists, so the first one is taken without a test; the row's butterfly selects its
        // additions: the tasks' chains interleave with no branch between them)
        auto row_value = [&](int q, int c) {
            const int l = lane & (lpr[q] - 1);  // lpr is a power of two
            const uint32_t* ht = img + (size_t)(it[q].first + c) * h_blocks * kImgLdsDw;
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < MAXUPL; ++m) {
                if (m == 0 || m < upl[q]) {
                    const uint32_t* im = ht + (size_t)(l + lpr[q] * m) * kUnitLdsDw;
                    Act2 a;
                    load_act_img2(im, a);
                    const float p01 = q2_unit_first(w[q][m], dw[q][m][0], a);
                    load_act_img2(im + 2 * kImgDw, a);
                    const float L = q2_unit_second(w[q][m], dw[q][m][1], p01, a);
                    acc = m == 0 ? L : acc + L;
                }
            }
            return group_sum_sel(acc, lpr[q]);
        };
        // the first column of every task at once, with no branch between them (a dead task works on item 0's first
        // column and stores nothing), so that the tasks' LDS reads and dots overlap; further columns task by task
        float v0[NT];
        if constexpr (MAXUPL == 1) {
            // one unit per lane: every task's two image halves are read from LDS before any dot, so the tasks share
            // one LDS round trip instead of two each (row_value's arithmetic, in its order)
            Act2 a0[NT], a1[NT];
#pragma unroll
            for (int q = 0; q < NT; ++q) {
                const int l = lane & (lpr[q] - 1);
                const uint32_t* im = img + (size_t)it[q].first * h_blocks * kImgLdsDw + (size_t)l * kUnitLdsDw;
                load_act_img2(im, a0[q]);
                load_act_img2(im + 2 * kImgDw, a1[q]);
            }
#pragma unroll
            for (int q = 0; q < NT; ++q) {
                const float p01 = q2_unit_first(w[q][0], dw[q][0][0], a0[q]);
                v0[q] = group_sum_sel(q2_unit_second(w[q][0], dw[q][0][1], p01, a1[q]), lpr[q]);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NT; ++q) v0[q] = row_value(q, 0);
        }
        if (tb == 0) SMOE_STAMP(1, 11);  // the first row values are formed
#pragma unroll
        for (int q = 0; q < NT; ++q) {
            if (!live[q]) continue;  // wave-uniform
            const int l = lane % lpr[q];
            const bool store = rloc[q] < kDcRows && r0 + rloc[q] < H && l == 0;
            for (int c = 0; c < it[q].ncol; ++c) {
                float v = v0[q];
                if (c > 0) {
                    pin_units(w);
                    v = row_value(q, c);
                }
                if (it[q].shared) v = v * sigmoid(sg[it[q].tok0 + c]);
                if (store) Ys[(it[q].first + c) * kDcRows + rloc[q]] = v;
            }
        }
    }
    __syncthreads();
    SMOE_STAMP(1, 12);  // every task's row values are parked
    if (tid < T * kDcRows) {
        const int t = tid / kDcRows, rl = tid - t * kDcRows;
        if (r0 + rl < H) {
            float acc = 0.0f;
            for (int s = 0; s < k; ++s) {
                const float v = Ys[s_slot[t * k + s] * kDcRows + rl], wv = s_wts[t * k + s];
                acc = s == 0 ? wv * v : __builtin_fmaf(wv, v, acc);
            }
            if (add_shared) acc = acc + Ys[(P + t) * kDcRows + rl];
            y[(size_t)t * H + r0 + rl] = acc;
        }
    }
}

template <int MAXUPL, int NT>
__global__ __launch_bounds__(256) void k_q2_down_combine(
    const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh, const uint32_t* __restrict__ himg,
    int h_blocks, const float* __restrict__ sg, const int4* __restrict__ items, int n_items, int npass, int H, int F,
    int Fs, const int32_t* __restrict__ slot, const float* __restrict__ wts, int T, int k, int add_shared,
    float* __restrict__ y) {
    typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ int s_slot[kSmallPairs];
    __shared__ float s_wts[kSmallPairs];
    __shared__ int4 s_items[2 * kDcItems];
    __shared__ float s_sg[kShCols];
    const int P = T * k, rows = P + T;
    const int pieces = rows * h_blocks * (kImgDw / 4);  // 16-byte pieces of the images
    float* Ys = reinterpret_cast<float*>(smem + (size_t)lds_piece(pieces) * 4);  // [rows][kDcRows]
    const int r0 = blockIdx.x * kDcRows;
    const int tid = threadIdx.x;

    // the first 1024 image pieces, the item table, the routing slots and weights: unconditional loads (clamped
    // indices), all in flight together, then one barrier before any weight load
    u32x4 pre[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pre[j] = reinterpret_cast<const u32x4*>(himg)[min(j * 256 + tid, pieces - 1)];
    int4 itv[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) itv[j] = items[min(j * 256 + tid, 2 * n_items - 1)];
    const int sl = slot[min(tid, P - 1)];
    const float wt = wts[min(tid, P - 1)];
    const float sgv = sg[min(tid, T - 1)];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (j * 256 + tid < pieces) reinterpret_cast<u32x4*>(smem)[lds_piece(j * 256 + tid)] = pre[j];
    if (tid < T) s_sg[tid] = sgv;
#pragma unroll
    for (int j = 0; j < 3; ++j)
        if (j * 256 + tid < 2 * n_items) s_items[j * 256 + tid] = itv[j];
    if (tid < P) {
        s_slot[tid] = sl;
        s_wts[tid] = wt;
    }
    for (int i = 1024 + tid; i < pieces; i += 256)
        reinterpret_cast<u32x4*>(smem)[lds_piece(i)] = reinterpret_cast<const u32x4*>(himg)[i];
    __syncthreads();

    down_combine_tasks<MAXUPL, NT>(down_exps, down_sh, smem, Ys, s_items, s_slot, s_wts, n_items, npass, r0, H, F, Fs,
                                   s_sg, T, k, add_shared, h_blocks, y, [] {});
}

// ------------------------------------------------------------------------------------------------ fused small batch
// The decode layer of a batch of at most kShCols tokens after the router, in one launch (k_q2_gu_route's gate/up
// work-groups, then k_q2_down_combine's down work-groups), so that the down rows' weight loads run beside the
// gate/up work instead of after a kernel boundary.  1-D grid: work-groups y * hbn + hb (y < max_items: item y,
// rows block hb; y = max_items, hb = 0: the writer of the routing, dispatch and item table), then the down
// work-groups, each owning kDcRows output rows of every item.  A down work-group routes the batch itself (ids and
// weights in LDS, bitwise the writer's) and issues its first batch of weight loads before it waits for h.  The h
// images pass through the workspace: every image dword in a tagged 64-bit word (q8_image_store with xchg), each
// checked by itself, so no fence is needed; the router kernel of the same call cleared the words.  The down
// work-groups come last in the grid: on every XCD all gate/up work-groups are dispatched before any down
// work-group that waits for them, and a down work-group gives up after a bounded wait (its rows are then NaN and
// its status word is 1; every down work-group writes its status word, 0 when it did not give up).
constexpr int kSpinLimit = 100000;  // polls of a bounded wait (each a round trip of ~1 us): ~0.1 s

// A bounded wait's end: `spin` polls done, all there or not.  A limit below zero gives up at once, without
// looking (the host's give-up switch, smoe_set_wait_limit, for tests of the give-up path).
__device__ __forceinline__ bool wait_gives_up(int spin, int limit) { return limit < 0 || spin >= limit; }

// The down work-group of the small-batch launches: rows r0 .. r0 + kDcRows - 1 of every item, then the combine.
// It routes the batch itself from the logits `lg` ([T][E]) and takes the shared gate dots from `sgv` (at least T),
// then issues its first batch of weight loads, waits for the h words (tag 1; a bounded wait), and forms its rows and
// y.  `gave` (uniform): an earlier wait of the caller's gave up -- the work-group then writes NaN
// rows without waiting.  status[r0 / kDcRows] = 1 when the rows are NaN, else 0.
template <int DMAXUPL, int DNT>
__device__ __forceinline__ void down_wg(int r0, uint32_t* smem, const float* lg, const float* sgv, bool gave,
                                        const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh,
                                        int T, int E, int k, int H, int F, int Fs, int has_shared, int h_blocks,
                                        const uint64_t* __restrict__ xchg, int spin_limit, int npass, int add_shared,
                                        float* __restrict__ y, int32_t* __restrict__ status) {
    __shared__ int s_slot[kSmallPairs];
    __shared__ float s_wts[kSmallPairs];
    __shared__ int4 s_items[2 * kDcItems];
    __shared__ int s_ids[64];
    __shared__ float s_sg[kShCols];
    __shared__ int s_bad, s_nt, s_fast;
    const int tid = threadIdx.x;
    const int P = T * k, n_sh = has_shared ? 1 : 0;
    const int rows = P + n_sh * T;
    const int lane = tid & 63, wave = tid >> 6;
    float* Ys = reinterpret_cast<float*>(smem + (size_t)(P + T) * h_blocks * kImgLdsDw);
    if (tid == 0) {
        s_bad = gave ? 1 : 0;
        if (has_shared) {
            s_items[0] = make_int4(kItemShared, P, T, 0);
            s_items[1] = make_int4(1, 2, 3, 0);
        }
    }
    if (tid < T) s_sg[tid] = sgv[tid];
    SMOE_STAMP(1, 4);
    // one token: wave 0 routes it with weights; candidate c (ascending id), selected at rank r, is the token's pair r
    // and the y-th touched expert (y = selected candidates below c), so its dispatch position is y
    const bool one = T == 1 && k <= 64;
    if (one) {
        if (wave == 0) {
            __shared__ uint2 s_cand1[64];
            const FastRoute R = E <= 512 ? route_fast_t<8, true>(lg, E, k, s_cand1)
                                         : route_fast_t<16, true>(lg, E, k, s_cand1);
            SMOE_STAMP(1, 14);
            if (R.ok) {
                const bool sel = R.crank < k;
                const unsigned long long sm = __ballot(sel);
                const int yc = __builtin_amdgcn_mbcnt_hi((uint32_t)(sm >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)sm, 0u));
                if (sel) {
                    s_slot[R.crank] = yc;
                    s_items[2 * (n_sh + yc)] = make_int4(R.cid, yc, 1, 0);
                    s_items[2 * (n_sh + yc) + 1] = make_int4(0, 0, 0, 0);
                }
                if (lane < k) s_wts[lane] = R.sel_w;
            }
            if (lane == 0) {
                s_fast = R.ok ? 1 : 0;
                s_nt = k;
            }
        }
        __syncthreads();
    }
    if (one && s_fast) {
    } else if (P <= 64) {
        // the batch's routing (one wave per token: ids and weights, bitwise the writer's), then one wave derives the
        // dispatch and the item table by cross-lane counts, lane p holding pair p: its slot is the pairs with a
        // smaller expert id plus the earlier pairs with its own; an expert's item sits at its rank among the
        // touched experts
        if (wave < T) route_token(lg + (size_t)wave * E, E, k, nullptr, nullptr, s_ids + wave * k, s_wts + wave * k);
        __syncthreads();
        if (wave == 0) {
            const int me = lane < P ? s_ids[lane] : 0x7FFFFFFF;
            int lt = 0, before = 0, cnt = 0, tk0 = 0, tk1 = 0, tk2 = 0, tk3 = 0;
            for (int q = 0; q < P; ++q) {
                const int o = __builtin_amdgcn_readlane(me, q);
                lt += o < me ? 1 : 0;
                if (o == me) {
                    tk0 = cnt == 0 ? q / k : tk0;
                    tk1 = cnt == 1 ? q / k : tk1;
                    tk2 = cnt == 2 ? q / k : tk2;
                    tk3 = cnt == 3 ? q / k : tk3;
                    before += q < lane ? 1 : 0;
                    ++cnt;
                }
            }
            const bool fst = lane < P && before == 0;
            const unsigned long long firsts = __ballot(fst);
            int rank = 0;
            for (unsigned long long m = firsts; m; m &= m - 1)
                rank += __builtin_amdgcn_readlane(me, __builtin_ctzll(m)) < me ? 1 : 0;
            if (lane < P) s_slot[lane] = lt + before;
            if (fst) {
                s_items[2 * (n_sh + rank)] = make_int4(me, lt, cnt, tk0);
                s_items[2 * (n_sh + rank) + 1] = make_int4(tk1, tk2, tk3, 0);
            }
            if (lane == 0) s_nt = __popcll(firsts);
        }
    } else {
        SmallDispatchLds& R = *reinterpret_cast<SmallDispatchLds*>(Ys + (size_t)(P + T) * kDcRows);
        small_route_dispatch(lg, T, E, k, false, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr, 0, has_shared, 1 << 30, kShCols, R);
        for (int j = tid; j < R.n_touched; j += 256) {
            const int e = R.el[j], first = R.off[e], n = R.cnt[e];
            int tk[4] = {0, 0, 0, 0};
            for (int q = 0; q < 4 && q < n; ++q) tk[q] = R.perm[first + q] / k;
            s_items[2 * (n_sh + j)] = make_int4(e, first, n, tk[0]);
            s_items[2 * (n_sh + j) + 1] = make_int4(tk[1], tk[2], tk[3], 0);
        }
        if (tid < P) {
            s_slot[R.perm[tid]] = tid;
            s_wts[tid] = R.wts[tid];
        }
        if (tid == 0) s_nt = R.n_touched;
    }
    __syncthreads();
    SMOE_STAMP(1, 6);  // the items are known
    const int n_items = n_sh + s_nt;
    auto wait_h = [&] {
        // every image word of the batch's h rows, eight per thread at a time: all loads in flight together (they
        // go out behind this work-group's weight loads, so they return once those have), then the words whose tag
        // is not set yet are read again until it is (a bounded wait)
        const int words = rows * h_blocks * kXchgSlots;
        bool ok = !gave && spin_limit >= 0;
        for (int base = 0; ok && base < words; base += 8 * 256) {
            uint64_t v[8];
            int at[8];
            bool need[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + j * 256 + tid;
                const int blk = i / kXchgSlots;
                const int r = blk / h_blocks, hb = blk - r * h_blocks;
                need[j] = i < words && hb * 32 < (r < P ? F : Fs);
                at[j] = min(i, words - 1);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = need[j] ? xchg_get(xchg + at[j]) : (1ull << 32);
            for (int spin = 0;; ++spin) {
                bool all = true;
#pragma unroll
                for (int j = 0; j < 8; ++j) all = all && (!need[j] || (v[j] >> 32) == 1u);
                if (all) break;
                if (wait_gives_up(spin, spin_limit)) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(4);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (need[j] && (v[j] >> 32) != 1u) v[j] = xchg_get(xchg + at[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + j * 256 + tid;
                const int blk = i / kXchgSlots, wd = i - blk * kXchgSlots;
                if (need[j]) smem[(size_t)lds_blk(blk) + wd] = (uint32_t)v[j];
            }
        }
        SMOE_STAMP(1, 8);  // this thread's h words arrived
        if (!ok) s_bad = 1;
        __syncthreads();
        SMOE_STAMP(1, 9);  // every h word arrived
    };
    down_combine_tasks<DMAXUPL, DNT>(down_exps, down_sh, smem, Ys, s_items, s_slot, s_wts, n_items, npass, r0, H, F,
                                     Fs, s_sg, T, k, add_shared, h_blocks, y, wait_h);
    __syncthreads();
    if (s_bad && tid < T * kDcRows) {  // a producer never arrived: the rows are not valid
        const int t = tid / kDcRows, rl = tid - t * kDcRows;
        if (r0 + rl < H) y[(size_t)t * H + r0 + rl] = __builtin_nanf("");
    }
    if (status && tid == 0) status[r0 / kDcRows] = s_bad;
    SMOE_STAMP(1, 10);
}

template <int NIT, int MAXUPL, int DMAXUPL, int DNT>
// (The arguments of the role split, the image loads, the routing and the exchange come first, T, k and has_shared
// packed into one dword (tkh = T | k << 8 | has_shared << 16), so that they fit the first 14 dwords, which arrive
// preloaded in SGPRs: a later argument is a scalar load, a round trip to memory, and the exchange pointer, which
// both roles hold from the start, would otherwise be waited for before the first loads.)
__global__ __launch_bounds__(256) void k_q2_moe_small(
    int max_items, int h_blocks, int E, int H, int F, int Fs, int tkh, int npass, const uint32_t* __restrict__ ximg,
    const float* __restrict__ logits, uint64_t* __restrict__ xchg, const float* __restrict__ sg,
    const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps, const uint8_t* __restrict__ gate_sh,
    const uint8_t* __restrict__ up_sh, const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh,
    int32_t* __restrict__ ids, float* __restrict__ wts, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm, int32_t* __restrict__ slot, int32_t* __restrict__ elist, int32_t* __restrict__ n_list,
    int4* __restrict__ items, int add_shared, float* __restrict__ y, int spin_limit, int32_t* __restrict__ status) {
    extern __shared__ __align__(16) uint32_t smem[];
    const int T = tkh & 0xFF, k = (tkh >> 8) & 0xFF, has_shared = (tkh >> 16) & 1;
    const int hbn = h_blocks;  // rows blocks of the widest expert
    const int n_gu = max_items * hbn + 1;
    const int id = blockIdx.x;
    SMOE_STAMP(1, 2);
#if defined(SMOE_STAMPS)
    {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        SMOE_STAMP_VAL(1, 1, xcc);  // the XCD
    }
    if (id >= n_gu) SMOE_STAMP_VAL(1, 0, 4);  // role: down
    else if (id / hbn == max_items) SMOE_STAMP_VAL(1, 0, 3);  // role: the writer
#endif
    if (id < n_gu) {  // gate/up (or the writer)
        const int yi = id / hbn, hb = id - yi * hbn;
        gu_route_wg<NIT, MAXUPL>(yi, hb, smem, gate_exps, up_exps, gate_sh, up_sh, ximg, logits, T, E, k, H, F, Fs,
                                 has_shared, ids, wts, counts, offsets, perm, slot, elist, n_list, items, max_items,
                                 nullptr, h_blocks, xchg);
        return;
    }
    down_wg<DMAXUPL, DNT>((id - n_gu) * kDcRows, smem, logits, sg, false, down_exps, down_sh, T, E, k, H, F, Fs,
                          has_shared, h_blocks, xchg, spin_limit, npass, add_shared, y, status);
}

// Generic Q2_0 GEMV over n_col columns of standard q8_1 activations (iq_mmvq's contract, metal/src/iq.mm:148-169).
// Grid (ceil(n_out / rows per block)); same unit and lane order as the expert kernels.
template <int NIT, int MAXUPL>
__global__ __launch_bounds__(256) void k_q2_mmvq(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xq, int n_in,
                                                  int n_out, int n_col, float* __restrict__ y) {
    const RowGeo G = row_geo(n_in);
    const int rpw = NIT * G.rpi;
    const size_t rb = (size_t)G.dpr * 36;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / G.lpr, l = lane - grp * G.lpr;
    const int row0 = blockIdx.x * 4 * rpw + wave * rpw;
    uint32_t wr[NIT][MAXUPL][9];
    bool live[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int r = row0 + it * G.rpi + grp;
        live[it] = r < n_out;
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m)
            if (live[it] && m < G.upl) load_unit(w + (size_t)r * rb + (size_t)(l + G.lpr * m) * 36, wr[it][m]);
    }
    float dw[NIT][MAXUPL][2];
#pragma unroll
    for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m) {
            dw[it][m][0] = unit_d0(wr[it][m]);
            dw[it][m][1] = unit_d1(wr[it][m]);
        }
    const int xb = n_in >> 5;
    for (int c = 0; c < n_col; ++c) {
        pin_units(wr);
        float acc[NIT];
#pragma unroll
        for (int m = 0; m < MAXUPL; ++m) {
            if (m < G.upl) {
                Act4 a;
                load_act_std(xq + ((size_t)c * xb + 4 * (l + G.lpr * m)) * 36, a);
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const float L = q2_unit_dot(wr[it][m], dw[it][m][0], dw[it][m][1], a);
                    acc[it] = m == 0 ? L : acc[it] + L;
                }
            }
        }
        int it;
        const float v = group_sum_rs<NIT>(acc, G.lpr, lane, it);
        const int r = row0 + it * G.rpi + grp;
        if (r < n_out && (l & 3) == 0 && (NIT > 1 || l == 0)) y[(size_t)c * n_out + r] = v;
    }
}

// ------------------------------------------------------------------------------------------------ combine
// y[t][j] = w0 * Y[slot0][j], then fma in selection order, then + shared (include/strata/kernels/native_moe.hpp:10-15).
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ Y, const int32_t* __restrict__ slot,
                                                  const float* __restrict__ wts, int k, int H, int P, int add_shared,
                                                  float* __restrict__ y) {
    asm volatile("" ::"s"(Y), "s"(slot), "s"(wts), "s"(y), "s"(k), "s"(H), "s"(P), "s"(add_shared));  // kernargs now
    const int t = blockIdx.x;
    const int32_t* sl = slot + (size_t)t * k;
    const float* wt = wts + (size_t)t * k;
    // the first 16 slots and weights in one go (scalar loads, past k: the last one again), so that the row loads
    // of the first two batches wait for one round trip
    int sl16[16];
    float wt16[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        sl16[i] = sl[min(i, k - 1)];
        wt16[i] = wt[min(i, k - 1)];
    }
    for (int j = blockIdx.y * 256 + threadIdx.x; j < H; j += gridDim.y * 256) {
        // the pair rows 16 at a time, all loads of a batch in flight together (past k: reloads of the last row)
        float acc = 0.0f;
        for (int s0 = 0; s0 < k; s0 += 16) {
            float v[16], wv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int s = min(s0 + i, k - 1);
                const int r = s0 == 0 ? sl16[i] : sl[s];
                v[i] = Y[(size_t)r * H + j];
                wv[i] = s0 == 0 ? wt16[i] : wt[s];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int s = s0 + i;
                if (s == 0) acc = wv[0] * v[0];
                else if (s < k) acc = __builtin_fmaf(wv[i], v[i], acc);
            }
        }
        if (add_shared) acc = acc + Y[(size_t)(P + t) * H + j];
        y[(size_t)t * H + j] = acc;
    }
}

// The same combine four neighbouring elements per thread (16-byte loads and stores; every element's sum is
// formed exactly as above), NB pair rows per batch (NB >= k where k <= 16, so that no batch reloads rows).
// H % 4 == 0, y 16-byte aligned.  NT: Y read and y written with streaming accesses (a Y larger than the caches).
template <int NB, bool NT>
__global__ __launch_bounds__(256) void k_combine4(const float* __restrict__ Y, const int32_t* __restrict__ slot,
                                                   const float* __restrict__ wts, int k, int H, int P, int add_shared,
                                                   float* __restrict__ y) {
    asm volatile("" ::"s"(Y), "s"(slot), "s"(wts), "s"(y), "s"(k), "s"(H), "s"(P), "s"(add_shared));  // kernargs now
    typedef float vf4 __attribute__((ext_vector_type(4)));
    auto ld = [](const float* p) -> float4 {
        if constexpr (NT) {
            const vf4 v = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
            return make_float4(v.x, v.y, v.z, v.w);
        } else {
            return *reinterpret_cast<const float4*>(p);
        }
    };
    const int t = blockIdx.x;
    const int32_t* sl = slot + (size_t)t * k;
    const float* wt = wts + (size_t)t * k;
    int slb[NB];
    float wtb[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        slb[i] = sl[min(i, k - 1)];
        wtb[i] = wt[min(i, k - 1)];
    }
    const int H4 = H >> 2;
    for (int j = blockIdx.y * 256 + threadIdx.x; j < H4; j += gridDim.y * 256) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int s0 = 0; s0 < k; s0 += NB) {
            float4 v[NB];
            float wv[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int s = min(s0 + i, k - 1);
                const int r = s0 == 0 ? slb[i] : sl[s];
                v[i] = ld(Y + (size_t)r * H + 4 * j);
                wv[i] = s0 == 0 ? wtb[i] : wt[s];
            }
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int s = s0 + i;
                if (s == 0) {
                    acc = make_float4(wv[0] * v[0].x, wv[0] * v[0].y, wv[0] * v[0].z, wv[0] * v[0].w);
                } else if (s < k) {
                    acc.x = __builtin_fmaf(wv[i], v[i].x, acc.x);
                    acc.y = __builtin_fmaf(wv[i], v[i].y, acc.y);
                    acc.z = __builtin_fmaf(wv[i], v[i].z, acc.z);
                    acc.w = __builtin_fmaf(wv[i], v[i].w, acc.w);
                }
            }
        }
        if (add_shared) {
            const float4 sh = ld(Y + (size_t)(P + t) * H + 4 * j);
            acc = make_float4(acc.x + sh.x, acc.y + sh.y, acc.z + sh.z, acc.w + sh.w);
        }
        if constexpr (NT)
            __builtin_nontemporal_store(vf4{acc.x, acc.y, acc.z, acc.w}, reinterpret_cast<vf4*>(y + (size_t)t * H) + j);
        else
            reinterpret_cast<float4*>(y + (size_t)t * H)[j] = acc;
    }
}

// out[t] = RMSNorm(x[t] + r[t]) with unit weight (r may be NULL), one work-group per row (residual_rmsnorm_row:
// the order of or_residual_rmsnorm_dev; out may alias x).  The stacked configuration's layer junction
// x_{l+1} = RMSNorm(x_l + MoE_l(x_l)).
template <bool VEC>
__global__ __launch_bounds__(256) void k_residual_rmsnorm(const float* x, const float* r, int n, float eps,
                                                           float* out) {
    __shared__ float wsum[4];
    __shared__ __align__(16) float row[VEC ? 4096 : 1];
    residual_rmsnorm_row<VEC>(x + (size_t)blockIdx.x * n, r ? r + (size_t)blockIdx.x * n : nullptr, n, eps,
                              out + (size_t)blockIdx.x * n, wsum, VEC ? row : nullptr);
}

hipError_t launch_residual_rmsnorm(const float* x, const float* r, int n_rows, int n, float eps, float* out,
                                   hipStream_t s) {
    const bool vec = n % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) |
                                     reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec) hipLaunchKernelGGL(k_residual_rmsnorm<true>, dim3((unsigned)n_rows), dim3(256), 0, s, x, r, n, eps, out);
    else hipLaunchKernelGGL(k_residual_rmsnorm<false>, dim3((unsigned)n_rows), dim3(256), 0, s, x, r, n, eps, out);
    return hipGetLastError();
}

// One token, parts contiguous [k][n] (the reference's moe_combine call shape).
__global__ __launch_bounds__(256) void k_combine_parts(const float* __restrict__ parts, const float* __restrict__ wts,
                                                        const float* __restrict__ shared, int k, int n,
                                                        float* __restrict__ y) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    float acc = wts[0] * parts[j];
    for (int s = 1; s < k; ++s) acc = __builtin_fmaf(wts[s], parts[(size_t)s * n + j], acc);
    if (shared) acc = acc + shared[j];
    y[j] = acc;
}

// ------------------------------------------------------------------------------------------------ q8_1 (stage API)
// x -> standard q8_1 blocks and/or bf16 bits, one thread per element, a q8_1 block per half wave.
__global__ __launch_bounds__(256) void k_prep(const float* __restrict__ x, int64_t n, uint8_t* __restrict__ xq,
                                               uint16_t* __restrict__ xb) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;
    const float v = live ? x[i] : 0.0f;
    if (xb && live) xb[i] = (uint16_t)f32_to_bf16(v);
    if (xq) {
        uint32_t ds;
        const int q = q8_1_value(v, &ds);
        if ((i - (threadIdx.x & 31)) < n) q8_1_store(q, ds, xq + (i >> 5) * 36);
    }
}

// SwiGLU + standard q8_1 over a flat vector (n % 32 == 0).
__global__ __launch_bounds__(256) void k_swiglu_q8(const float* __restrict__ gate, const float* __restrict__ up,
                                                    int64_t n, uint8_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;
    const float h = live ? silu_mul(gate[i], up[i]) : 0.0f;
    uint32_t ds;
    const int q = q8_1_value(h, &ds);
    if ((i - (threadIdx.x & 31)) < n) q8_1_store(q, ds, y + (i >> 5) * 36);
}

// ------------------------------------------------------------------------------------------------ launchers

namespace {
int lanes_per_row_host(int dpr) {
    const int l = dpr & -dpr;
    return l > 16 ? 16 : l;
}
// gate/up kernel: passes per wave (16 rows per wave), units per lane
void gu_shape(int n_in, int& nit, int& upl) {
    const int dpr = n_in >> 7, lpr = lanes_per_row_host(dpr);
    upl = dpr / lpr;
    nit = lpr >= 4 ? lpr / 4 : 1;
}
// row kernels: passes per wave (at least 16 rows per wave; group_sum_rs needs lpr = 4 passes when there are
// several), units per lane, rows per wave
void rows_shape(int n_in, int& nit, int& upl, int& rpw) {
    const int dpr = n_in >> 7, lpr = lanes_per_row_host(dpr);
    upl = dpr / lpr;
    const int rpi = 64 / lpr;
    nit = rpi >= 16 ? 1 : 16 / rpi;
    rpw = nit * rpi;
}
// the down kernel: as rows_shape; with many work items (`wide`) then up to 4 passes until a lane holds 2 units
// (a work-group streams tens of KB per staging of its h images; passes that do not fit one reduce-scatter are
// summed one by one), with few the narrower shape keeps more work-groups in flight.  Two units per lane, not 4
// nor 1, at decode b=16 (F = 512): 11.8 us against 13.6 and 13.8 -- the grid runs as two rounds of resident
// work-groups, so one round's dots overlap the next round's loads.
void down_shape(int n_in, bool wide, int& nit, int& upl, int& rpw) {
    rows_shape(n_in, nit, upl, rpw);
    if (!wide) return;
    while (nit * upl < 2 && nit < 4) nit *= 2;
    rpw = nit * (64 / lanes_per_row_host(n_in >> 7));
}
constexpr int kDownWideItems = 32;  // work items from which the down kernel takes the wide shape
}  // namespace

bool gemv_shape_ok(int n_in) {
    if (n_in <= 0 || n_in % 128) return false;
    int nit, upl;
    gu_shape(n_in, nit, upl);
    return upl <= 8 && nit <= 4;
}

bool down_shapes_match(int F, int Fs) {
    int a, b, c, d, e, f;
    for (const bool wide : {false, true}) {
        down_shape(F, wide, a, b, c);
        down_shape(Fs, wide, d, e, f);
        if (a != d || b != e) return false;
    }
    return true;
}

size_t img_bytes(int64_t n_blocks) { return (size_t)n_blocks * kImgDw * 4; }

hipError_t launch_prep(const float* x, int64_t n, uint8_t* xq, uint16_t* xb, hipStream_t s) {
    hipLaunchKernelGGL(k_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n, xq, xb);
    return hipGetLastError();
}

// The router grid's x extent: with several token tiles, rounded up to a multiple of 8, so that the token tiles of a
// row block (linear ids x + g * grid.x) are dealt to one XCD and its weight rows come from that XCD's L2 after the
// first tile (the padding blocks are image blocks past the images: they do nothing).
static unsigned router_grid_x(int blocks, int T, int tile) {
    return (unsigned)(T > tile ? (blocks + 7) / 8 * 8 : blocks);
}

hipError_t launch_router(const float* xf, const uint16_t* xb, const void* W, const uint16_t* w_inp,
                         const float* bias, int H, int E, int rows_total, int T, float* logits, int ld_logits, float* sg,
                         uint32_t* ximg, int tile_rows, int img_natural, hipStream_t s, const float* rprev, float eps,
                         float* xout, uint4* clear, int clear_n16, int w_f32) {
    // the fused junction is the row-per-wave path's, for rows up to 4096; so is the clearing of the exchange
    if (rprev && (tile_rows || !xf || H > 4096)) return hipErrorInvalidValue;
    // the rows are E and, with w_inp, the shared gate's (the kernels count them so); images are made from f32 x
    if (rows_total != E + (w_inp ? 1 : 0) || (ximg && !xf)) return hipErrorInvalidValue;
    if (clear_n16 && (tile_rows || !clear)) return hipErrorInvalidValue;
    // the f32 router runs on the row-per-wave path from f32 x
    if (w_f32 && (tile_rows || !xf || H % 4 || H > 4096)) return hipErrorInvalidValue;
    if (w_f32) {
        const int maxc4 = (H / 4 + 63) / 64;
        int tile = T <= 64 ? 4 : 16384 / H;  // f32 tile in LDS: at most 64 KiB
        if (tile > 16) tile = 16;
        if (tile > T) tile = T;
        if (tile < 1) tile = 1;
        const int img_blocks = ximg ? (tile * (H / 32) + 7) / 8 : 0;
        dim3 grid(router_grid_x((rows_total + 3) / 4 + img_blocks, T, tile), (unsigned)((T + tile - 1) / tile));
        const size_t lds = (size_t)tile * H * 4;
#define SMOE_ROUTER_F32(C)                                                                                          \
    hipLaunchKernelGGL((k_router<C, true>), grid, dim3(256), lds, s, H, E, T, tile, W, w_inp, bias, xf, rprev,     \
                       clear_n16, xb, logits, ld_logits, sg, ximg, img_natural, eps, xout, clear)
        if (maxc4 <= 2) SMOE_ROUTER_F32(2);
        else if (maxc4 <= 4) SMOE_ROUTER_F32(4);
        else if (maxc4 <= 8) SMOE_ROUTER_F32(8);
        else SMOE_ROUTER_F32(16);
#undef SMOE_ROUTER_F32
        return hipGetLastError();
    }
    const int chunks = H / 8;
    const int maxc = (chunks + 63) / 64;
    // tokens staged per block: 4 for decode batches (more blocks, short staging), 16 (<= 64 KiB of bf16) beyond
    if (tile_rows)  // many tokens: bf16 x and W on the matrix cores
        return launch_router_mfma(xb, static_cast<const uint16_t*>(W), w_inp, bias, H, E, rows_total, T, logits,
                                  ld_logits, sg, s);
    int tile = T <= 64 ? 4 : 32768 / H;
    if (tile > 16) tile = 16;
    if (tile > T) tile = T;
    if (tile < 1) tile = 1;
    // row blocks (4 weight rows each), then with ximg the image blocks (8 q8_1 blocks of the tile each)
    const int img_blocks = ximg ? (tile * (H / 32) + 7) / 8 : 0;
    dim3 grid(router_grid_x((rows_total + 3) / 4 + img_blocks, T, tile), (unsigned)((T + tile - 1) / tile));
    const size_t lds = (size_t)tile * H * 2;
#define SMOE_ROUTER(C)                                                                                          \
    hipLaunchKernelGGL((k_router<C, false>), grid, dim3(256), lds, s, H, E, T, tile, W, w_inp, bias, xf, rprev,    \
                       clear_n16, xb, logits, ld_logits, sg, ximg, img_natural, eps, xout, clear)
    if (maxc <= 2) SMOE_ROUTER(2);
    else if (maxc <= 4) SMOE_ROUTER(4);
    else if (maxc <= 8) SMOE_ROUTER(8);
    else SMOE_ROUTER(16);
#undef SMOE_ROUTER
    return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int ld_logits, int T, int E, int k, int32_t* ids, float* wts, hipStream_t s) {
    hipLaunchKernelGGL(k_topk, dim3((unsigned)T), dim3(64), 0, s, logits, ld_logits, T, E, k, ids, wts);
    return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t* ids, int P, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                           int32_t* slot, int32_t* elist, int32_t* n_list, int4* items, int max_items, int T, int k,
                           int has_shared, int chunk, int sh_chunk, hipStream_t s) {
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, ids, P, E, counts, offsets, perm, slot, elist, n_list,
                       items, max_items, T, k, has_shared, chunk, sh_chunk);
    return hipGetLastError();
}

size_t dispatch_work_bytes(int64_t P, int E) {
    const int64_t chunks = (P + kDispatchChunk - 1) / kDispatchChunk;
    return (size_t)(chunks * E + 2 * (int64_t)E) * 4;
}

hipError_t launch_dispatch_multi(const int32_t* ids, int P, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                                 int32_t* slot, int32_t* elist, int32_t* n_list, int4* items, int max_items, int T,
                                 int k, int has_shared, int chunk, int sh_chunk, int32_t* work, hipStream_t s) {
    if (!counts) return hipErrorInvalidValue;  // the rank pass reads them
    const int chunks = (P + kDispatchChunk - 1) / kDispatchChunk;
    int32_t* hist = work;
    int32_t* item_of = work + (size_t)chunks * E;
    // the chunk counts in the scan's own LDS for few chunks (one launch fewer), else by k_dispatch_hist
    const bool in_lds = chunks <= kScanLdsChunks && chunks * E <= kScanLdsCounts;
    if (!in_lds) hipLaunchKernelGGL(k_dispatch_hist, dim3((unsigned)chunks), dim3(1024), 0, s, ids, P, E, hist);
    hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(1024), 0, s, hist, chunks, P, E, counts, offsets, elist, n_list,
                       items, item_of, max_items, T, has_shared, chunk, sh_chunk, in_lds ? ids : nullptr);
    hipLaunchKernelGGL(k_dispatch_rank, dim3((unsigned)chunks), dim3(1024), 0, s, ids, P, E, hist, counts, offsets,
                       item_of, perm, slot, items, k, chunk);
    return hipGetLastError();
}

hipError_t launch_topk_dispatch(const float* logits, int T, int E, int k, int32_t* ids, float* wts, int32_t* counts,
                                int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                                int4* items, int max_items, int has_shared, int chunk, int sh_chunk, hipStream_t s) {
    hipLaunchKernelGGL(k_topk_dispatch, dim3(1), dim3(256), 0, s, logits, T, E, k, ids, wts, counts, offsets, perm,
                       slot, elist, n_list, items, max_items, has_shared, chunk, sh_chunk);
    return hipGetLastError();
}

int shared_items(int T) { return (T + kShCols - 1) / kShCols; }
int gemv_shared_chunk() { return kShCols; }


#define SMOE_SHAPE_DISPATCH(KERNEL_MACRO)              \
    if (nit == 4 && upl == 1) KERNEL_MACRO(4, 1);      \
    else if (nit == 4) KERNEL_MACRO(4, 2);             \
    else if (nit == 2 && upl == 1) KERNEL_MACRO(2, 1); \
    else if (nit == 2) KERNEL_MACRO(2, 4);             \
    else if (upl <= 2) KERNEL_MACRO(1, 2);             \
    else if (upl <= 4) KERNEL_MACRO(1, 4);             \
    else KERNEL_MACRO(1, 8);

hipError_t launch_q2_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint32_t* ximg, const int4* items, const int32_t* perm, int k, int H, int F, int Fs,
                        int has_shared, int max_items, uint32_t* himg, int h_blocks, hipStream_t s, const StageOut* so,
                        const uint64_t* eptr) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    dim3 grid((unsigned)(Fmax / 32), (unsigned)max_items);
    int nit, upl;
    gu_shape(H, nit, upl);
    const size_t lds = (size_t)kGuCols * (H >> 5) * kImgLdsDw * 4 + 16;  // + the dead staging slot
    // the traced variant (the trace's expert stages) is its own instantiation: the plain kernel keeps its registers
    const StageOut none{};
    const bool traced = so && so->any();
#define SMOE_GU(N, U)                                                                                                \
    if (traced)                                                                                                      \
        hipLaunchKernelGGL((k_q2_gu<N, U, true>), grid, dim3(256), lds, s, items, ximg, gate_exps, up_exps, eptr, H,  \
                           F, Fs, k, gate_sh, up_sh, perm, himg, h_blocks, *so);                                     \
    else                                                                                                             \
        hipLaunchKernelGGL((k_q2_gu<N, U, false>), grid, dim3(256), lds, s, items, ximg, gate_exps, up_exps, eptr, H, \
                           F, Fs, k, gate_sh, up_sh, perm, himg, h_blocks, none)
    SMOE_SHAPE_DISPATCH(SMOE_GU)
#undef SMOE_GU
    return hipGetLastError();
}

hipError_t launch_q2_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                          const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                          hipStream_t s, const uint64_t* eptr, const int32_t* dmap) {
    int nit, upl, rpw;
    const bool wide = max_items >= kDownWideItems;
    down_shape(F, wide, nit, upl, rpw);  // the caller guarantees the shared width has the same passes and units
    if (Fs > 0) {                  // ... but its rows per wave may be fewer: the grid covers H rows for both
        int a, b, rpw_s;
        down_shape(Fs, wide, a, b, rpw_s);
        rpw = rpw_s < rpw ? rpw_s : rpw;
    }
    dim3 grid((unsigned)((H + 4 * rpw - 1) / (4 * rpw)), (unsigned)max_items);
    const size_t col_bytes = (size_t)h_blocks * kImgLdsDw * 4;
    int cps = (int)(24576 / col_bytes);
    cps = cps < 1 ? 1 : cps > 16 ? 16 : cps;
    const size_t lds = (size_t)cps * col_bytes + 16;  // + the dead staging slot
#define SMOE_DOWN(N, U)                                                                                            \
    hipLaunchKernelGGL((k_q2_down<N, U>), grid, dim3(256), lds, s, items, himg, down_exps, eptr, H, F, Fs, h_blocks, \
                       cps, down_sh, sg, Y, dmap)
    SMOE_SHAPE_DISPATCH(SMOE_DOWN)
#undef SMOE_DOWN
    return hipGetLastError();
}

hipError_t launch_q2_gu_route(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh,
                              const uint8_t* up_sh, const uint32_t* ximg, const float* logits, int T, int E, int k, int H,
                              int F, int Fs, int has_shared, int32_t* ids, float* wts, int32_t* counts,
                              int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                              int4* items, int max_items, uint32_t* himg, int h_blocks, hipStream_t s) {
    if (T < 1 || T > kShCols || T * k > kSmallPairs || E > 1024) return hipErrorInvalidValue;
    const int Fmax = has_shared && Fs > F ? Fs : F;
    dim3 grid((unsigned)(Fmax / 32), (unsigned)max_items + 1);  // + the writer row
    int nit, upl;
    gu_shape(H, nit, upl);
    size_t lds = (size_t)kGuCols * (H >> 5) * kImgLdsDw * 4 + 16 + sizeof(GuRouteLds);
    if (lds < sizeof(SmallDispatchLds)) lds = sizeof(SmallDispatchLds);
#define SMOE_GUR(N, U)                                                                                             \
    hipLaunchKernelGGL((k_q2_gu_route<N, U>), grid, dim3(256), lds, s, gate_exps, up_exps, gate_sh, up_sh, ximg,   \
                       logits, T, E, k, H, F, Fs, has_shared, ids, wts, counts, offsets, perm, slot, elist, n_list, \
                       items, max_items, himg, h_blocks)
    SMOE_SHAPE_DISPATCH(SMOE_GUR)
#undef SMOE_GUR
    return hipGetLastError();
}

size_t down_combine_lds(int T, int k, int h_blocks) {
    const size_t rows = (size_t)T * k + T;
    return rows * h_blocks * kImgLdsDw * 4 + rows * kDcRows * 4;
}

bool down_combine_ok(int T, int k, int h_blocks) {
    return T >= 1 && T <= kShCols && T * k <= kSmallPairs && down_combine_lds(T, k, h_blocks) <= kDownCombineLds;
}
static_assert(kSmallPairs + kShCols <= kDcItems && 2 * kDcItems <= 3 * 256, "the item table of a small batch in LDS");

hipError_t launch_q2_down_combine(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                                  const float* sg, const int4* items, int n_items, int H, int F, int Fs,
                                  const int32_t* slot, const float* wts, int T, int k, int add_shared, float* y,
                                  hipStream_t s) {
    if (!down_combine_ok(T, k, h_blocks)) return hipErrorInvalidValue;
    int npass = 1, maxupl = 1;
    for (const int Fe : {F, Fs}) {
        if (Fe <= 0) continue;
        const int dpr = Fe >> 7, lpr = lanes_per_row_host(dpr), rpi = 64 / lpr;
        const int np = (kDcRows + rpi - 1) / rpi, u = dpr / lpr;
        npass = np > npass ? np : npass;
        maxupl = u > maxupl ? u : maxupl;
    }
    if (maxupl > 8) return hipErrorInvalidValue;
    dim3 grid((unsigned)((H + kDcRows - 1) / kDcRows));
    const size_t lds = down_combine_lds(T, k, h_blocks);
#define SMOE_DC(U, N)                                                                                               \
    hipLaunchKernelGGL((k_q2_down_combine<U, N>), grid, dim3(256), lds, s, down_exps, down_sh, himg, h_blocks, sg, \
                       items, n_items, npass, H, F, Fs, slot, wts, T, k, add_shared, y)
    if (maxupl == 1) SMOE_DC(1, 4);
    else if (maxupl == 2) SMOE_DC(2, 4);
    else if (maxupl <= 4) SMOE_DC(4, 2);
    else SMOE_DC(8, 1);
#undef SMOE_DC
    return hipGetLastError();
}

size_t moe_small_lds(int T, int k, int H, int h_blocks) {
    const size_t rows = (size_t)T * k + T;
    const size_t down = rows * h_blocks * kImgLdsDw * 4 + rows * kDcRows * 4 + sizeof(SmallDispatchLds);
    size_t gu = (size_t)kGuCols * (H >> 5) * kImgLdsDw * 4 + 16 + sizeof(GuRouteLds);
    if (gu < sizeof(SmallDispatchLds)) gu = sizeof(SmallDispatchLds);
    return down > gu ? down : gu;
}

size_t moe_small_xchg_bytes(int T, int k, int max_items, int h_blocks) {
    const size_t rows = (size_t)T * k + T;
    (void)max_items;
    const size_t bytes = rows * h_blocks * kXchgSlots * 8;
    return (bytes + 15) / 16 * 16;
}

bool moe_small_ok(int T, int k, int H, int F, int Fs, int has_shared, int h_blocks) {
    if (!down_combine_ok(T, k, h_blocks)) return false;
    if (moe_small_lds(T, k, H, h_blocks) > 96 * 1024) return false;
    int nit, upl;
    gu_shape(H, nit, upl);
    for (const int Fe : {F, has_shared ? Fs : 0}) {
        if (Fe <= 0) continue;
        const int dpr = Fe >> 7, lpr = lanes_per_row_host(dpr);
        if (dpr / lpr > 2) return false;  // down rows of at most 2 units per lane (F up to 1024 x 2^a)
    }
    return true;
}

namespace {
std::atomic<int> g_wait_limit{kSpinLimit};
}
int wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }
int default_wait_limit() { return kSpinLimit; }
void set_wait_limit(int limit) { g_wait_limit.store(limit, std::memory_order_relaxed); }

// down rows: passes per wave and units per lane of the widest of the routed and shared down rows
static void small_down_shape(int F, int Fs, int has_shared, int& npass, int& dmaxupl) {
    npass = 1;
    dmaxupl = 1;
    for (const int Fe : {F, has_shared ? Fs : 0}) {
        if (Fe <= 0) continue;
        const int dpr = Fe >> 7, lpr = lanes_per_row_host(dpr), rpi = 64 / lpr;
        const int np = (kDcRows + rpi - 1) / rpi, u = dpr / lpr;
        npass = np > npass ? np : npass;
        dmaxupl = u > dmaxupl ? u : dmaxupl;
    }
}

hipError_t launch_q2_moe_small(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh,
                               const uint8_t* up_sh, const uint8_t* down_exps, const uint8_t* down_sh,
                               const uint32_t* ximg, const float* logits, const float* sg, int T, int E, int k, int H,
                               int F, int Fs, int has_shared, int32_t* ids, float* wts, int32_t* counts,
                               int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                               int4* items, int max_items, int h_blocks, uint8_t* xchg, int add_shared, float* y,
                               int32_t* status, hipStream_t s) {
    if (T < 1 || T > kShCols || T * k > kSmallPairs || E > 1024 || max_items + 1 > kDcItems || k < 1 || k > 255 ||
        !moe_small_ok(T, k, H, F, Fs, has_shared, h_blocks))
        return hipErrorInvalidValue;
    const int tkh = T | (k << 8) | ((has_shared ? 1 : 0) << 16);  // (the kernel's packed T, k, has_shared)
    int npass, dmaxupl;
    small_down_shape(F, Fs, has_shared, npass, dmaxupl);
    uint64_t* xw = reinterpret_cast<uint64_t*>(xchg);
    const int n_gu = max_items * h_blocks + 1;
    dim3 grid((unsigned)(n_gu + (H + kDcRows - 1) / kDcRows));
    int nit, upl;
    gu_shape(H, nit, upl);
    const size_t lds = moe_small_lds(T, k, H, h_blocks);
    const int spin = wait_limit();
    // (a down work-group's tasks in one batch of three per wave when they fit: the b = 1 layer's 11 items)
    const bool d3 = dmaxupl == 1 && max_items * npass <= 12;
#define SMOE_MS(N, U)                                                                                                \
    do {                                                                                                             \
        if (d3)                                                                                                      \
            hipLaunchKernelGGL((k_q2_moe_small<N, U, 1, 3>), grid, dim3(256), lds, s, max_items, h_blocks, E, H, F,  \
                               Fs, tkh, npass, ximg, logits, xw, sg, gate_exps, up_exps, gate_sh, up_sh, down_exps,   \
                               down_sh, ids, wts, counts, offsets, perm, slot, elist, n_list, items, add_shared, y,   \
                               spin, status);                                                                         \
        else if (dmaxupl == 1)                                                                                       \
            hipLaunchKernelGGL((k_q2_moe_small<N, U, 1, 4>), grid, dim3(256), lds, s, max_items, h_blocks, E, H, F,  \
                               Fs, tkh, npass, ximg, logits, xw, sg, gate_exps, up_exps, gate_sh, up_sh, down_exps,   \
                               down_sh, ids, wts, counts, offsets, perm, slot, elist, n_list, items, add_shared, y,   \
                               spin, status);                                                                         \
        else                                                                                                         \
            hipLaunchKernelGGL((k_q2_moe_small<N, U, 2, 4>), grid, dim3(256), lds, s, max_items, h_blocks, E, H, F,  \
                               Fs, tkh, npass, ximg, logits, xw, sg, gate_exps, up_exps, gate_sh, up_sh, down_exps,   \
                               down_sh, ids, wts, counts, offsets, perm, slot, elist, n_list, items, add_shared, y,   \
                               spin, status);                                                                         \
    } while (0)
    SMOE_SHAPE_DISPATCH(SMOE_MS)
#undef SMOE_MS
    return hipGetLastError();
}

int fused_status_words(int H) { return (H + kDcRows - 1) / kDcRows; }

hipError_t launch_combine(const float* Y, const int32_t* slot, const float* wts, int k, int H, int P, int T,
                          int add_shared, float* y, hipStream_t s, int nt) {
    if (H % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
        const int ychunks = (H / 4 + 255) / 256;
        dim3 grid((unsigned)T, (unsigned)(ychunks < 8 ? ychunks : 8));
#define SMOE_C4(NB)                                                                                                   \
    do {                                                                                                               \
        if (nt) hipLaunchKernelGGL((k_combine4<NB, true>), grid, dim3(256), 0, s, Y, slot, wts, k, H, P, add_shared, y); \
        else hipLaunchKernelGGL((k_combine4<NB, false>), grid, dim3(256), 0, s, Y, slot, wts, k, H, P, add_shared, y);  \
    } while (0)
        if (k <= 4) SMOE_C4(4);
        else if (k <= 8) SMOE_C4(8);
        else if (k == 10) SMOE_C4(10);  // (the configs' top-k: no batch slot reloads a row)
        else if (k <= 12) SMOE_C4(12);
        else SMOE_C4(16);
#undef SMOE_C4
        return hipGetLastError();
    }
    const int ychunks = (H + 255) / 256;
    dim3 grid((unsigned)T, (unsigned)(ychunks < 8 ? ychunks : 8));
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, s, Y, slot, wts, k, H, P, add_shared, y);
    return hipGetLastError();
}

hipError_t launch_combine_parts(const float* parts, const float* wts, const float* shared, int k, int n, float* y,
                                hipStream_t s) {
    hipLaunchKernelGGL(k_combine_parts, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, parts, wts, shared, k, n, y);
    return hipGetLastError();
}

hipError_t launch_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y, hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gate, up, n, y);
    return hipGetLastError();
}

hipError_t launch_q2_mmvq(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y, hipStream_t s) {
    int nit, upl, rpw;
    rows_shape(n_in, nit, upl, rpw);
    dim3 grid((unsigned)((n_out + 4 * rpw - 1) / (4 * rpw)));
#define SMOE_MMVQ(N, U) hipLaunchKernelGGL((k_q2_mmvq<N, U>), grid, dim3(256), 0, s, w, xq, n_in, n_out, n_col, y)
    SMOE_SHAPE_DISPATCH(SMOE_MMVQ)
#undef SMOE_MMVQ
    return hipGetLastError();
}

}  // namespace smoe

#if defined(SMOE_STAMPS)
// The stamp buffer of the timeline build (device memory of 2 x 4096 x 32 u64, or NULL to stop stamping).
extern "C" int smoe_debug_set_stamps(void* p) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(smoe::g_stamp), &p, sizeof(p));
}
#endif
