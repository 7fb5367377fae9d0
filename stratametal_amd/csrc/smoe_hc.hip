// stratametal_amd/csrc/smoe_hc.hip - the hyper-connection ends of the layer call (gfx950, wave64).
//
// FfnExec::run reads the layer's input from hc residual streams through the gated residual and writes the MoE
// block's output back onto every stream (metal/src/layer_exec.cpp:469,531; metal/include/strata/metal/gr.hpp:1-48).
// Per token, R is [hc][n] f32 (stream c at c * n):
//   read:  xn = R * rs_c * w_norm (rs_c = 1 / sqrt(mean(R_c^2) + eps); w_norm is the stored (1 + w)), act = bf16(xn);
//          proj_r = act . down_r (r < hc_lr), lq = bf16(silu(proj_r / hc)); gate_i = lq . up_i (i < hc * n);
//          mixed_d = (sum_c xn_cd * sigmoid(gate_cd)) / hc;  inject_c = act . inj_c;
//   write: out_cd = R_cd + y_d * 2 sigmoid(inject_c / hc).
// The read is two bandwidth-bound bf16 GEMVs in a chain (about 10.5 MB of weights per token at n 2048, hc 4, hc_lr 320,
// as much as the MoE block itself), so it is two launches: k_hc_proj (the norm, the activations staged in LDS, the
// down and inject rows) and k_hc_mix (lq, the up rows, the gated mean).  The write is a third; the stacked call forms
// it inside the next layer's k_hc_proj.  Reduction orders are fixed and restated by the test oracle
// (or_hc_read_dev, or_hc_write_dev).
#include "smoe_device.hpp"
#include "smoe_gemv.hpp"
#include "smoe_launch.hpp"

namespace smoe {

namespace {

// Per-stream scale rs_c of one token: thread i of 256 adds fmaf(v, v, acc) over d = i, i + 256, ... from 0, the wave
// butterfly 32..1, the four wave sums ((w0 + w1) + w2) + w3 (LDS `wsum`: 4 floats per stream); rs = 1 / sqrtf(ss / n
// + eps).  Every thread returns with rs of every stream in `rs_s` (LDS, hc floats).  `v[c][m]` holds R_c[tid + 256 m].
template <int HC, int NM>
__device__ __forceinline__ void stream_scales(const float (&v)[HC][NM], int hc, int n, float eps, float (*wsum)[4],
                                              float* rs_s) {
    const int tid = threadIdx.x;
    float acc[HC];
#pragma unroll
    for (int c = 0; c < HC; ++c) {
        acc[c] = 0.0f;
#pragma unroll
        for (int m = 0; m < NM; ++m)
            if (tid + 256 * m < n) acc[c] = __builtin_fmaf(v[c][m], v[c][m], acc[c]);
    }
    wave_sum_xor_fast_n<HC>(acc);
    if ((tid & 63) == 0) {
#pragma unroll
        for (int c = 0; c < HC; ++c) wsum[c][tid >> 6] = acc[c];
    }
    __syncthreads();
    if (tid < hc) {
        const float ss = ((wsum[tid][0] + wsum[tid][1]) + wsum[tid][2]) + wsum[tid][3];
        rs_s[tid] = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
    }
    __syncthreads();
}

}  // namespace

// k_hc_proj: grid (ceil((hc_lr + hc) / 4), T), 256 threads; block (b, t) takes rows 4b .. 4b + 3 of [down; inj] for
// token t, one row per wave (lane l adds the 8-element chunks l, l + 64, ... in element order, then the xor butterfly
// 32..1, as the router).  Every block forms the token's scales and stages act = bf16((R * rs) * w_norm) in LDS; block
// (0, t) also writes rs[t][c] for k_hc_mix.  With `rprev` the layer's streams are first formed from the layer before,
// R = rprev + y_prev * 2 sigmoid(inj_prev / hc) (the stacked call's write, fused), and block (0, t) stores them to R.
template <int HC, int NM, int MAXC>
__global__ __launch_bounds__(256) void k_hc_proj(float* __restrict__ R, const float* __restrict__ norm,
                                                  const uint16_t* __restrict__ down, const uint16_t* __restrict__ inj,
                                                  int n, int hc, int hc_lr, float eps, float* __restrict__ proj,
                                                  float* __restrict__ inject, float* __restrict__ rs_out,
                                                  const float* __restrict__ rprev, const float* __restrict__ yprev,
                                                  const float* __restrict__ injprev) {
    extern __shared__ __align__(16) uint16_t act_s[];  // hc * n bf16
    __shared__ float wsum[HC][4];
    __shared__ float rs_s[HC];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int hd = hc * n;
    const int rows = hc_lr + hc;
    const int row = min((int)blockIdx.x * 4 + (tid >> 6), rows - 1);  // clamped: every load in bounds
    const uint16_t* wr = row < hc_lr ? down + (size_t)row * hd : inj + (size_t)(row - hc_lr) * hd;
    const int chunks = hd >> 3;
    uint4 wv[MAXC];
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {  // the wave's weight row first: in flight while the scales are formed
        const int c = lane + 64 * j;
        wv[j] = c < chunks ? *reinterpret_cast<const uint4*>(wr + 8 * c) : make_uint4(0, 0, 0, 0);
    }
    float* Rt = R + (size_t)t * hd;
    float v[HC][NM];
#pragma unroll
    for (int c = 0; c < HC; ++c) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const int d = tid + 256 * m;
            float x = 0.0f;
            if (c < hc && d < n) {
                const size_t i = (size_t)c * n + d;
                if (rprev) {
                    const float s = sigmoid(injprev[(size_t)t * hc + c] / (float)hc);
                    x = rprev[(size_t)t * hd + i] + yprev[(size_t)t * n + d] * (2.0f * s);
                } else {
                    x = Rt[i];
                }
            }
            v[c][m] = x;
        }
    }
    if (rprev && blockIdx.x == 0) {
#pragma unroll
        for (int c = 0; c < HC; ++c)
#pragma unroll
            for (int m = 0; m < NM; ++m)
                if (c < hc && tid + 256 * m < n) Rt[(size_t)c * n + tid + 256 * m] = v[c][m];
    }
    stream_scales<HC, NM>(v, hc, n, eps, wsum, rs_s);
    if (blockIdx.x == 0 && tid < hc) rs_out[(size_t)t * hc + tid] = rs_s[tid];
#pragma unroll
    for (int c = 0; c < HC; ++c) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const int d = tid + 256 * m;
            if (c < hc && d < n) {
                const size_t i = (size_t)c * n + d;
                act_s[i] = (uint16_t)f32_to_bf16((v[c][m] * rs_s[c]) * norm[i]);
            }
        }
    }
    __syncthreads();
    if ((int)blockIdx.x * 4 + (tid >> 6) >= rows) return;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
            const uint4 xv = *reinterpret_cast<const uint4*>(act_s + 8 * c);
            const uint32_t xq[4] = {xv.x, xv.y, xv.z, xv.w};
            const uint32_t wq[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc = __builtin_fmaf(u2f(xq[q] << 16), u2f(wq[q] << 16), acc);
                acc = __builtin_fmaf(u2f(xq[q] & 0xFFFF0000u), u2f(wq[q] & 0xFFFF0000u), acc);
            }
        }
    }
    acc = wave_sum_xor_fast(acc);
    if (lane == 0) {
        if (row < hc_lr) proj[(size_t)t * hc_lr + row] = acc;
        else if (inject) inject[(size_t)t * hc + row - hc_lr] = acc;
    }
}

// k_hc_mix: grid (n / 8, T), 256 threads; block (b, t) forms mixed[t][8b .. 8b + 7].  lq = bf16(silu(proj / hc)) in
// LDS; the 8 hc rows i = c * n + d of `up` (hc_lr bf16 each) go 8 lanes per row (lane l adds the 8-element chunks
// l, l + 8, ... in element order, then the xor butterfly 4, 2, 1), wave w taking the rows of streams w, w + 4, ...;
// gated = xn * sigmoid(gate) with xn = (R * rs) * w_norm as k_hc_proj forms it; mixed = (((0 + g_0) + g_1) + ...) / hc.
template <int LQC>
__global__ __launch_bounds__(256) void k_hc_mix(const float* __restrict__ R, const float* __restrict__ norm,
                                                 const uint16_t* __restrict__ up, const float* __restrict__ proj,
                                                 const float* __restrict__ rs, int n, int hc, int hc_lr,
                                                 float* __restrict__ mixed) {
    __shared__ __align__(16) uint16_t lq_s[64 * LQC];
    __shared__ float gated[8][8];  // [stream][d - 8b], hc <= 8
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d0 = blockIdx.x * 8;
    const int hd = hc * n;
    const int lchunks = hc_lr >> 3;  // 8-element chunks of a row
    const int g = lane >> 3, l = lane & 7;
    // the first row of this 8-lane group (stream `wave`, d0 + g), loaded before lq is formed
    uint4 wv[LQC];
    {
        const int c = min(wave, hc - 1);
        const uint16_t* wr = up + ((size_t)c * n + d0 + g) * hc_lr;
#pragma unroll
        for (int j = 0; j < LQC; ++j) {
            const int ch = l + 8 * j;
            wv[j] = ch < lchunks ? *reinterpret_cast<const uint4*>(wr + 8 * ch) : make_uint4(0, 0, 0, 0);
        }
    }
    for (int i = tid; i < hc_lr; i += 256) {
        const float z = proj[(size_t)t * hc_lr + i] / (float)hc;
        lq_s[i] = (uint16_t)f32_to_bf16(z / (1.0f + expf_smoe(-z)));
    }
    __syncthreads();
    for (int c = wave; c < hc; c += 4) {
        const size_t i = (size_t)c * n + d0 + g;
        if (c != wave) {  // streams beyond the first four: this wave's next row
            const uint16_t* wr = up + i * hc_lr;
#pragma unroll
            for (int j = 0; j < LQC; ++j) {
                const int ch = l + 8 * j;
                wv[j] = ch < lchunks ? *reinterpret_cast<const uint4*>(wr + 8 * ch) : make_uint4(0, 0, 0, 0);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < LQC; ++j) {
            const int ch = l + 8 * j;
            if (ch < lchunks) {
                const uint4 xq4 = *reinterpret_cast<const uint4*>(lq_s + 8 * ch);
                const uint32_t xq[4] = {xq4.x, xq4.y, xq4.z, xq4.w};
                const uint32_t wq[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc = __builtin_fmaf(u2f(xq[q] << 16), u2f(wq[q] << 16), acc);
                    acc = __builtin_fmaf(u2f(xq[q] & 0xFFFF0000u), u2f(wq[q] & 0xFFFF0000u), acc);
                }
            }
        }
        acc = acc + xor_swap<4>(acc);
        acc = acc + xor_swap<2>(acc);
        acc = acc + xor_swap<1>(acc);
        if (l == 0) {
            const float xn = (R[(size_t)t * hd + i] * rs[(size_t)t * hc + c]) * norm[i];
            gated[c][g] = xn * sigmoid(acc);
        }
    }
    __syncthreads();
    if (tid < 8) {
        float m = 0.0f;
        for (int c = 0; c < hc; ++c) m = m + gated[c][tid];
        mixed[(size_t)t * n + d0 + tid] = m / (float)hc;
    }
}

// k_hc_write: out[t][c][d] = R[t][c][d] + y[t][d] * (2 * sigmoid(inject[t][c] / hc)); out may be R.
__global__ __launch_bounds__(256) void k_hc_write(const float* R, const float* __restrict__ y,
                                                   const float* __restrict__ inject, int n, int hc, int64_t total,
                                                   float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t row = i / n;  // t * hc + c
    const int d = (int)(i - row * n);
    const int64_t t = row / hc;
    const float s = sigmoid(inject[row] / (float)hc);
    out[i] = R[i] + y[t * n + d] * (2.0f * s);
}

bool hc_shape_ok(int n, int hc, int hc_lr) {
    if (n <= 0 || hc <= 0 || hc_lr <= 0) return false;
    if (n % 8 || hc_lr % 8 || n > 4096 || hc > 8 || hc_lr > 2048) return false;
    return (int64_t)hc * n <= 16384;  // the activations in LDS: 32 KiB of bf16
}

hipError_t launch_hc_read(float* R, const float* norm, const uint16_t* down, const uint16_t* up, const uint16_t* inj,
                          int n_tok, int n, int hc, int hc_lr, float eps, float* proj, float* rs, float* mixed,
                          float* inject, const float* rprev, const float* yprev, const float* injprev, hipStream_t s) {
    if (!hc_shape_ok(n, hc, hc_lr) || n_tok <= 0) return hipErrorInvalidValue;
    const int hd = hc * n;
    const int maxc = (hd / 8 + 63) / 64;
    const int nm = (n + 255) / 256;
    dim3 g1((unsigned)((hc_lr + hc + 3) / 4), (unsigned)n_tok);
    const size_t lds = (size_t)hd * 2;
#define SMOE_HCP(HCv, NMv, C)                                                                                       \
    hipLaunchKernelGGL((k_hc_proj<HCv, NMv, C>), g1, dim3(256), lds, s, R, norm, down, inj, n, hc, hc_lr, eps, proj, \
                       inject, rs, rprev, yprev, injprev)
#define SMOE_HCP_C(HCv, NMv)             \
    if (maxc <= 8) SMOE_HCP(HCv, NMv, 8);  \
    else if (maxc <= 16) SMOE_HCP(HCv, NMv, 16); \
    else if (maxc <= 24) SMOE_HCP(HCv, NMv, 24); \
    else SMOE_HCP(HCv, NMv, 32);
#define SMOE_HCP_NM(HCv)                 \
    if (nm <= 2) { SMOE_HCP_C(HCv, 2) }  \
    else if (nm <= 8) { SMOE_HCP_C(HCv, 8) } \
    else { SMOE_HCP_C(HCv, 16) }
    if (hc <= 4) { SMOE_HCP_NM(4) }
    else { SMOE_HCP_NM(8) }
#undef SMOE_HCP_NM
#undef SMOE_HCP_C
#undef SMOE_HCP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int lqc = (hc_lr / 8 + 7) / 8;  // chunks per lane of an up row
    dim3 g2((unsigned)(n / 8), (unsigned)n_tok);
    if (lqc <= 5) hipLaunchKernelGGL((k_hc_mix<5>), g2, dim3(256), 0, s, R, norm, up, proj, rs, n, hc, hc_lr, mixed);
    else if (lqc <= 8) hipLaunchKernelGGL((k_hc_mix<8>), g2, dim3(256), 0, s, R, norm, up, proj, rs, n, hc, hc_lr, mixed);
    else hipLaunchKernelGGL((k_hc_mix<32>), g2, dim3(256), 0, s, R, norm, up, proj, rs, n, hc, hc_lr, mixed);
    return hipGetLastError();
}

hipError_t launch_hc_write(const float* R, const float* y, const float* inject, int n_tok, int n, int hc, float* out,
                           hipStream_t s) {
    const int64_t total = (int64_t)n_tok * hc * n;
    if (total <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hc_write, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, R, y, inject, n, hc, total,
                       out);
    return hipGetLastError();
}

}  // namespace smoe
