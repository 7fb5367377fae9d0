// stratametal_amd/csrc/smoe_decode.hip - the decode-contract kernels of the MoE block (gfx950, wave64).
//
// Decode is a bandwidth-bound dequant-GEMV: each expert's 2-bit rows are streamed once, with coalesced
// dword loads, unpacked in registers and multiplied with v_dot4_i32_i8 against q8_1 activations held in
// LDS.  No MFMA.  One launch sequence per call:
//   k_prep     x -> q8_1 (one quantisation serves routed and shared experts) and bf16 (router input)
//   k_router   router logits + the shared expert's gate dot, one wave per weight row
//   k_topk     softmax / top-k / renormalise, one wave per token
//   k_dispatch canonical stable dispatch of the (token, slot) pairs, the touched-expert list
//   k_q2_gu    per (touched expert | shared, 32 rows of h): gate and up rows, SwiGLU, q8_1 of h
//   k_q2_down  per (touched expert | shared, 64 output rows): the down rows (times the shared gate)
//   k_combine  y = routing-weighted sum of the pair rows + the shared row
// Reduction orders are fixed and restated on the host by the test oracle (oracle/smoe_oracle.c).
#include "smoe_device.hpp"
#include "smoe_launch.hpp"

namespace smoe {

// ------------------------------------------------------------------------------------------------ prep
// One thread per element.  Each 32-lane half wave is one q8_1 block.  x: [n] f32 (n % 32 == 0).
__global__ __launch_bounds__(256) void k_prep(const float* __restrict__ x, int64_t n, uint8_t* __restrict__ xq,
                                               uint16_t* __restrict__ xb) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;
    const float v = live ? x[i] : 0.0f;
    if (xb && live) xb[i] = (uint16_t)f32_to_bf16(v);
    if (xq) {
        uint32_t ds;
        const int q = q8_1_value(v, &ds);
        const int64_t blk = i >> 5;
        if (((i - (threadIdx.x & 31)) < n)) q8_1_store(q, ds, xq + blk * 36);
    }
}

// ------------------------------------------------------------------------------------------------ router
// logits[t][row] = sum_i f32(bf16 x[t][i]) * f32(bf16 W[row][i]); row == E is the shared gate row
// (w_inp) and goes to sg[t].  One wave per row; lane l owns the 8-element chunks l, l+64, ...; each lane
// accumulates its chunks in element order from 0, then an xor butterfly 32..1 (oracle: or_bf16_gemv_dev).
// Every product of two bf16 values is exact in f32, so fmaf(x, w, acc) == acc + x * w.
template <int MAXC>
__global__ __launch_bounds__(256) void k_router(const uint16_t* __restrict__ xb, const uint16_t* __restrict__ W,
                                                 const uint16_t* __restrict__ w_inp, const float* __restrict__ bias,
                                                 int H, int E, int rows_total, int T, int tok_per_block,
                                                 float* __restrict__ logits, int ld_logits, float* __restrict__ sg) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows_total) return;
    const uint16_t* wr = row < E ? W + (size_t)row * H : w_inp;
    const int chunks = H >> 3;
    uint4 wv[MAXC];
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) wv[j] = *reinterpret_cast<const uint4*>(wr + 8 * c);
        else wv[j] = make_uint4(0, 0, 0, 0);
    }
    const int t0 = blockIdx.y * tok_per_block;
    const int t1 = min(T, t0 + tok_per_block);
    for (int t = t0; t < t1; ++t) {
        const uint16_t* xr = xb + (size_t)t * H;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXC; ++j) {
            const int c = lane + 64 * j;
            if (c < chunks) {
                const uint4 xv = *reinterpret_cast<const uint4*>(xr + 8 * c);
                const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
                const uint32_t ws[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc = __builtin_fmaf(u2f(xs[q] << 16), u2f(ws[q] << 16), acc);
                    acc = __builtin_fmaf(u2f(xs[q] & 0xFFFF0000u), u2f(ws[q] & 0xFFFF0000u), acc);
                }
            }
        }
        acc = wave_sum_xor(acc);
        if (lane == 0) {
            if (row < E) logits[(size_t)t * ld_logits + row] = bias ? acc + bias[row] : acc;
            else sg[t] = acc;
        }
    }
}

// ------------------------------------------------------------------------------------------------ top-k
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

// One wave per token, E <= 1024 (16 logits per lane, lane l owns e = l + 64 j).  Selection by (logit desc,
// id asc), a NaN logit ranks as -inf.  ex_e = exp(l_e - max); S = per-lane sums in j order, then the xor
// butterfly; p_i = ex_i / S; w_i = p_i / max(sum of the k p_i in selection order, 2^-14)
// (metal/shaders/router.metal:30-132; oracle: or_route_dev).
__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ logits, int ld_logits, int T, int E, int k,
                                              int32_t* __restrict__ ids, float* __restrict__ wts) {
    const int t = blockIdx.x;
    if (t >= T) return;
    const int lane = threadIdx.x;
    const float* l = logits + (size_t)t * ld_logits;
    float key[16], ex[16];
    uint32_t taken = 0;
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int e = lane + 64 * j;
        float v = -__builtin_inff();
        if (e < E) {
            v = l[e];
            if (v != v) v = -__builtin_inff();
        } else {
            taken |= 1u << j;
        }
        key[j] = v;
        mx = __builtin_fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        ex[j] = 0.0f;
        if (!((taken >> j) & 1u)) {
            ex[j] = expf_smoe(key[j] - mx);
            acc = acc + ex[j];
        }
    }
    const float S = wave_sum_xor(acc);
    float ssel = 0.0f, my_p = 0.0f;
    for (int i = 0; i < k; ++i) {
        float bv = -__builtin_inff(), bx = 0.0f;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int e = lane + 64 * j;
            if (!((taken >> j) & 1u) && better(key[j], e, bv, bi)) {
                bv = key[j];
                bi = e;
                bx = ex[j];
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, kWave);
            const int oi = __shfl_xor(bi, o, kWave);
            const float ox = __shfl_xor(bx, o, kWave);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
                bx = ox;
            }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        const float p = bx / S;
        if (lane == i) my_p = p;
        ssel = ssel + p;
        if (lane == 0) ids[(size_t)t * k + i] = bi;
    }
    const float den = __builtin_fmaxf(ssel, 6.103515625e-05f);
    if (lane < k) wts[(size_t)t * k + lane] = my_p / den;
}

// ------------------------------------------------------------------------------------------------ dispatch
// One work-group of 1024 threads.  counts by LDS atomics (order-free), offsets by an exclusive scan,
// ranks by a ballot match inside each wave and per-wave counts in LDS, 1024 pairs per pass, so a pair's
// position is offsets[e] + (number of earlier pairs with the same expert): the stable counting sort of the
// oracle's or_dispatch.  Also the ascending list of touched experts.
__device__ __forceinline__ int block_exclusive_scan_1024(int v, int* scratch /*>= 17 ints*/, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += u;
    }
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int w = 0; w < 16; ++w) {
            const int c = scratch[w];
            scratch[w] = run;
            run += c;
        }
        scratch[16] = run;
    }
    __syncthreads();
    const int r = scratch[wave] + incl - v;
    *total = scratch[16];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t* __restrict__ ids, int P, int E,
                                                    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                    int32_t* __restrict__ perm, int32_t* __restrict__ slot,
                                                    int32_t* __restrict__ elist, int32_t* __restrict__ n_list) {
    __shared__ int cnt[1024];
    __shared__ int run[1024];
    __shared__ uint8_t wcnt[16][1024];
    __shared__ int scan_scratch[17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    cnt[tid] = 0;
    for (int w = 0; w < 16; ++w) wcnt[w][tid] = 0;
    __syncthreads();
    for (int i = tid; i < P; i += 1024) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    int total;
    const int off = block_exclusive_scan_1024(c, scan_scratch, &total);
    const int flag = c > 0 ? 1 : 0;
    int n_touched;
    const int fpos = block_exclusive_scan_1024(flag, scan_scratch, &n_touched);
    if (tid < E) {
        if (counts) counts[tid] = c;
        offsets[tid] = off;
        run[tid] = off;
        if (flag && elist) elist[fpos] = tid;
    }
    if (tid == 0) {
        offsets[E] = total;
        if (n_list) *n_list = n_touched;
    }
    __syncthreads();
    const unsigned long long lt = (1ull << lane) - 1ull;
    for (int base = 0; base < P; base += 1024) {
        const int i = base + tid;
        const int id = i < P ? ids[i] : -1;
        const bool valid = id >= 0 && id < E;  // an out-of-range id is not dispatched: slot[i] = -1
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
        if (valid && leader) wcnt[wave][key] = (uint8_t)cnt_w;
        __syncthreads();
        if (valid) {
            int pos = run[key] + rank_w;
            for (int w = 0; w < wave; ++w) pos += wcnt[w][key];
            perm[pos] = i;
            slot[i] = pos;
        }
        __syncthreads();
        if (valid && leader) {
            atomicAdd(&run[key], cnt_w);
            wcnt[wave][key] = 0;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ Q2_0 rows
// A "unit" is one 36-byte double block (two Q2_0 blocks, 128 weights, dword aligned): 9 dwords
//   w0 = {d0, codes0[0..1]}, w1..w3 = codes0[2..13], w4 = {codes0[14..15], d1}, w5..w8 = codes1[0..15].
// Activations for the unit's four q8_1 blocks sit in LDS in the permuted form below.  Unit part
// L = ((P0 + P1) + P2) + P3 with P_h = (f32(d_w) * f32(d_x)) * (float) sumi_h and
// sumi_h = sum(code * q) - sum(q) = sum((code - 1) * q) (metal/shaders/iq.metal:444-456).

// LDS image of one q8_1 block: 8 dwords of q permuted so that dword c of each 16-group holds
// q[c], q[c+4], q[c+8], q[c+12] (the order (codes >> 2c) & 0x03030303 delivers), then f32 d, int sum q.
constexpr int kActDw = 12;  // dwords per q8_1 block image (16-byte aligned)

__device__ __forceinline__ void transpose4x4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t* o) {
    const uint32_t t0 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);  // a0b0 a1b0 a0b1 a1b1
    const uint32_t u0 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);  // a2b0 a3b0 a2b1 a3b1
    const uint32_t t1 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);  // a0b2 a1b2 a0b3 a1b3
    const uint32_t u1 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);  // a2b2 a3b2 a2b3 a3b3
    o[0] = __builtin_amdgcn_perm(u0, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(u0, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(u1, t1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(u1, t1, 0x07060302u);
}

// q8_1 block (9 dwords in global memory) -> LDS image
__device__ __forceinline__ void stage_q8(const uint32_t* __restrict__ src, uint32_t* dst) {
    uint32_t b[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) b[i] = src[i];
    uint32_t o[8];
    transpose4x4(b[1], b[2], b[3], b[4], o);
    transpose4x4(b[5], b[6], b[7], b[8], o + 4);
    int sq = 0;
#pragma unroll
    for (int i = 1; i < 9; ++i) sq = __builtin_amdgcn_sdot4((int)b[i], 0x01010101, sq, false);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    d4[0] = make_uint4(o[0], o[1], o[2], o[3]);
    d4[1] = make_uint4(o[4], o[5], o[6], o[7]);
    d4[2] = make_uint4(f2u(f16_to_f32(b[0] & 0xFFFFu)), (uint32_t)sq, 0u, 0u);
}

__device__ __forceinline__ int q2_half_dot(uint32_t a, uint32_t b, const uint32_t* X) {
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

// act: LDS images of the unit's 4 q8_1 blocks (4 * kActDw dwords)
__device__ __forceinline__ float q2_unit_dot(const uint32_t (&w)[9], const uint32_t* act) {
    const float d0 = f16_to_f32(w[0] & 0xFFFFu);
    const float d1 = f16_to_f32(w[4] >> 16);
    uint32_t c[8];
    c[0] = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
    c[1] = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
    c[2] = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
    c[3] = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
    c[4] = w[5];
    c[5] = w[6];
    c[6] = w[7];
    c[7] = w[8];
    float L = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const uint32_t* X = act + h * kActDw;
        const uint4 x0 = *reinterpret_cast<const uint4*>(X);
        const uint4 x1 = *reinterpret_cast<const uint4*>(X + 4);
        const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float dx = u2f(X[8]);
        const int sq = (int)X[9];
        const int sumi = q2_half_dot(c[2 * h], c[2 * h + 1], xs) - sq;
        const float P = ((h < 2 ? d0 : d1) * dx) * (float)sumi;
        L = h == 0 ? P : L + P;
    }
    return L;
}

__device__ __forceinline__ void load_unit(const uint8_t* p, uint32_t (&w)[9]) {
    // 4-byte aligned (units are 36 bytes from a 4-byte aligned tensor base)
    const uint32_t* q = reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(p, 4));
    __builtin_memcpy(w, q, 36);
}

// Column source of a GEMV tile: token / output row of column c.
struct Cols {
    int n;          // number of columns
    int first;      // first slot (routed) or token (shared)
    const int32_t* perm;  // routed: pair index at each dispatch position; null for the shared expert
    int k;
};

__device__ __forceinline__ int col_token(const Cols& cs, int c) {
    return cs.perm ? cs.perm[cs.first + c] / cs.k : cs.first + c;
}

constexpr int kColBatch = 4;

// ------------------------------------------------------------------------------------------------ gate/up
// Grid (FF/32, max work items).  Work item wi < n_list: routed expert elist[wi] with its pairs at
// dispatch positions offsets[e]..offsets[e+1]; wi == n_list (when has_shared): the shared expert with
// every token.  The block computes gate rows [32 hb, 32 hb + 32) and the same up rows for each column,
// SwiGLU, and the q8_1 block hb of h, stored at hq[(slot or P + t) * hq_blocks + hb].
// Row value = ((L_0 + L_1) + ...) over the row's units in order (oracle: or_q2_0_gemv_dev).
template <int MAXU>
__global__ __launch_bounds__(256) void k_q2_gu(const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps,
                                                const uint8_t* __restrict__ gate_sh, const uint8_t* __restrict__ up_sh,
                                                const uint8_t* __restrict__ xq, const int32_t* __restrict__ offsets,
                                                const int32_t* __restrict__ perm, const int32_t* __restrict__ elist,
                                                const int32_t* __restrict__ n_list, int k, int T, int H, int F, int Fs,
                                                int has_shared, int P, uint8_t* __restrict__ hq, int hq_blocks) {
    extern __shared__ __align__(16) uint32_t smem[];
    const int hb = blockIdx.x;
    const int wi = blockIdx.y;
    const int nl = *n_list;
    const bool shared = has_shared && wi == nl;
    if (wi > nl || (wi == nl && !shared)) return;
    const int Fe = shared ? Fs : F;
    if (hb * 32 >= Fe) return;
    const int e = shared ? -1 : elist[wi];
    const int dpr = H >> 7;
    const size_t rb = (size_t)dpr * 36;
    const uint8_t* g0 = shared ? gate_sh : gate_exps + (size_t)e * F * rb;
    const uint8_t* u0 = shared ? up_sh : up_exps + (size_t)e * F * rb;
    g0 += (size_t)hb * 32 * rb;
    u0 += (size_t)hb * 32 * rb;
    const int half_units = 32 * dpr;
    const int nunits = 2 * half_units;

    uint32_t w[MAXU][9];
#pragma unroll
    for (int j = 0; j < MAXU; ++j) {
        const int u = threadIdx.x + 256 * j;
        if (u < nunits) load_unit(u < half_units ? g0 + (size_t)u * 36 : u0 + (size_t)(u - half_units) * 36, w[j]);
    }

    Cols cs;
    if (shared) cs = Cols{T, 0, nullptr, k};
    else cs = Cols{offsets[e + 1] - offsets[e], offsets[e], perm, k};

    const int qb_per_col = H >> 5;
    const int lp_stride = dpr + 1;
    uint32_t* act = smem;                                         // kColBatch * qb_per_col * kActDw
    float* lp = reinterpret_cast<float*>(act + kColBatch * qb_per_col * kActDw);  // kColBatch * 64 * lp_stride
    float* gu = lp + kColBatch * 64 * lp_stride;                  // kColBatch * 64

    for (int c0 = 0; c0 < cs.n; c0 += kColBatch) {
        const int nb = min(kColBatch, cs.n - c0);
        for (int idx = threadIdx.x; idx < nb * qb_per_col; idx += 256) {
            const int c = idx / qb_per_col, qb = idx - c * qb_per_col;
            const int tok = col_token(cs, c0 + c);
            stage_q8(reinterpret_cast<const uint32_t*>(xq + ((size_t)tok * qb_per_col + qb) * 36),
                     act + (c * qb_per_col + qb) * kActDw);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MAXU; ++j) {
            const int u = threadIdx.x + 256 * j;
            if (u < nunits) {
                const int r = u / dpr, g = u - r * dpr;
                for (int c = 0; c < nb; ++c)
                    lp[(c * 64 + r) * lp_stride + g] = q2_unit_dot(w[j], act + (c * qb_per_col + 4 * g) * kActDw);
            }
        }
        __syncthreads();
        {
            const int c = threadIdx.x >> 6, r = threadIdx.x & 63;
            if (c < nb) {
                const float* s = lp + (c * 64 + r) * lp_stride;
                float acc = s[0];
                for (int g = 1; g < dpr; ++g) acc = acc + s[g];
                gu[c * 64 + r] = acc;
            }
        }
        __syncthreads();
        {
            const int c = threadIdx.x >> 6, l = threadIdx.x & 63;
            if (c < nb) {
                const float h = l < 32 ? silu_mul(gu[c * 64 + l], gu[c * 64 + 32 + l]) : 0.0f;
                uint32_t ds;
                const int q = q8_1_value(h, &ds);
                const int row = shared ? P + (c0 + c) : cs.first + c0 + c;
                if (l < 32) q8_1_store(q, ds, hq + ((size_t)row * hq_blocks + hb) * 36);
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ down
// Grid (H/64, max work items).  Rows [64 bx, 64 bx + 64) of the work item's down matrix against each
// column's q8_1 h; the shared rows are multiplied by sigmoid(sg[t]) (metal/shaders/shared_expert.metal:24-32).
template <int MAXU>
__global__ __launch_bounds__(256) void k_q2_down(const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh,
                                                  const uint8_t* __restrict__ hq, int hq_blocks, const float* __restrict__ sg,
                                                  const int32_t* __restrict__ offsets, const int32_t* __restrict__ elist,
                                                  const int32_t* __restrict__ n_list, int T, int H, int F, int Fs,
                                                  int has_shared, int P, float* __restrict__ Y) {
    extern __shared__ __align__(16) uint32_t smem[];
    const int bx = blockIdx.x;
    const int wi = blockIdx.y;
    const int nl = *n_list;
    const bool shared = has_shared && wi == nl;
    if (wi > nl || (wi == nl && !shared)) return;
    const int Fe = shared ? Fs : F;
    const int e = shared ? -1 : elist[wi];
    const int dpr = Fe >> 7;
    const size_t rb = (size_t)dpr * 36;
    const uint8_t* base = (shared ? down_sh : down_exps + (size_t)e * H * ((size_t)(F >> 7) * 36)) + (size_t)bx * 64 * rb;
    const int nrows = min(64, H - bx * 64);
    const int nunits = nrows * dpr;

    uint32_t w[MAXU][9];
#pragma unroll
    for (int j = 0; j < MAXU; ++j) {
        const int u = threadIdx.x + 256 * j;
        if (u < nunits) load_unit(base + (size_t)u * 36, w[j]);
    }
    const int ncol = shared ? T : offsets[e + 1] - offsets[e];
    const int first = shared ? P : offsets[e];

    const int qb_per_col = Fe >> 5;
    const int lp_stride = dpr + 1;
    uint32_t* act = smem;
    float* lp = reinterpret_cast<float*>(act + kColBatch * qb_per_col * kActDw);

    for (int c0 = 0; c0 < ncol; c0 += kColBatch) {
        const int nb = min(kColBatch, ncol - c0);
        for (int idx = threadIdx.x; idx < nb * qb_per_col; idx += 256) {
            const int c = idx / qb_per_col, qb = idx - c * qb_per_col;
            stage_q8(reinterpret_cast<const uint32_t*>(hq + ((size_t)(first + c0 + c) * hq_blocks + qb) * 36),
                     act + (c * qb_per_col + qb) * kActDw);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MAXU; ++j) {
            const int u = threadIdx.x + 256 * j;
            if (u < nunits) {
                const int r = u / dpr, g = u - r * dpr;
                for (int c = 0; c < nb; ++c)
                    lp[(c * 64 + r) * lp_stride + g] = q2_unit_dot(w[j], act + (c * qb_per_col + 4 * g) * kActDw);
            }
        }
        __syncthreads();
        {
            const int c = threadIdx.x >> 6, r = threadIdx.x & 63;
            if (c < nb && r < nrows) {
                const float* s = lp + (c * 64 + r) * lp_stride;
                float acc = s[0];
                for (int g = 1; g < dpr; ++g) acc = acc + s[g];
                const int yrow = first + c0 + c;
                if (shared) acc = acc * sigmoid(sg[c0 + c]);
                Y[(size_t)yrow * H + bx * 64 + r] = acc;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ combine
// y[t][j] = w0 * Y[slot0][j], then fma in selection order, then + shared (include/strata/kernels/native_moe.hpp:10-15).
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ Y, const int32_t* __restrict__ slot,
                                                  const float* __restrict__ wts, int k, int H, int P, int add_shared,
                                                  float* __restrict__ y) {
    const int t = blockIdx.y;
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= H) return;
    const int32_t* sl = slot + (size_t)t * k;
    const float* wt = wts + (size_t)t * k;
    float acc = wt[0] * Y[(size_t)sl[0] * H + j];
    for (int s = 1; s < k; ++s) acc = __builtin_fmaf(wt[s], Y[(size_t)sl[s] * H + j], acc);
    if (add_shared) acc = acc + Y[(size_t)(P + t) * H + j];
    y[(size_t)t * H + j] = acc;
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

// SwiGLU + q8_1 over a flat vector (n % 32 == 0).
__global__ __launch_bounds__(256) void k_swiglu_q8(const float* __restrict__ gate, const float* __restrict__ up,
                                                    int64_t n, uint8_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;
    const float h = live ? silu_mul(gate[i], up[i]) : 0.0f;
    uint32_t ds;
    const int q = q8_1_value(h, &ds);
    if ((i - (threadIdx.x & 31)) < n) q8_1_store(q, ds, y + (i >> 5) * 36);
}

// Generic Q2_0 GEMV over n_col columns of q8_1 activations (iq_mmvq's contract, metal/src/iq.mm:148-169):
// grid (ceil(n_out / 64), 1); same unit order as the expert kernels.
template <int MAXU>
__global__ __launch_bounds__(256) void k_q2_mmvq(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xq, int n_in,
                                                  int n_out, int n_col, float* __restrict__ y) {
    extern __shared__ __align__(16) uint32_t smem[];
    const int bx = blockIdx.x;
    const int dpr = n_in >> 7;
    const size_t rb = (size_t)dpr * 36;
    const uint8_t* base = w + (size_t)bx * 64 * rb;
    const int nrows = min(64, n_out - bx * 64);
    const int nunits = nrows * dpr;
    uint32_t wr[MAXU][9];
#pragma unroll
    for (int j = 0; j < MAXU; ++j) {
        const int u = threadIdx.x + 256 * j;
        if (u < nunits) load_unit(base + (size_t)u * 36, wr[j]);
    }
    const int qb_per_col = n_in >> 5;
    const int lp_stride = dpr + 1;
    uint32_t* act = smem;
    float* lp = reinterpret_cast<float*>(act + kColBatch * qb_per_col * kActDw);
    for (int c0 = 0; c0 < n_col; c0 += kColBatch) {
        const int nb = min(kColBatch, n_col - c0);
        for (int idx = threadIdx.x; idx < nb * qb_per_col; idx += 256) {
            const int c = idx / qb_per_col, qb = idx - c * qb_per_col;
            stage_q8(reinterpret_cast<const uint32_t*>(xq + ((size_t)(c0 + c) * qb_per_col + qb) * 36),
                     act + (c * qb_per_col + qb) * kActDw);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MAXU; ++j) {
            const int u = threadIdx.x + 256 * j;
            if (u < nunits) {
                const int r = u / dpr, g = u - r * dpr;
                for (int c = 0; c < nb; ++c)
                    lp[(c * 64 + r) * lp_stride + g] = q2_unit_dot(wr[j], act + (c * qb_per_col + 4 * g) * kActDw);
            }
        }
        __syncthreads();
        {
            const int c = threadIdx.x >> 6, r = threadIdx.x & 63;
            if (c < nb && r < nrows) {
                const float* s = lp + (c * 64 + r) * lp_stride;
                float acc = s[0];
                for (int g = 1; g < dpr; ++g) acc = acc + s[g];
                y[(size_t)(c0 + c) * n_out + bx * 64 + r] = acc;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ launchers

size_t gemv_lds_bytes(int n_in) {
    const int dpr = n_in >> 7;
    return (size_t)kColBatch * (n_in >> 5) * kActDw * 4 + (size_t)kColBatch * 64 * (dpr + 1) * 4 + kColBatch * 64 * 4;
}

hipError_t launch_prep(const float* x, int64_t n, uint8_t* xq, uint16_t* xb, hipStream_t s) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(k_prep, dim3(blocks), dim3(256), 0, s, x, n, xq, xb);
    return hipGetLastError();
}

hipError_t launch_router(const uint16_t* xb, const uint16_t* W, const uint16_t* w_inp, const float* bias, int H, int E,
                         int rows_total, int T, float* logits, int ld_logits, float* sg, hipStream_t s) {
    const int chunks = H / 8;
    const int maxc = (chunks + 63) / 64;
    const int tok_per_block = T <= 16 ? T : 16;
    dim3 grid((unsigned)((rows_total + 3) / 4), (unsigned)((T + tok_per_block - 1) / tok_per_block));
#define SMOE_ROUTER(C)                                                                                         \
    hipLaunchKernelGGL(k_router<C>, grid, dim3(256), 0, s, xb, W, w_inp, bias, H, E, rows_total, T, tok_per_block, \
                       logits, ld_logits, sg)
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
                           int32_t* slot, int32_t* elist, int32_t* n_list, hipStream_t s) {
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, ids, P, E, counts, offsets, perm, slot, elist, n_list);
    return hipGetLastError();
}

hipError_t launch_q2_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint8_t* xq, const int32_t* offsets, const int32_t* perm, const int32_t* elist,
                        const int32_t* n_list, int k, int T, int H, int F, int Fs, int has_shared, int P, int max_items,
                        uint8_t* hq, int hq_blocks, hipStream_t s) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    dim3 grid((unsigned)(Fmax / 32), (unsigned)max_items);
    const size_t lds = gemv_lds_bytes(H);
    const int units = 64 * (H >> 7);
    const int upt = (units + 255) / 256;
#define SMOE_GU(U)                                                                                                \
    hipLaunchKernelGGL(k_q2_gu<U>, grid, dim3(256), lds, s, gate_exps, up_exps, gate_sh, up_sh, xq, offsets, perm, \
                       elist, n_list, k, T, H, F, Fs, has_shared, P, hq, hq_blocks)
    if (upt <= 2) SMOE_GU(2);
    else if (upt <= 4) SMOE_GU(4);
    else if (upt <= 6) SMOE_GU(6);
    else SMOE_GU(8);
#undef SMOE_GU
    return hipGetLastError();
}

hipError_t launch_q2_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint8_t* hq, int hq_blocks,
                          const float* sg, const int32_t* offsets, const int32_t* elist, const int32_t* n_list, int T,
                          int H, int F, int Fs, int has_shared, int P, int max_items, float* Y, hipStream_t s) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    dim3 grid((unsigned)((H + 63) / 64), (unsigned)max_items);
    const size_t lds = gemv_lds_bytes(Fmax);
    const int units = 64 * (Fmax >> 7);
    const int upt = (units + 255) / 256;
#define SMOE_DOWN(U)                                                                                          \
    hipLaunchKernelGGL(k_q2_down<U>, grid, dim3(256), lds, s, down_exps, down_sh, hq, hq_blocks, sg, offsets, \
                       elist, n_list, T, H, F, Fs, has_shared, P, Y)
    if (upt <= 1) SMOE_DOWN(1);
    else if (upt <= 2) SMOE_DOWN(2);
    else if (upt <= 4) SMOE_DOWN(4);
    else SMOE_DOWN(8);
#undef SMOE_DOWN
    return hipGetLastError();
}

hipError_t launch_combine(const float* Y, const int32_t* slot, const float* wts, int k, int H, int P, int T,
                          int add_shared, float* y, hipStream_t s) {
    dim3 grid((unsigned)((H + 255) / 256), (unsigned)T);
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
    const size_t lds = gemv_lds_bytes(n_in);
    const int units = 64 * (n_in >> 7);
    const int upt = (units + 255) / 256;
    dim3 grid((unsigned)((n_out + 63) / 64));
#define SMOE_MMVQ(U) hipLaunchKernelGGL(k_q2_mmvq<U>, grid, dim3(256), lds, s, w, xq, n_in, n_out, n_col, y)
    if (upt <= 1) SMOE_MMVQ(1);
    else if (upt <= 2) SMOE_MMVQ(2);
    else if (upt <= 4) SMOE_MMVQ(4);
    else SMOE_MMVQ(8);
#undef SMOE_MMVQ
    return hipGetLastError();
}

}  // namespace smoe
