// stratametal_amd/csrc/smoe_prefill.hip - the prefill contract's expert products on bf16 MFMA (gfx950).
//
// Contract (oracle: or_moe_prefill): activations rounded to bf16; Q2_0 weights used exactly as
// (code - 1) * f32(d); SwiGLU in f32; h rounded to bf16 for the down product; f32 accumulation.  The
// reference's float prompt path is a dequantising GEMM (include/strata/prefill/gemm.hpp:28-40,
// include/strata/prefill/kernels.hpp:54-57,97-98, include/strata/prefill/moe_fused.hpp:52-62).
//
// How the exact weights reach the matrix cores.  A 64-weight block contributes
//     d * sum_k (c_k - 1) a_k = d * (sum_k c_k a_k - A),   A = sum_k a_k,
// so the MFMA B operand is the raw code c in {0, 1, 2, 3} (exact in bf16; one v_cvt_scalef32_pk_bf16_fp4
// turns a byte of two 2-bit codes, masked into the low bits of two fp4 nibbles, into two bf16 values with the
// scale 2: fp4 e2m1 nibble c has the value c / 2), the accumulator input of the block's first MFMA is -A
// (carried with every activation record), and the block's f32 result is scaled by d into the running sum.
//
// Activation records.  Each 64-value block of an activation row (x for gate/up, h for down) is one 144-byte
// record: 64 bf16 in MFMA order, then -A as f32, then 12 unused bytes.  Position p = 32 s + 8 q + e holds
// element 16 q + 8 s + pi(e), pi = (0 2 1 3 4 6 5 7): the order in which a lane of quarter q meets the
// codes of code dword q of the block in the two 32-deep MFMA steps s.
//
// MFMA tiles (v_mfma_f32_16x16x32_bf16, lane l = 16 q + i): A[i][k] = activation of token i, B[k][j] = code
// of weight row j, C[4 q + r][j] in register r.  A work-group of 4 waves owns 64 weight rows (gate/up: 64
// rows of each) and a work item of at most 128 tokens (8 tiles of 16); each wave owns 16 rows and every tile.
// The raw Q2_0 rows and the tile's activation records are staged in LDS one 128-value unit (two blocks) at a
// time; the codes are expanded in registers and reused across the token tiles.
#include "smoe_device.hpp"
#include "smoe_items.hpp"
#include "smoe_launch.hpp"

#include <climits>

namespace smoe {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int kRecDw = 36;       // dwords per activation record
constexpr int kChunk = 64;       // tokens per work item
constexpr int kTiles = kChunk / 16;
constexpr int kActStride = 76;   // LDS dwords per staged token: two records + 4 dwords against bank conflicts

__device__ __forceinline__ int perm8(int e) { return (e == 1 || e == 5) ? e + 1 : (e == 2 || e == 6) ? e - 1 : e; }
// record position of block element kappa (pi is an involution)
__device__ __forceinline__ int rec_pos(int kappa) {
    return 32 * ((kappa >> 3) & 1) + 8 * (kappa >> 4) + perm8(kappa & 7);
}

// ------------------------------------------------------------------------------------------------ records of x
// One thread per 8 positions (a 16-byte chunk) of a record; eight consecutive lanes form one record and add
// their chunk sums by an xor butterfly for -A.
__global__ __launch_bounds__(256) void k_act_records(const float* __restrict__ x, int64_t n_rec,
                                                     uint32_t* __restrict__ rec) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t r = g >> 3;
    const int ch = (int)(g & 7);
    const bool live = r < n_rec;
    const int s = ch >> 2, q = ch & 3;
    float v[8];
    if (live) {
        const float4* src = reinterpret_cast<const float4*>(x + r * 64 + 16 * q + 8 * s);
        const float4 lo = src[0], hi = src[1];
        v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
        v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = f32_to_bf16(v[perm8(e)]);
    float sm = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sm = sm + bf16_to_f32(b[e]);
    sm = sm + __shfl_xor(sm, 1, kWave);
    sm = sm + __shfl_xor(sm, 2, kWave);
    sm = sm + __shfl_xor(sm, 4, kWave);
    if (live) {
        uint32_t* dst = rec + r * kRecDw;
        reinterpret_cast<uint4*>(dst)[ch] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                                                       b[6] | (b[7] << 16));
        if (ch == 0) dst[32] = f2u(-sm);
    }
}

// ------------------------------------------------------------------------------------------------ codes -> B
__device__ __forceinline__ bf16x8 cat4(bf16x2 a, bf16x2 b, bf16x2 c, bf16x2 d) {
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}

// Code dword cw (16 codes) -> the B operands of the two 32-deep steps: x holds codes 0, 2 of each byte in
// the low bits of its nibbles, y codes 1, 3.
__device__ __forceinline__ void expand_codes(uint32_t cw, bf16x8& s0, bf16x8& s1) {
    const uint32_t x = cw & 0x33333333u, y = (cw >> 2) & 0x33333333u;
    s0 = cat4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 0), __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(y, 2.0f, 0),
              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 1), __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(y, 2.0f, 1));
    s1 = cat4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 2), __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(y, 2.0f, 2),
              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 3), __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(y, 2.0f, 3));
}

// Staging of one 128-value unit through registers: the global loads of unit u + 1 are issued before the
// matrix work on unit u, and land in LDS after it.  Thread t loads the 36-byte unit of weight row t
// (t < nrows) and up to kStageA 16-byte chunks of the columns' activation records: chunk idx = t + 256 m is
// column idx / 18, record (idx % 18) / 9 of the unit, 16-byte piece idx % 9 (piece 8 carries -A).
constexpr int kStageA = (kChunk * 18 + 255) / 256;
constexpr int kDeadSlot = kChunk * (kActStride / 4);  // 16-byte slot past the staged columns

struct Stager {
    const uint8_t* wrow;            // this thread's weight row (a valid row for every thread; stored if has_w)
    const uint32_t* __restrict__ recs;
    bool has_w;
    uint32_t src[kStageA];          // dword offset of chunk m in unit 0 (0 when unused: a harmless valid load)
    int dst[kStageA];               // 16-byte slot in the staged activations (kDeadSlot when unused)
    uint32_t w[9];
    uint4 a[kStageA];

    // Every load and store is unconditional (unused slots read a valid address and land in a dead slot) so that
    // the loads issue back to back and the stores need no branches.
    __device__ void init(const uint8_t* row, bool has_row, const uint32_t* r, const int* rowidx, int ncol,
                         int rec_per_row) {
        wrow = row;
        has_w = has_row;
        recs = r;
#pragma unroll
        for (int m = 0; m < kStageA; ++m) {
            const int idx = (int)threadIdx.x + 256 * m, c = idx / 18, p = idx - 18 * c, h = p >= 9 ? 1 : 0,
                      ch = p - 9 * h;
            const bool live = c < ncol;
            src[m] = live ? (uint32_t)(((size_t)rowidx[c] * rec_per_row + h) * kRecDw + 4 * ch) : 0u;
            dst[m] = live ? c * (kActStride / 4) + h * (kRecDw / 4) + ch : kDeadSlot;
        }
    }
    __device__ void load(int u) {
        __builtin_memcpy(w, __builtin_assume_aligned(wrow + (size_t)u * 36, 4), 36);
#pragma unroll
        for (int m = 0; m < kStageA; ++m) a[m] = *reinterpret_cast<const uint4*>(recs + src[m] + (size_t)u * 2 * kRecDw);
    }
    __device__ void store(uint32_t* wt, uint4* act) const {
        if (has_w) {
#pragma unroll
            for (int i = 0; i < 9; ++i) wt[threadIdx.x * 9 + i] = w[i];
        }
#pragma unroll
        for (int m = 0; m < kStageA; ++m) act[dst[m]] = a[m];
    }
};

// -A of block h for the four tokens 4 q .. 4 q + 3 of tile n (record dword 32 of each token's staged record)
__device__ __forceinline__ f32x4 neg_sums(const uint32_t* act, int n, int h, int q) {
    const uint32_t* p = act + (16 * n + 4 * q) * kActStride + h * kRecDw + 32;
    return f32x4{u2f(p[0]), u2f(p[kActStride]), u2f(p[2 * kActStride]), u2f(p[3 * kActStride])};
}

// One staged unit against NS weight-row sets per wave: for block h of the unit, the B operands of the NS sets
// (lane row i of set s at LDS row rows[s]) are expanded, then every live token tile n loads its activation
// fragments once and feeds all NS sets: acc[n][s] += d_s * (C = -A; C += A0 B0; C += A1 B1).
template <int NS>
__device__ __forceinline__ void mma_unit(f32x4 (&acc)[kTiles][NS], const uint32_t* wt, const int (&rows)[NS],
                                         const uint32_t* act, int ntiles, int i, int q) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bf16x8 b0[NS], b1[NS];
        float d[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t* w = wt + rows[s] * 9;
            const uint32_t cw = h == 0 ? __builtin_amdgcn_alignbyte(w[q + 1], w[q], 2) : w[5 + q];
            d[s] = h == 0 ? (float)__builtin_bit_cast(_Float16, (uint16_t)(w[0] & 0xFFFFu))
                          : (float)__builtin_bit_cast(_Float16, (uint16_t)(w[4] >> 16));
            expand_codes(cw, b0[s], b1[s]);
        }
#pragma unroll
        for (int n = 0; n < kTiles; ++n) {
            if (n < ntiles) {
                const uint32_t* ar = act + (16 * n + i) * kActStride + h * kRecDw;
                const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(ar + 4 * q);
                const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(ar + 16 + 4 * q);
                const f32x4 na = neg_sums(act, n, h, q);
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0[s], na, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[s], c, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[n][s][r] = __builtin_fmaf(d[s], c[r], acc[n][s][r]);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ gate/up
// Grid (Fmax / 128, work items).  Work-group rt of an item computes gate and up rows [128 rt, 128 rt + 128)
// for the item's columns: wave w the rows 32 w .. 32 w + 31 of each (sets 0, 1 gate; 2, 3 up), then
// h = bf16(silu(gate) * up) into records 2 rt and 2 rt + 1 of each column's h row.
__global__ __launch_bounds__(256) void k_mm_gu(const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps,
                                               const uint8_t* __restrict__ gate_sh, const uint8_t* __restrict__ up_sh,
                                               const uint32_t* __restrict__ xrec, const int4* __restrict__ items,
                                               const int32_t* __restrict__ perm, int k, int H, int F, int Fs,
                                               uint32_t* __restrict__ hrec, int h_rec) {
    __shared__ uint32_t wt[256 * 9];
    __shared__ __align__(16) uint32_t act[kChunk * kActStride + 4];
    __shared__ int rowidx[kChunk];
    Item item;
    if (!work_item(items, blockIdx.y, item)) return;
    const int rt = blockIdx.x;
    const int Fe = item.shared ? Fs : F;
    if (128 * rt >= Fe) return;
    const int ncol = item.ncol, ntiles = (ncol + 15) >> 4;
    const int units = H >> 7;
    const size_t rb = (size_t)units * 36;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, i = lane & 15, q = lane >> 4;
    for (int c = tid; c < ncol; c += 256) rowidx[c] = item_token(item, perm, k, c);
    __syncthreads();
    Stager stg;
    {
        const uint8_t* base = tid < 128 ? (item.shared ? gate_sh : gate_exps + (size_t)item.e * F * rb)
                                        : (item.shared ? up_sh : up_exps + (size_t)item.e * F * rb);
        stg.init(base + (size_t)(128 * rt + (tid & 127)) * rb, true, xrec, rowidx, ncol, H >> 6);
    }
    stg.load(0);
    const int rows[4] = {32 * wave + i, 32 * wave + 16 + i, 128 + 32 * wave + i, 128 + 32 * wave + 16 + i};

    f32x4 acc[kTiles][4];
#pragma unroll
    for (int n = 0; n < kTiles; ++n)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[n][s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int u = 0; u < units; ++u) {
        stg.store(wt, reinterpret_cast<uint4*>(act));
        __syncthreads();
        if (u + 1 < units) stg.load(u + 1);
        mma_unit<4>(acc, wt, rows, act, ntiles, i, q);
        __syncthreads();
    }
    // h tile [column][128 rows in record order] as bf16 in the activation buffer
    uint16_t* ht = reinterpret_cast<uint16_t*>(act);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int f = 32 * wave + 16 * s + i;  // row within the work-group's 128
        const int pos = 64 * (f >> 6) + rec_pos(f & 63);
#pragma unroll
        for (int n = 0; n < kTiles; ++n) {
            if (n < ntiles) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = 16 * n + 4 * q + r;
                    if (c < ncol) ht[c * 128 + pos] = (uint16_t)f32_to_bf16(silu_mul(acc[n][s][r], acc[n][s + 2][r]));
                }
            }
        }
    }
    __syncthreads();
    for (int base = 0; base < ncol * 16; base += 256) {  // 16 chunks (two records) per column
        const int idx = base + tid, c = idx >> 4, rr = (idx >> 3) & 1, ch = idx & 7;
        const bool live = c < ncol;
        const uint4 v = live ? reinterpret_cast<const uint4*>(ht + c * 128 + 64 * rr)[ch] : make_uint4(0, 0, 0, 0);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
        float sm = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) sm = (sm + u2f(wv[m] << 16)) + u2f(wv[m] & 0xFFFF0000u);
        sm = sm + __shfl_xor(sm, 1, kWave);
        sm = sm + __shfl_xor(sm, 2, kWave);
        sm = sm + __shfl_xor(sm, 4, kWave);
        if (live) {
            uint32_t* dst = hrec + ((size_t)(item.first + c) * h_rec + 2 * rt + rr) * kRecDw;
            reinterpret_cast<uint4*>(dst)[ch] = v;
            if (ch == 0) dst[32] = f2u(-sm);
        }
    }
}

// ------------------------------------------------------------------------------------------------ down
// Grid (H / 128, work items).  Work-group rt computes down rows [128 rt, 128 rt + 128) of the item's columns
// (wave w rows 32 w .. 32 w + 31, two sets) into Y[first + c] (the shared expert's rows times sigmoid(sg[t])).
__global__ __launch_bounds__(256) void k_mm_down(const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh,
                                                 const uint32_t* __restrict__ hrec, int h_rec, const float* __restrict__ sg,
                                                 const int4* __restrict__ items, int H, int F, int Fs,
                                                 float* __restrict__ Y) {
    __shared__ uint32_t wt[128 * 9];
    __shared__ __align__(16) uint32_t act[kChunk * kActStride + 4];
    __shared__ int rowidx[kChunk];
    Item item;
    if (!work_item(items, blockIdx.y, item)) return;
    const int rt = blockIdx.x;
    const int Fe = item.shared ? Fs : F;
    const int ncol = item.ncol, ntiles = (ncol + 15) >> 4;
    const int units = Fe >> 7;
    const size_t rb = (size_t)units * 36;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, i = lane & 15, q = lane >> 4;
    for (int c = tid; c < ncol; c += 256) rowidx[c] = item.first + c;
    __syncthreads();
    Stager stg;
    {
        const uint8_t* base = item.shared ? down_sh : down_exps + (size_t)item.e * H * ((size_t)(F >> 7) * 36);
        stg.init(base + (size_t)(128 * rt + (tid & 127)) * rb, tid < 128, hrec, rowidx, ncol, h_rec);
    }
    stg.load(0);
    const int rows[2] = {32 * wave + i, 32 * wave + 16 + i};

    f32x4 acc[kTiles][2];
#pragma unroll
    for (int n = 0; n < kTiles; ++n)
#pragma unroll
        for (int s = 0; s < 2; ++s) acc[n][s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int u = 0; u < units; ++u) {
        stg.store(wt, reinterpret_cast<uint4*>(act));
        __syncthreads();
        if (u + 1 < units) stg.load(u + 1);
        mma_unit<2>(acc, wt, rows, act, ntiles, i, q);
        __syncthreads();
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int col = 128 * rt + 32 * wave + 16 * s + i;
#pragma unroll
        for (int n = 0; n < kTiles; ++n) {
            if (n < ntiles) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = 16 * n + 4 * q + r;
                    if (c < ncol) {
                        float v = acc[n][s][r];
                        if (item.shared) v = v * sigmoid(sg[item.tok0 + c]);
                        Y[(size_t)(item.first + c) * H + col] = v;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ launchers
int mfma_chunk() { return kChunk; }
size_t act_rec_bytes(int64_t n_rec) { return (size_t)n_rec * kRecDw * 4; }

hipError_t launch_act_records(const float* x, int64_t n_rec, uint32_t* rec, hipStream_t s) {
    hipLaunchKernelGGL(k_act_records, dim3((unsigned)((n_rec * 8 + 255) / 256)), dim3(256), 0, s, x, n_rec, rec);
    return hipGetLastError();
}

hipError_t launch_mm_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint32_t* xrec, const int4* items, const int32_t* perm, int k, int H, int F, int Fs,
                        int has_shared, int max_items, uint32_t* hrec, int h_rec, hipStream_t s) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    hipLaunchKernelGGL(k_mm_gu, dim3((unsigned)(Fmax / 128), (unsigned)max_items), dim3(256), 0, s, gate_exps, up_exps,
                       gate_sh, up_sh, xrec, items, perm, k, H, F, Fs, hrec, h_rec);
    return hipGetLastError();
}

hipError_t launch_mm_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* hrec, int h_rec,
                          const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_mm_down, dim3((unsigned)(H / 128), (unsigned)max_items), dim3(256), 0, s, down_exps, down_sh,
                       hrec, h_rec, sg, items, H, F, Fs, Y);
    return hipGetLastError();
}

}  // namespace smoe
