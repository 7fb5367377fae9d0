// stratametal_amd/csrc/smoe_iq2.hip - IQ2_S (ggml type 22) expert products of the decode contract (gfx950).
//
// IQ2_S block: 82 bytes for 256 weights: fp16 d @0, qs[32] @2 (grid index low bytes), signs[32] @34, qh[8]
// @66 (grid index high bits, 2 per group), scales[8] @74 (two 4-bit scales per 32-weight sub-block).  The dot
// of sub-block ib against a q8_1 block (metal/shaders/iq.metal:152-180; oracle iq2s_partial):
//     sum0 / sum1 = integer dots of groups 0-1 / 2-3 (8 weights each, magnitude grid[idx] with signs),
//     sumi = (sum0 * ls0 + sum1 * ls1 + (sum0 + sum1) / 2) / 4   (C integer division),
//     P = (f32(d_w) * f32(d_x)) * (float) sumi.
//
// A lane owns one block of a row.  It decodes the block once per work item into 64 dwords of signed int8
// weights (natural order), then every column costs 8 v_dot4_i32_i8 per sub-block.  The decode folds the
// signs into the magnitude lookup: the LDS table holds each grid entry's eight magnitude indices (0..2) as
// bytes, and one v_perm over the byte table {8, 25, 43, 0, -8, -25, -43, 0} with selector index | 4 * sign
// yields four signed weights.
//
// Device order (oracle: or_iq2_s_gemv_dev): lane value L = ((P_0 + P_1) + ...) + P_7 over its block's
// sub-blocks; the row is the xor butterfly over the row's nb lanes, distance nb / 2 first (nb = blocks per
// row, a power of two).
//
// Activations are q8_1 images in natural order (image dword c holds q[4c .. 4c + 3]).
#include "smoe_gemv.hpp"
#include "smoe_launch.hpp"

namespace smoe {

// The grid as LDS wants it, built at compile time from the codes: entry i = the eight 2-bit magnitude indices of
// grid entry i, one per byte (low dword: weights 0-3).  A work-group copies the 8 KB into LDS with 16-byte loads.
namespace {
constexpr uint16_t kIq2sCodeList[1024] = {
#include "iq2s_grid_codes.inc"
};
constexpr int kIq2sTabEntries = 1024;
constexpr int kIq2sTabPieces = kIq2sTabEntries / 2;  // 16-byte pieces
struct Iq2sTable {
    uint64_t e[kIq2sTabEntries];
};
constexpr Iq2sTable make_iq2s_table() {
    Iq2sTable t{};
    for (int i = 0; i < 1024; ++i) {
        const uint32_t c = kIq2sCodeList[i];
        uint64_t lo = 0, hi = 0;
        for (int q = 0; q < 4; ++q) {
            lo |= (uint64_t)((c >> (2 * q)) & 3u) << (8 * q);
            hi |= (uint64_t)((c >> (8 + 2 * q)) & 3u) << (8 * q);
        }
        t.e[i] = lo | (hi << 32);
    }
    return t;
}
__device__ const Iq2sTable kIq2sTab = make_iq2s_table();
}  // namespace

constexpr uint32_t kMagPos = 0x002B1908u;  // bytes 8, 25, 43, 0
constexpr uint32_t kMagNeg = 0x00D5E7F8u;  // bytes -8, -25, -43, 0

// The LDS table in two steps, so that a kernel can issue the table loads first and its other loads behind them:
// grid_codes_load (16-byte pieces tid + NTH j, unconditional), grid_table_store (waits for those loads alone).
// Pieces per thread of the table copy (the last round is partial).
template <int NTH>
constexpr int kTabRounds = (kIq2sTabPieces + NTH - 1) / NTH;
template <int NTH>
__device__ __forceinline__ void grid_codes_load(uint4 (&c)[kTabRounds<NTH>]) {
    const uint4* src = reinterpret_cast<const uint4*>(kIq2sTab.e);
#pragma unroll
    for (int j = 0; j < kTabRounds<NTH>; ++j) {
        const int i = (int)threadIdx.x + NTH * j;
        c[j] = src[i < kIq2sTabPieces ? i : 0];
    }
}
template <int NTH>
__device__ __forceinline__ void grid_table_store(const uint4 (&c)[kTabRounds<NTH>], uint2* tab) {
#pragma unroll
    for (int j = 0; j < kTabRounds<NTH>; ++j) {
        const int i = (int)threadIdx.x + NTH * j;
        if (i < kIq2sTabPieces) reinterpret_cast<uint4*>(tab)[i] = c[j];
    }
}

// Four signed weights from four magnitude indices (bytes) and their four sign bits.
__device__ __forceinline__ uint32_t signed_mags(uint32_t idx4, uint32_t nib) {
    // sign bit j -> bit 2 of byte j (a 24-bit multiply: nib < 16, the product < 2^28, the four partial products
    // in disjoint bits)
    const uint32_t sel = (__umul24(nib, 0x00810204u) & 0x04040404u) | idx4;
    return __builtin_amdgcn_perm(kMagNeg, kMagPos, sel);
}

struct Iq2Block {
    uint32_t w[64];  // signed int8 weights: dword 2 (4 ib + grp) + h = weights 8 (4 ib + grp) + 4 h .. + 3
    uint32_t sc[2];  // the eight scale bytes
    float d;
};

// Block b of a row (rows are a whole number of block pairs, 164 bytes, so dword aligned).  Every field after the
// scale (qs @2, signs @34, qh @66, scales @74) starts at byte 2 modulo 4, so the block is loaded so that each
// field dword is one alignbyte of two raw dwords with a per-lane shift: an even block's 80 bytes from its first
// byte (shift 2), an odd block's from its byte 2 (shift 0, the pair's bytes 84 .. 163); raw[20] is the pair's
// dword 20 for both (the even block's bytes 80-83, the odd block's scale in its high half).  Returns the shift.
__device__ __forceinline__ uint32_t load_block_raw(const uint8_t* row, int b, uint32_t (&raw)[21]) {
    const uint8_t* pair = row + (size_t)(b >> 1) * 164;
    __builtin_memcpy(raw, __builtin_assume_aligned(pair + ((b & 1) ? 84 : 0), 4), 80);
    raw[20] = *reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(pair + 80, 4));
    return (b & 1) ? 0u : 2u;
}

__device__ __forceinline__ void decode_block(const uint32_t (&raw)[21], uint32_t sh, const uint2* __restrict__ tab,
                                             Iq2Block& B) {
    // field dword m (m = 0 .. 19 from byte 2: qs 0-7, signs 8-15, qh 16-17, scales 18-19)
    auto fd = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
    const uint32_t dbits = sh ? (raw[0] & 0xFFFFu) : (raw[20] >> 16);
    B.d = (float)__builtin_bit_cast(_Float16, (uint16_t)dbits);
    const uint32_t qh0 = fd(16), qh1 = fd(17);  // qh bytes 0..3, 4..7
    B.sc[0] = fd(18);
    B.sc[1] = fd(19);
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t qsd = fd(ib);
        const uint32_t sgd = fd(8 + ib);
        const uint32_t qhd = ib < 4 ? qh0 : qh1;
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            const uint32_t idx = ((qsd >> (8 * grp)) & 0xFFu) | (((qhd >> (8 * (ib & 3) + 2 * grp)) & 3u) << 8);
            const uint2 e = tab[idx];
            const uint32_t sb = (sgd >> (8 * grp)) & 0xFFu;
            B.w[2 * (4 * ib + grp)] = signed_mags(e.x, sb & 15u);
            B.w[2 * (4 * ib + grp) + 1] = signed_mags(e.y, sb >> 4);
        }
    }
}

// Marks the decoded weights as rewritten, so the compiler keeps them as they are instead of rematerialising.
template <int NIT>
__device__ __forceinline__ void pin_blocks(Iq2Block (&B)[NIT]) {
#pragma unroll
    for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int i = 0; i < 64; ++i) asm volatile("" : "+v"(B[it].w[i]));
}

// Sub-block ib against one natural-order q8_1 image (8 dwords of q, then f32 d).
__device__ __forceinline__ float iq2_sub(const Iq2Block& B, int ib, const uint32_t* q, float dx) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) s0 = __builtin_amdgcn_sdot4((int)B.w[8 * ib + c], (int)q[c], s0, false);
#pragma unroll
    for (int c = 4; c < 8; ++c) s1 = __builtin_amdgcn_sdot4((int)B.w[8 * ib + c], (int)q[c], s1, false);
    const uint32_t scb = (B.sc[ib >> 2] >> (8 * (ib & 3))) & 0xFFu;
    const int ls0 = (int)(scb & 15u), ls1 = (int)(scb >> 4);
    // 24-bit multiplies: |s| <= 16 * 43 * 127 < 2^23 and ls <= 15, so the products are exact
    const int v = __mul24(s0, ls0) + __mul24(s1, ls1) + (s0 + s1) / 2;
    const int sumi = (v + (int)(((uint32_t)v >> 31) * 3u)) >> 2;  // v / 4, truncated toward zero
    return (B.d * dx) * (float)sumi;
}

// The block's lane value against a column's images (img = the column's image row, block b's images 8 b ..).
__device__ __forceinline__ float iq2_block_dot_img(const Iq2Block& B, const uint32_t* img, int b) {
    float L = 0.0f;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint4* p = reinterpret_cast<const uint4*>(img + (size_t)lds_blk(8 * b + ib));
        const uint4 lo = p[0], hi = p[1], ds = p[2];
        const uint32_t q[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const float P = iq2_sub(B, ib, q, u2f(ds.x));
        L = ib == 0 ? P : L + P;
    }
    return L;
}

// The same against standard 36-byte q8_1 blocks (the stage API's input).
__device__ __forceinline__ float iq2_block_dot_std(const Iq2Block& B, const uint8_t* __restrict__ xq, int b) {
    float L = 0.0f;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t w9[9];
        __builtin_memcpy(w9, __builtin_assume_aligned(xq + (size_t)(8 * b + ib) * 36, 4), 36);
        const float P = iq2_sub(B, ib, w9 + 1, f16_to_f32(w9[0] & 0xFFFFu));
        L = ib == 0 ? P : L + P;
    }
    return L;
}

// ------------------------------------------------------------------------------------------------ gate/up
// Grid (Fmax / 32, work items), NW = nb waves (64 NW threads).  The work-group computes gate rows
// [32 hb, 32 hb + 32) and the same up rows: row rho = wave * (64 / nb) + lane / nb (rho < 32 gate, else up),
// nb lanes per row, one block per lane, decoded once.  Columns go in stages of 2 NW: their x images are
// copied to LDS, every column's 64 row values parked in LDS, then each half wave quantises one column's 32 h
// values into natural-order image block hb.
// (What a routed item's work-group reads before its image and weight loads is in the first 14 dwords of the
// arguments, which arrive preloaded in SGPRs; the later ones are scalar loads waited for where they are used.)
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_iq2_gu(const int4* __restrict__ items, const uint32_t* __restrict__ ximg,
                                                     const uint8_t* __restrict__ gate_exps,
                                                     const uint8_t* __restrict__ up_exps,
                                                     const uint64_t* __restrict__ eptr, int H, int F, int Fs, int k,
                                                     const uint8_t* __restrict__ gate_sh,
                                                     const uint8_t* __restrict__ up_sh, const int32_t* __restrict__ perm,
                                                     uint32_t* __restrict__ himg, int h_blocks, const StageOut so) {
    constexpr int kCols = 2 * NW;
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ uint2 tab[kIq2sTabEntries];
    __shared__ float rowv[kCols][64];
    __shared__ uint8_t qsc[kCols][32];
    Item item;
    if (!work_item(items, blockIdx.y, item)) return;
    const int hb = blockIdx.x;
    const int Fe = item.shared ? Fs : F;
    if (hb * 32 >= Fe) return;
    const int nb = H >> 8;  // == NW
    const size_t rb = (size_t)nb * 82;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rho = wave * (64 / nb) + lane / nb, b = lane % nb;
    if (eptr && !item.shared) {  // a pointer per routed item: its blob holds the gate rows, then the up rows
        gate_exps = reinterpret_cast<const uint8_t*>(eptr[item.e]);
        up_exps = gate_exps + (size_t)F * rb;
        item.e = 0;
    }
    const uint8_t* base = (rho < 32 ? (item.shared ? gate_sh : gate_exps + (size_t)item.e * F * rb)
                                    : (item.shared ? up_sh : up_exps + (size_t)item.e * F * rb));
    const uint8_t* rowp = base + (size_t)(32 * hb + (rho & 31)) * rb;
    const int qb = H >> 5;
    // loads in the order their data is needed: the grid codes, the first column batch's images (when their rows
    // need no memory read), then the weights; the table store waits for the codes alone, the image commit for
    // the images alone
    uint4 codes[kTabRounds<64 * NW>];
    grid_codes_load<64 * NW>(codes);
    const int nc0 = min(kCols, item.ncol);
    uint32_t raw[21];
    uint32_t off;
    if (stage_direct(item, 0, nc0, true)) {  // straight-line inside each branch, so no wait lands between the loads
        StagePieces sp;
        stage_issue_direct<64 * NW>(sp, ximg, qb, 0, nc0, kCols, 0, item, true);
        __builtin_amdgcn_sched_barrier(0);
        off = load_block_raw(rowp, b, raw);
        __builtin_amdgcn_sched_barrier(0);
        grid_table_store<64 * NW>(codes, tab);
        stage_commit_direct(sp, smem);
    } else {
        off = load_block_raw(rowp, b, raw);
        grid_table_store<64 * NW>(codes, tab);
        stage_images<64 * NW>(smem, ximg, qb, 0, nc0, kCols, item, perm, k, true, 0, 4 * 64 * NW);
    }
    stage_images<64 * NW>(smem, ximg, qb, 0, nc0, kCols, item, perm, k, true, 4 * 64 * NW);  // rounds beyond the first
    __syncthreads();
    Iq2Block B[1];
    decode_block(raw, off, tab, B[0]);

    for (int c0 = 0; c0 < item.ncol; c0 += kCols) {
        const int nc = min(kCols, item.ncol - c0);
        if (c0 > 0) {
            stage_images<64 * NW>(smem, ximg, qb, c0, nc, kCols, item, perm, k, true);
            __syncthreads();
        }
        for (int c = 0; c < nc; ++c) {
            const uint32_t* xt = smem + (size_t)c * qb * kImgLdsDw;
            pin_blocks(B);
            const float v = group_sum(iq2_block_dot_img(B[0], xt, b), nb);
            if (b == 0) rowv[c][rho] = v;
        }
        __syncthreads();
        {
            const int hw = threadIdx.x >> 5;  // half wave = column
            const bool live_c = hw < nc;
            const int i = lane & 31;
            const float h = live_c ? silu_mul(rowv[hw][i], rowv[hw][32 + i]) : 0.0f;
            const int row = item.first + c0 + (live_c ? hw : 0);
            q8_image_store(h, live_c, qsc[hw], himg + ((size_t)row * h_blocks + hb) * kImgDw, true);
            if (so.any())  // the trace's stages: gate and up dots, the standard q8_1 block of h
                stage_store(so, row, hb, live_c ? rowv[hw][i] : 0.0f, live_c ? rowv[hw][32 + i] : 0.0f, h, live_c, F, Fs);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ down
// Grid (H / (4 * 64 / nbf), work items); nbf = F / 256 lanes per row, 64 / nbf rows per wave.  The item's h
// images are copied to LDS `cps` columns at a time; each group leader writes Y[first + c][row] (the shared
// rows times sigmoid(sg[t])).
// (Arguments ordered as k_iq2_gu's.)
__global__ __launch_bounds__(256) void k_iq2_down(const int4* __restrict__ items, const uint32_t* __restrict__ himg,
                                                   const uint8_t* __restrict__ down_exps,
                                                   const uint64_t* __restrict__ eptr, int H, int F, int Fs,
                                                   int h_blocks, int cps, const uint8_t* __restrict__ down_sh,
                                                   const float* __restrict__ sg, float* __restrict__ Y,
                                                   const int32_t* __restrict__ dmap) {
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ uint2 tab[kIq2sTabEntries];
    Item item;
    if (!work_item(items, blockIdx.y, item)) return;
    const int Fe = item.shared ? Fs : F;
    const int nb = Fe >> 8;
    const size_t rb = (size_t)nb * 82;
    const uint8_t* base =
        item.shared ? down_sh
        : eptr      ? reinterpret_cast<const uint8_t*>(eptr[item.e]) + (size_t)2 * F * ((size_t)(H >> 8) * 82)
                    : down_exps + (size_t)item.e * H * ((size_t)(F >> 8) * 82);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rpw = 64 / nb, grp = lane / nb, b = lane - grp * nb;
    const int r = blockIdx.x * 4 * rpw + wave * rpw + grp;
    const bool live = r < H;
    // loads in the order their data is needed (see k_iq2_gu): grid codes, the first column batch's h images,
    // then the weights
    uint4 codes[kTabRounds<256>];
    grid_codes_load<256>(codes);
    const int nc0 = min(cps, item.ncol);
    StagePieces sp;
    stage_issue_direct<256>(sp, himg, h_blocks, 0, nc0, cps, 0, item, false);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t raw[21];
    uint32_t off;
    off = load_block_raw(base + (size_t)(live ? r : 0) * rb, b, raw);
    __builtin_amdgcn_sched_barrier(0);
    grid_table_store<256>(codes, tab);
    stage_commit_direct(sp, smem);
    stage_images<256>(smem, himg, h_blocks, 0, nc0, cps, item, nullptr, 1, false, 4 * 256);  // rounds beyond the first
    __syncthreads();
    Iq2Block B[1];
    decode_block(raw, off, tab, B[0]);
    for (int c0 = 0; c0 < item.ncol; c0 += cps) {
        const int nc = min(cps, item.ncol - c0);
        if (c0 > 0) {
            stage_images<256>(smem, himg, h_blocks, c0, nc, cps, item, nullptr, 1, false);
            __syncthreads();
        }
        for (int c = 0; c < nc; ++c) {
            const uint32_t* ht = smem + (size_t)c * h_blocks * kImgLdsDw;
            pin_blocks(B);
            float v = group_sum(iq2_block_dot_img(B[0], ht, b), nb);
            if (item.shared) v = v * sigmoid(sg[item.tok0 + c0 + c]);
            const int orow = (dmap && !item.shared) ? dmap[item.first + c0 + c] : item.first + c0 + c;
            if (orow >= 0 && live && b == 0) Y[(size_t)orow * H + r] = v;
        }
        __syncthreads();
    }
}

// Generic IQ2_S GEMV over n_col columns of standard q8_1 blocks (iq_mmvq's contract, metal/src/iq.mm:148-169).
__global__ __launch_bounds__(256) void k_iq2_mmvq(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xq, int n_in,
                                                   int n_out, int n_col, float* __restrict__ y) {
    __shared__ uint2 tab[kIq2sTabEntries];
    {
        uint4 codes[kTabRounds<256>];
        grid_codes_load<256>(codes);
        grid_table_store<256>(codes, tab);
    }
    const int nb = n_in >> 8;
    const size_t rb = (size_t)nb * 82;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rpw = 64 / nb, grp = lane / nb, b = lane - grp * nb;
    const int r = blockIdx.x * 4 * rpw + wave * rpw + grp;
    const bool live = r < n_out;
    __syncthreads();
    Iq2Block B[1];
    {
        uint32_t raw[21];
        uint32_t off;
        off = load_block_raw(w + (size_t)(live ? r : 0) * rb, b, raw);
        decode_block(raw, off, tab, B[0]);
    }
    const int xb = n_in >> 5;
    for (int c = 0; c < n_col; ++c) {
        pin_blocks(B);
        const float v = group_sum(iq2_block_dot_std(B[0], xq + (size_t)c * xb * 36, b), nb);
        if (live && b == 0) y[(size_t)c * n_out + r] = v;
    }
}

// ------------------------------------------------------------------------------------------------ launchers
// Rows the IQ2_S kernels tile: n_in = 256 nb with nb in {2, 4, 8} (a row is a whole number of block pairs,
// one block per lane, at most 8 lanes per row).
bool iq2_shape_ok(int n_in) {
    if (n_in <= 0 || n_in % 256) return false;
    const int nb = n_in / 256;
    return nb == 2 || nb == 4 || nb == 8;
}

hipError_t launch_iq2_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                         const uint32_t* ximg, const int4* items, const int32_t* perm, int k, int H, int F, int Fs,
                         int has_shared, int max_items, uint32_t* himg, int h_blocks, hipStream_t s, const StageOut* so,
                         const uint64_t* eptr) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    dim3 grid((unsigned)(Fmax / 32), (unsigned)max_items);
    const int nb = H / 256;
    const size_t lds = (size_t)(2 * nb) * (H >> 5) * kImgLdsDw * 4 + 16;  // + the dead staging slot
#define SMOE_IQ2_GU(NW)                                                                                           \
    hipLaunchKernelGGL((k_iq2_gu<NW>), grid, dim3(64 * (NW)), lds, s, items, ximg, gate_exps, up_exps, eptr, H, F, Fs, \
                       k, gate_sh, up_sh, perm, himg, h_blocks, so ? *so : StageOut{})
    if (nb == 2) SMOE_IQ2_GU(2);
    else if (nb == 4) SMOE_IQ2_GU(4);
    else SMOE_IQ2_GU(8);
#undef SMOE_IQ2_GU
    return hipGetLastError();
}

hipError_t launch_iq2_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                           const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                           hipStream_t s, const uint64_t* eptr, const int32_t* dmap) {
    const int rpw = 64 / (F / 256);  // the caller guarantees the shared width has the same row shape
    dim3 grid((unsigned)((H + 4 * rpw - 1) / (4 * rpw)), (unsigned)max_items);
    const size_t col_bytes = (size_t)h_blocks * kImgLdsDw * 4;
    int cps = (int)(24576 / col_bytes);
    cps = cps < 1 ? 1 : cps > 16 ? 16 : cps;
    hipLaunchKernelGGL(k_iq2_down, grid, dim3(256), (size_t)cps * col_bytes + 16, s, items, himg, down_exps, eptr, H, F,
                       Fs, h_blocks, cps, down_sh, sg, Y, dmap);
    return hipGetLastError();
}

hipError_t launch_iq2_mmvq(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y, hipStream_t s) {
    const int rpw = 64 / (n_in / 256);
    dim3 grid((unsigned)((n_out + 4 * rpw - 1) / (4 * rpw)));
    hipLaunchKernelGGL(k_iq2_mmvq, grid, dim3(256), 0, s, w, xq, n_in, n_out, n_col, y);
    return hipGetLastError();
}

}  // namespace smoe
