// stratametal_amd/csrc/smoe_prefill.hip - the prefill contract's expert products on the matrix cores (gfx950).
//
// Contract (oracle: or_moe_prefill): activations rounded to bf16; Q2_0 weights used exactly as
// (code - 1) * f32(d); SwiGLU in f32; h rounded to bf16 for the down product; f32 accumulation.  The
// reference's float prompt path is a dequantising GEMM (include/strata/prefill/gemm.hpp:28-40,
// include/strata/prefill/kernels.hpp:54-57,97-98, include/strata/prefill/moe_fused.hpp:52-62).
//
// How the exact products reach the matrix cores: both operands are fp16 and the MFMA is
// v_mfma_f32_16x16x32_f16 (exact products, f32 sums).
//  - An activation a is its bf16 value held in fp16, which is exact for 2^-17 <= |a| < 65520 (fp16 keeps 11
//    significant bits and reaches 2^-24; bf16 has 8).  Smaller magnitudes round in fp16 (an error below 2^-25
//    per element); larger ones do not fit: the contract's activations and h are required to stay below 65520.
//  - A weight (c - 1) * d, c in {0, 1, 2, 3}, d the block's fp16 scale, is one of {-d, 0, d, 2d}: exact in fp16
//    (for |d| < 32752).  It is made in two steps: v_cvt_scalef32_pk_f16_fp4 turns a byte of two 2-bit codes,
//    masked into the low bits of two fp4 nibbles, into the fp16 pair (c0, c1) (nibble c is the e2m1 value c / 2,
//    scale 2), then v_pk_fma_f16(c, d, -d) gives (c - 1) * d with one rounding of an exact value.
// The K loop is one chain of MFMAs per output tile; nothing in it waits for an MFMA result.
//
// Activation records.  Each 64-value block of an activation row (x for gate/up, h for down) is one 128-byte
// record of 64 fp16 in MFMA order: position p = 32 s + 8 q + e holds element 16 q + 8 s + pi(e),
// pi = (0 2 1 3 4 6 5 7), the order in which a lane of quarter q meets the codes of code dword q of the block
// in the two 32-deep MFMA steps s.
//
// MFMA tiles (lane l = 16 q + i): A[i][k] = weight of row i, B[k][j] = activation of column (token) j,
// C[4 q + r][j] in register r: a lane holds four consecutive rows of one column, which the epilogues store as one
// piece (measured: down 82 -> 72 us at the benchmark's prefill 512, whose stores had been one dword per row).
#include "smoe_device.hpp"
#include "smoe_gemv.hpp"
#include "smoe_items.hpp"
#include "smoe_launch.hpp"

#include <climits>
#include <type_traits>

namespace smoe {

typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int kRecBytes = 128;   // bytes per 64-value activation record
constexpr int kChunk = 128;      // columns (tokens) per work item

__device__ __forceinline__ int perm8(int e) { return (e == 1 || e == 5) ? e + 1 : (e == 2 || e == 6) ? e - 1 : e; }
// record position of block element kappa (pi is an involution)
__device__ __forceinline__ int rec_pos(int kappa) {
    return 32 * ((kappa >> 3) & 1) + 8 * (kappa >> 4) + perm8(kappa & 7);
}
// fp16 bits of the bf16 rounding of v
__device__ __forceinline__ uint32_t bf16_as_f16(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)bf16_to_f32(f32_to_bf16(v)));
}

// ------------------------------------------------------------------------------------------------ records of x
// Chunk ch (8 positions, 16 bytes) of record r from the 8 values it holds, v[e] = element 16 q + 8 s + e of the
// record's 64-value block (s = ch / 4, q = ch % 4); with `xb`, the same 8 values also as bf16 bits in natural order
// (the router's exact operand).
__device__ __forceinline__ void store_record_chunk(const float (&v)[8], int64_t r, int ch, uint32_t* __restrict__ rec,
                                                   uint16_t* __restrict__ xb) {
    const int s = ch >> 2, q = ch & 3;
    if (xb) {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = f32_to_bf16(v[e]);
        *reinterpret_cast<uint4*>(xb + r * 64 + 16 * q + 8 * s) =
            make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = bf16_as_f16(v[perm8(e)]);
    reinterpret_cast<uint4*>(rec + r * (kRecBytes / 4))[ch] =
        make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
}

// Whether a finite value's bf16 rounding lies beyond fp16 (65520 or more in magnitude: the MFMA operand would be
// inf); the per-work-group flags of such values feed smoe_trace.overflow.
__device__ __forceinline__ bool f16_overflow(float v) {
    return __builtin_isfinite(v) && !(__builtin_fabsf(bf16_to_f32(f32_to_bf16(v))) < 65520.0f);
}
__device__ __forceinline__ bool f16_overflow8(const float (&v)[8]) {
    bool o = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) o |= f16_overflow(v[e]);
    return o;
}

// One thread per 8 positions (a 16-byte chunk) of a record.  With `flags`, work-group b writes flags[b] = whether
// any of its values is an fp16 overflow.
__global__ __launch_bounds__(256) void k_act_records(const float* __restrict__ x, int64_t n_rec,
                                                     uint32_t* __restrict__ rec, uint16_t* __restrict__ xb,
                                                     int32_t* __restrict__ flags) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t r = g >> 3;
    bool ovf = false;
    if (r < n_rec) {
        const int ch = (int)(g & 7);
        const float4* src = reinterpret_cast<const float4*>(x + r * 64 + 16 * (ch & 3) + 8 * (ch >> 2));
        const float4 lo = src[0], hi = src[1];
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        store_record_chunk(v, r, ch, rec, xb);
        ovf = f16_overflow8(v);
    }
    if (flags) {
        const int any = __syncthreads_or(ovf ? 1 : 0);
        if (threadIdx.x == 0) flags[blockIdx.x] = any ? 1 : 0;
    }
}

// The stack junction of the prefill path and the records of its output in one launch, one work-group per row:
// x = RMSNorm(x_prev + r_prev) exactly as k_residual_rmsnorm forms it (written to `out`), then the row's
// records and bf16 copy exactly as k_act_records forms them from x, read back from LDS.  n <= 4096, n % 64 == 0,
// x, r and out 16-byte aligned.
__global__ __launch_bounds__(256) void k_junction_records(const float* __restrict__ x, const float* __restrict__ r,
                                                          int n, float eps, float* __restrict__ out,
                                                          uint32_t* __restrict__ rec, uint16_t* __restrict__ xb,
                                                          int32_t* __restrict__ flags) {
    __shared__ float wsum[4];
    __shared__ __align__(16) float row[4096];
    residual_rmsnorm_row<true>(x + (size_t)blockIdx.x * n, r + (size_t)blockIdx.x * n, n, eps,
                               out + (size_t)blockIdx.x * n, wsum, row);
    __syncthreads();
    const int rpr = n >> 6;
    bool ovf = false;
    for (int g = threadIdx.x; g < rpr * 8; g += 256) {
        const int rl = g >> 3, ch = g & 7;
        const float4* src = reinterpret_cast<const float4*>(row + rl * 64 + 16 * (ch & 3) + 8 * (ch >> 2));
        const float4 lo = src[0], hi = src[1];
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        store_record_chunk(v, (int64_t)blockIdx.x * rpr + rl, ch, rec, xb);
        ovf |= f16_overflow8(v);
    }
    if (flags) {
        const int any = __syncthreads_or(ovf ? 1 : 0);
        if (threadIdx.x == 0) flags[blockIdx.x] = any ? 1 : 0;
    }
}

// ------------------------------------------------------------------------------------------------ codes -> B
__device__ __forceinline__ f16x8 cat4(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}
// (c - 1) * d for a pair of codes c (as fp16 values)
__device__ __forceinline__ f16x2 scale_pair(f16x2 c, f16x2 d, f16x2 nd) { return __builtin_elementwise_fma(c, d, nd); }

// Code dword cw (16 codes) of a block with scale d (fp16 bits) -> the B operands of the two 32-deep steps:
// x holds codes 0, 2 of each byte in the low bits of its nibbles, y codes 1, 3.
__device__ __forceinline__ void expand_codes(uint32_t cw, uint32_t dbits, f16x8& s0, f16x8& s1) {
    const uint32_t x = cw & 0x33333333u, y = (cw >> 2) & 0x33333333u;
    const uint32_t dd = dbits | (dbits << 16);
    const f16x2 d = __builtin_bit_cast(f16x2, dd), nd = __builtin_bit_cast(f16x2, dd ^ 0x80008000u);
    s0 = cat4(scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 2.0f, 0), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 2.0f, 0), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 2.0f, 1), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 2.0f, 1), d, nd));
    s1 = cat4(scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 2.0f, 2), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 2.0f, 2), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 2.0f, 3), d, nd),
              scale_pair(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 2.0f, 3), d, nd));
}

// Staging.  Both operands reach LDS by buffer loads that write LDS directly (`buffer_load_dwordx4 ... lds`:
// lane L of an instruction lands at M0 + 16 L), several stages deep: while the waves multiply stage u, the
// loads of the next stages are in flight.  A stage is one 128-value unit (two blocks) of K:
//   activations: the item's columns x 17 pieces of 16 bytes (the column's two records, then one pad piece
//                that spreads the columns over the LDS banks);
//   weights:     256 rows x a 48-byte window holding the row's 36-byte unit (the window starts at the 16-byte
//                boundary at or below the unit, 4 (u % 4) bytes before it).
// Every wave issues the same number of instructions per stage (those past the real ones land in a dummy slot),
// so `s_waitcnt vmcnt(n * slots)` means "my loads of all but the n newest stages are done"; the barrier after
// it makes everyone's visible.  Columns past the item and pad pieces read at an offset beyond the buffer
// (range-checked: no memory access, zeros written), so a short item moves only its own activation bytes.
//
// Three work-group shapes share one LDS ring (the item's column count picks one):
//   wide (65..128 columns): 3 stages of 128 columns;
//   narrow (17..64 columns): 5 stages of 64 columns;
//   thin (<= 16 columns):   2 stages of four units each for 16 columns, rows as narrow: these work-groups stream
//                           weights, and a four-unit stage brings each row's weights as one 144-byte window
//                           (its columns as 65 pieces: 8 records and a pad).  They run at ~13 GB/s of weights
//                           per CU whatever the depth (a third stage for 8 columns was slower), so the depth
//                           stays at one stage in flight.
// In every shape wave w owns two 16-row sets (gate/up: gate rows 16 w .. + 15 and the same up rows; down: rows
// 32 w .. + 31) and every column, so each row's codes are expanded once per work-group.
constexpr int kWgRows = 256;
// Down work-groups (other than thin) take kDownRbw consecutive row blocks of their item, one K loop over all of
// them: the ring runs on across the row blocks, so the next block's first stages load while the last units and
// the stores of the one before run (a down K loop is only n_ff / 128 units).
constexpr int kDownRbw = 2;
constexpr int kWaves = 8;
constexpr uint32_t kOob = 0x80000000u;
constexpr int kRing = 148480;           // bytes of the stage ring
constexpr int kDummy = kRing;           // 1 KB landing slot of the padding instructions
constexpr int kLds = kRing + 1024;

// MODE 0 (thin, <= kThinCols columns): stages of four units each (see below), rows as narrow.  MODE 3 is the same
// shape with a ring of one stage: k_mm_down_thin takes 55 KB of LDS, so two of its work-groups share a CU and one's
// loads overlap the other's products (measured: the thin down items 8 us faster at the benchmark's prefill; the
// same split of gate/up, whose thin work-groups stream four stages, gained nothing).
// MODE 4 (k_mm_down_thin): MODE 3 over half the rows, 128 per work-group, one 16-row set per wave: 36 KB of LDS, so
// four work-groups share a CU.
// MODE 5 (k_mm_gu_thin): the thin gate/up shape over 64 gate and 64 up rows per work-group, one 16-row set per wave
// (waves 0-3 gate, 4-7 up), kThinGStages stages: several work-groups share a CU (one stage: 37 KB, four per CU;
// measured at prefill 512: thin items 68 us against 74 with two stages and two per CU, and the whole gate/up stage
// 110 us against 123 with the thin items inside k_mm_gu).
enum { kThin = 0, kNarrow = 1, kWide = 2, kThin1 = 3, kThinH = 4, kThinG = 5 };
constexpr int kThinGStages = 1;
// Thin gate/up items run in k_mm_gu_thin below this many routed pairs per expert on average (prefill 512 of the
// benchmark: 10, the thin items the bulk of the work; 4096 tokens: 80, a few thin remainders that k_mm_gu's tail hides,
// where the extra launch after it cost ~6 us per layer).
constexpr int kThinApartPairs = 32;
constexpr int kMaxTiles = 8;  // column tiles of 16 per wave at most (the wide shape's 128 columns)
constexpr int kThinCols = 16;
template <int MODE>
struct Shape {
    static constexpr bool kIsThin = MODE == kThin || MODE == kThin1 || MODE == kThinH || MODE == kThinG;
    static constexpr int kTok = MODE == kWide ? 128 : MODE == kNarrow ? 64 : kThinCols;
    static constexpr int MT = (kTok + 15) / 16;  // column tiles of a wave: every wave has every column
    static constexpr int kStages =
        MODE == kWide ? 3 : MODE == kNarrow ? 5 : MODE == kThin ? 2 : MODE == kThinG ? kThinGStages : 1;
    static constexpr int kRows = MODE == kThinH || MODE == kThinG ? kWgRows / 2 : kWgRows;  // a work-group's weight rows
    static constexpr int NS = kRows / (16 * kWaves);                       // 16-row sets of a wave
    // units of 128 values per stage: the thin shape streams weights, four units at a time, so that a row's
    // weights arrive as one 144-byte window (16-byte aligned, 9 pieces) instead of four 48-byte ones
    static constexpr int UPS = kIsThin ? 4 : 1;
    static constexpr int kColPieces = 16 * UPS + 1;                // a column's records, then one pad piece
    static constexpr int kRowPieces = UPS == 1 ? 3 : 9 * UPS / 4;  // a row's weight window
    static constexpr int kRowDw = 4 * kRowPieces;
    static constexpr int kAPieces = (kTok * kColPieces + 63) / 64 * 64;  // whole DMA instructions
    static constexpr int kAIns = kAPieces / 64;
    static constexpr int kWPieces = kRows * kRowPieces;
    static constexpr int kWIns = kWPieces / 64;
    static constexpr int kASlots = (kAIns + kWaves - 1) / kWaves;
    static constexpr int kWSlots = (kWIns + kWaves - 1) / kWaves;
    static constexpr int kSlots = kASlots + kWSlots;
    static constexpr int kABytes = kAPieces * 16;
    static constexpr int kStage = kABytes + kWPieces * 16;
    static constexpr int kDummyAt =
        MODE == kThin1 || MODE == kThinH || MODE == kThinG ? kStages * kStage : kDummy;  // the padding's slot
    static constexpr int kLdsBytes = kDummyAt + 1024;
    static_assert(UPS == 1 || UPS == 4, "one or four units per stage");
    static_assert(kAPieces % 64 == 0 && kWPieces % 64 == 0, "whole DMA instructions");
    static_assert(kStages * kStage <= kRing && kLdsBytes <= kLds, "ring");
    static_assert((kStages - 2) * kSlots <= 63, "vmcnt range");
    static_assert(kStages - 2 <= 6, "wait_stages cases");
};

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Raw buffer resource over [base, base + bytes) (no swizzle, no stride; out-of-range lanes read nothing).
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return i32x4{(int)(uint32_t)b, (int)(uint32_t)(b >> 32), (int)bytes, 0x00020000};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_u8*)p; }
// M0 is written one instruction before the load that reads it (one wait state for LDS DMA).
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, i32x4 rsrc, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
                 "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until this wave's loads of all but the `after` newest stages are done.
template <int SLOTS>
__device__ __forceinline__ void wait_stages(int after) {
    switch (after) {
        case 0: vmcnt<0>(); break;
        case 1: vmcnt<SLOTS>(); break;
        case 2: vmcnt<2 * SLOTS>(); break;
        case 3: vmcnt<3 * SLOTS>(); break;
        case 4: vmcnt<4 * SLOTS>(); break;
        case 5: vmcnt<5 * SLOTS>(); break;
        default: vmcnt<6 * SLOTS>(); break;
    }
}

// One wave's DMA plan: per slot the byte offset within a stage (uniform; -1 for the dummy) and the lane's
// buffer offset at unit 0.
template <int MODE>
struct MmPlan {
    using S = Shape<MODE>;
    uint32_t a_off[S::kASlots], w_off[S::kWSlots];
    int a_at[S::kASlots], w_at[S::kWSlots];
    i32x4 w_rsrc[S::kWSlots];  // the slot's weight tensor (the up rows' for the second half of gate/up)
    // a work-group that runs several row blocks (down, one weight tensor): unit u of the K loop is unit u % upr of
    // row block u / upr, whose weight rows are the rbs bytes from wbase + (u / upr) rbs (of wbytes in all); each row
    // block gets a buffer resource of its own, so rows past the tensor read as zeros (one row block: upr = the K
    // loop's units, and w_rsrc as set by init)
    int upr = 1 << 30;
    uint32_t rbs = 0, wbytes = 0;
    const uint8_t* wbase = nullptr;

    // rowidx: activation row of each column; rpr: records per activation row; rb: weight row bytes; split: rows
    // of the first weight tensor (gate/up: 128; down: 256, i.e. one tensor); rw0 / rw1: the two weight tensors.
    __device__ __forceinline__ void init(const int* rowidx, int wave, int lane, int ncol, int rpr, uint32_t rb,
                                         int split, i32x4 rw0, i32x4 rw1) {
#pragma unroll
        for (int m = 0; m < S::kASlots; ++m) {
            const int j = wave + kWaves * m;
            const int P = 64 * j + lane, t = P / S::kColPieces, p = P - S::kColPieces * t;
            const bool live = j < S::kAIns && t < ncol && p < 16 * S::UPS;
            const int row = rowidx[t < ncol ? t : 0];
            a_off[m] = live ? (uint32_t)(row * rpr * kRecBytes + 16 * p) : kOob;
            a_at[m] = j < S::kAIns ? 1024 * j : -1;
        }
#pragma unroll
        for (int m = 0; m < S::kWSlots; ++m) {
            const int j = wave + kWaves * m;
            const int P = 64 * j + lane, row = P / S::kRowPieces, p = P - S::kRowPieces * row;
            const bool real = j < S::kWIns;
            const int r = row >= split ? row - split : row;
            static_assert((S::kRowPieces * 128) % 64 == 0, "whole instructions per weight tensor");
            w_rsrc[m] = 64 * j >= S::kRowPieces * split ? rw1 : rw0;  // whole instructions per tensor
            w_off[m] = real ? (uint32_t)r * rb + 16u * p : kOob;
            w_at[m] = real ? S::kABytes + 1024 * j : -1;
        }
    }

    // Issue the stage of units u .. u + UPS - 1 into ring stage b (u a multiple of UPS).  One unit: the row's
    // 48-byte window starts at the 16-byte boundary at or below the unit; four: at the unit (36 u = 144 u / 4).
    __device__ __forceinline__ void issue(uint32_t lds0, int b, int u, i32x4 ra) const {
        const uint32_t st = (uint32_t)(b * S::kStage);
        const int rbl = u / upr, ur = u - rbl * upr;
        const uint32_t sa = __builtin_amdgcn_readfirstlane((uint32_t)ur * (2 * kRecBytes));
        const uint32_t sw = __builtin_amdgcn_readfirstlane((uint32_t)(S::UPS == 1 ? 36 * ur - 4 * (ur & 3) : 36 * ur));
        const uint32_t wofs = (uint32_t)rbl * rbs;
        const i32x4 wr = buffer_rsrc(wbase + wofs, wbytes - wofs < rbs ? wbytes - wofs : rbs);
#pragma unroll
        for (int m = 0; m < S::kASlots; ++m) {
            const uint32_t at = a_at[m] < 0 ? (uint32_t)S::kDummyAt : st + (uint32_t)a_at[m];
            dma16(__builtin_amdgcn_readfirstlane(lds0 + at), a_off[m], ra, sa);
        }
#pragma unroll
        for (int m = 0; m < S::kWSlots; ++m) {
            const uint32_t at = w_at[m] < 0 ? (uint32_t)S::kDummyAt : st + (uint32_t)w_at[m];
            dma16(__builtin_amdgcn_readfirstlane(lds0 + at), w_off[m], wbase ? wr : w_rsrc[m], sw);
        }
    }
};

// One staged unit: the activation fragments of all NT column tiles (columns tok0 + 16 n ..; CP pieces per column
// in LDS, A at the unit's first piece) are loaded first; then for each block h and row set s (LDS row rows[s] of
// RD dwords; the unit starts `wofs` dwords into the row's window)
// the set's weight operands are expanded and fed to every tile: acc[n][s] += W0 A0 + W1 A1.  Set s + 1 is expanded
// while the matrix cores work on set s.
template <int NS, int NT, int CP = 17, int RD = 12>
__device__ __forceinline__ void mm_unit(f32x4 (&acc)[kMaxTiles][NS], const uint32_t* W, int wofs, const int (&rows)[NS],
                                        const uint4* A, int tok0, int i, int q) {
    f16x8 a[2][NT][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const uint4* ar = A + (tok0 + 16 * n + i) * CP + 8 * h;
            a[h][n][0] = __builtin_bit_cast(f16x8, ar[q]);
            a[h][n][1] = __builtin_bit_cast(f16x8, ar[4 + q]);
        }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t* w = W + rows[s] * RD + wofs;
            const uint32_t cw = h == 0 ? __builtin_amdgcn_alignbyte(w[q + 1], w[q], 2) : w[5 + q];
            const uint32_t db = h == 0 ? (w[0] & 0xFFFFu) : (w[4] >> 16);
            f16x8 b0, b1;
            expand_codes(cw, db, b0, b1);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                acc[n][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b0, a[h][n][0], acc[n][s], 0, 0, 0);
                acc[n][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b1, a[h][n][1], acc[n][s], 0, 0, 0);
            }
        }
    }
}

// The K loop of both kernels: stages of UPS units of 128 values through the ring, kStages - 1 stages in flight.
// NT: the wave's live column tiles.  With several row blocks (pl.upr units each, one unit per stage), epi(rbl) runs
// after the last unit of row block rbl: it stores the wave's results of that block and clears acc, while the next
// block's first stages are already in flight.
struct NoEpi {
    __device__ __forceinline__ void operator()(int) const {}
};
template <int MODE, int NT, class Epi>
__device__ __forceinline__ void mm_loop_nt(f32x4 (&acc)[kMaxTiles][Shape<MODE>::NS], uint8_t* lds, const MmPlan<MODE>& pl,
                                           int units, i32x4 ra, const int (&rows)[Shape<MODE>::NS], int tok0, int i,
                                           int q, const Epi& epi) {
    using S = Shape<MODE>;
    constexpr int ST = S::kStages;
    const uint32_t lds0 = lds_addr(lds);
    const int nst = (units + S::UPS - 1) / S::UPS;
    int ur = 0, rbl = 0;  // (UPS == 1) the consumed stage's unit within its row block, and that row block
    auto stage = [&](int g, int b) {  // the units of stage g, in ring stage b
        const uint8_t* stg = lds + b * S::kStage;
        const uint32_t* W = reinterpret_cast<const uint32_t*>(stg + S::kABytes);
        const uint4* A = reinterpret_cast<const uint4*>(stg);
        if constexpr (S::UPS == 1) {
            mm_unit<S::NS, NT>(acc, W, ur & 3, rows, A, tok0, i, q);
            if (++ur == pl.upr) {
                epi(rbl++);
                ur = 0;
            }
        } else {
#pragma unroll
            for (int uu = 0; uu < S::UPS; ++uu)
                if (S::UPS * g + uu < units)
                    mm_unit<S::NS, NT, S::kColPieces, S::kRowDw>(acc, W, 9 * uu, rows, A + 16 * uu, tok0, i, q);
        }
    };
    if constexpr (ST == 1) {  // one ring stage: load, wait, multiply; the CU's other work-group fills the gaps
        for (int g = 0; g < nst; ++g) {
            if (g) __syncthreads();  // everyone is done with stage g - 1
            pl.issue(lds0, 0, S::UPS * g, ra);
            vmcnt<0>();
            __syncthreads();
            stage(g, 0);
        }
    } else {
#pragma unroll
        for (int b = 0; b < ST - 1; ++b)
            if (b < nst) pl.issue(lds0, b, S::UPS * b, ra);
        int b = 0, g = 0;  // ring stage of stage g
        // steady state: every iteration consumes stage g, with the ST - 2 stages after it still in flight, and issues
        // stage g + ST - 1 (a constant wait, no test)
        for (; g + ST - 1 < nst; ++g) {
            vmcnt<(ST - 2) * S::kSlots>();
            __syncthreads();  // stage g is in LDS for everyone; everyone is done with stage g - 1
            pl.issue(lds0, b == 0 ? ST - 1 : b - 1, S::UPS * (g + ST - 1), ra);
            stage(g, b);
            b = b + 1 == ST ? 0 : b + 1;
        }
        // the last stages (all of them when there are fewer than ST - 1): nothing left to issue, the waits shrink
        for (; g < nst; ++g) {
            wait_stages<S::kSlots>(nst - 1 - g);
            __syncthreads();
            stage(g, b);
            b = b + 1 == ST ? 0 : b + 1;
        }
    }
}

template <int MODE, class Epi = NoEpi>
__device__ __forceinline__ void mm_loop(f32x4 (&acc)[kMaxTiles][Shape<MODE>::NS], uint8_t* lds, const MmPlan<MODE>& pl,
                                        int units, i32x4 ra, const int (&rows)[Shape<MODE>::NS], int tok0, int ntiles,
                                        int i, int q, const Epi& epi = Epi{}) {
#pragma unroll
    for (int n = 0; n < kMaxTiles; ++n)
#pragma unroll
        for (int s = 0; s < Shape<MODE>::NS; ++s) acc[n][s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (Shape<MODE>::kIsThin) {  // one tile
        mm_loop_nt<MODE, 1>(acc, lds, pl, units, ra, rows, tok0, i, q, epi);
        return;
    } else if constexpr (MODE == kNarrow) {
        switch (ntiles) {  // work-group-uniform: 2 .. 4 live tiles
            case 1: mm_loop_nt<MODE, 1>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            case 2: mm_loop_nt<MODE, 2>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            case 3: mm_loop_nt<MODE, 3>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            default: mm_loop_nt<MODE, 4>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
        }
    } else {
        switch (ntiles) {  // work-group-uniform: 5 .. 8 live tiles
            case 5: mm_loop_nt<MODE, 5>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            case 6: mm_loop_nt<MODE, 6>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            case 7: mm_loop_nt<MODE, 7>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
            default: mm_loop_nt<MODE, 8>(acc, lds, pl, units, ra, rows, tok0, i, q, epi); break;
        }
    }
}

// ------------------------------------------------------------------------------------------------ gate/up
// Grid (Fmax / 128, work items), 8 waves.  Work-group rt computes gate and up rows [128 rt, 128 rt + 128) for the
// item's (at most 128) columns, then h = bf16(silu(gate) * up) into records 2 rt and 2 rt + 1 of each column's h
// row.  Wave w has gate rows 16 w .. + 15 (set 0) and the same up rows (set 1).
// SwiGLU of the prefill contract: silu(g) * u with the hardware exp2 and reciprocal (a few ulp).  h is rounded to
// bf16 next and the contract is held to 1e-3 per row; the decode contract keeps silu_mul's exact order.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// The expert GEMMs' 1-D grids: work-group id -> (work item y, row block rb).  The dispatcher deals linear ids round
// robin over the 8 XCDs, so the n_rb row blocks of item y are given the ids 8 (n_rb (y / 8) + rb) + y % 8: one XCD,
// dispatched back to back, reading the item's activation records from memory once and then from that XCD's L2 (a 2-D
// grid of (row block, item) put each row block of an item on another XCD).  The grid holds n_rb * (max_items rounded
// up to 8) work-groups; false past max_items.
__device__ __forceinline__ bool xcd_item(int n_rb, int max_items, int& y, int& rb) {
    const int id = blockIdx.x, xcd = id & 7, slot = id >> 3, g = slot / n_rb;
    y = 8 * g + xcd;
    rb = slot - n_rb * g;
    return y < max_items;
}
__host__ __device__ inline unsigned xcd_grid(int n_rb, int max_items) {
    return (unsigned)(n_rb * ((max_items + 7) / 8) * 8);
}

template <int MODE>
__device__ __forceinline__ void mm_gu_body(uint8_t* lds, const int* rowidx, const Item& item, int ncol, int rt,
                                           const uint8_t* g0, const uint8_t* u0, const uint32_t* xrec,
                                           uint32_t xrec_bytes, int H, uint32_t* hrec, int h_rec, int32_t* flag) {
    using S = Shape<MODE>;
    constexpr int NS = S::NS;
    const int units = H >> 7;
    const uint32_t rb = (uint32_t)units * 36u;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, i = lane & 15,
              q = lane >> 4;
    const i32x4 ra = buffer_rsrc(xrec, xrec_bytes);
    const i32x4 rg0 = buffer_rsrc(g0 + (size_t)128 * rt * rb, 128u * rb);
    const i32x4 ru0 = buffer_rsrc(u0 + (size_t)128 * rt * rb, 128u * rb);
    MmPlan<MODE> pl;
    pl.init(rowidx, wave, lane, ncol, H >> 6, rb, 128, rg0, ru0);
    int rows[NS];
    const int fbase = 16 * wave;  // first of the wave's gate rows within the work-group's 128
    rows[0] = fbase + i;
    rows[1] = 128 + fbase + i;
    const int tok0 = 0;
    const int ntiles = min(S::MT, (ncol + 15) >> 4);
    f32x4 acc[kMaxTiles][NS];
    mm_loop<MODE>(acc, lds, pl, units, ra, rows, tok0, ntiles, i, q);
    __syncthreads();  // every wave is done with the ring: its start becomes the h tile
    // h tile [column][128 rows in record order] as fp16 bits of bf16 values
    // lane (q, i) holds rows fbase + 4 q .. + 3 of column 16 n + i: their record positions are one aligned group of
    // four, in the order (0 2 1 3), written as one 8-byte store
    uint16_t* ht = reinterpret_cast<uint16_t*>(lds);
    bool ovf = false;
    static_assert(NS == 2, "one gate set and one up set");
    const int f4 = fbase + 4 * q;
    const int pos4 = 64 * (f4 >> 6) + rec_pos(f4 & 63);
#pragma unroll
    for (int n = 0; n < S::MT; ++n) {
        const int c = tok0 + 16 * n + i;
        if (n < ntiles && c < ncol) {
            uint32_t hb[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float h = silu_mul_fast(acc[n][0][r], acc[n][1][r]);
                hb[r] = bf16_as_f16(h);
                if (flag) ovf |= f16_overflow(h);
            }
            *reinterpret_cast<uint2*>(ht + c * 128 + pos4) = make_uint2(hb[0] | (hb[2] << 16), hb[1] | (hb[3] << 16));
        }
    }
    if (flag) {
        const int any = __syncthreads_or(ovf ? 1 : 0);
        if (threadIdx.x == 0) {
            flag[0] = any ? 1 : 0;
            flag[1] = 0;
        }
    } else {
        __syncthreads();
    }
    for (int idx = tid; idx < ncol * 16; idx += 512) {  // 16 chunks (two records) per column
        const int c = idx >> 4, rr = (idx >> 3) & 1, ch = idx & 7;
        const uint4 v = reinterpret_cast<const uint4*>(ht + c * 128 + 64 * rr)[ch];
        reinterpret_cast<uint4*>(hrec + ((size_t)(item.first + c) * h_rec + 2 * rt + rr) * (kRecBytes / 4))[ch] = v;
    }
}

__global__ __launch_bounds__(512) void k_mm_gu(const uint8_t* __restrict__ gate_exps, const uint8_t* __restrict__ up_exps,
                                               const uint8_t* __restrict__ gate_sh, const uint8_t* __restrict__ up_sh,
                                               const uint32_t* __restrict__ xrec, uint32_t xrec_bytes,
                                               const int4* __restrict__ items, int max_items, int n_rb,
                                               const int32_t* __restrict__ perm, int k, int H, int F, int Fs,
                                               uint32_t* __restrict__ hrec, int h_rec, int32_t* __restrict__ flags,
                                               int thin_apart) {
    __shared__ __align__(16) uint8_t lds[kLds];
    __shared__ int rowidx[kChunk];
    int y, rt;
    if (!xcd_item(n_rb, max_items, y, rt)) return;
    // with `flags`, this work-group's words (per 64 h rows, as k_mm_gu_thin writes them: the block's two): whether
    // one of its h values is an fp16 overflow (0 when it has no work; a thin item's, k_mm_gu_thin writes after this)
    int32_t* flag = flags ? flags + ((size_t)y * n_rb + rt) * 2 : nullptr;
    Item item;
    if (!work_item(items, y, item)) {
        if (flag && threadIdx.x == 0) flag[0] = flag[1] = 0;
        return;
    }
    const int Fe = item.shared ? Fs : F;
    if (128 * rt >= Fe || (thin_apart && item.ncol <= kThinCols)) {  // (thin items apart: k_mm_gu_thin's)
        if (flag && threadIdx.x == 0) flag[0] = flag[1] = 0;
        return;
    }
    const int ncol = item.ncol;
    if ((int)threadIdx.x < ncol) rowidx[threadIdx.x] = item_token(item, perm, k, threadIdx.x);
    __syncthreads();
    const size_t rb = (size_t)(H >> 7) * 36;
    const uint8_t* g0 = item.shared ? gate_sh : gate_exps + (size_t)item.e * F * rb;
    const uint8_t* u0 = item.shared ? up_sh : up_exps + (size_t)item.e * F * rb;
    if (ncol > 64) mm_gu_body<kWide>(lds, rowidx, item, ncol, rt, g0, u0, xrec, xrec_bytes, H, hrec, h_rec, flag);
    else if (ncol > kThinCols)
        mm_gu_body<kNarrow>(lds, rowidx, item, ncol, rt, g0, u0, xrec, xrec_bytes, H, hrec, h_rec, flag);
    else mm_gu_body<kThin>(lds, rowidx, item, ncol, rt, g0, u0, xrec, xrec_bytes, H, hrec, h_rec, flag);
}

// The thin gate/up items (<= kThinCols columns), launched after k_mm_gu: 64 h rows per work-group (waves 0-3 own
// 16 gate rows each, waves 4-7 the same up rows), a ring of kThinGStages stages of four units, so that several
// work-groups share a CU and one's weight stream overlaps the others' products and epilogues.  After the K
// loop the up waves hand their sums to the gate waves through LDS; h = bf16(silu(gate) * up) goes to record rt of
// each column's h row.
__device__ __forceinline__ void mm_gu_thin_body(uint8_t* lds, const int* rowidx, const Item& item, int ncol, int rt,
                                                const uint8_t* g0, const uint8_t* u0, const uint32_t* xrec,
                                                uint32_t xrec_bytes, int H, uint32_t* hrec, int h_rec, int32_t* flag) {
    using S = Shape<kThinG>;
    static_assert(S::NS == 1 && S::MT == 1, "one 16-row set and one column tile per wave");
    const int units = H >> 7;
    const uint32_t rb = (uint32_t)units * 36u;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, i = lane & 15,
              q = lane >> 4;
    const i32x4 ra = buffer_rsrc(xrec, xrec_bytes);
    const i32x4 rg0 = buffer_rsrc(g0 + (size_t)64 * rt * rb, 64u * rb);
    const i32x4 ru0 = buffer_rsrc(u0 + (size_t)64 * rt * rb, 64u * rb);
    MmPlan<kThinG> pl;
    pl.init(rowidx, wave, lane, ncol, H >> 6, rb, 64, rg0, ru0);
    const bool up_wave = wave >= kWaves / 2;
    const int fbase = 16 * (wave & 3);  // the wave's 16 rows within the work-group's 64 h rows
    int rows[1];
    rows[0] = (up_wave ? 64 : 0) + fbase + i;
    f32x4 acc[kMaxTiles][1];
    mm_loop<kThinG>(acc, lds, pl, units, ra, rows, 0, 1, i, q);
    __syncthreads();  // every wave is done with the ring
    f32x4* xs = reinterpret_cast<f32x4*>(lds + 4096);  // the up waves' sums (after the h tile)
    if (up_wave) xs[(wave - kWaves / 2) * 64 + lane] = acc[0][0];
    __syncthreads();
    // h tile [column][64 rows in record order] as fp16 bits of bf16 values; lane (q, i) of a gate wave holds rows
    // fbase + 4 q .. + 3 of column i, one aligned group of four record positions in the order (0 2 1 3)
    uint16_t* ht = reinterpret_cast<uint16_t*>(lds);
    bool ovf = false;
    if (!up_wave && i < ncol) {
        const f32x4 up = xs[wave * 64 + lane];
        const int pos4 = rec_pos(fbase + 4 * q);
        uint32_t hb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float h = silu_mul_fast(acc[0][0][r], up[r]);
            hb[r] = bf16_as_f16(h);
            if (flag) ovf |= f16_overflow(h);
        }
        *reinterpret_cast<uint2*>(ht + i * 64 + pos4) = make_uint2(hb[0] | (hb[2] << 16), hb[1] | (hb[3] << 16));
    }
    if (flag) {
        const int any = __syncthreads_or(ovf ? 1 : 0);
        if (threadIdx.x == 0) *flag = any ? 1 : 0;
    } else {
        __syncthreads();
    }
    for (int idx = tid; idx < ncol * 8; idx += 512) {  // 8 chunks (one record) per column
        const int c = idx >> 3, ch = idx & 7;
        const uint4 v = reinterpret_cast<const uint4*>(ht + c * 64)[ch];
        reinterpret_cast<uint4*>(hrec + ((size_t)(item.first + c) * h_rec + rt) * (kRecBytes / 4))[ch] = v;
    }
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(8))) void k_mm_gu_thin(const uint8_t* __restrict__ gate_exps,
                                                    const uint8_t* __restrict__ up_exps,
                                                    const uint8_t* __restrict__ gate_sh,
                                                    const uint8_t* __restrict__ up_sh,
                                                    const uint32_t* __restrict__ xrec, uint32_t xrec_bytes,
                                                    const int4* __restrict__ items, int max_items, int n_rb,
                                                    const int32_t* __restrict__ perm, int k, int H, int F, int Fs,
                                                    uint32_t* __restrict__ hrec, int h_rec, int32_t* __restrict__ flags) {
    __shared__ __align__(16) uint8_t lds[Shape<kThinG>::kLdsBytes];
    __shared__ int rowidx[kThinCols];
    int y, rt;
    if (!xcd_item(n_rb, max_items, y, rt)) return;
    Item item;
    if (!work_item(items, y, item) || item.ncol > kThinCols) return;
    const int Fe = item.shared ? Fs : F;
    if (64 * rt >= Fe) return;
    int32_t* flag = flags ? flags + (size_t)y * n_rb + rt : nullptr;
    const int ncol = item.ncol;
    if ((int)threadIdx.x < ncol) rowidx[threadIdx.x] = item_token(item, perm, k, threadIdx.x);
    __syncthreads();
    const size_t rb = (size_t)(H >> 7) * 36;
    const uint8_t* g0 = item.shared ? gate_sh : gate_exps + (size_t)item.e * F * rb;
    const uint8_t* u0 = item.shared ? up_sh : up_exps + (size_t)item.e * F * rb;
    mm_gu_thin_body(lds, rowidx, item, ncol, rt, g0, u0, xrec, xrec_bytes, H, hrec, h_rec, flag);
}

// ------------------------------------------------------------------------------------------------ down
// 8 waves.  A work-group computes down rows [R rt, R rt + R) (R = Shape::kRows) of the item's columns for its nrb row blocks rt
// from rt0 (k_mm_down: kDownRbw; k_mm_down_thin: one) into Y[first + c] (the shared expert's rows times
// sigmoid(sg[t])).  Wave w has rows 16 NS w .. + 16 NS - 1 of each row block (NS sets: two, one for kThinH).
template <int MODE>
__device__ __forceinline__ void mm_down_body(uint8_t* lds, const int* rowidx, const Item& item, int ncol, int units,
                                             int rt0, int nrb, const uint8_t* d0, const uint32_t* hrec,
                                             uint32_t hrec_bytes, int h_rec, const float* sg, int H, float* Y, bool nt) {
    using S = Shape<MODE>;
    constexpr int NS = S::NS;
    const uint32_t rb = (uint32_t)units * 36u;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, i = lane & 15,
              q = lane >> 4;
    constexpr int RW = S::kRows;
    const int nrows = min(RW * nrb, H - RW * rt0);
    const i32x4 ra = buffer_rsrc(hrec, hrec_bytes);
    const uint8_t* dr = d0 + (size_t)RW * rt0 * rb;
    const i32x4 rd = buffer_rsrc(dr, (uint32_t)min(RW, nrows) * rb);
    MmPlan<MODE> pl;
    pl.init(rowidx, wave, lane, ncol, h_rec, rb, RW, rd, rd);
    pl.upr = units;  // (the K loop's epilogue hook stores each row block's results)
    if (nrb > 1) {
        pl.rbs = (uint32_t)RW * rb;
        pl.wbytes = (uint32_t)nrows * rb;
        pl.wbase = dr;
    }
    int rows[NS];
    const int r0 = 16 * NS * wave;
#pragma unroll
    for (int s = 0; s < NS; ++s) rows[s] = r0 + 16 * s + i;
    const int tok0 = 0;
    const int ntiles = min(S::MT, (ncol + 15) >> 4);
    f32x4 acc[kMaxTiles][NS];
    // lane (q, i) holds rows r0 + 16 s + 4 q .. + 3 of column 16 n + i: one 16-byte store (H % 128 == 0); with `nt`
    // a streaming store (Y larger than the caches: its lines would evict the records and weights other work-groups of
    // this XCD still read)
    auto store = [&](int rbl) {
#pragma unroll
        for (int n = 0; n < S::MT; ++n) {
            const int c = tok0 + 16 * n + i;
            if (n < ntiles && c < ncol) {
                const float gs = item.shared ? sigmoid(sg[item.tok0 + c]) : 1.0f;
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int row = RW * (rt0 + rbl) + r0 + 16 * s + 4 * q;
                    if (row < H) {
                        f32x4 v = acc[n][s];
                        if (item.shared) v = f32x4{v[0] * gs, v[1] * gs, v[2] * gs, v[3] * gs};
                        f32x4* dst = reinterpret_cast<f32x4*>(Y + (size_t)(item.first + c) * H + row);
                        if (nt) __builtin_nontemporal_store(v, dst);
                        else *dst = v;
                    }
                }
            }
        }
    };
    if constexpr (S::UPS == 1) {  // each row block's results leave from inside the K loop
        auto epi = [&](int rbl) {
            store(rbl);
#pragma unroll
            for (int n = 0; n < kMaxTiles; ++n)
#pragma unroll
                for (int s = 0; s < NS; ++s) acc[n][s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        };
        mm_loop<MODE>(acc, lds, pl, nrb * units, ra, rows, tok0, ntiles, i, q, epi);
    } else {  // (one row block)
        mm_loop<MODE>(acc, lds, pl, units, ra, rows, tok0, ntiles, i, q);
        store(0);
    }
}

__global__ __launch_bounds__(512) void k_mm_down(const uint8_t* __restrict__ down_exps, const uint8_t* __restrict__ down_sh,
                                                 const uint32_t* __restrict__ hrec, uint32_t hrec_bytes, int h_rec,
                                                 const float* __restrict__ sg, const int4* __restrict__ items,
                                                 int max_items, int n_rg, int n_rb, int H, int F, int Fs,
                                                 float* __restrict__ Y, int nt) {
    __shared__ __align__(16) uint8_t lds[kLds];
    __shared__ int rowidx[kChunk];
    int y, rg;
    if (!xcd_item(n_rg, max_items, y, rg)) return;
    Item item;
    if (!work_item(items, y, item)) return;
    const int Fe = item.shared ? Fs : F;
    const int ncol = item.ncol;
    if (ncol <= kThinCols) return;  // k_mm_down_thin's
    if ((int)threadIdx.x < ncol) rowidx[threadIdx.x] = item.first + threadIdx.x;
    __syncthreads();
    const int units = Fe >> 7;
    const uint8_t* d0 = item.shared ? down_sh : down_exps + (size_t)item.e * H * ((size_t)(F >> 7) * 36);
    const int rt0 = kDownRbw * rg, nrb = min(kDownRbw, n_rb - rt0);
    if (ncol > 64)
        mm_down_body<kWide>(lds, rowidx, item, ncol, units, rt0, nrb, d0, hrec, hrec_bytes, h_rec, sg, H, Y, nt);
    else mm_down_body<kNarrow>(lds, rowidx, item, ncol, units, rt0, nrb, d0, hrec, hrec_bytes, h_rec, sg, H, Y, nt);
}

// The thin items (<= kThinCols columns), launched after k_mm_down: 128 rows per work-group, one-stage ring (36 KB of
// LDS), four work-groups per CU.  A thin down work-group's K is one stage at n_ff <= 512, so it would otherwise hold a
// CU idle while its only stage loads.
__global__ __launch_bounds__(512) void k_mm_down_thin(const uint8_t* __restrict__ down_exps,
                                                      const uint8_t* __restrict__ down_sh,
                                                      const uint32_t* __restrict__ hrec, uint32_t hrec_bytes, int h_rec,
                                                      const float* __restrict__ sg, const int4* __restrict__ items,
                                                      int max_items, int n_rb, int H, int F, int Fs,
                                                      float* __restrict__ Y, int nt) {
    __shared__ __align__(16) uint8_t lds[Shape<kThinH>::kLdsBytes];
    __shared__ int rowidx[kThinCols];
    int y, rt;
    if (!xcd_item(n_rb, max_items, y, rt)) return;
    Item item;
    if (!work_item(items, y, item) || item.ncol > kThinCols) return;
    const int Fe = item.shared ? Fs : F;
    const int ncol = item.ncol;
    if ((int)threadIdx.x < ncol) rowidx[threadIdx.x] = item.first + threadIdx.x;
    __syncthreads();
    const int units = Fe >> 7;
    const uint8_t* d0 = item.shared ? down_sh : down_exps + (size_t)item.e * H * ((size_t)(F >> 7) * 36);
    mm_down_body<kThinH>(lds, rowidx, item, ncol, units, rt, 1, d0, hrec, hrec_bytes, h_rec, sg, H, Y, nt);
}

// ------------------------------------------------------------------------------------------------ launchers
int mfma_chunk() { return kChunk; }
size_t act_rec_bytes(int64_t n_rec) { return (size_t)n_rec * kRecBytes; }

hipError_t launch_junction_records(const float* x, const float* r, int n_rows, int n, float eps, float* out,
                                   uint32_t* rec, uint16_t* xb, hipStream_t s, int32_t* flags) {
    if (n > 4096 || n % 64 || !r ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(out)) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_junction_records, dim3((unsigned)n_rows), dim3(256), 0, s, x, r, n, eps, out, rec, xb, flags);
    return hipGetLastError();
}

int64_t act_records_blocks(int64_t n_rec) { return (n_rec * 8 + 255) / 256; }

hipError_t launch_act_records(const float* x, int64_t n_rec, uint32_t* rec, uint16_t* xb, hipStream_t s,
                              int32_t* flags) {
    hipLaunchKernelGGL(k_act_records, dim3((unsigned)act_records_blocks(n_rec)), dim3(256), 0, s, x, n_rec, rec, xb,
                       flags);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------ router
// The prefill path's router on the matrix cores (bf16 routers, from kMfmaTokens tokens): logits[t][e] =
// sum_h bf16(x[t][h]) * bf16(W[e][h]) (+ bias[e]), and row E (w_inp) the shared gate sg[t].
// v_mfma_f32_16x16x32_bf16: every bf16 product is exact in f32; the sums are the matrix core's f32 accumulation, in
// the hardware's order, so the logits are the exact dot to ~1e-7 relative (not bit for bit the decode path's router);
// the routing and dispatch of the device's logits are exact.
// Work-group tile: 32 tokens x 64 rows; wave w takes rows 16 w .. 16 w + 15 of the 32 tokens (two 16 x 16 tiles; lane
// 16 q + i: A[i][8 q + e] = x of token i, B[8 q + e][j] = weight row j, C[4 q + r][j] in register r).  K runs in
// chunks of 128 through two LDS buffers (rows at a 272-byte pitch: a 16-row fragment read covers the 64 banks once);
// every thread keeps the global loads of the next two chunks in flight, one barrier per chunk.  At 512 tokens the grid
// is 144 work-groups, so the kernel is bound by load latency (one round trip per two chunks), not by the matrix cores:
// the chunk is as deep as the registers of two chunks in flight allow.  The work-groups of one token block take
// consecutive row blocks on one XCD (linear id mod 8), so that the block's x rows are read from memory once per XCD
// and then from its L2.
constexpr int kRtTok = 32, kRtRows = 64, kRtK = 128, kRtPitch = kRtK * 2 + 16, kRtM = kRtTok / 16;
constexpr int kRtPieces = kRtK / 8, kRtPass = 256 / kRtPieces;  // 16-byte pieces per row; rows per pass of 256 threads
constexpr int kRtLa = kRtTok / kRtPass, kRtLb = kRtRows / kRtPass;  // a thread's x and weight pieces per chunk
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_router_mfma(const uint16_t* __restrict__ xb, const uint16_t* __restrict__ W,
                                                      const uint16_t* __restrict__ w_inp, const float* __restrict__ bias,
                                                      int H, int E, int rows_total, int T, int n_tb, int n_rb,
                                                      float* __restrict__ logits, int ld_logits, float* __restrict__ sg) {
    __shared__ __align__(16) uint8_t sa[2][kRtTok * kRtPitch];
    __shared__ __align__(16) uint8_t sb[2][kRtRows * kRtPitch];
    const int id = blockIdx.x;
    const int tb = (id & 7) + 8 * ((id >> 3) / n_rb), rb = (id >> 3) % n_rb;
    if (tb >= n_tb) return;  // (the grid pads the token blocks to a multiple of 8)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, i = lane & 15;
    const int t0 = tb * kRtTok, r0 = rb * kRtRows;
    // a thread's 16-byte pieces of a chunk: piece tid % kRtPieces of x rows and weight rows tid / kRtPieces + kRtPass j
    // (rows clamped: the tail's loads stay in bounds, its results are not stored)
    const int pc = tid % kRtPieces, pr = tid / kRtPieces;
    const uint16_t* asrc[kRtLa];
    const uint16_t* bsrc[kRtLb];
#pragma unroll
    for (int j = 0; j < kRtLa; ++j) asrc[j] = xb + (size_t)min(t0 + pr + kRtPass * j, T - 1) * H + 8 * pc;
#pragma unroll
    for (int j = 0; j < kRtLb; ++j) {
        const int r = min(r0 + pr + kRtPass * j, rows_total - 1);
        bsrc[j] = (r < E ? W + (size_t)r * H : w_inp) + 8 * pc;
    }
    u32x4 ra[2][kRtLa], rw[2][kRtLb];
    auto load = [&](auto slot, int k0) {
        constexpr int P = decltype(slot)::value;
#pragma unroll
        for (int j = 0; j < kRtLa; ++j) ra[P][j] = *reinterpret_cast<const u32x4*>(asrc[j] + k0);
#pragma unroll
        for (int j = 0; j < kRtLb; ++j) rw[P][j] = *reinterpret_cast<const u32x4*>(bsrc[j] + k0);
    };
    auto stash = [&](auto slot) {  // register slot P into LDS buffer P
        constexpr int P = decltype(slot)::value;
#pragma unroll
        for (int j = 0; j < kRtLa; ++j)
            *reinterpret_cast<u32x4*>(&sa[P][(pr + kRtPass * j) * kRtPitch + 16 * pc]) = ra[P][j];
#pragma unroll
        for (int j = 0; j < kRtLb; ++j)
            *reinterpret_cast<u32x4*>(&sb[P][(pr + kRtPass * j) * kRtPitch + 16 * pc]) = rw[P][j];
    };
    using Zero = std::integral_constant<int, 0>;
    using One = std::integral_constant<int, 1>;
    const int nk = H / kRtK;
    load(Zero{}, 0);
    load(One{}, min(1, nk - 1) * kRtK);
    stash(Zero{});
    __syncthreads();
    f32x4 acc[kRtM];
#pragma unroll
    for (int m = 0; m < kRtM; ++m) acc[m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // chunk c lives in register slot c & 1 and LDS buffer c & 1; the loop is unrolled by two so that every register
    // slot is a constant (an indexed slot would wait for its loads at once)
    auto chunk = [&](int kc, auto parity) {
        constexpr int P = decltype(parity)::value;
        using Q = std::integral_constant<int, 1 - P>;
        // chunk kc + 2's loads go out now (unconditionally, past the end the last chunk again: a load under a branch
        // would make the wait below count the loads in flight as zero); chunk kc + 1's, issued a chunk ago, reach LDS
        // after the products
        load(parity, min(kc + 2, nk - 1) * kRtK);
        __builtin_amdgcn_sched_barrier(0);  // (the loads stay ahead of the products and of the stash below)
#pragma unroll
        for (int st = 0; st < kRtK / 32; ++st) {  // the chunk's 32-deep steps
            const bf16x8 b = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(&sb[P][(16 * wave + i) * kRtPitch + 2 * (32 * st + 8 * q)]));
#pragma unroll
            for (int m = 0; m < kRtM; ++m) {
                const bf16x8 a = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(&sa[P][(16 * m + i) * kRtPitch + 2 * (32 * st + 8 * q)]));
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[m], 0, 0, 0);
            }
        }
        stash(Q{});  // (past the end: a copy nobody reads)
        __syncthreads();
    };
    int kc = 0;
    for (; kc + 1 < nk; kc += 2) {
        chunk(kc, Zero{});
        chunk(kc + 1, One{});
    }
    if (kc < nk) chunk(kc, Zero{});  // an odd chunk count's last chunk
    const int row = r0 + 16 * wave + i;
    if (row >= rows_total) return;
    const float bv = (bias && row < E) ? bias[row] : 0.0f;
#pragma unroll
    for (int m = 0; m < kRtM; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 16 * m + 4 * q + r;
            if (t >= T) continue;
            if (row < E) logits[(size_t)t * ld_logits + row] = bias ? acc[m][r] + bv : acc[m][r];
            else sg[t] = acc[m][r];
        }
}

hipError_t launch_router_mfma(const uint16_t* xb, const uint16_t* W, const uint16_t* w_inp, const float* bias, int H,
                              int E, int rows_total, int T, float* logits, int ld_logits, float* sg, hipStream_t s) {
    if (H % kRtK || T < 1 || rows_total < E || rows_total > E + 1 || (rows_total > E && !w_inp))
        return hipErrorInvalidValue;
    const int n_tb = (T + kRtTok - 1) / kRtTok, n_rb = (rows_total + kRtRows - 1) / kRtRows;
    const int n_tb8 = (n_tb + 7) / 8 * 8;
    hipLaunchKernelGGL(k_router_mfma, dim3((unsigned)(n_tb8 * n_rb)), dim3(256), 0, s, xb, W, w_inp, bias, H, E,
                       rows_total, T, n_tb, n_rb, logits, ld_logits, sg);
    return hipGetLastError();
}

hipError_t launch_mm_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint32_t* xrec, int64_t n_xrec, const int4* items, const int32_t* perm, int k, int H,
                        int F, int Fs, int has_shared, int max_items, uint32_t* hrec, int h_rec, hipStream_t s,
                        int32_t* flags, int n_expert) {
    const int Fmax = has_shared && Fs > F ? Fs : F;
    const size_t bytes = act_rec_bytes(n_xrec);
    if (bytes >= kOob) return hipErrorInvalidValue;  // buffer offsets are 31-bit
    const int n_rb = Fmax / 128;
    // the thin items in a kernel of their own when they are many (fewer than kThinApartPairs pairs per expert on
    // average); with many pairs per expert they are few, and inside k_mm_gu they run in its tail instead of after it
    const int P = (int)(n_xrec / (H / 64)) * k;
    const int thin_apart = P < kThinApartPairs * n_expert ? 1 : 0;
    hipLaunchKernelGGL(k_mm_gu, dim3(xcd_grid(n_rb, max_items)), dim3(512), 0, s, gate_exps, up_exps, gate_sh, up_sh,
                       xrec, (uint32_t)bytes, items, max_items, n_rb, perm, k, H, F, Fs, hrec, h_rec, flags,
                       thin_apart);
    if (thin_apart)
        hipLaunchKernelGGL(k_mm_gu_thin, dim3(xcd_grid(2 * n_rb, max_items)), dim3(512), 0, s, gate_exps, up_exps,
                           gate_sh, up_sh, xrec, (uint32_t)bytes, items, max_items, 2 * n_rb, perm, k, H, F, Fs, hrec,
                           h_rec, flags);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_copy_f32(const float* __restrict__ src, int64_t n, float* __restrict__ dst) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy_f32(const float* src, int64_t n, float* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)blocks), dim3(256), 0, s, src, n, dst);
    return hipGetLastError();
}

// The overflow mask of smoe_trace: bit 0 when a flag of fx is set, bit 1 when one of fh is (one work-group).
// The call's status mask from its flag words: bit 0 any x flag, bit 1 any h flag (the prefill path's fp16 operand
// limits), bit 2 any wait flag (a fused decode launch's bounded wait gave up).
__global__ __launch_bounds__(256) void k_flags_mask(const int32_t* __restrict__ fx, int64_t nx,
                                                    const int32_t* __restrict__ fh, int64_t nh,
                                                    const int32_t* __restrict__ fw, int64_t nw, int32_t* __restrict__ out) {
    int ax = 0, ah = 0, aw = 0;
    for (int64_t i = threadIdx.x; i < nx; i += 256) ax |= fx[i];
    for (int64_t i = threadIdx.x; i < nh; i += 256) ah |= fh[i];
    for (int64_t i = threadIdx.x; i < nw; i += 256) aw |= fw[i];
    ax = __syncthreads_or(ax);
    ah = __syncthreads_or(ah);
    aw = __syncthreads_or(aw);
    if (threadIdx.x == 0) *out = (ax ? 1 : 0) | (ah ? 2 : 0) | (aw ? 4 : 0);
}

hipError_t launch_flags_mask(const int32_t* fx, int64_t nx, const int32_t* fh, int64_t nh, int32_t* out,
                             hipStream_t s, const int32_t* fw, int64_t nw) {
    hipLaunchKernelGGL(k_flags_mask, dim3(1), dim3(256), 0, s, fx, nx, fh, nh, fw, nw, out);
    return hipGetLastError();
}

hipError_t launch_mm_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* hrec, int64_t n_hrec,
                          int h_rec, const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                          int nt, hipStream_t s) {
    const size_t bytes = act_rec_bytes(n_hrec);
    if (bytes >= kOob) return hipErrorInvalidValue;
    // the thin items after the others: their kernel's smaller LDS lets two work-groups share a CU
    const int n_rb = (H + kWgRows - 1) / kWgRows, n_rg = (n_rb + kDownRbw - 1) / kDownRbw;
    hipLaunchKernelGGL(k_mm_down, dim3(xcd_grid(n_rg, max_items)), dim3(512), 0, s, down_exps, down_sh, hrec,
                       (uint32_t)bytes, h_rec, sg, items, max_items, n_rg, n_rb, H, F, Fs, Y, nt);
    const int n_rb_thin = (H + Shape<kThinH>::kRows - 1) / Shape<kThinH>::kRows;
    hipLaunchKernelGGL(k_mm_down_thin, dim3(xcd_grid(n_rb_thin, max_items)), dim3(512), 0, s, down_exps, down_sh,
                       hrec, (uint32_t)bytes, h_rec, sg, items, max_items, n_rb_thin, H, F, Fs, Y, nt);
    return hipGetLastError();
}

}  // namespace smoe
