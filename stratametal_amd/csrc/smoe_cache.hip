// stratametal_amd/csrc/smoe_cache.hip - the expert tier's device-side lists: routed entries grouped by expert
// through a table of one blob pointer per expert (the hit/miss split), the work-item table of the grouped expert
// kernels, and q8_1 blocks turned into the expert kernels' activation images.
//
// An entry is one routed (token, expert) pair, i = t * k + s of the router's ids.  The split (the reference's
// moe_hit_select / moe_hit_select_multi / moe_group_resident, include/strata/kernels/s2_expert_grouped.hpp:92-112):
// an entry whose expert has a blob (eptr[e] != 0) is a hit, the others (no blob, or an id outside the table) are
// misses.  Hits are grouped by expert: groups in ascending expert id, a group's entries in ascending i, so that each
// blob row is read once for all of its entries (moe_grouped_s2 / native_expert_grouped, s2_expert_grouped.hpp:
// 104-108, include/strata/kernels/iq_kernels.hpp:70-80); misses are listed in ascending i.  Counts stay on the
// device, so a captured graph replays for any split.
#include <hip/hip_runtime.h>

#include "smoe_device.hpp"
#include "smoe_gemv.hpp"
#include "smoe_items.hpp"
#include "smoe_launch.hpp"

namespace smoe {

namespace {

constexpr int kGroupThreads = 1024;

struct GroupLds {
    int cnt[kMaxGroupExperts];   // hits per expert
    int next[kMaxGroupExperts];  // the next free entry of the expert's group
    int res[kMaxGroupExperts];   // the expert has a blob
    int ids[kGroupThreads];      // the pass's hit experts (-1: a miss or past n)
    int gstart[kMaxGroupExperts + 1];
    int etok[kMaxGroupEntries];  // every entry's token, for the items' first four columns
    int scratch[2 * 17];
};

// One work-group of 1024 threads.  Counting sort of the hits by expert (LDS counts, one scan for the group and
// entry offsets packed in one int: groups << 16 | entries), then the entries placed in passes of 1024 in ascending
// i: an entry's rank among the earlier entries of its expert in the pass comes from the pass's ids in LDS, the
// misses' positions from a scan.  With `items`, the work-item table of the expert kernels as well: slot g < cap_groups
// is group g (e = g, so that the kernels read the blob at grp_ptr[g]), the rest empty, then the shared expert's
// token chunks (rows P + t); and `slot_id` = i for the combine of the rows in entry order.
__global__ __launch_bounds__(kGroupThreads) void k_expert_group(
    const int32_t* __restrict__ ids, int n, int kpt, int E, const uint64_t* __restrict__ eptr,
    uint64_t* __restrict__ grp_ptr, int32_t* __restrict__ grp_start, int32_t* __restrict__ grp_expert,
    int32_t* __restrict__ ent_dst, int32_t* __restrict__ ent_tok, int32_t* __restrict__ miss_dst,
    int32_t* __restrict__ counts, int4* __restrict__ items, int cap_groups, int n_sh_items, int P, int T,
    int32_t* __restrict__ slot_id) {
    __shared__ GroupLds s;
    const int tid = threadIdx.x;
    // every expert's blob flag and count (E <= 1024 = one thread each)
    if (tid < E) {
        s.res[tid] = eptr[tid] != 0 ? 1 : 0;
        s.cnt[tid] = 0;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kGroupThreads) {
        const int e = ids[i];
        if (e >= 0 && e < E && s.res[e]) atomicAdd(&s.cnt[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? s.cnt[tid] : 0;
    int sc[1], tot[1];
    block_exclusive_scan_1024<1>({(c > 0 ? 1 << 16 : 0) | c}, s.scratch, sc, tot);
    const int n_groups = tot[0] >> 16, n_hit = tot[0] & 0xFFFF;
    if (c > 0) {
        const int g = sc[0] >> 16, first = sc[0] & 0xFFFF;
        grp_ptr[g] = eptr[tid];
        grp_start[g] = first;
        if (grp_expert) grp_expert[g] = tid;
        s.gstart[g] = first;
        s.next[tid] = first;
    }
    if (tid == 0) {
        grp_start[n_groups] = n_hit;
        s.gstart[n_groups] = n_hit;
    }
    int miss_base = 0;
    for (int i0 = 0; i0 < n; i0 += kGroupThreads) {
        const int i = i0 + tid;
        const int e = i < n ? ids[i] : -1;
        const bool hit = i < n && e >= 0 && e < E && s.res[e];
        const bool miss = i < n && !hit;
        __syncthreads();  // the previous pass's reads of s.ids and s.scratch are done
        s.ids[tid] = hit ? e : -1;
        int ms[1], mt[1];
        block_exclusive_scan_1024<1>({miss ? 1 : 0}, s.scratch + 17, ms, mt);  // its barrier publishes s.ids
        if (hit) {
            int rank = 0;
            for (int j = 0; j < tid; ++j) rank += s.ids[j] == e ? 1 : 0;
            const int pos = s.next[e] + rank;
            ent_dst[pos] = i;
            ent_tok[pos] = i / kpt;
            s.etok[pos] = i / kpt;
        }
        if (miss) miss_dst[miss_base + ms[0]] = i;
        __syncthreads();  // every rank read s.next
        if (hit) atomicAdd(&s.next[e], 1);
        miss_base += mt[0];
    }
    if (tid == 0) {
        counts[0] = n_groups;
        counts[1] = n_hit;
        counts[2] = miss_base;
        counts[3] = 0;
    }
    if (!items) return;
    __syncthreads();  // s.etok complete
    for (int wi = tid; wi < cap_groups + n_sh_items; wi += kGroupThreads) {
        int4 a = make_int4(kItemEmpty, 0, 0, 0), b = make_int4(0, 0, 0, 0);
        if (wi < n_groups) {
            const int first = s.gstart[wi], ncol = s.gstart[wi + 1] - first;
            int tk[4] = {0, 0, 0, 0};
            for (int j = 0; j < 4 && j < ncol; ++j) tk[j] = s.etok[first + j];
            a = make_int4(wi, first, ncol, tk[0]);
            b = make_int4(tk[1], tk[2], tk[3], 0);
        } else if (wi >= cap_groups) {
            const int t0 = (wi - cap_groups) * kShCols;
            a = make_int4(kItemShared, P + t0, min(kShCols, T - t0), t0);
            b = make_int4(t0 + 1, t0 + 2, t0 + 3, 0);
        }
        items[2 * wi] = a;
        items[2 * wi + 1] = b;
    }
    for (int i = tid; slot_id && i < n; i += kGroupThreads) slot_id[i] = i;
}

// The work-item table of caller-made group lists (counts[0] groups; group g's blob at grp_ptr[g], its entries
// [grp_start[g], grp_start[g + 1]) reading token ent_tok[j] and writing row ent_dst[j]), checked on the device so
// that no list can send a kernel outside its buffers: groups beyond cap_groups are dropped, a group's entries are
// clipped to [0, cap_entries), a group without a blob is empty, and an entry whose token is not below n_tok or
// whose row is not below n_rows gets token 0 and row -1 (computed, not written).  The checked tokens and rows go
// to etok / edst, which the kernels read instead of the caller's.
__global__ __launch_bounds__(256) void k_group_items(const uint64_t* __restrict__ grp_ptr,
                                                      const int32_t* __restrict__ grp_start,
                                                      const int32_t* __restrict__ ent_tok,
                                                      const int32_t* __restrict__ ent_dst,
                                                      const int32_t* __restrict__ counts, int cap_groups,
                                                      int cap_entries, int n_tok, int n_rows, int4* __restrict__ items,
                                                      int32_t* __restrict__ etok, int32_t* __restrict__ edst) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    auto checked_tok = [&](int j) {
        const int t = ent_tok[j], d = ent_dst[j];
        return (t >= 0 && t < n_tok && d >= 0 && d < n_rows) ? t : 0;
    };
    if (i < cap_entries) {
        const int t = ent_tok[i], d = ent_dst[i];
        const bool ok = t >= 0 && t < n_tok && d >= 0 && d < n_rows;
        etok[i] = ok ? t : 0;
        edst[i] = ok ? d : -1;
    }
    if (i >= cap_groups) return;
    const int n_groups = min(counts[0], cap_groups);
    int4 a = make_int4(kItemEmpty, 0, 0, 0), b = make_int4(0, 0, 0, 0);
    if (i < n_groups && grp_ptr[i] != 0) {
        const int first = min(max(grp_start[i], 0), cap_entries);
        const int last = min(max(grp_start[i + 1], first), cap_entries);
        const int ncol = last - first;
        if (ncol > 0) {
            int tk[4] = {0, 0, 0, 0};
            for (int j = 0; j < 4 && j < ncol; ++j) tk[j] = checked_tok(first + j);
            a = make_int4(i, first, ncol, tk[0]);
            b = make_int4(tk[1], tk[2], tk[3], 0);
        }
    }
    items[2 * i] = a;
    items[2 * i + 1] = b;
}

// q8_1 blocks (36 bytes: fp16 d, fp16 s, 32 int8) -> activation images (kImgDw dwords: the 32 values split into
// nibbles, or in natural byte order, then f32 of d and the integer sum of the values), one thread per block.  The
// image equals the one the router kernel writes for the same activation row (both come from the same quantiser).
__global__ __launch_bounds__(256) void k_q8_images(const uint8_t* __restrict__ xq, int64_t n_blocks, int natural,
                                                    uint32_t* __restrict__ img) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t* p = xq + b * 36;
    const uint32_t d16 = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    int q[32];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        q[i] = (int)(int8_t)p[4 + i];
        sum += q[i];
    }
    uint32_t w[8];
    if (natural) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            w[c] = (uint32_t)(uint8_t)q[4 * c] | ((uint32_t)(uint8_t)q[4 * c + 1] << 8) |
                   ((uint32_t)(uint8_t)q[4 * c + 2] << 16) | ((uint32_t)(uint8_t)q[4 * c + 3] << 24);
    } else {
        // position p: 16-group g = p >> 4, parity p & 1, nibble (p & 15) >> 1 of dword 4 g + 2 (p & 1) (high
        // nibbles of the value) and of the dword after it (low nibbles)
#pragma unroll
        for (int c = 0; c < 8; ++c) w[c] = 0;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int dw = 4 * (i >> 4) + 2 * (i & 1), sh = 4 * ((i & 15) >> 1);
            w[dw] |= (uint32_t)((q[i] >> 4) & 15) << sh;
            w[dw + 1] |= (uint32_t)(q[i] & 15) << sh;
        }
    }
    uint4* o = reinterpret_cast<uint4*>(img + b * kImgDw);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
    o[2] = make_uint4(f2u(f16_to_f32(d16)), (uint32_t)sum, 0u, 0u);
}

// p[i] = i (the combine's slots of rows kept in entry order)
__global__ __launch_bounds__(256) void k_iota(int32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = i;
}

}  // namespace

hipError_t launch_iota(int32_t* p, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_iota, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

hipError_t launch_expert_group(const int32_t* ids, int n, int kpt, int E, const uint64_t* eptr, uint64_t* grp_ptr,
                               int32_t* grp_start, int32_t* grp_expert, int32_t* ent_dst, int32_t* ent_tok,
                               int32_t* miss_dst, int32_t* counts, int4* items, int cap_groups, int n_sh_items, int P,
                               int T, int32_t* slot_id, hipStream_t s) {
    hipLaunchKernelGGL(k_expert_group, dim3(1), dim3(kGroupThreads), 0, s, ids, n, kpt, E, eptr, grp_ptr, grp_start,
                       grp_expert, ent_dst, ent_tok, miss_dst, counts, items, cap_groups, n_sh_items, P, T, slot_id);
    return hipGetLastError();
}

hipError_t launch_group_items(const uint64_t* grp_ptr, const int32_t* grp_start, const int32_t* ent_tok,
                              const int32_t* ent_dst, const int32_t* counts, int cap_groups, int cap_entries, int n_tok,
                              int n_rows, int4* items, int32_t* etok, int32_t* edst, hipStream_t s) {
    const int n = cap_groups > cap_entries ? cap_groups : cap_entries;
    hipLaunchKernelGGL(k_group_items, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, grp_ptr, grp_start, ent_tok,
                       ent_dst, counts, cap_groups, cap_entries, n_tok, n_rows, items, etok, edst);
    return hipGetLastError();
}

hipError_t launch_q8_images(const uint8_t* xq, int64_t n_blocks, int natural, uint32_t* img, hipStream_t s) {
    hipLaunchKernelGGL(k_q8_images, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, s, xq, n_blocks, natural,
                       img);
    return hipGetLastError();
}

}  // namespace smoe
