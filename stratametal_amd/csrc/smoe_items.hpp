// stratametal_amd/csrc/smoe_items.hpp - the work-item table the dispatch writes and the expert kernels read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smoe {

// Work-item table of the expert kernels, 8 ints per item (one 32-byte load): a routed chunk
// {e, first, ncol, tok0 | tok1, tok2, tok3, 0} (the tokens of its first four pairs), shared-expert chunk
// {-1, P + t0, ncol, t0 | t0 + 1, t0 + 2, t0 + 3, 0}, unused {-2, ...}.
constexpr int kShCols = 4;
constexpr int kItemEmpty = -2, kItemShared = -1;

// Work item wi of the expert kernels, from the table the dispatch wrote: a routed expert with its pairs at
// dispatch positions first .. first + ncol, or a chunk of the shared expert's tokens (rows P + t).  Column c
// reads token tok(c) and writes row first + c of the pair-row buffers.
struct Item {
    bool shared;
    int e, ncol, first, tok0;
    int tk[4];
};
__device__ __forceinline__ bool work_item(const int4* __restrict__ items, int wi, Item& it) {
    const int4 a = items[2 * wi], b = items[2 * wi + 1];
    if (a.x == kItemEmpty) return false;
    it.shared = a.x == kItemShared;
    it.e = a.x;
    it.first = a.y;
    it.ncol = a.z;
    it.tok0 = a.w;
    it.tk[0] = a.w;
    it.tk[1] = b.x;
    it.tk[2] = b.y;
    it.tk[3] = b.z;
    return true;
}

// work_item for a work-group-uniform wi: the whole 32-byte entry in one scalar load, all of it in SGPRs before the
// test (so that the compiler does not split the load around the branch and wait twice).
__device__ __forceinline__ bool work_item_uniform(const int4* __restrict__ items, int wi, Item& it) {
    typedef int v8i __attribute__((ext_vector_type(8)));
    v8i v = *reinterpret_cast<const v8i*>(items + 2 * wi);
    asm volatile("" : "+s"(v));
    const int4 a = make_int4(v[0], v[1], v[2], v[3]), b = make_int4(v[4], v[5], v[6], v[7]);
    if (a.x == kItemEmpty) return false;
    it.shared = a.x == kItemShared;
    it.e = a.x;
    it.first = a.y;
    it.ncol = a.z;
    it.tok0 = a.w;
    it.tk[0] = a.w;
    it.tk[1] = b.x;
    it.tk[2] = b.y;
    it.tk[3] = b.z;
    return true;
}

// The token of a routed item's column c < 4, by selects (no branch, no memory read).
__device__ __forceinline__ int item_token_head(const Item& it, int c) {
    return c == 0 ? it.tk[0] : c == 1 ? it.tk[1] : c == 2 ? it.tk[2] : it.tk[3];
}

__device__ __forceinline__ int item_token(const Item& it, const int32_t* perm, int k, int c) {
    if (it.shared) return it.tok0 + c;
    if (c < 4) return c == 0 ? it.tk[0] : c == 1 ? it.tk[1] : c == 2 ? it.tk[2] : it.tk[3];
    return perm[it.first + c] / k;
}

}  // namespace smoe
