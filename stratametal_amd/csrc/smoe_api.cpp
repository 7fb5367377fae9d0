// stratametal_amd/csrc/smoe_api.cpp - the C ABI (include/smoe.h): argument checks, workspace layout and
// the launch sequence.  Every refusal happens before the first launch, so a refused call leaves all
// outputs untouched; a zero count returns before launching (metal/src/router.mm:33-37,
// metal/src/iq.mm:150-158, metal/src/moe_combine.mm:32-34).
#include "smoe.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "smoe_launch.hpp"

namespace {

thread_local std::string g_last;

smoe_status fail(smoe_status s, const std::string& why) {
    g_last = why;
    return s;
}
smoe_status ok() {
    g_last.clear();
    return SMOE_OK;
}

constexpr size_t kAlign = 256;
size_t up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int row_values(int type) { return type == SMOE_Q2_0 ? 128 : type == SMOE_IQ2_S ? 256 : 0; }

// The shared expert's projection types (0 in the geometry: sh_type).  A shared expert whose three types equal the
// routed type runs inside the expert kernels ("fused"); any other runs the q8_1 GEMV chain ("native").
int sh_gate_t(const smoe_geom& g) { return g.sh_gate_type ? g.sh_gate_type : g.sh_type; }
int sh_up_t(const smoe_geom& g) { return g.sh_up_type ? g.sh_up_type : g.sh_type; }
int sh_down_t(const smoe_geom& g) { return g.sh_down_type ? g.sh_down_type : g.sh_type; }
bool sh_native(const smoe_geom& g) {
    return g.sh_type >= 0 && (sh_gate_t(g) != g.w_type || sh_up_t(g) != g.w_type || sh_down_t(g) != g.w_type);
}
bool sh_fused(const smoe_geom& g) { return g.sh_type >= 0 && !sh_native(g); }
bool gemv_type(int t) { return t == SMOE_Q2_0 || t == SMOE_IQ2_S || smoe::native_type(t); }

// GEMV-path tiling limits: a row of n_embd is at most 32 double blocks (4096 values).
constexpr int kMaxEmbd = 4096;
constexpr int kMaxFF = 4096;
constexpr int kMaxExpert = 1024;
constexpr int kMaxK = 64;
// Up to this many tokens top-k and dispatch run as one work-group (k_topk_dispatch: one wave per token, at most
// one per SIMD); beyond it the tokens are routed by one work-group each (k_topk), then dispatched (k_dispatch).
constexpr int kFusedRouteTokens = 4;
// From this many pairs the dispatch runs as three launches over chunks of 1024 pairs (k_dispatch_hist,
// k_dispatch_scan, k_dispatch_rank) instead of one work-group.
constexpr int kDispatchMultiPairs = 2048;
// SMOE_PATH_AUTO runs the MFMA (prefill) contract from this many tokens on.
constexpr int kMfmaTokens = 128;
// The MFMA kernels' buffer offsets into the activation and h records are 31-bit.
constexpr size_t kMfmaRecordLimit = (size_t)1 << 31;
// The prefill path's Y (f32 per-pair rows) from this size on is stored and read with streaming accesses (half the
// 256 MB Infinity Cache).
constexpr size_t kYStreamBytes = (size_t)128 << 20;

smoe_status check_geom(const smoe_geom* g) {
    if (!g) return fail(SMOE_ENULL, "geometry is NULL");
    if (g->w_type != SMOE_Q2_0 && g->w_type != SMOE_IQ2_S)
        return fail(SMOE_ETYPE, "routed expert type " + std::to_string(g->w_type) + " is not Q2_0 (42) or IQ2_S (22)");
    if (g->sh_type != -1 && !gemv_type(g->sh_type))
        return fail(SMOE_ETYPE, "shared expert type " + std::to_string(g->sh_type) + " is not a supported type or -1");
    for (const int t : {g->sh_gate_type, g->sh_up_type, g->sh_down_type})
        if (t != 0 && !gemv_type(t))
            return fail(SMOE_ETYPE, "shared projection type " + std::to_string(t) + " is not a supported type");
    if (g->router_dtype != SMOE_ROUTER_BF16 && g->router_dtype != SMOE_ROUTER_F32)
        return fail(SMOE_EINVAL, "router_dtype must be 0 (bf16) or 1 (f32)");
    if (g->n_expert < 1 || g->n_expert > kMaxExpert) return fail(SMOE_EINVAL, "n_expert must be in 1..1024");
    if (g->top_k < 1 || g->top_k > kMaxK) return fail(SMOE_EINVAL, "top_k must be in 1..64");
    if (g->top_k > g->n_expert) return fail(SMOE_EINVAL, "top_k exceeds n_expert");
    const int rv = row_values(g->w_type);
    if (g->n_embd <= 0 || g->n_embd % rv || g->n_embd > kMaxEmbd)
        return fail(SMOE_EINVAL, "n_embd must be a positive multiple of " + std::to_string(rv) + ", at most 4096");
    if (g->n_ff <= 0 || g->n_ff % rv || g->n_ff > kMaxFF)
        return fail(SMOE_EINVAL, "n_ff must be a positive multiple of " + std::to_string(rv) + ", at most 4096");
    const bool has_sh = sh_fused(*g), nat = sh_native(*g);
    if (has_sh && (g->n_ff_shared <= 0 || g->n_ff_shared % rv || g->n_ff_shared > kMaxFF))
        return fail(SMOE_EINVAL, "n_ff_shared must be a positive multiple of " + std::to_string(rv) + ", at most 4096");
    if (nat) {  // each projection's rows a whole number of its blocks, in a shape its GEMV tiles
        const int Fs = g->n_ff_shared;
        if (Fs <= 0 || Fs % 32 || Fs > kMaxFF)
            return fail(SMOE_EINVAL, "a native shared expert's n_ff_shared must be a positive multiple of 32, at most 4096");
        const struct { int type, n; const char* what; } proj[3] = {
            {sh_gate_t(*g), g->n_embd, "gate"}, {sh_up_t(*g), g->n_embd, "up"}, {sh_down_t(*g), Fs, "down"}};
        for (const auto& p : proj) {
            const bool ok = p.type == SMOE_Q2_0    ? (p.n % 128 == 0 && p.n <= kMaxFF && smoe::gemv_shape_ok(p.n))
                            : p.type == SMOE_IQ2_S ? smoe::iq2_shape_ok(p.n)
                                                   : smoe::native_row_bytes(p.type, p.n) > 0;
            if (!ok)
                return fail(SMOE_EINVAL, std::string("shared ") + p.what + " rows of " + std::to_string(p.n) +
                                             " values do not fit type " + std::to_string(p.type) + "'s blocks");
        }
    }
    if (g->w_type == SMOE_Q2_0) {
        if (!smoe::gemv_shape_ok(g->n_embd) || !smoe::gemv_shape_ok(g->n_ff))
            return fail(SMOE_EINVAL, "n_embd / 128 and n_ff / 128 must each be a power of two times at most 8");
        if (has_sh && !smoe::down_shapes_match(g->n_ff, g->n_ff_shared))
            return fail(SMOE_EINVAL, "n_ff_shared must split into down-row units like n_ff (same power-of-two factor)");
    } else {
        if (!smoe::iq2_shape_ok(g->n_embd) || !smoe::iq2_shape_ok(g->n_ff))
            return fail(SMOE_EINVAL, "IQ2_S: n_embd and n_ff must be 512, 1024 or 2048");
        if (has_sh && g->n_ff_shared != g->n_ff)
            return fail(SMOE_EINVAL, "IQ2_S: n_ff_shared must equal n_ff");
    }
    return SMOE_OK;
}

struct Layout {
    size_t ximg, xbf, logits, sg, ids, wts, counts, offsets, perm, slot, elist, nlist, items, himg, Y, dwork, xchg,
        oflags, status, nxq, ngu, nhq, total;
    int h_blocks;  // q8_1 blocks per h row (GEMV path)
    int h_rec;     // 64-value records per h row (MFMA path)
    int64_t n_xflags, n_hflags;  // the MFMA path's per-work-group overflow flags (a trace asking for the mask)
};

// Work items: every touched expert plus the shared expert's token chunks (GEMV path); the MFMA path splits
// an expert's pairs and the shared tokens into chunks of mfma_chunk() columns.
constexpr int64_t kMaxGridY = 65535;  // the largest y dimension of a launch grid

int max_items_gemv(const smoe_geom& g, int64_t T) {
    const int64_t P = T * g.top_k;
    return (int)((P < g.n_expert ? P : g.n_expert) + (sh_fused(g) ? smoe::shared_items((int)T) : 0));
}
int max_items_mfma(const smoe_geom& g, int64_t T) {
    const int64_t P = T * g.top_k, C = smoe::mfma_chunk();
    return (int)((P < g.n_expert ? P : g.n_expert) + P / C + (sh_fused(g) ? (T + C - 1) / C : 0));
}

Layout layout(const smoe_geom& g, int64_t T) {
    Layout L{};
    const int64_t H = g.n_embd, E = g.n_expert, K = g.top_k;
    const int64_t P = T * K;
    const int64_t Fmax = (sh_fused(g) && g.n_ff_shared > g.n_ff) ? g.n_ff_shared : g.n_ff;
    L.h_blocks = (int)(Fmax / 32);
    L.h_rec = (int)(Fmax / 64);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = up(o + bytes);
        return at;
    };
    auto most = [](size_t a, size_t b) { return a > b ? a : b; };
    // x: q8_1 images (GEMV) or bf16 records (MFMA); h likewise
    L.ximg = take(most(smoe::img_bytes(T * (H / 32)), smoe::act_rec_bytes(T * (H / 64))));
    L.xbf = take((size_t)T * H * 2);  // bf16 x of the MFMA path (the router's exact operand)
    L.logits = take((size_t)T * E * 4);
    L.sg = take((size_t)T * 4);
    L.ids = take((size_t)P * 4);
    L.wts = take((size_t)P * 4);
    L.counts = take((size_t)E * 4);
    L.offsets = take((size_t)(E + 1) * 4);
    L.perm = take((size_t)P * 4);
    L.slot = take((size_t)P * 4);
    L.elist = take((size_t)(E + 1) * 4);
    L.nlist = take(16);
    L.items = take((size_t)most(max_items_gemv(g, T), max_items_mfma(g, T)) * 32);
    L.himg = take(most(smoe::img_bytes((P + T) * L.h_blocks), smoe::act_rec_bytes((P + T) * L.h_rec)));
    L.Y = take((size_t)(P + T) * H * 4);
    L.dwork = take(smoe::dispatch_work_bytes(P, (int)E));  // chunk histograms of the many-pair dispatch
    // the h exchange of the fused small-batch launch, sized for its largest batch whatever T is (so that a workspace
    // sized for max_tokens holds every smaller call's layout)
    L.xchg = take(smoe::moe_small_xchg_bytes(kFusedRouteTokens, (int)K, max_items_gemv(g, kFusedRouteTokens),
                                             L.h_blocks));
    L.n_xflags = most(smoe::act_records_blocks(T * (H / 64)), T);
    L.n_hflags = (Fmax / 64) * (int64_t)max_items_mfma(g, T);  // one per 64 h rows of every work item
    L.oflags = take((size_t)(L.n_xflags + L.n_hflags) * 4);
    L.status = take((size_t)smoe::fused_status_words((int)H) * 4);  // the fused decode launch's wait flags
    if (sh_native(g)) {  // the native shared expert's chain: x as q8_1 blocks, gate and up rows, q8_1 of h
        const int64_t Fs = g.n_ff_shared;
        L.nxq = take((size_t)T * (H / 32) * 36);
        L.ngu = take((size_t)2 * T * Fs * 4);
        L.nhq = take((size_t)T * (Fs / 32) * 36);
    }
    L.total = o;
    return L;
}

hipStream_t stream_of(void* s) { return reinterpret_cast<hipStream_t>(s); }

smoe_status launched(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(SMOE_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return SMOE_OK;
}

#define SMOE_TRY(call, what)                              \
    do {                                                  \
        const smoe_status _s = launched((call), (what));  \
        if (_s != SMOE_OK) return _s;                     \
    } while (0)

}  // namespace

namespace smoe {
// The thread's last error for the other translation units of the library (the model reader).
smoe_status report(smoe_status s, const std::string& why) { return s == SMOE_OK ? ok() : fail(s, why); }
}  // namespace smoe

extern "C" {

const char* smoe_status_str(smoe_status s) {
    switch (s) {
        case SMOE_OK: return "ok";
        case SMOE_EINVAL: return "invalid argument";
        case SMOE_ESIZE: return "buffer too small";
        case SMOE_ETYPE: return "unsupported ggml type";
        case SMOE_EDEVICE: return "HIP runtime error";
        case SMOE_EALIGN: return "misaligned pointer";
        case SMOE_ENULL: return "NULL pointer";
    }
    return "unknown status";
}

const char* smoe_last_error(void) { return g_last.c_str(); }

int32_t smoe_abi_version(void) { return 109; }

size_t smoe_workspace_bytes(const smoe_geom* g, int32_t max_tokens) {
    if (check_geom(g) != SMOE_OK || max_tokens < 0) return 0;
    return layout(*g, max_tokens).total;
}

namespace {
bool overlaps(const void* a, const void* b, size_t bytes) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), z = reinterpret_cast<uintptr_t>(b);
    return x < z + bytes && z < x + bytes;
}
// [a, a + na) and [b, b + nb) share a byte
bool overlaps_n(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), z = reinterpret_cast<uintptr_t>(b);
    return x < z + nb && z < x + na;
}

// Every check of a block call that can refuse it, made before its first launch (smoe_ffn_run runs it ahead of
// its own first launch too).
smoe_status check_forward(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, const float* y,
                          const void* workspace, size_t workspace_bytes, int32_t path, const float* x_prev,
                          const float* r_prev) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (!w) return fail(SMOE_ENULL, "weights is NULL");
    if (n_tokens < 0) return fail(SMOE_EINVAL, "n_tokens is negative");
    if (path < SMOE_PATH_AUTO || path > SMOE_PATH_MFMA) return fail(SMOE_EINVAL, "unknown path");
    if ((int64_t)n_tokens * g->top_k > (1 << 24)) return fail(SMOE_EINVAL, "n_tokens * top_k exceeds 2^24");
    if (!w->gate_exps || !w->up_exps || !w->down_exps || !w->router)
        return fail(SMOE_ENULL, "a routed expert tensor or the router is NULL");
    const bool has_sh = g->sh_type >= 0;
    if (has_sh && (!w->gate_sh || !w->up_sh || !w->down_sh || !w->gate_inp_sh))
        return fail(SMOE_ENULL, "a shared expert tensor is NULL (set sh_type = -1 for a layer without one)");
    if (!aligned(w->gate_exps, 4) || !aligned(w->up_exps, 4) || !aligned(w->down_exps, 4))
        return fail(SMOE_EALIGN, "expert tensors must be 4-byte aligned");
    if (!aligned(w->router, 16)) return fail(SMOE_EALIGN, "the router must be 16-byte aligned");
    if (has_sh && (!aligned(w->gate_sh, 4) || !aligned(w->up_sh, 4) || !aligned(w->down_sh, 4) ||
                   !aligned(w->gate_inp_sh, 16)))
        return fail(SMOE_EALIGN, "shared tensors must be 4-byte aligned (gate_inp_shexp 16-byte)");
    if (w->logit_bias && !aligned(w->logit_bias, 4)) return fail(SMOE_EALIGN, "logit_bias must be 4-byte aligned");
    if (n_tokens == 0) return ok();  // empty x / y may be NULL: nothing is read or written
    if (!x || !y) return fail(SMOE_ENULL, "x or y is NULL");
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(SMOE_EALIGN, "x and y must be 4-byte aligned");
    if (x_prev) {
        const size_t bytes = (size_t)n_tokens * g->n_embd * 4;
        if (!r_prev) return fail(SMOE_ENULL, "r_prev is NULL");
        if (g->n_embd > 4096) return fail(SMOE_EINVAL, "the fused junction takes rows up to 4096");
        if (!aligned(x_prev, 16) || !aligned(r_prev, 16) || !aligned(x, 16))
            return fail(SMOE_EALIGN, "x_prev, r_prev and x must be 16-byte aligned");
        if (overlaps(x, x_prev, bytes) || overlaps(x, r_prev, bytes) || overlaps(x, y, bytes))
            return fail(SMOE_EINVAL, "x must not overlap x_prev, r_prev or y");
    }
    const bool iq2 = g->w_type == SMOE_IQ2_S;
    if (iq2 && path == SMOE_PATH_MFMA) return fail(SMOE_ETYPE, "the MFMA (prefill) path is built for Q2_0 experts only");
    const bool mfma = !iq2 && (path == SMOE_PATH_MFMA || (path == SMOE_PATH_AUTO && n_tokens >= kMfmaTokens));

    // grids take tokens and work items on their y dimension, at most 65535: refused here, before any launch
    if (n_tokens > kMaxGridY)
        return fail(SMOE_EINVAL, std::to_string(n_tokens) + " tokens exceed " + std::to_string(kMaxGridY) +
                                     " per call; split the batch");
    const int64_t n_items = mfma ? max_items_mfma(*g, n_tokens) : max_items_gemv(*g, n_tokens);
    if (n_items > kMaxGridY)
        return fail(SMOE_EINVAL, std::to_string(n_items) + " expert work items exceed " + std::to_string(kMaxGridY) +
                                     " per call; split the batch");
    const Layout L = layout(*g, n_tokens);
    if (mfma) {  // the MFMA kernels address the activation and h records with 31-bit buffer offsets
        const int64_t P = (int64_t)n_tokens * g->top_k;
        if (smoe::act_rec_bytes((int64_t)n_tokens * (g->n_embd / 64)) >= kMfmaRecordLimit ||
            smoe::act_rec_bytes((P + n_tokens) * L.h_rec) >= kMfmaRecordLimit)
            return fail(SMOE_EINVAL, "the MFMA path's activation or h records of " + std::to_string(n_tokens) +
                                         " tokens exceed 2 GiB; split the batch");
    }
    if (!workspace) return fail(SMOE_ENULL, "workspace is NULL");
    if (!aligned(workspace, kAlign)) return fail(SMOE_EALIGN, "workspace must be 256-byte aligned");
    if (workspace_bytes < L.total)
        return fail(SMOE_ESIZE, "workspace is " + std::to_string(workspace_bytes) + " bytes, needs " +
                                    std::to_string(L.total));
    return SMOE_OK;
}

#define SMOE_TRY_S(call)                    \
    do {                                    \
        const smoe_status _s = (call);      \
        if (_s != SMOE_OK) return _s;       \
    } while (0)

// Where a call left its flag words in the workspace: the prefill path's fp16 operand flags of its records kernel and
// k_mm_gu (bits 0 and 1 of the status mask), the fused decode launch's wait flags, one per down work-group (bit 2).
struct FlagWords {
    const void* ws = nullptr;
    size_t x = 0, h = 0, w = 0;  // byte offsets in the workspace
    int64_t nx = 0, nh = 0, nw = 0;
};
void flag_words(const smoe_geom& g, const Layout& L, int T, bool mfma, bool fused, bool junction, const void* ws,
                FlagWords& f) {
    f = FlagWords{};
    f.ws = ws;
    const int H = g.n_embd, F = g.n_ff, Fs = sh_fused(g) ? g.n_ff_shared : 0;
    if (mfma) {
        f.x = L.oflags;
        f.nx = junction ? T : smoe::act_records_blocks((int64_t)T * (H / 64));
        f.h = L.oflags + (size_t)L.n_xflags * 4;
        f.nh = (int64_t)(F > Fs ? F : Fs) / 128 * max_items_mfma(g, T);
    }
    if (fused) {
        f.w = L.status;
        f.nw = smoe::fused_status_words(H);
    }
}
smoe_status fold_status(const FlagWords& f, int32_t* out, hipStream_t st) {
    const uint8_t* ws = static_cast<const uint8_t*>(f.ws);
    SMOE_TRY(smoe::launch_flags_mask(reinterpret_cast<const int32_t*>(ws + f.x), f.nx,
                                     reinterpret_cast<const int32_t*>(ws + f.h), f.nh, out, st,
                                     reinterpret_cast<const int32_t*>(ws + f.w), f.nw),
             "status mask");
    return SMOE_OK;
}

// The flag words of the last call enqueued on each of the most recent workspaces (smoe_forward_status's table).
constexpr int kFlagTable = 64;
std::mutex g_flag_mu;
FlagWords g_flag_table[kFlagTable];
int g_flag_next = 0;
void remember_flags(const FlagWords& f) {
    std::lock_guard<std::mutex> lock(g_flag_mu);
    for (FlagWords& e : g_flag_table)
        if (e.ws == f.ws) {
            e = f;
            return;
        }
    g_flag_table[g_flag_next] = f;
    g_flag_next = (g_flag_next + 1) % kFlagTable;
}
bool recall_flags(const void* ws, FlagWords& f) {
    std::lock_guard<std::mutex> lock(g_flag_mu);
    for (const FlagWords& e : g_flag_table)
        if (e.ws && e.ws == ws) {
            f = e;
            return true;
        }
    return false;
}

// The native shared expert (its projections in their own types): q8_1 of x, gate and up, SwiGLU + q8_1, down
// times sigmoid(sg[t]) into out[t] (T rows of n_embd), in the workspace's native-chain slots.
smoe_status native_shared(const smoe_geom& g, const smoe_weights* w, const float* x, int T, uint8_t* ws,
                          const Layout& L, float* out, const float* sg, hipStream_t st) {
    const int H = g.n_embd, Fn = g.n_ff_shared;
    uint8_t* nxq = ws + L.nxq;
    float* ngu = reinterpret_cast<float*>(ws + L.ngu);
    uint8_t* nhq = ws + L.nhq;
    SMOE_TRY(smoe::launch_prep(x, (int64_t)T * H, nxq, nullptr, st), "shared q8_1");
    auto gemv = [&](int type, const void* wt, const uint8_t* xq, int n_in, int n_out, float* y,
                    const float* gate) -> hipError_t {
        const uint8_t* wb = static_cast<const uint8_t*>(wt);
        if (smoe::native_type(type)) return smoe::launch_mmvq_native(type, wb, xq, n_in, n_out, T, y, n_out, gate, st);
        hipError_t e = type == SMOE_IQ2_S ? smoe::launch_iq2_mmvq(wb, xq, n_in, n_out, T, y, st)
                                          : smoe::launch_q2_mmvq(wb, xq, n_in, n_out, T, y, st);
        if (e == hipSuccess && gate) e = smoe::launch_sigmoid_rows(y, T, n_out, gate, st);
        return e;
    };
    SMOE_TRY(gemv(sh_gate_t(g), w->gate_sh, nxq, H, Fn, ngu, nullptr), "shared gate");
    SMOE_TRY(gemv(sh_up_t(g), w->up_sh, nxq, H, Fn, ngu + (size_t)T * Fn, nullptr), "shared up");
    SMOE_TRY(smoe::launch_swiglu_q8(ngu, ngu + (size_t)T * Fn, (int64_t)T * Fn, nhq, st), "shared swiglu");
    SMOE_TRY(gemv(sh_down_t(g), w->down_sh, nhq, Fn, H, out, sg), "shared down");
    return SMOE_OK;
}

// The forward call; with x_prev, x = RMSNorm(x_prev + r_prev) is formed first (fused into the router kernel on the
// GEMV path, a junction kernel before the call on the MFMA path) and written to x.
smoe_status forward_impl(const smoe_geom* g, const smoe_weights* w, float* x_io, int32_t n_tokens, float* y,
                         int32_t add_shared, void* workspace, size_t workspace_bytes, const smoe_trace* trace,
                         int32_t path, void* hip_stream, const float* x_prev, const float* r_prev, float eps) {
    const float* x = x_io;
    smoe_status s = check_forward(g, w, x, n_tokens, y, workspace, workspace_bytes, path, x_prev, r_prev);
    if (s != SMOE_OK || n_tokens == 0) return s == SMOE_OK ? ok() : s;
    const bool has_sh = g->sh_type >= 0;  // the router's shared gate row
    const bool nat = sh_native(*g);         // the shared expert as its own q8_1 GEMV chain, into Y's shared rows
    const bool shf = has_sh && !nat;        // the shared expert inside the expert kernels
    const bool iq2 = g->w_type == SMOE_IQ2_S;
    const bool mfma = !iq2 && (path == SMOE_PATH_MFMA || (path == SMOE_PATH_AUTO && n_tokens >= kMfmaTokens));
    const Layout L = layout(*g, n_tokens);

    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const int T = n_tokens, H = g->n_embd, E = g->n_expert, K = g->top_k, F = g->n_ff;
    const int Fs = shf ? g->n_ff_shared : 0;
    const int P = T * K;
    uint32_t* ximg = reinterpret_cast<uint32_t*>(ws + L.ximg);
    float* logits = (trace && trace->logits) ? trace->logits : reinterpret_cast<float*>(ws + L.logits);
    float* sg = (trace && trace->sgate) ? trace->sgate : reinterpret_cast<float*>(ws + L.sg);
    int32_t* ids = (trace && trace->ids) ? trace->ids : reinterpret_cast<int32_t*>(ws + L.ids);
    float* wts = (trace && trace->weights) ? trace->weights : reinterpret_cast<float*>(ws + L.wts);
    int32_t* counts = (trace && trace->counts) ? trace->counts : reinterpret_cast<int32_t*>(ws + L.counts);
    int32_t* offsets = (trace && trace->offsets) ? trace->offsets : reinterpret_cast<int32_t*>(ws + L.offsets);
    int32_t* perm = (trace && trace->perm) ? trace->perm : reinterpret_cast<int32_t*>(ws + L.perm);
    int32_t* slot = (trace && trace->slot) ? trace->slot : reinterpret_cast<int32_t*>(ws + L.slot);
    int32_t* elist = reinterpret_cast<int32_t*>(ws + L.elist);
    int32_t* nlist = reinterpret_cast<int32_t*>(ws + L.nlist);
    int4* items = reinterpret_cast<int4*>(ws + L.items);
    uint32_t* himg = reinterpret_cast<uint32_t*>(ws + L.himg);
    float* Y = reinterpret_cast<float*>(ws + L.Y);
    const hipStream_t st = stream_of(hip_stream);
    const int n_items = mfma ? max_items_mfma(*g, T) : max_items_gemv(*g, T);
    const int chunk = mfma ? smoe::mfma_chunk() : (1 << 30);
    // the prefill path's per-pair rows Y past kYStreamBytes: the down kernels store them and the combine reads them
    // (and writes y) with streaming accesses, which keep them out of the XCDs' L2 (measured at 4096 tokens of the
    // benchmark's layer, 369 MB of Y: 50 us less per layer; at 512 tokens, 46 MB, the combine reads Y back from the
    // Infinity Cache and the streaming loads cost it 1.5 us)
    const bool y_stream = mfma && (size_t)(P + T) * (size_t)H * sizeof(float) > kYStreamBytes;
    const int sh_chunk = mfma ? smoe::mfma_chunk() : smoe::gemv_shared_chunk();

    void* const* ev = trace ? trace->stage_events : nullptr;
    int ev_i = 0;
    auto mark = [&]() -> smoe_status {
        if (!ev) return SMOE_OK;
        const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(ev[ev_i++]), st);
        return launched(e, "stage event");
    };
#define SMOE_MARK()                          \
    do {                                     \
        const smoe_status _m = mark();       \
        if (_m != SMOE_OK) return _m;        \
    } while (0)
    SMOE_MARK();
    const bool fused_norm = x_prev && !mfma;
    // the expert stages of the trace: the decode path's unfused kernels, so that every stage lands in memory
    const bool stages = trace && (trace->xq || trace->hq || trace->parts || trace->shared || trace->egate ||
                                  trace->eup || trace->sgu || trace->shq);
    // the prefill path's per-work-group flags of its fp16 operand limits (folded by a trace or smoe_forward_status)
    int32_t* xflags = mfma ? reinterpret_cast<int32_t*>(ws + L.oflags) : nullptr;
    int32_t* hflags = xflags ? xflags + L.n_xflags : nullptr;
    // batches of at most kFusedRouteTokens tokens on the Q2_0 GEMV path: the gate/up kernel routes the batch itself,
    // and (when the batch's h images fit in LDS) the down kernel applies the combine; where the shapes allow, both
    // run as one launch whose exchange words the router kernel clears (its down work-groups' wait flags: wflags)
    const bool small = !mfma && !iq2 && !stages && T <= kFusedRouteTokens;
    const bool small_down = small && smoe::down_combine_ok(T, K, L.h_blocks);
    const bool fused = small_down && smoe::moe_small_ok(T, K, H, F, Fs, shf ? 1 : 0, L.h_blocks);
    int32_t* wflags = fused ? reinterpret_cast<int32_t*>(ws + L.status) : nullptr;
    uint8_t* xchg = ws + L.xchg;
    const size_t xchg_bytes = fused ? smoe::moe_small_xchg_bytes(T, K, n_items, L.h_blocks) : 0;
    uint16_t* xbf = mfma ? reinterpret_cast<uint16_t*>(ws + L.xbf) : nullptr;
    // the prefill path's junction and the records of its output in one launch, before the call on that output
    if (x_prev && mfma)
        SMOE_TRY(smoe::launch_junction_records(x_prev, r_prev, T, H, eps, x_io, ximg, xbf, st, xflags),
                 "junction records");
    if (mfma && !x_prev)
        SMOE_TRY(smoe::launch_act_records(x, (int64_t)T * (H / 64), ximg, xbf, st, xflags), "activation records");
    // the f32 router (router_dtype 1) reads f32 x on the row-per-wave path, also for many tokens
    const bool f32r = g->router_dtype == SMOE_ROUTER_F32;
    SMOE_TRY(smoe::launch_router(fused_norm ? x_prev : x, f32r ? nullptr : xbf, w->router,
                                 has_sh ? w->gate_inp_sh : nullptr, w->logit_bias, H, E, E + (has_sh ? 1 : 0), T, logits,
                                 E, sg, mfma ? nullptr : ximg, (mfma && !f32r) ? 1 : 0, iq2 ? 1 : 0, st,
                                 fused_norm ? r_prev : nullptr, eps, fused_norm ? x_io : nullptr,
                                 fused ? reinterpret_cast<uint4*>(xchg) : nullptr, (int)(xchg_bytes / 16), f32r ? 1 : 0),
             "router");
    SMOE_MARK();
    if (small) {
        // no route kernel: the stage boundary marks stay, the route stage is empty
    } else if (T <= kFusedRouteTokens) {
        SMOE_TRY(smoe::launch_topk_dispatch(logits, T, E, K, ids, wts, counts, offsets, perm, slot, elist, nlist, items,
                                            n_items, shf ? 1 : 0, chunk, sh_chunk, st),
                 "route");
    } else {
        SMOE_TRY(smoe::launch_topk(logits, E, T, E, K, ids, wts, st), "topk");
        if (P > kDispatchMultiPairs)
            SMOE_TRY(smoe::launch_dispatch_multi(ids, P, E, counts, offsets, perm, slot, elist, nlist, items, n_items,
                                                 T, K, shf ? 1 : 0, chunk, sh_chunk,
                                                 reinterpret_cast<int32_t*>(ws + L.dwork), st),
                     "dispatch");
        else
            SMOE_TRY(smoe::launch_dispatch(ids, P, E, counts, offsets, perm, slot, elist, nlist, items, n_items, T, K,
                                           shf ? 1 : 0, chunk, sh_chunk, st),
                     "dispatch");
    }
    SMOE_MARK();
    const uint8_t* ge = static_cast<const uint8_t*>(w->gate_exps);
    const uint8_t* ue = static_cast<const uint8_t*>(w->up_exps);
    const uint8_t* de = static_cast<const uint8_t*>(w->down_exps);
    const uint8_t* gs = static_cast<const uint8_t*>(w->gate_sh);
    const uint8_t* us = static_cast<const uint8_t*>(w->up_sh);
    const uint8_t* ds = static_cast<const uint8_t*>(w->down_sh);
    // the expert stages of a traced decode-path call, written by the gate/up kernels
    smoe::StageOut so{};
    if (trace && !mfma) {
        so.hq = trace->hq;
        so.egate = trace->egate;
        so.eup = trace->eup;
        if (!nat) {
            so.sgu = trace->sgu;
            so.shq = trace->shq;
        }
        so.P = P;
        so.T = T;
    }
    if (mfma) {
        SMOE_TRY(smoe::launch_mm_gu(ge, ue, gs, us, ximg, (int64_t)T * (H / 64), items, perm, K, H, F, Fs,
                                    shf ? 1 : 0, n_items, himg, L.h_rec, st, hflags, E),
                 "gate/up");
        SMOE_MARK();
        SMOE_TRY(smoe::launch_mm_down(de, ds, himg, (int64_t)(P + T) * L.h_rec, L.h_rec, sg, items, H, F, Fs, n_items,
                                      Y, y_stream ? 1 : 0, st),
                 "down");
    } else if (iq2) {
        SMOE_TRY(smoe::launch_iq2_gu(ge, ue, gs, us, ximg, items, perm, K, H, F, Fs, shf ? 1 : 0, n_items, himg,
                                     L.h_blocks, st, &so),
                 "gate/up");
        SMOE_MARK();
        SMOE_TRY(smoe::launch_iq2_down(de, ds, himg, L.h_blocks, sg, items, H, F, Fs, n_items, Y, st), "down");
    } else if (fused) {
        SMOE_TRY(smoe::launch_q2_moe_small(ge, ue, gs, us, de, ds, ximg, logits, sg, T, E, K, H, F, Fs, shf ? 1 : 0,
                                           ids, wts, counts, offsets, perm, slot, elist, nlist, items, n_items, L.h_blocks,
                                           xchg, (shf && add_shared) ? 1 : 0, y, wflags, st),
                 "route + gate/up + down + combine");
        SMOE_MARK();  // gate/up, down and combine are one launch: the later stage boundaries are empty
    } else {
        if (small)
            SMOE_TRY(smoe::launch_q2_gu_route(ge, ue, gs, us, ximg, logits, T, E, K, H, F, Fs, shf ? 1 : 0, ids, wts,
                                              counts, offsets, perm, slot, elist, nlist, items, n_items, himg,
                                              L.h_blocks, st),
                     "route + gate/up");
        else
            SMOE_TRY(smoe::launch_q2_gu(ge, ue, gs, us, ximg, items, perm, K, H, F, Fs, shf ? 1 : 0, n_items, himg,
                                        L.h_blocks, st, &so),
                     "gate/up");
        SMOE_MARK();
        if (small_down)
            SMOE_TRY(smoe::launch_q2_down_combine(de, ds, himg, L.h_blocks, sg, items, n_items, H, F, Fs, slot, wts, T, K,
                                                  (shf && add_shared) ? 1 : 0, y, st),
                     "down + combine");
        else
            SMOE_TRY(smoe::launch_q2_down(de, ds, himg, L.h_blocks, sg, items, H, F, Fs, n_items, Y, st), "down");
    }
    SMOE_MARK();
    if (nat) SMOE_TRY_S(native_shared(*g, w, x_io, T, ws, L, Y + (size_t)P * H, sg, st));
    if (!small_down)
        SMOE_TRY(smoe::launch_combine(Y, slot, wts, K, H, P, T, (has_sh && add_shared) ? 1 : 0, y, st,
                                      y_stream ? 1 : 0),
                 "combine");
    else if (nat && add_shared)  // the fused combine left the shared rows out: the same last addition, after it
        SMOE_TRY(smoe::launch_add_rows(y, Y + (size_t)P * H, T, H, st), "shared add");
    SMOE_MARK();
#undef SMOE_MARK
    FlagWords flags;
    flag_words(*g, L, T, mfma, fused, x_prev != nullptr, workspace, flags);
    remember_flags(flags);
    // the trace's expert stages and overflow mask, after the last stage event
    if (trace) {
        if (trace->xq && !mfma)
            SMOE_TRY(smoe::launch_prep(x_io, (int64_t)T * H, trace->xq, nullptr, st), "trace xq");
        if (trace->parts) SMOE_TRY(smoe::launch_copy_f32(Y, (int64_t)P * H, trace->parts, st), "trace parts");
        if (trace->shared && has_sh)
            SMOE_TRY(smoe::launch_copy_f32(Y + (size_t)P * H, (int64_t)T * H, trace->shared, st), "trace shared");
        if (nat && !mfma) {  // the native shared chain's own stages: its gate and up dots, the q8_1 of its h
            const int Fn = g->n_ff_shared;
            if (trace->sgu)
                SMOE_TRY(smoe::launch_copy_f32(reinterpret_cast<const float*>(ws + L.ngu), 2 * (int64_t)T * Fn,
                                               trace->sgu, st),
                         "trace shared gate/up");
            if (trace->shq)  // 36-byte blocks: whole dwords
                SMOE_TRY(smoe::launch_copy_f32(reinterpret_cast<const float*>(ws + L.nhq), (int64_t)T * (Fn / 32) * 9,
                                               reinterpret_cast<float*>(trace->shq), st),
                         "trace shared h");
        }
        if (trace->overflow) SMOE_TRY_S(fold_status(flags, trace->overflow, st));
    }
    return ok();
}
}  // namespace

smoe_status smoe_forward_path(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                              int32_t add_shared, void* workspace, size_t workspace_bytes, const smoe_trace* trace,
                              int32_t path, void* hip_stream) {
    return forward_impl(g, w, const_cast<float*>(x), n_tokens, y, add_shared, workspace, workspace_bytes, trace, path,
                        hip_stream, nullptr, nullptr, 0.0f);
}

smoe_status smoe_forward_residual(const smoe_geom* g, const smoe_weights* w, const float* x_prev, const float* r_prev,
                                  float eps, float* x, int32_t n_tokens, float* y, int32_t add_shared, void* workspace,
                                  size_t workspace_bytes, const smoe_trace* trace, void* hip_stream) {
    if (n_tokens > 0 && (!x_prev || !x)) return fail(SMOE_ENULL, "x_prev or x is NULL");
    if (!(eps >= 0.0f) || eps == INFINITY) return fail(SMOE_EINVAL, "forward_residual: eps must be finite and non-negative");
    return forward_impl(g, w, x, n_tokens, y, add_shared, workspace, workspace_bytes, trace, SMOE_PATH_AUTO, hip_stream,
                        x_prev, r_prev, eps);
}

smoe_status smoe_forward(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                         int32_t add_shared, void* workspace, size_t workspace_bytes, const smoe_trace* trace,
                         void* hip_stream) {
    return smoe_forward_path(g, w, x, n_tokens, y, add_shared, workspace, workspace_bytes, trace, SMOE_PATH_AUTO,
                             hip_stream);
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------ layer ends
namespace {
// gr_read's scratch: proj [T][hc_lr] and rs [T][hc]
struct HcLayout {
    size_t proj, rs, total;
};
HcLayout hc_layout(const smoe_hc& h, int64_t T) {
    HcLayout L{};
    size_t o = 0;
    L.proj = o;
    o = up(o + (size_t)T * h.hc_lr * 4);
    L.rs = o;
    o = up(o + (size_t)T * h.hc * 4);
    L.total = o;
    return L;
}

smoe_status check_hc(const smoe_hc* h, int32_t n_embd) {
    if (!h) return fail(SMOE_ENULL, "hyper-connection weights are NULL");
    if (!smoe::hc_shape_ok(n_embd, h->hc, h->hc_lr))
        return fail(SMOE_EINVAL, "hyper connection: n_embd % 8 == 0 and <= 4096, hc in 1..8, hc * n_embd <= 16384, "
                                 "hc_lr % 8 == 0 and <= 2048");
    if (!(h->eps >= 0.0f) || h->eps == INFINITY) return fail(SMOE_EINVAL, "hyper connection: eps must be finite and >= 0");
    if (!h->norm || !h->down || !h->up || !h->inject) return fail(SMOE_ENULL, "a hyper-connection tensor is NULL");
    if (!aligned(h->norm, 4) || !aligned(h->down, 16) || !aligned(h->up, 16) || !aligned(h->inject, 16))
        return fail(SMOE_EALIGN, "hyper-connection tensors: norm 4-byte, down/up/inject 16-byte aligned");
    return SMOE_OK;
}
}  // namespace

extern "C" {

size_t smoe_hc_read_workspace_bytes(const smoe_hc* hc, int32_t n_embd, int32_t max_tokens) {
    if (check_hc(hc, n_embd) != SMOE_OK || max_tokens < 0) return 0;
    return hc_layout(*hc, max_tokens).total;
}

smoe_status smoe_hc_read(const smoe_hc* hc, int32_t n_embd, const float* R, int32_t n_tokens, float* mixed,
                         float* inject, void* workspace, size_t workspace_bytes, void* hip_stream) {
    smoe_status s = check_hc(hc, n_embd);
    if (s != SMOE_OK) return s;
    if (n_tokens < 0) return fail(SMOE_EINVAL, "hc_read: negative token count");
    if (n_tokens == 0) return ok();
    if (!R || !mixed || !workspace) return fail(SMOE_ENULL, "hc_read: NULL buffer");
    if (!aligned(R, 4) || !aligned(mixed, 4) || (inject && !aligned(inject, 4)) || !aligned(workspace, kAlign))
        return fail(SMOE_EALIGN, "hc_read: R, mixed, inject 4-byte, workspace 256-byte aligned");
    const HcLayout L = hc_layout(*hc, n_tokens);
    if (workspace_bytes < L.total)
        return fail(SMOE_ESIZE, "hc_read workspace is " + std::to_string(workspace_bytes) + " bytes, needs " +
                                    std::to_string(L.total));
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    SMOE_TRY(smoe::launch_hc_read(const_cast<float*>(R), hc->norm, hc->down, hc->up, hc->inject, n_tokens, n_embd,
                                  hc->hc, hc->hc_lr, hc->eps, reinterpret_cast<float*>(ws + L.proj),
                                  reinterpret_cast<float*>(ws + L.rs), mixed, inject, nullptr, nullptr, nullptr,
                                  stream_of(hip_stream)),
             "hc_read");
    return ok();
}

smoe_status smoe_hc_write(const smoe_hc* hc, int32_t n_embd, const float* R, const float* y, const float* inject,
                          int32_t n_tokens, float* R_out, void* hip_stream) {
    if (!hc) return fail(SMOE_ENULL, "hyper-connection geometry is NULL");
    if (n_embd < 0 || n_tokens < 0 || hc->hc < 0) return fail(SMOE_EINVAL, "hc_write: negative size");
    if (n_embd == 0 || n_tokens == 0 || hc->hc == 0) return ok();
    if ((int64_t)n_tokens * hc->hc * n_embd > ((int64_t)1 << 38)) return fail(SMOE_EINVAL, "hc_write: too many values");
    if (!R || !y || !inject || !R_out) return fail(SMOE_ENULL, "hc_write: NULL buffer");
    if (!aligned(R, 4) || !aligned(y, 4) || !aligned(inject, 4) || !aligned(R_out, 4))
        return fail(SMOE_EALIGN, "hc_write: R, y, inject and R_out must be 4-byte aligned");
    SMOE_TRY(smoe::launch_hc_write(R, y, inject, n_tokens, n_embd, hc->hc, R_out, stream_of(hip_stream)), "hc_write");
    return ok();
}

}  // extern "C"

namespace {
// smoe_ffn_run's workspace: the block's own, then mixed [T][n], inject [T][hc], y [T][n], gr_read's scratch
struct FfnLayout {
    size_t moe, mixed, inject, y, hc, total;
};
FfnLayout ffn_layout(const smoe_geom& g, const smoe_hc& h, int64_t T) {
    FfnLayout L{};
    size_t o = 0;
    L.moe = o;
    o = up(o + layout(g, T).total);
    L.mixed = o;
    o = up(o + (size_t)T * g.n_embd * 4);
    L.inject = o;
    o = up(o + (size_t)T * h.hc * 4);
    L.y = o;
    o = up(o + (size_t)T * g.n_embd * 4);
    L.hc = o;
    o = up(o + hc_layout(h, T).total);
    L.total = o;
    return L;
}
}  // namespace

extern "C" {

size_t smoe_ffn_workspace_bytes(const smoe_geom* g, const smoe_hc* hc, int32_t max_tokens) {
    if (check_geom(g) != SMOE_OK || max_tokens < 0) return 0;
    if (check_hc(hc, g->n_embd) != SMOE_OK) return 0;
    return ffn_layout(*g, *hc, max_tokens).total;
}

smoe_status smoe_ffn_run(const smoe_geom* g, const smoe_weights* w, const smoe_hc* hc, const float* residual,
                         int32_t n_tokens, float* out, int32_t add_shared, void* workspace, size_t workspace_bytes,
                         const smoe_trace* trace, void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    s = check_hc(hc, g->n_embd);
    if (s != SMOE_OK) return s;
    if (n_tokens < 0) return fail(SMOE_EINVAL, "ffn_run: negative token count");
    if (n_tokens == 0) return ok();
    if (!residual || !out || !workspace) return fail(SMOE_ENULL, "ffn_run: NULL buffer");
    if (!aligned(residual, 4) || !aligned(out, 4) || !aligned(workspace, kAlign))
        return fail(SMOE_EALIGN, "ffn_run: residual and out 4-byte, workspace 256-byte aligned");
    const FfnLayout L = ffn_layout(*g, *hc, n_tokens);
    if (workspace_bytes < L.total)
        return fail(SMOE_ESIZE, "ffn_run workspace is " + std::to_string(workspace_bytes) + " bytes, needs " +
                                    std::to_string(L.total));
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    float* mixed = reinterpret_cast<float*>(ws + L.mixed);
    float* inj = reinterpret_cast<float*>(ws + L.inject);
    float* yb = reinterpret_cast<float*>(ws + L.y);
    // every check of the block itself before the first launch
    const size_t moe_bytes = layout(*g, n_tokens).total;
    s = check_forward(g, w, mixed, n_tokens, yb, ws + L.moe, moe_bytes, SMOE_PATH_AUTO, nullptr, nullptr);
    if (s != SMOE_OK) return s;
    const HcLayout H = hc_layout(*hc, n_tokens);
    SMOE_TRY(smoe::launch_hc_read(const_cast<float*>(residual), hc->norm, hc->down, hc->up, hc->inject, n_tokens,
                                  g->n_embd, hc->hc, hc->hc_lr, hc->eps,
                                  reinterpret_cast<float*>(ws + L.hc + H.proj), reinterpret_cast<float*>(ws + L.hc + H.rs),
                                  mixed, inj, nullptr, nullptr, nullptr, stream_of(hip_stream)),
             "hc_read");
    s = forward_impl(g, w, mixed, n_tokens, yb, add_shared, ws + L.moe, moe_bytes, trace, SMOE_PATH_AUTO, hip_stream,
                     nullptr, nullptr, 0.0f);
    if (s != SMOE_OK) return s;
    SMOE_TRY(smoe::launch_hc_write(residual, yb, inj, n_tokens, g->n_embd, hc->hc, out, stream_of(hip_stream)),
             "hc_write");
    return ok();
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------ no allocation
// smoe_forward_static's scratch: one copy of this array lives on every GPU the library runs on, from the code
// object's load until the process ends.  Host code never passes `scratch` itself to a kernel (in host code the
// name is a host-side stand-in, not a device address): it uses the device address hipGetSymbolAddress returns,
// looked up once per device on that device's first call.
static __device__ __align__(256) uint8_t scratch[SMOE_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The device address of the current device's copy of `scratch`, or NULL with the reason in g_last.
void* device_scratch() {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        fail(SMOE_EDEVICE, std::string("hipGetDevice: ") + hipGetErrorString(e));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        fail(SMOE_EDEVICE, "device ordinal " + std::to_string(dev) + " is beyond the library's 64");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || !p) {
            fail(SMOE_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(r));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

smoe_status smoe_forward_static(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                                int32_t add_shared, const smoe_trace* trace, void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (n_tokens < 0) return fail(SMOE_EINVAL, "n_tokens is negative");
    if ((int64_t)n_tokens * g->top_k > (1 << 24)) return fail(SMOE_EINVAL, "n_tokens * top_k exceeds 2^24");
    if (n_tokens == 0) return forward_impl(g, w, const_cast<float*>(x), 0, y, add_shared, nullptr, 0, trace,
                                           SMOE_PATH_AUTO, hip_stream, nullptr, nullptr, 0.0f);
    const size_t need = layout(*g, n_tokens).total;
    if (need > SMOE_STATIC_SCRATCH_BYTES)
        return fail(SMOE_ESIZE, std::to_string(n_tokens) + " tokens need " + std::to_string(need) +
                                    " bytes of scratch; the static scratch holds " +
                                    std::to_string((size_t)SMOE_STATIC_SCRATCH_BYTES) +
                                    " (call smoe_forward with a workspace for this batch)");
    void* ws = device_scratch();
    if (!ws) return SMOE_EDEVICE;
    return forward_impl(g, w, const_cast<float*>(x), n_tokens, y, add_shared, ws, SMOE_STATIC_SCRATCH_BYTES, trace,
                        SMOE_PATH_AUTO, hip_stream, nullptr, nullptr, 0.0f);
}

smoe_status smoe_forward_status(const void* workspace, int32_t* status, void* hip_stream) {
    if (!status) return fail(SMOE_ENULL, "forward_status: status is NULL");
    if (!aligned(status, 4)) return fail(SMOE_EALIGN, "forward_status: status must be 4-byte aligned");
    const void* ws = workspace ? workspace : device_scratch();
    if (!ws) return SMOE_EDEVICE;
    FlagWords f;
    if (!recall_flags(ws, f))
        return fail(SMOE_EINVAL, "forward_status: no call on this workspace is known (the library keeps the last " +
                                     std::to_string(kFlagTable) + " workspaces)");
    SMOE_TRY_S(fold_status(f, status, stream_of(hip_stream)));
    return ok();
}

int32_t smoe_set_wait_limit(int32_t polls) {
    const int32_t prev = smoe::wait_limit();
    smoe::set_wait_limit(polls < 0 ? -1 : polls == 0 ? smoe::default_wait_limit() : polls);
    return prev;
}

// ------------------------------------------------------------------------------------------------ stages

smoe_status smoe_router_topk(const float* logits, int32_t n_tokens, int32_t n_expert, int32_t k, int32_t* ids,
                             float* weights, void* hip_stream) {
    if (n_tokens < 0 || n_expert < 0 || k < 0) return fail(SMOE_EINVAL, "router_topk: negative size");
    if (n_tokens == 0 || n_expert == 0 || k == 0) return ok();
    if (k > kMaxK) return fail(SMOE_EINVAL, "router_topk: k exceeds 64");
    if (n_expert > kMaxExpert) return fail(SMOE_EINVAL, "router_topk: n_expert exceeds 1024");
    if (k > n_expert) return fail(SMOE_EINVAL, "router_topk: k exceeds n_expert");
    if (!logits || !ids || !weights) return fail(SMOE_ENULL, "router_topk: NULL buffer");
    SMOE_TRY(smoe::launch_topk(logits, n_expert, n_tokens, n_expert, k, ids, weights, stream_of(hip_stream)), "topk");
    return ok();
}

smoe_status smoe_router_margin(const float* logits, int32_t n_tokens, int32_t n_expert, int32_t k, float* stats,
                               int32_t* ids, void* hip_stream) {
    if (n_tokens < 0 || n_expert < 0 || k < 0) return fail(SMOE_EINVAL, "router_margin: negative size");
    if (n_tokens == 0) return ok();
    if (k < 1 || k >= n_expert) return fail(SMOE_EINVAL, "router_margin: needs 1 <= k < n_expert");
    if (n_expert > kMaxExpert) return fail(SMOE_EINVAL, "router_margin: n_expert exceeds 1024");
    if (!logits || !stats || !ids) return fail(SMOE_ENULL, "router_margin: NULL buffer");
    if (!aligned(logits, 4) || !aligned(stats, 4) || !aligned(ids, 4))
        return fail(SMOE_EALIGN, "router_margin: buffers must be 4-byte aligned");
    SMOE_TRY(smoe::launch_router_margin(logits, n_tokens, n_expert, k, stats, ids, stream_of(hip_stream)),
             "router_margin");
    return ok();
}

smoe_status smoe_f32_to_bf16(const float* x, int64_t n, uint16_t* y, void* hip_stream) {
    if (n < 0) return fail(SMOE_EINVAL, "f32_to_bf16: negative length");
    if (n == 0) return ok();
    if (!x || !y) return fail(SMOE_ENULL, "f32_to_bf16: NULL buffer");
    if (n % 32) {
        return fail(SMOE_EINVAL, "f32_to_bf16: length must be a multiple of 32");
    }
    SMOE_TRY(smoe::launch_prep(x, n, nullptr, y, stream_of(hip_stream)), "f32_to_bf16");
    return ok();
}

smoe_status smoe_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int32_t n_in, int32_t n_out, int32_t n_tok,
                           void* hip_stream) {
    if (n_in < 0 || n_out < 0 || n_tok < 0) return fail(SMOE_EINVAL, "bf16_gemv: negative size");
    if (n_in == 0 || n_out == 0 || n_tok == 0) return ok();
    if (!x || !w || !y) return fail(SMOE_ENULL, "bf16_gemv: NULL buffer");
    if (n_in % 8 || n_in > 8192) return fail(SMOE_EINVAL, "bf16_gemv: n_in must be a multiple of 8, at most 8192");
    if ((int64_t)n_tok * n_in % 2) return fail(SMOE_EINVAL, "bf16_gemv: odd element count");
    if (!aligned(x, 16) || !aligned(w, 16)) return fail(SMOE_EALIGN, "bf16_gemv: x and w must be 16-byte aligned");
    SMOE_TRY(smoe::launch_router(nullptr, x, w, nullptr, nullptr, n_in, n_out, n_out, n_tok, y, n_out, nullptr, nullptr,
                                 0, 0, stream_of(hip_stream)),
             "bf16_gemv");
    return ok();
}

smoe_status smoe_quantize_q8_1(const float* x, int64_t n, uint8_t* y, void* hip_stream) {
    if (n < 0) return fail(SMOE_EINVAL, "quantize_q8_1: negative length");
    if (n == 0) return ok();
    if (n % 32) return fail(SMOE_EINVAL, "quantize_q8_1: length must be a multiple of 32");
    if (!x || !y) return fail(SMOE_ENULL, "quantize_q8_1: NULL buffer");
    if (!aligned(y, 4)) return fail(SMOE_EALIGN, "quantize_q8_1: y must be 4-byte aligned");
    SMOE_TRY(smoe::launch_prep(x, n, y, nullptr, stream_of(hip_stream)), "quantize_q8_1");
    return ok();
}

smoe_status smoe_mmvq(int32_t type, const void* w, int64_t byte_off, const uint8_t* x_q8, int32_t n_in, int32_t n_out,
                      int32_t n_col, float* y, void* hip_stream) {
    if (n_in < 0 || n_out < 0 || n_col < 0 || byte_off < 0) return fail(SMOE_EINVAL, "mmvq: negative size");
    if (n_in == 0 || n_out == 0 || n_col == 0) return ok();
    if (!gemv_type(type))
        return fail(SMOE_ETYPE, "mmvq: type " + std::to_string(type) + " has no GEMV here");
    if (smoe::native_type(type) && smoe::native_row_bytes(type, n_in) <= 0)
        return fail(SMOE_EINVAL, "mmvq: n_in must be a multiple of " + std::to_string(smoe::native_block_values(type)));
    if (type == SMOE_Q2_0 && (n_in > kMaxFF || !smoe::gemv_shape_ok(n_in)))
        return fail(SMOE_EINVAL, "mmvq: n_in must be 128 times a power of two times at most 8, at most 4096");
    if (type == SMOE_IQ2_S && !smoe::iq2_shape_ok(n_in))
        return fail(SMOE_EINVAL, "mmvq: IQ2_S n_in must be 512, 1024 or 2048");
    if (!w || !x_q8 || !y) return fail(SMOE_ENULL, "mmvq: NULL buffer");
    const uint8_t* base = static_cast<const uint8_t*>(w) + byte_off;
    if (!aligned(base, 4) || !aligned(x_q8, 4)) return fail(SMOE_EALIGN, "mmvq: w + byte_off and x must be 4-byte aligned");
    if (smoe::native_type(type))
        SMOE_TRY(smoe::launch_mmvq_native(type, base, x_q8, n_in, n_out, n_col, y, n_out, nullptr, stream_of(hip_stream)),
                 "mmvq");
    else if (type == SMOE_IQ2_S) SMOE_TRY(smoe::launch_iq2_mmvq(base, x_q8, n_in, n_out, n_col, y, stream_of(hip_stream)), "mmvq");
    else SMOE_TRY(smoe::launch_q2_mmvq(base, x_q8, n_in, n_out, n_col, y, stream_of(hip_stream)), "mmvq");
    return ok();
}

smoe_status smoe_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y, void* hip_stream) {
    if (n < 0) return fail(SMOE_EINVAL, "swiglu_q8: negative length");
    if (n == 0) return ok();
    if (n % 32) return fail(SMOE_EINVAL, "swiglu_q8: length must be a multiple of 32");
    if (!gate || !up || !y) return fail(SMOE_ENULL, "swiglu_q8: NULL buffer");
    if (!aligned(y, 4)) return fail(SMOE_EALIGN, "swiglu_q8: y must be 4-byte aligned");
    SMOE_TRY(smoe::launch_swiglu_q8(gate, up, n, y, stream_of(hip_stream)), "swiglu_q8");
    return ok();
}

namespace {
int64_t type_row_bytes(int32_t type, int64_t n) {
    return type == SMOE_Q2_0 ? n / 64 * 18 : type == SMOE_IQ2_S ? n / 256 * 82 : -1;
}
// The reference's iq_expert_bytes checks (metal/src/iq.mm:171-180); "" when the expert is well formed.
std::string expert_refusal(int32_t gu_type, int32_t d_type, int64_t n_embd, int64_t n_ff, smoe_status& code) {
    code = SMOE_ETYPE;
    if ((gu_type != SMOE_Q2_0 && gu_type != SMOE_IQ2_S) || (d_type != SMOE_Q2_0 && d_type != SMOE_IQ2_S))
        return "expert: type is not Q2_0 or IQ2_S";
    if (gu_type != SMOE_IQ2_S) return "expert: gate type is a down quant (64-value blocks)";
    code = SMOE_EINVAL;
    if (n_embd <= 0 || n_ff <= 0) return "expert: empty expert";
    if (n_ff % 32) return "expert: n_ff must be a multiple of 32";
    if (!smoe::iq2_shape_ok((int)n_embd) || n_embd > kMaxEmbd) return "expert: IQ2_S n_embd must be 512, 1024 or 2048";
    if (d_type == SMOE_Q2_0 && (n_ff > kMaxFF || !smoe::gemv_shape_ok((int)n_ff)))
        return "expert: Q2_0 n_ff must be 128 times a power of two times at most 8";
    if (d_type == SMOE_IQ2_S && !smoe::iq2_shape_ok((int)n_ff)) return "expert: IQ2_S n_ff must be 512, 1024 or 2048";
    return "";
}
}  // namespace

size_t smoe_expert_bytes(int32_t gu_type, int32_t d_type, int64_t n_embd, int64_t n_ff) {
    smoe_status code;
    const std::string why = expert_refusal(gu_type, d_type, n_embd, n_ff, code);
    if (!why.empty()) {
        fail(code, why);
        return 0;
    }
    ok();
    return (size_t)(2 * n_ff * type_row_bytes(gu_type, n_embd) + n_embd * type_row_bytes(d_type, n_ff));
}

size_t smoe_expert_scratch_bytes(int64_t n_embd, int64_t n_ff, int64_t n_tok) {
    (void)n_embd;
    if (n_tok < 0 || n_ff < 0) return 0;
    const size_t f32 = up((size_t)(n_tok * n_ff * 4));
    return 2 * f32 + up((size_t)(n_tok * (n_ff / 32) * 36));
}

smoe_status smoe_expert(const void* blob, size_t blob_bytes, const uint8_t* x_q8, int32_t gu_type, int32_t d_type,
                        int64_t n_embd, int64_t n_ff, int64_t n_tok, float* y, void* scratch, size_t scratch_bytes,
                        void* hip_stream) {
    if (n_tok == 0) return ok();
    if (n_tok < 0) return fail(SMOE_EINVAL, "expert: negative token count");
    if (n_tok > (1 << 20)) return fail(SMOE_EINVAL, "expert: more than 2^20 tokens");
    smoe_status code;
    const std::string why = expert_refusal(gu_type, d_type, n_embd, n_ff, code);
    if (!why.empty()) return fail(code, why);
    const size_t need = (size_t)(2 * n_ff * type_row_bytes(gu_type, n_embd) + n_embd * type_row_bytes(d_type, n_ff));
    if (blob_bytes < need)
        return fail(SMOE_ESIZE, "expert blob is " + std::to_string(blob_bytes) + " bytes, needs " + std::to_string(need));
    const size_t sneed = smoe_expert_scratch_bytes(n_embd, n_ff, n_tok);
    if (scratch_bytes < sneed)
        return fail(SMOE_ESIZE, "expert scratch is " + std::to_string(scratch_bytes) + " bytes, needs " + std::to_string(sneed));
    if (!blob || !x_q8 || !y || !scratch) return fail(SMOE_ENULL, "expert: NULL buffer");
    if (!aligned(blob, 4) || !aligned(x_q8, 4) || !aligned(y, 4)) return fail(SMOE_EALIGN, "expert: buffers must be 4-byte aligned");
    if (!aligned(scratch, kAlign)) return fail(SMOE_EALIGN, "expert: scratch must be 256-byte aligned");
    uint8_t* sc = static_cast<uint8_t*>(scratch);
    const size_t f32 = up((size_t)(n_tok * n_ff * 4));
    float* gate = reinterpret_cast<float*>(sc);
    float* upv = reinterpret_cast<float*>(sc + f32);
    uint8_t* hq = sc + 2 * f32;
    const int64_t up_off = n_ff * type_row_bytes(gu_type, n_embd), down_off = 2 * up_off;
    const uint8_t* b = static_cast<const uint8_t*>(blob);
    const hipStream_t st = stream_of(hip_stream);
    if (gu_type == SMOE_IQ2_S) {
        SMOE_TRY(smoe::launch_iq2_mmvq(b, x_q8, (int)n_embd, (int)n_ff, (int)n_tok, gate, st), "expert gate");
        SMOE_TRY(smoe::launch_iq2_mmvq(b + up_off, x_q8, (int)n_embd, (int)n_ff, (int)n_tok, upv, st), "expert up");
    }
    SMOE_TRY(smoe::launch_swiglu_q8(gate, upv, n_tok * n_ff, hq, st), "expert swiglu");
    if (d_type == SMOE_IQ2_S) SMOE_TRY(smoe::launch_iq2_mmvq(b + down_off, hq, (int)n_ff, (int)n_embd, (int)n_tok, y, st), "expert down");
    else SMOE_TRY(smoe::launch_q2_mmvq(b + down_off, hq, (int)n_ff, (int)n_embd, (int)n_tok, y, st), "expert down");
    return ok();
}

smoe_status smoe_residual_rmsnorm(const float* x, const float* r, int32_t n_rows, int32_t n, float eps, float* out,
                                  void* hip_stream) {
    if (n_rows < 0 || n < 0) return fail(SMOE_EINVAL, "residual_rmsnorm: negative size");
    if (n_rows == 0 || n == 0) return ok();
    if (n > 4096) return fail(SMOE_EINVAL, "residual_rmsnorm: rows longer than 4096");
    if (!(eps >= 0.0f) || eps == INFINITY) return fail(SMOE_EINVAL, "residual_rmsnorm: eps must be finite and non-negative");
    if (!x || !out) return fail(SMOE_ENULL, "residual_rmsnorm: NULL buffer");
    SMOE_TRY(smoe::launch_residual_rmsnorm(x, r, n_rows, n, eps, out, stream_of(hip_stream)), "residual_rmsnorm");
    return ok();
}

smoe_status smoe_combine(const float* parts, const float* weights, const float* shared, float* y, int32_t n_embd,
                         int32_t k, void* hip_stream) {
    if (n_embd < 0 || k < 0) return fail(SMOE_EINVAL, "combine: negative size");
    if (n_embd == 0 || k == 0) return ok();
    if (k > kMaxK) return fail(SMOE_EINVAL, "combine: k exceeds 64");
    if (!parts || !weights || !y) return fail(SMOE_ENULL, "combine: NULL buffer");
    SMOE_TRY(smoe::launch_combine_parts(parts, weights, shared, k, n_embd, y, stream_of(hip_stream)), "combine");
    return ok();
}

smoe_status smoe_dispatch(const int32_t* ids, int32_t n_tokens, int32_t k, int32_t n_expert, int32_t* counts,
                          int32_t* offsets, int32_t* perm, int32_t* slot, void* hip_stream) {
    if (n_tokens < 0 || k < 0 || n_expert < 0) return fail(SMOE_EINVAL, "dispatch: negative size");
    if (n_tokens == 0 || k == 0 || n_expert == 0) return ok();
    if (n_expert > kMaxExpert) return fail(SMOE_EINVAL, "dispatch: n_expert exceeds 1024");
    if ((int64_t)n_tokens * k > (1 << 24)) return fail(SMOE_EINVAL, "dispatch: more than 2^24 pairs");
    if (!ids || !offsets || !perm || !slot) return fail(SMOE_ENULL, "dispatch: NULL buffer");
    SMOE_TRY(smoe::launch_dispatch(ids, n_tokens * k, n_expert, counts, offsets, perm, slot, nullptr, nullptr, nullptr,
                                   0, n_tokens, k, 0, 1 << 30, smoe::gemv_shared_chunk(), stream_of(hip_stream)),
             "dispatch");
    return ok();
}

smoe_status smoe_synth_blocks(int32_t type, uint64_t seed, uint64_t stream_id, int64_t n_values, float sigma, void* out,
                              void* hip_stream) {
    if (type != SMOE_Q2_0 && type != SMOE_IQ2_S) return fail(SMOE_ETYPE, "synth_blocks: type is not Q2_0 or IQ2_S");
    const int64_t per = type == SMOE_Q2_0 ? 64 : 256;
    if (n_values < 0 || n_values % per) return fail(SMOE_EINVAL, "synth_blocks: n_values must be whole blocks");
    if (n_values == 0) return ok();
    if (!out) return fail(SMOE_ENULL, "synth_blocks: NULL buffer");
    SMOE_TRY(smoe::launch_synth_blocks(type, seed, stream_id, n_values / per, sigma, static_cast<uint8_t*>(out),
                                       stream_of(hip_stream)),
             "synth_blocks");
    return ok();
}

smoe_status smoe_synth_bf16(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, uint16_t* out, void* hip_stream) {
    if (n < 0) return fail(SMOE_EINVAL, "synth_bf16: negative length");
    if (n == 0) return ok();
    if (!out) return fail(SMOE_ENULL, "synth_bf16: NULL buffer");
    SMOE_TRY(smoe::launch_synth_bf16(seed, stream_id, n, sigma, out, stream_of(hip_stream)), "synth_bf16");
    return ok();
}

smoe_status smoe_synth_normal(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, float* out, void* hip_stream) {
    if (n < 0) return fail(SMOE_EINVAL, "synth_normal: negative length");
    if (n == 0) return ok();
    if (!out) return fail(SMOE_ENULL, "synth_normal: NULL buffer");
    SMOE_TRY(smoe::launch_synth_normal(seed, stream_id, n, sigma, out, stream_of(hip_stream)), "synth_normal");
    return ok();
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------ expert tier
namespace {

int64_t routed_row_bytes(int type, int64_t n) { return type == SMOE_Q2_0 ? n / 64 * 18 : n / 256 * 82; }

// [gate rows | up rows | down rows] of one routed expert
size_t blob_bytes(const smoe_geom& g) {
    return (size_t)(2 * (int64_t)g.n_ff * routed_row_bytes(g.w_type, g.n_embd) +
                    (int64_t)g.n_embd * routed_row_bytes(g.w_type, g.n_ff));
}

// smoe_expert_grouped's workspace: x images, the item table, the checked tokens and rows, the h images
struct GroupedLayout {
    size_t ximg, items, etok, edst, himg, total;
};
GroupedLayout grouped_layout(const smoe_geom& g, int64_t T, int64_t cap_groups, int64_t cap_entries) {
    GroupedLayout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = up(o + bytes);
        return at;
    };
    L.ximg = take(smoe::img_bytes(T * (g.n_embd / 32)));
    L.items = take((size_t)cap_groups * 32);
    L.etok = take((size_t)cap_entries * 4);
    L.edst = take((size_t)cap_entries * 4);
    L.himg = take(smoe::img_bytes(cap_entries * (g.n_ff / 32)));
    L.total = o;
    return L;
}

// The verify window's workspace: the router's outputs, the group lists, the item table (groups, then the shared
// chunks of a fused shared expert), the h images of every entry and shared token, the combine's slots, and the
// native shared expert's chain (in `nat`, whose other offsets are unused).
struct VerifyLayout {
    size_t ximg, logits, sg, grp_ptr, grp_start, ent_dst, ent_tok, items, himg, slot, total;
    int cap_groups, n_items, h_blocks;
    Layout nat;
};
VerifyLayout verify_layout(const smoe_geom& g, int64_t T) {
    VerifyLayout L{};
    const int64_t H = g.n_embd, E = g.n_expert, P = T * g.top_k;
    const int64_t Fmax = (sh_fused(g) && g.n_ff_shared > g.n_ff) ? g.n_ff_shared : g.n_ff;
    L.cap_groups = (int)(P < E ? P : E);
    L.n_items = L.cap_groups + (sh_fused(g) ? smoe::shared_items((int)T) : 0);
    L.h_blocks = (int)(Fmax / 32);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = up(o + bytes);
        return at;
    };
    L.ximg = take(smoe::img_bytes(T * (H / 32)));
    L.logits = take((size_t)T * E * 4);
    L.sg = take((size_t)T * 4);
    L.grp_ptr = take((size_t)L.cap_groups * 8);
    L.grp_start = take((size_t)(L.cap_groups + 1) * 4);
    L.ent_dst = take((size_t)P * 4);
    L.ent_tok = take((size_t)P * 4);
    L.items = take((size_t)L.n_items * 32);
    L.himg = take(smoe::img_bytes((P + T) * L.h_blocks));
    L.slot = take((size_t)P * 4);
    if (sh_native(g)) {
        const int64_t Fs = g.n_ff_shared;
        L.nat.nxq = take((size_t)T * (H / 32) * 36);
        L.nat.ngu = take((size_t)2 * T * Fs * 4);
        L.nat.nhq = take((size_t)T * (Fs / 32) * 36);
    }
    L.total = o;
    return L;
}

}  // namespace

extern "C" {

size_t smoe_expert_blob_bytes(const smoe_geom* g) { return check_geom(g) == SMOE_OK ? blob_bytes(*g) : 0; }

smoe_status smoe_expert_pack(const smoe_geom* g, const smoe_weights* w, int32_t expert, void* blob, void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (!w || !w->gate_exps || !w->up_exps || !w->down_exps || !blob)
        return fail(SMOE_ENULL, "expert_pack: NULL routed planes or blob");
    if (expert < 0 || expert >= g->n_expert) return fail(SMOE_EINVAL, "expert_pack: expert id out of range");
    const size_t gu = (size_t)g->n_ff * (size_t)routed_row_bytes(g->w_type, g->n_embd);
    const size_t dn = (size_t)g->n_embd * (size_t)routed_row_bytes(g->w_type, g->n_ff);
    uint8_t* b = static_cast<uint8_t*>(blob);
    const hipStream_t st = stream_of(hip_stream);
    SMOE_TRY(hipMemcpyAsync(b, static_cast<const uint8_t*>(w->gate_exps) + (size_t)expert * gu, gu, hipMemcpyDefault, st),
             "expert_pack gate");
    SMOE_TRY(hipMemcpyAsync(b + gu, static_cast<const uint8_t*>(w->up_exps) + (size_t)expert * gu, gu, hipMemcpyDefault,
                            st),
             "expert_pack up");
    SMOE_TRY(hipMemcpyAsync(b + 2 * gu, static_cast<const uint8_t*>(w->down_exps) + (size_t)expert * dn, dn,
                            hipMemcpyDefault, st),
             "expert_pack down");
    return ok();
}

smoe_status smoe_expert_group(const int32_t* ids, int32_t n, int32_t k_per_tok, int32_t n_expert,
                              const uint64_t* expert_ptr, uint64_t* grp_ptr, int32_t* grp_start, int32_t* grp_expert,
                              int32_t* ent_dst, int32_t* ent_tok, int32_t* miss_dst, int32_t* counts,
                              void* hip_stream) {
    if (n < 0 || n > smoe::kMaxGroupEntries) return fail(SMOE_EINVAL, "expert_group: n must be in 0..4096");
    if (k_per_tok < 1) return fail(SMOE_EINVAL, "expert_group: k_per_tok must be at least 1");
    if (n_expert < 1 || n_expert > smoe::kMaxGroupExperts) return fail(SMOE_EINVAL, "expert_group: n_expert must be in 1..1024");
    if (!expert_ptr || !grp_ptr || !grp_start || !ent_dst || !ent_tok || !miss_dst || !counts || (n > 0 && !ids))
        return fail(SMOE_ENULL, "expert_group: NULL buffer");
    if (!aligned(expert_ptr, 8) || !aligned(grp_ptr, 8)) return fail(SMOE_EALIGN, "expert_group: pointer tables must be 8-byte aligned");
    SMOE_TRY(smoe::launch_expert_group(ids, n, k_per_tok, n_expert, expert_ptr, grp_ptr, grp_start, grp_expert, ent_dst,
                                       ent_tok, miss_dst, counts, nullptr, 0, 0, n, 0, nullptr, stream_of(hip_stream)),
             "expert_group");
    return ok();
}

size_t smoe_expert_grouped_workspace_bytes(const smoe_geom* g, int32_t n_tokens, int32_t cap_groups,
                                           int32_t cap_entries) {
    if (check_geom(g) != SMOE_OK || n_tokens < 0 || cap_groups < 0 || cap_entries < 0) return 0;
    return grouped_layout(*g, n_tokens, cap_groups, cap_entries).total;
}

smoe_status smoe_expert_grouped(const smoe_geom* g, const uint64_t* grp_ptr, const int32_t* grp_start,
                                const int32_t* ent_dst, const int32_t* ent_tok, const int32_t* counts,
                                int32_t cap_groups, int32_t cap_entries, const uint8_t* x_q8_1, int32_t n_tokens,
                                float* out, int32_t n_out_rows, void* workspace, size_t workspace_bytes,
                                void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (n_tokens < 0 || cap_groups < 0 || cap_entries < 0 || n_out_rows < 0)
        return fail(SMOE_EINVAL, "expert_grouped: negative size");
    // one work-group row per group: the launch's second grid dimension holds at most 65535
    if (cap_groups > 65535 || cap_entries > (1 << 24))
        return fail(SMOE_EINVAL, "expert_grouped: cap_groups must be at most 65535 and cap_entries at most 2^24");
    if (n_tokens == 0 || cap_groups == 0 || cap_entries == 0 || n_out_rows == 0) return ok();
    if (!grp_ptr || !grp_start || !ent_dst || !ent_tok || !counts || !x_q8_1 || !out || !workspace)
        return fail(SMOE_ENULL, "expert_grouped: NULL buffer");
    const GroupedLayout L = grouped_layout(*g, n_tokens, cap_groups, cap_entries);
    if (workspace_bytes < L.total) return fail(SMOE_ESIZE, "expert_grouped: workspace too small");
    if (!aligned(workspace, kAlign)) return fail(SMOE_EALIGN, "expert_grouped: workspace must be 256-byte aligned");
    if (!aligned(grp_ptr, 8) || !aligned(x_q8_1, 4) || !aligned(out, 4))
        return fail(SMOE_EALIGN, "expert_grouped: grp_ptr must be 8-byte and x, out 4-byte aligned");
    const int H = g->n_embd, F = g->n_ff;
    const bool iq2 = g->w_type == SMOE_IQ2_S;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint32_t* ximg = reinterpret_cast<uint32_t*>(ws + L.ximg);
    int4* items = reinterpret_cast<int4*>(ws + L.items);
    int32_t* etok = reinterpret_cast<int32_t*>(ws + L.etok);
    int32_t* edst = reinterpret_cast<int32_t*>(ws + L.edst);
    uint32_t* himg = reinterpret_cast<uint32_t*>(ws + L.himg);
    const int hb = F / 32;
    const hipStream_t st = stream_of(hip_stream);
    SMOE_TRY(smoe::launch_q8_images(x_q8_1, (int64_t)n_tokens * (H / 32), iq2 ? 1 : 0, ximg, st), "grouped images");
    SMOE_TRY(smoe::launch_group_items(grp_ptr, grp_start, ent_tok, ent_dst, counts, cap_groups, cap_entries, n_tokens,
                                      n_out_rows, items, etok, edst, st),
             "grouped items");
    if (iq2) {
        SMOE_TRY(smoe::launch_iq2_gu(nullptr, nullptr, nullptr, nullptr, ximg, items, etok, 1, H, F, 0, 0, cap_groups,
                                     himg, hb, st, nullptr, grp_ptr),
                 "grouped gate/up");
        SMOE_TRY(smoe::launch_iq2_down(nullptr, nullptr, himg, hb, nullptr, items, H, F, 0, cap_groups, out, st,
                                       grp_ptr, edst),
                 "grouped down");
    } else {
        SMOE_TRY(smoe::launch_q2_gu(nullptr, nullptr, nullptr, nullptr, ximg, items, etok, 1, H, F, 0, 0, cap_groups,
                                    himg, hb, st, nullptr, grp_ptr),
                 "grouped gate/up");
        SMOE_TRY(smoe::launch_q2_down(nullptr, nullptr, himg, hb, nullptr, items, H, F, 0, cap_groups, out, st, grp_ptr,
                                      edst),
                 "grouped down");
    }
    return ok();
}

size_t smoe_verify_workspace_bytes(const smoe_geom* g, int32_t max_tokens) {
    if (check_geom(g) != SMOE_OK || max_tokens < 0 || (int64_t)max_tokens * g->top_k > smoe::kMaxGroupEntries) return 0;
    return verify_layout(*g, max_tokens).total;
}

smoe_status smoe_verify_begin(const smoe_geom* g, const smoe_weights* w, const uint64_t* expert_ptr, const float* x,
                              int32_t n_tokens, float* rows, int32_t* ids, float* weights, int32_t* miss_dst,
                              int32_t* counts, void* workspace, size_t workspace_bytes, void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (!w) return fail(SMOE_ENULL, "verify_begin: weights is NULL");
    if (n_tokens < 0) return fail(SMOE_EINVAL, "verify_begin: n_tokens is negative");
    if ((int64_t)n_tokens * g->top_k > smoe::kMaxGroupEntries)
        return fail(SMOE_EINVAL, "verify_begin: n_tokens * top_k exceeds 4096");
    if (n_tokens == 0) return ok();
    const bool has_sh = g->sh_type >= 0, nat = sh_native(*g), shf = has_sh && !nat;
    if (!w->router) return fail(SMOE_ENULL, "verify_begin: the router is NULL");
    if (has_sh && (!w->gate_sh || !w->up_sh || !w->down_sh || !w->gate_inp_sh))
        return fail(SMOE_ENULL, "verify_begin: a shared expert tensor is NULL (set sh_type = -1 for a layer without one)");
    if (!expert_ptr || !x || !rows || !ids || !weights || !miss_dst || !counts || !workspace)
        return fail(SMOE_ENULL, "verify_begin: NULL buffer");
    const VerifyLayout L = verify_layout(*g, n_tokens);
    if (workspace_bytes < L.total) return fail(SMOE_ESIZE, "verify_begin: workspace too small");
    if (!aligned(workspace, kAlign)) return fail(SMOE_EALIGN, "verify_begin: workspace must be 256-byte aligned");
    if (!aligned(expert_ptr, 8) || !aligned(x, 16) || !aligned(rows, 4) || !aligned(ids, 4) || !aligned(weights, 4))
        return fail(SMOE_EALIGN, "verify_begin: expert_ptr 8-byte, x 16-byte, rows, ids and weights 4-byte aligned");
    const int T = n_tokens, H = g->n_embd, E = g->n_expert, K = g->top_k, F = g->n_ff, P = T * K;
    const int Fs = shf ? g->n_ff_shared : 0;
    if (overlaps_n(x, (size_t)T * H * 4, rows, (size_t)(P + T) * H * 4))
        return fail(SMOE_EINVAL, "verify_begin: rows overlaps x");
    const bool iq2 = g->w_type == SMOE_IQ2_S, f32r = g->router_dtype == SMOE_ROUTER_F32;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint32_t* ximg = reinterpret_cast<uint32_t*>(ws + L.ximg);
    float* logits = reinterpret_cast<float*>(ws + L.logits);
    float* sg = reinterpret_cast<float*>(ws + L.sg);
    uint64_t* grp_ptr = reinterpret_cast<uint64_t*>(ws + L.grp_ptr);
    int32_t* grp_start = reinterpret_cast<int32_t*>(ws + L.grp_start);
    int32_t* ent_dst = reinterpret_cast<int32_t*>(ws + L.ent_dst);
    int32_t* ent_tok = reinterpret_cast<int32_t*>(ws + L.ent_tok);
    int4* items = reinterpret_cast<int4*>(ws + L.items);
    uint32_t* himg = reinterpret_cast<uint32_t*>(ws + L.himg);
    const hipStream_t st = stream_of(hip_stream);
    // the router as the block's decode path runs it (the same x images, logits, shared gate dots and routing)
    SMOE_TRY(smoe::launch_router(x, nullptr, w->router, has_sh ? w->gate_inp_sh : nullptr, w->logit_bias, H, E,
                                 E + (has_sh ? 1 : 0), T, logits, E, sg, ximg, 0, iq2 ? 1 : 0, st, nullptr, 0.0f,
                                 nullptr, nullptr, 0, f32r ? 1 : 0),
             "verify router");
    SMOE_TRY(smoe::launch_topk(logits, E, T, E, K, ids, weights, st), "verify topk");
    SMOE_TRY(smoe::launch_expert_group(ids, P, K, E, expert_ptr, grp_ptr, grp_start, nullptr, ent_dst, ent_tok,
                                       miss_dst, counts, items, L.cap_groups, L.n_items - L.cap_groups, P, T, nullptr,
                                       st),
             "verify split");
    const uint8_t* gs = static_cast<const uint8_t*>(w->gate_sh);
    const uint8_t* us = static_cast<const uint8_t*>(w->up_sh);
    const uint8_t* ds = static_cast<const uint8_t*>(w->down_sh);
    if (iq2) {
        SMOE_TRY(smoe::launch_iq2_gu(nullptr, nullptr, gs, us, ximg, items, ent_tok, 1, H, F, Fs, shf ? 1 : 0, L.n_items,
                                     himg, L.h_blocks, st, nullptr, grp_ptr),
                 "verify gate/up");
        SMOE_TRY(smoe::launch_iq2_down(nullptr, ds, himg, L.h_blocks, sg, items, H, F, Fs, L.n_items, rows, st, grp_ptr,
                                       ent_dst),
                 "verify down");
    } else {
        SMOE_TRY(smoe::launch_q2_gu(nullptr, nullptr, gs, us, ximg, items, ent_tok, 1, H, F, Fs, shf ? 1 : 0, L.n_items,
                                    himg, L.h_blocks, st, nullptr, grp_ptr),
                 "verify gate/up");
        SMOE_TRY(smoe::launch_q2_down(nullptr, ds, himg, L.h_blocks, sg, items, H, F, Fs, L.n_items, rows, st, grp_ptr,
                                      ent_dst),
                 "verify down");
    }
    if (nat) SMOE_TRY_S(native_shared(*g, w, x, T, ws, L.nat, rows + (size_t)P * H, sg, st));
    return ok();
}

smoe_status smoe_verify_end(const smoe_geom* g, int32_t n_tokens, const float* rows, const float* weights,
                            int32_t add_shared, float* y, void* workspace, size_t workspace_bytes, void* hip_stream) {
    smoe_status s = check_geom(g);
    if (s != SMOE_OK) return s;
    if (n_tokens < 0) return fail(SMOE_EINVAL, "verify_end: n_tokens is negative");
    if ((int64_t)n_tokens * g->top_k > smoe::kMaxGroupEntries)
        return fail(SMOE_EINVAL, "verify_end: n_tokens * top_k exceeds 4096");
    if (n_tokens == 0) return ok();
    if (!rows || !weights || !y || !workspace) return fail(SMOE_ENULL, "verify_end: NULL buffer");
    const VerifyLayout L = verify_layout(*g, n_tokens);
    if (workspace_bytes < L.total) return fail(SMOE_ESIZE, "verify_end: workspace too small");
    if (!aligned(workspace, kAlign)) return fail(SMOE_EALIGN, "verify_end: workspace must be 256-byte aligned");
    if (!aligned(rows, 4) || !aligned(weights, 4) || !aligned(y, 4))
        return fail(SMOE_EALIGN, "verify_end: rows, weights and y must be 4-byte aligned");
    const int T = n_tokens, H = g->n_embd, K = g->top_k, P = T * K;
    if (overlaps_n(y, (size_t)T * H * 4, rows, (size_t)(P + T) * H * 4))
        return fail(SMOE_EINVAL, "verify_end: y overlaps rows");
    int32_t* slot = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + L.slot);
    const hipStream_t st = stream_of(hip_stream);
    SMOE_TRY(smoe::launch_iota(slot, P, st), "verify slots");
    SMOE_TRY(smoe::launch_combine(rows, slot, weights, K, H, P, T, (g->sh_type >= 0 && add_shared) ? 1 : 0, y, st),
             "verify combine");
    return ok();
}

}  // extern "C"
