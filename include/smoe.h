/* include/smoe.h - C ABI of the MI355X (gfx950) quantized mixture-of-experts block.
 *
 * The drop-in boundary for StrataMetal's per-layer MoE call: `FfnExec::run`'s interior from `mixed` to
 * `combined` (metal/src/layer_exec.cpp:470-530) and the kernel-level calls it is built from.  Plain
 * pointers and sizes only; no exceptions cross this boundary.  Pointers are DEVICE pointers unless a
 * comment says otherwise.  Every entry point validates its arguments before launching anything and
 * returns a status; a refused call launches nothing and leaves every output untouched; a call with a
 * zero count returns SMOE_OK without launching (metal/src/router.mm:33-37, metal/src/iq.mm:150-158).
 * All work is enqueued on `hip_stream` (a hipStream_t; NULL = the null stream): no host
 * synchronisation, no allocation.
 *
 * Weight layouts are GGUF's, unchanged:
 *   Q2_0  (ggml type 42): 18-byte blocks {fp16 d; 16 code bytes} of 64 weights, value (code - 1) * d
 *         (include/strata/artifact/dequant.hpp:8-13,69-78).
 *   IQ2_S (ggml type 22): 82-byte blocks of 256 weights (include/strata/artifact/gguf_reader.hpp:197-200).
 *   A 3-D expert tensor holds expert e at e * rows * row_bytes (metal/src/layer_exec.cpp:115-120).
 *   q8_1 activations: 36-byte blocks {fp16 d; fp16 s; int8 q[32]} (metal/include/strata/metal/iq.hpp:42-43).
 *   The other native types of real layers (the shared expert's projections, the down quants), GGUF's blocks:
 *   Q8_0 (8, 34 B / 32), Q4_0 (2, 18 B / 32), Q5_0 (6, 22 B / 32), IQ4_NL (20, 18 B / 32), IQ4_XS (23, 136 B / 256),
 *   Q3_K (11, 110 B / 256), Q4_K (12, 144 B / 256), Q5_K (13, 176 B / 256), Q6_K (14, 210 B / 256)
 *   (include/strata/artifact/dequant.hpp:81-280).
 */
#ifndef SMOE_H
#define SMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    SMOE_OK = 0,
    SMOE_EINVAL = -1, /* a count, shape or option is out of range */
    SMOE_ESIZE = -2,  /* a caller-provided buffer (workspace) is too small */
    SMOE_ETYPE = -3,  /* a ggml type this block does not implement */
    SMOE_EDEVICE = -4,/* the HIP runtime reported an error at launch */
    SMOE_EALIGN = -5, /* a pointer is not aligned as the layout requires */
    SMOE_ENULL = -6   /* a required pointer is NULL */
} smoe_status;

enum { SMOE_Q2_0 = 42, SMOE_IQ2_S = 22 };
enum {
    SMOE_Q8_0 = 8, SMOE_Q4_0 = 2, SMOE_Q5_0 = 6, SMOE_IQ4_NL = 20, SMOE_IQ4_XS = 23,
    SMOE_Q3_K = 11, SMOE_Q4_K = 12, SMOE_Q5_K = 13, SMOE_Q6_K = 14
};

/* Which arithmetic contract runs the expert products. */
enum {
    SMOE_PATH_AUTO = 0, /* GEMV for n_tokens < 128, MFMA otherwise */
    SMOE_PATH_GEMV = 1, /* q8_1 activations, integer dot (the decode contract) */
    SMOE_PATH_MFMA = 2  /* bf16 activations, bf16 MFMA with exact per-block weight scales (the prefill contract);
                           the matrix cores take bf16 activations and h as fp16, which holds them below 65520 in
                           magnitude (smoe_trace.overflow reports tokens beyond), and block scales below 32752 */
};

#define SMOE_ROUTER_BF16 0
#define SMOE_ROUTER_F32 1

/* Layer geometry.  ModelGeometry's MoE fields (include/strata/core/layout.hpp:27-59) plus the types. */
typedef struct {
    int32_t n_embd;       /* H: 128 * 2^a * b with b <= 8 (2048, 2560, 4096 ...), at most 4096 */
    int32_t n_ff;         /* routed expert width: same form (512, 640 ...), at most 4096 */
    int32_t n_ff_shared;  /* shared expert width (ignored when sh_type < 0) */
    int32_t n_expert;     /* E: 1..1024 (metal/src/router.mm:33-37) */
    int32_t top_k;        /* k: 1..64, k <= E */
    int32_t w_type;       /* routed experts: SMOE_Q2_0 or SMOE_IQ2_S */
    int32_t sh_type;      /* shared expert: its type (any type below), or -1 = no shared expert */
    int32_t router_dtype; /* 0 = bf16 (the repo's contract: include/strata/core/layer.hpp:131-136); 1 = f32 router
                             weights and f32 activations in the router (the literal benchmark configuration; the
                             shared gate stays bf16); SMOE_ROUTER_F32 */
    /* The shared expert's gate, up and down projections in their own types (0: sh_type), as real layers store
     * them (include/strata/kernels/shared_expert.hpp:54-58: NativeSharedWeights).  A shared expert whose three
     * types all equal w_type runs inside the expert kernels; any other one (a "native" shared expert: Q2_0, IQ2_S
     * or the SMOE_Q8_0 .. SMOE_Q6_K types, each projection its own) runs the q8_1 GEMV contract on every path
     * (x as q8_1 blocks, the types' integer dots in the reference's 32-lane order, SwiGLU + q8_1, down times
     * sigmoid(gate_inp_shexp . x)).  n_ff_shared % 32 == 0; each projection's row length a whole number of its
     * blocks (Q2_0: 128 * 2^a * b, b <= 8; IQ2_S: 512, 1024 or 2048); n_ff_shared at most 4096. */
    int32_t sh_gate_type, sh_up_type, sh_down_type;
} smoe_geom;

/* One layer's tensors, all resident in device memory (4-byte aligned). */
typedef struct {
    const void* gate_exps;       /* ffn_gate_exps: [E][n_ff] rows of n_embd */
    const void* up_exps;         /* ffn_up_exps:   [E][n_ff] rows of n_embd */
    const void* down_exps;       /* ffn_down_exps: [E][n_embd] rows of n_ff */
    const void* router;          /* ffn_gate_inp: [E][n_embd] bf16, or f32 with router_dtype 1 (16-byte aligned) */
    const void* gate_sh;         /* ffn_gate_shexp: [n_ff_shared] rows of n_embd */
    const void* up_sh;           /* ffn_up_shexp */
    const void* down_sh;         /* ffn_down_shexp: [n_embd] rows of n_ff_shared */
    const uint16_t* gate_inp_sh; /* ffn_gate_inp_shexp: [n_embd] bf16 */
    const float* logit_bias;     /* [E] added to the router logits before top-k, or NULL (synthetic routing only) */
} smoe_weights;

/* Optional device copies of intermediate results (FfnTrace, metal/include/strata/metal/layer_exec.hpp:100-109).
 * Any pointer may be NULL. */
typedef struct {
    float* logits;    /* [T][E] router logits (bias included) */
    int32_t* ids;     /* [T][k] selected experts, selection order */
    float* weights;   /* [T][k] renormalised routing weights */
    int32_t* counts;  /* [E] pairs per expert */
    int32_t* offsets; /* [E+1] exclusive prefix sum of counts */
    int32_t* perm;    /* [T*k] pair index t*k+s at each dispatch position */
    int32_t* slot;    /* [T*k] dispatch position of pair t*k+s */
    float* sgate;     /* [T] shared expert gate dot (before the sigmoid) */
    /* NULL, or SMOE_STAGE_EVENTS hipEvent_t recorded on hip_stream at the stage boundaries of smoe_forward
     * (before the first kernel and after each stage: router, route (q8_1 + top-k + dispatch), gate/up, down,
     * combine),
     * for per-stage timing (the upstream engine's event-pair stage timing, include/strata/core/layer.hpp:317-337). */
    void* const* stage_events;
    /* The expert stages (FfnTrace's exq, ehq, edown and shared).  A call asking for any of xq, hq, parts or shared
     * runs the decode path's unfused kernels (top-k and dispatch, gate/up, down, combine; the same bits as the fused
     * launches of small batches). */
    uint8_t* xq;      /* [T][n_embd/32] q8_1 blocks (36 bytes: fp16 d, fp16 s, 32 int8) of x (decode path only) */
    uint8_t* hq;      /* [T*k][n_ff/32] q8_1 blocks of each pair's h, by dispatch position (decode path only) */
    float* parts;     /* [T*k][n_embd] each pair's expert output before its routing weight, by dispatch position */
    float* shared;    /* [T][n_embd] the shared expert's output times sigmoid(sgate) (layers with a shared expert) */
    /* [1] the call's status mask (smoe_forward_status's): 0, or bit 0 -- an activation whose bf16 value is 65520 or
     * more in magnitude (finite x) met the prefill path's fp16 operands, bit 1 -- such an h value (the affected
     * tokens' outputs are then not the prefill contract's: inf or NaN), bit 2 -- a bounded wait of the fused decode
     * launch gave up (the rows of its down work-groups are NaN). */
    int32_t* overflow;
    /* More of FfnTrace's expert stages (egate, eup; sgate, sup, sh_hq), for the reference's stage-wise check
     * (metal/src/pack_parity.cpp:8584-8600): the products of each stage from the device's own q8_1 inputs.  Decode
     * path only; asking for any of them runs the unfused kernels, as above. */
    float* egate;     /* [T*k][n_ff] each pair's gate dots (before SwiGLU), by dispatch position */
    float* eup;       /* [T*k][n_ff] each pair's up dots */
    float* sgu;       /* [2][T][n_ff_shared] the shared expert's gate dots, then its up dots (layers with a shared
                         expert) */
    uint8_t* shq;     /* [T][n_ff_shared/32] q8_1 blocks of the shared expert's h (layers with a shared expert) */
} smoe_trace;

#define SMOE_STAGE_EVENTS 6

/* ---------------------------------------------------------------------------------------------- block */

/* Bits of a call's status mask (smoe_forward_status, smoe_trace.overflow). */
#define SMOE_STATUS_X_FP16 1 /* an activation at or beyond 65520 in magnitude met the prefill path's fp16 operands */
#define SMOE_STATUS_H_FP16 2 /* such an h value */
#define SMOE_STATUS_WAIT 4   /* a bounded wait of the fused decode launch gave up: its down work-groups' y rows are NaN */

/* Workspace bytes smoe_forward needs for up to `max_tokens` tokens (either path); 0 on bad geometry. */
size_t smoe_workspace_bytes(const smoe_geom* g, int32_t max_tokens);

/* y[T][n_embd] = MoE(x[T][n_embd]): router, top-k, dispatch, expert products with SwiGLU, the shared
 * expert times sigmoid(gate_inp_shexp . x) (added only when add_shared != 0), and the weighted combine.
 * Replaces FfnExec::run's interior (metal/src/layer_exec.cpp:470-530) and the upstream per-layer
 * moe_layer / moe_route + moe_finish (include/strata/core/layer.hpp:140-189).  `workspace` is
 * device memory of at least smoe_workspace_bytes(g, n_tokens) bytes, 256-byte aligned; concurrent
 * calls need distinct workspaces.  A call takes at most 65535 tokens (n_tokens * top_k at most 2^24).
 * Batches of at most 4 tokens on the decode path run as the router launch and one launch of the rest, whose down
 * work-groups wait for the gate/up work-groups' h (a bounded wait).  Should a wait give up (a producer never arrived,
 * e.g. its work-group was starved of a CU for ~0.1 s), the affected rows of y are NaN and smoe_forward_status reports
 * SMOE_STATUS_WAIT; the call still returns SMOE_OK, as no host synchronisation happens on the call path. */
smoe_status smoe_forward(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                         int32_t add_shared, void* workspace, size_t workspace_bytes, const smoe_trace* trace,
                         void* hip_stream);

/* smoe_forward with an explicit contract (SMOE_PATH_*). */
smoe_status smoe_forward_path(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                              int32_t add_shared, void* workspace, size_t workspace_bytes, const smoe_trace* trace,
                              int32_t path, void* hip_stream);

/* The stacked configuration's layer junction fused into the next layer's call: x = RMSNorm(x_prev + r_prev)
 * (unit weight; as smoe_residual_rmsnorm forms it) is written to x, then y = MoE(x) as smoe_forward.  On the
 * decode (GEMV) path the norm is formed inside the router kernel; on the prefill path a junction kernel runs
 * first.  Bitwise equal to smoe_residual_rmsnorm followed by smoe_forward.  x must not overlap x_prev, r_prev
 * or y (y may be r_prev); x_prev, r_prev and x 16-byte aligned.  No counterpart in the reference's MoE block
 * (its layer walk normalises in the hyper-connection read, out of this block's scope). */
smoe_status smoe_forward_residual(const smoe_geom* g, const smoe_weights* w, const float* x_prev, const float* r_prev,
                                  float eps, float* x, int32_t n_tokens, float* y, int32_t add_shared,
                                  void* workspace, size_t workspace_bytes, const smoe_trace* trace, void* hip_stream);

/* ---------------------------------------------------------------------------------------------- layer ends */

/* The hyper-connection ends of the layer call: FfnExec::run reads the MoE block's input from hc residual streams
 * through the gated residual (gr_read) and adds the block's output back onto every stream (gr_write)
 * (metal/src/layer_exec.cpp:469,531; metal/include/strata/metal/gr.hpp:22-48).  Per token R is [hc][n_embd] f32:
 *   xn = R * rs_c * norm (rs_c = 1 / sqrt(mean(R_c^2) + eps)), act = bf16(xn);
 *   lq = bf16(silu((act . down_r) / hc)); mixed_d = (sum_c xn_cd * sigmoid(lq . up_{c n_embd + d})) / hc;
 *   inject_c = act . inject_c;   out_cd = R_cd + y_d * 2 sigmoid(inject_c / hc).
 * Shapes: n_embd % 8 == 0 and at most 4096, hc <= 8, hc * n_embd <= 16384, hc_lr % 8 == 0 and at most 2048. */
typedef struct {
    int32_t hc;             /* residual streams (the reference model's 4: include/strata/core/layout.hpp:48-49) */
    int32_t hc_lr;          /* width of the gate's low-rank projection (320) */
    float eps;              /* the per-stream RMSNorm's epsilon (FfnExec::run passes 1e-6) */
    const float* norm;      /* hc_norm: [hc][n_embd] f32, the stored (1 + w) */
    const uint16_t* down;   /* hc_down: [hc_lr][hc * n_embd] bf16 */
    const uint16_t* up;     /* hc_up: [hc * n_embd][hc_lr] bf16 */
    const uint16_t* inject; /* hc_inj: [hc][hc * n_embd] bf16 */
} smoe_hc;

/* Workspace bytes of smoe_hc_read for up to max_tokens tokens (0 on a bad shape). */
size_t smoe_hc_read_workspace_bytes(const smoe_hc* hc, int32_t n_embd, int32_t max_tokens);

/* gr_read for n_tokens tokens: R [T][hc][n_embd] -> mixed [T][n_embd], inject [T][hc] (inject may be NULL: the
 * final mixer, nothing written).  Replaces gr_read (metal/include/strata/metal/gr.hpp:44-46) with bf16 activations. */
smoe_status smoe_hc_read(const smoe_hc* hc, int32_t n_embd, const float* R, int32_t n_tokens, float* mixed,
                         float* inject, void* workspace, size_t workspace_bytes, void* hip_stream);

/* gr_write: R_out[t][c][d] = R[t][c][d] + y[t][d] * 2 sigmoid(inject[t][c] / hc); R_out may be R.
 * Replaces gr_write (metal/include/strata/metal/gr.hpp:48). */
smoe_status smoe_hc_write(const smoe_hc* hc, int32_t n_embd, const float* R, const float* y, const float* inject,
                          int32_t n_tokens, float* R_out, void* hip_stream);

/* Workspace bytes of smoe_ffn_run for up to max_tokens tokens (0 on bad geometry). */
size_t smoe_ffn_workspace_bytes(const smoe_geom* g, const smoe_hc* hc, int32_t max_tokens);

/* The whole layer call FfnExec::run(residual, out, add_shared, trace) (metal/include/strata/metal/layer_exec.hpp:
 * 135-137, metal/src/layer_exec.cpp:462-531): gr_read of the residual streams, the MoE block on `mixed`
 * (smoe_forward, SMOE_PATH_AUTO), gr_write of its output back onto the streams.  residual and out are
 * [T][hc][n_embd] f32 (out may be residual); `trace` covers the MoE block as in smoe_forward. */
smoe_status smoe_ffn_run(const smoe_geom* g, const smoe_weights* w, const smoe_hc* hc, const float* residual,
                         int32_t n_tokens, float* out, int32_t add_shared, void* workspace, size_t workspace_bytes,
                         const smoe_trace* trace, void* hip_stream);

/* ---------------------------------------------------------------------------------------------- GGUF models */

/* A model in GGUF v3 files, read on the host: every shard of a split model (`<stem>-NNNNN-of-MMMMM.gguf`, any
 * shard's path opens all; the metadata in shard 1), mapped read-only.  Replaces GgufFile / GgufModel and
 * ModelTensors (include/strata/artifact/gguf_reader.hpp:340-566, metal/include/strata/metal/layer_tensors.hpp:87-212).
 * Refused: a missing shard, bad magic, a version other than 3, a header that ends early, a tensor listed twice or
 * in two shards, split.count / split.no / split.tensors.count that disagree. */
typedef struct smoe_model smoe_model;

typedef struct {
    int32_t type;         /* ggml type */
    int32_t n_dims;
    int32_t shard;        /* the shard holding it (0 = the first) */
    int32_t reserved;
    uint64_t ne[4];       /* GGUF order: ne[0] is a row (it varies fastest); unused dimensions are 1 */
    uint64_t bytes;       /* payload bytes */
    uint64_t file_offset; /* byte offset of the payload in its shard */
    const void* host;     /* the payload in the read-only mapping (valid until smoe_model_close) */
} smoe_tensor_info;

smoe_status smoe_model_open(const char* any_shard_path, smoe_model** out);
void smoe_model_close(smoe_model* m);
int32_t smoe_model_n_shards(const smoe_model* m);
int64_t smoe_model_n_tensors(const smoe_model* m);
/* A tensor by its full name (blk.<layer>.<suffix> for a layer's), refused when absent, of a type without a known
 * block size, or not inside its file. */
smoe_status smoe_model_tensor(const smoe_model* m, const char* name, smoe_tensor_info* info);
/* The i-th tensor (shard by shard, directory order) and its name (name_cap bytes, NUL included). */
smoe_status smoe_model_tensor_at(const smoe_model* m, int64_t i, char* name, size_t name_cap, smoe_tensor_info* info);
/* Metadata of the first shard: an integer or bool value (an array: its element count), or a string. */
smoe_status smoe_model_meta_u64(const smoe_model* m, const char* key, uint64_t* value);
smoe_status smoe_model_meta_str(const smoe_model* m, const char* key, char* buf, size_t cap);

/* One layer's MoE block from the model, the tensor side of FfnExec::load (metal/src/layer_exec.cpp:369-431):
 * blk.<layer>.ffn_{gate,up,down}_exps, ffn_gate_inp, and with_shared the shared expert's ffn_{gate,up,down}_shexp
 * and ffn_gate_inp_shexp (each projection its own type), and the hyper-connection tensors hc_ffn_{norm,down,up,
 * inject} when present (all four or none).  The geometry comes from the tensors' shapes and types (ffn_gate_inp
 * BF16: router_dtype 0, F32: 1; ffn_gate_inp_shexp BF16, or F32 rounded to bf16 on upload), top_k from the call
 * (> 0) or the model's <general.architecture>.expert_used_count; the plan is refused when the block does not take
 * the geometry (smoe_workspace_bytes's checks). */
typedef struct {
    smoe_geom geom;
    smoe_hc hc;          /* hc, hc_lr and eps 1e-6 of the hyper-connection tensors (hc 0: none); pointers NULL */
    size_t device_bytes; /* bytes smoe_layer_upload writes */
    size_t off[12];      /* slot offsets in the device buffer (256-byte aligned) */
    int32_t layer, with_shared;
} smoe_layer_plan;

smoe_status smoe_layer_plan_for(const smoe_model* m, int32_t layer, int32_t top_k, int32_t with_shared,
                                smoe_layer_plan* plan);
/* Copies the planned tensors into `device` (256-byte aligned, at least plan->device_bytes) on hip_stream and waits
 * for the copies; fills `w` (device pointers into `device`) and, when `hc` is given, the hyper-connection tensors. */
smoe_status smoe_layer_upload(const smoe_model* m, const smoe_layer_plan* plan, void* device, size_t device_bytes,
                              smoe_weights* w, smoe_hc* hc, void* hip_stream);

/* ---------------------------------------------------------------------------------------------- expert tier */

/* Routed experts addressed one pointer each: expert e's blob is [gate rows | up rows | down rows] of the routed
 * type (n_ff rows of n_embd values twice, then n_embd rows of n_ff values), the layout of NativeExpertLayout
 * (include/strata/kernels/iq_kernels.hpp:56-65).  A table `expert_ptr` [n_expert] of device-readable addresses
 * (HBM, or pinned host memory the GPU reads over the bus) holds each expert's blob, 0 for an expert the table does
 * not hold.  Every result is bitwise the block's decode contract (smoe_forward's routed pair rows and output). */
size_t smoe_expert_blob_bytes(const smoe_geom* g); /* 0 when the geometry is refused */
/* Copies expert `expert`'s rows from the planes of `w` into `blob` (smoe_expert_blob_bytes) on hip_stream. */
smoe_status smoe_expert_pack(const smoe_geom* g, const smoe_weights* w, int32_t expert, void* blob, void* hip_stream);

/* The hit/miss split on the device.  Entry i of ids[n] (T tokens x k_per_tok, flattened: token i / k_per_tok) is a
 * hit when expert_ptr[ids[i]] != 0, else (no blob, or an id outside [0, n_expert)) a miss.  Hits are grouped by
 * expert, groups in ascending expert id and a group's entries in ascending i: group g's blob grp_ptr[g], expert
 * grp_expert[g] (may be NULL), entries [grp_start[g], grp_start[g + 1]) with ent_dst[j] = i and ent_tok[j] =
 * i / k_per_tok.  Misses go to miss_dst in ascending i.  counts [4] = {groups, hit entries, misses, 0}, all on the
 * device (nothing is read back).  Sizes: grp_ptr, grp_expert min(n, n_expert); grp_start that + 1; ent_dst,
 * ent_tok, miss_dst n.  n <= 4096, n_expert <= 1024.  Replaces moe_hit_select / moe_hit_select_multi /
 * moe_group_resident (include/strata/kernels/s2_expert_grouped.hpp:92-112). */
smoe_status smoe_expert_group(const int32_t* ids, int32_t n, int32_t k_per_tok, int32_t n_expert,
                              const uint64_t* expert_ptr, uint64_t* grp_ptr, int32_t* grp_start, int32_t* grp_expert,
                              int32_t* ent_dst, int32_t* ent_tok, int32_t* miss_dst, int32_t* counts,
                              void* hip_stream);

/* Grouped experts: group g < counts[0] (at most cap_groups) has its blob at grp_ptr[g] and the entries
 * [grp_start[g], grp_start[g + 1]) (within [0, cap_entries)); entry j reads token ent_tok[j]'s activation (x_q8_1:
 * n_tokens rows of n_embd / 32 q8_1 blocks, smoe_quantize_q8_1's format) and writes the expert's output (before the
 * routing weight) to row ent_dst[j] of out (n_out_rows rows of n_embd f32).  Each blob row is read once for all of
 * its group's entries.  The lists are read on the device and checked there: an entry whose token or row is out of
 * range, and a group whose blob is 0, write nothing.  The launch is sized by the caps, so a captured graph replays
 * for any lists.  Sizes: grp_ptr cap_groups, grp_start cap_groups + 1, ent_dst and ent_tok cap_entries
 * (cap_groups <= 65535, cap_entries <= 2^24).
 * Replaces moe_grouped_s2 / native_expert_grouped / moe_hit_grouped_s2_dev (s2_expert_grouped.hpp:104-108,
 * iq_kernels.hpp:70-80). */
size_t smoe_expert_grouped_workspace_bytes(const smoe_geom* g, int32_t n_tokens, int32_t cap_groups,
                                           int32_t cap_entries);
smoe_status smoe_expert_grouped(const smoe_geom* g, const uint64_t* grp_ptr, const int32_t* grp_start,
                                const int32_t* ent_dst, const int32_t* ent_tok, const int32_t* counts,
                                int32_t cap_groups, int32_t cap_entries, const uint8_t* x_q8_1, int32_t n_tokens,
                                float* out, int32_t n_out_rows, void* workspace, size_t workspace_bytes,
                                void* hip_stream);

/* The verify window with the hit/miss split: n_tokens tokens (n_tokens * top_k <= 4096) through the layer, the
 * routed experts from the table.  smoe_verify_begin runs the router and the routing (ids, weights [T][k], as
 * smoe_forward's), the split (miss_dst, counts as smoe_expert_group), the hits into rows[i] (i = t * k + s, the
 * entry's row) and the shared expert into rows[T * k + t] (times sigmoid of its gate): rows is [(T * k + T)][n_embd]
 * f32.  The caller then writes each miss's row (rows[miss_dst[j]], j < counts[2]: its own expert pool, or
 * smoe_expert_grouped over another table), and smoe_verify_end forms y [T][n_embd] from rows and weights as
 * smoe_forward's combine does.  w->gate_exps / up_exps / down_exps are not read (may be NULL).  Both calls take the
 * same workspace (smoe_verify_workspace_bytes of at least n_tokens).  With every expert in the table, begin + end
 * give smoe_forward's y bitwise; a miss computed by smoe_expert_grouped gives the same row as a hit.
 * Replaces the verify window's moe_hit_select_multi + moe_hit_grouped_s2_multi + moe_hit_add + moe_combine
 * (s2_expert_grouped.hpp:92-99). */
size_t smoe_verify_workspace_bytes(const smoe_geom* g, int32_t max_tokens);
smoe_status smoe_verify_begin(const smoe_geom* g, const smoe_weights* w, const uint64_t* expert_ptr, const float* x,
                              int32_t n_tokens, float* rows, int32_t* ids, float* weights, int32_t* miss_dst,
                              int32_t* counts, void* workspace, size_t workspace_bytes, void* hip_stream);
smoe_status smoe_verify_end(const smoe_geom* g, int32_t n_tokens, const float* rows, const float* weights,
                            int32_t add_shared, float* y, void* workspace, size_t workspace_bytes, void* hip_stream);

/* ---------------------------------------------------------------------------------------------- no allocation */

/* Bytes of the library's static device scratch (one array per GPU, held from the library's load until the
 * process ends). */
#define SMOE_STATIC_SCRATCH_BYTES (32u << 20)

/* smoe_forward (SMOE_PATH_AUTO) with the library's own static device scratch in place of a caller workspace: it
 * calls no hipMalloc, hipFree or other allocating routine, so it suits callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Limit: a call whose smoe_workspace_bytes(g, n_tokens) exceeds SMOE_STATIC_SCRATCH_BYTES is refused with
 * SMOE_ESIZE (at the benchmark geometry, H 2048 / E 512 / k 10 / FF 512, that is 299 tokens).
 * `hip_stream` must belong to the current device.  Every call on one GPU shares that GPU's scratch and leaves
 * its contents behind: calls that overlap in time on one GPU (other streams, other host threads) race, so the
 * caller serialises them.  The first call on a device looks up the scratch's device address once. */
smoe_status smoe_forward_static(const smoe_geom* g, const smoe_weights* w, const float* x, int32_t n_tokens, float* y,
                                int32_t add_shared, const smoe_trace* trace, void* hip_stream);

/* The status of the last block call enqueued on `workspace` (smoe_forward, smoe_forward_path, smoe_forward_residual,
 * smoe_ffn_run; NULL: the current GPU's scratch of smoe_forward_static), folded on hip_stream into *status (device
 * memory, one int32) after that call: 0, or a mask of the SMOE_STATUS_* bits above.  The affected tokens' outputs are
 * then not the contract's; the caller can rerun them (on SMOE_PATH_GEMV for the fp16 bits).  The library keeps the
 * flag places of the last call on each of its 64 most recent workspaces (a workspace beyond them: SMOE_EINVAL).  No
 * counterpart in the reference (its prompt path shares the fp16 limit, include/strata/prefill/kernels.hpp:97-98). */
smoe_status smoe_forward_status(const void* workspace, int32_t* status, void* hip_stream);

/* The bound of the fused decode launch's waits, in polls (each a memory round trip, ~1 us): polls > 0 sets it, 0
 * restores the default (100000), a negative value makes every wait give up at once -- for tests of the give-up path.
 * Returns the previous bound.  Applies to launches enqueued after it (a captured graph keeps its own). */
int32_t smoe_set_wait_limit(int32_t polls);

/* ---------------------------------------------------------------------------------------------- stages */

/* logits (n_tokens, n_expert) f32 -> ids, weights (n_tokens, k): softmax over every expert, top k by
 * (logit desc, id asc), weights renormalised by max(sum, 2^-14).  k <= 64, n_expert <= 1024.
 * Replaces router_top10 (metal/include/strata/metal/router.hpp:16). */
smoe_status smoe_router_topk(const float* logits, int32_t n_tokens, int32_t n_expert, int32_t k, int32_t* ids,
                             float* weights, void* hip_stream);

/* The router-margin diagnostic (metal/src/forward.cpp:441-513), for reading an expert-id mismatch: per token, the
 * k-th and (k+1)-th experts ranked by softmax probability (ties to the lower id), stats [T][4] = {p_k - p_k1 (the
 * margin, before renormalisation), logits[id_k] - logits[id_k1], p_k, p_k1}, ids [T][2] = {id_k, id_k1}.
 * 1 <= k < n_expert <= 1024. */
smoe_status smoe_router_margin(const float* logits, int32_t n_tokens, int32_t n_expert, int32_t k, float* stats,
                               int32_t* ids, void* hip_stream);

/* x [n] f32 -> bf16 bits, round to nearest even, NaN quieted.
 * Replaces f32_to_bf16_bulk (metal/include/strata/metal/elementwise.hpp:27). */
smoe_status smoe_f32_to_bf16(const float* x, int64_t n, uint16_t* y, void* hip_stream);

/* y[o] = sum_i f32(x[i]) * f32(w[o][i]) for n_tok rows of bf16 x; y is (n_tok, n_out).
 * Replaces bf16_gemv (metal/include/strata/metal/bf16_gemv.hpp:25). */
smoe_status smoe_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int32_t n_in, int32_t n_out,
                           int32_t n_tok, void* hip_stream);

/* x [n] f32 -> q8_1 blocks (n % 32 == 0).  Replaces iq_quantize_q8_1 (metal/include/strata/metal/iq.hpp:46). */
smoe_status smoe_quantize_q8_1(const float* x, int64_t n, uint8_t* y, void* hip_stream);

/* y[c * n_out + r] = W[r] . x[c] for n_col q8_1 columns; W is n_out rows of n_in values of `type`, the first
 * at `w + byte_off`.  Types: Q2_0, IQ2_S, and SMOE_Q8_0 .. SMOE_Q6_K (n_in a multiple of the type's block: 32 or
 * 256; w + byte_off 4-byte aligned).  Replaces iq_mmvq (metal/include/strata/metal/iq.hpp:50-51; its per-type
 * dots metal/shaders/iq.metal:224-513). */
smoe_status smoe_mmvq(int32_t type, const void* w, int64_t byte_off, const uint8_t* x_q8, int32_t n_in,
                      int32_t n_out, int32_t n_col, float* y, void* hip_stream);

/* y = q8_1(silu(gate) * up), n % 32 == 0.  Replaces iq_swiglu_q8 (metal/include/strata/metal/iq.hpp:54). */
smoe_status smoe_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y, void* hip_stream);

/* y = sum_{s<k} w[s] * parts[s] (+ shared), one token; k <= 64.
 * Replaces moe_combine (metal/include/strata/metal/moe_combine.hpp:15). */
smoe_status smoe_combine(const float* parts, const float* weights, const float* shared, float* y, int32_t n_embd,
                         int32_t k, void* hip_stream);

/* One expert's whole FFN on an assembled blob [gate rows | up rows | down rows] (each row n_embd values of
 * gu_type, resp. n_ff values of d_type): gate = W_g x, up = W_u x, hq = q8_1(silu(gate) * up), y = W_d hq for
 * n_tok q8_1 rows x_q8 of n_embd; y is (n_tok, n_embd) f32.  As the reference, the gate/up type must have
 * 256-value blocks (here IQ2_S; a 64-value type such as Q2_0 is a down quant and refused with SMOE_ETYPE),
 * n_ff % 32 == 0, and the blob must hold smoe_expert_bytes.  `scratch` (smoe_expert_scratch_bytes, 256-byte
 * aligned) holds gate, up and hq; nothing is allocated.
 * Replaces iq_expert / iq_expert_bytes (metal/include/strata/metal/iq.hpp:56-65, metal/src/iq.mm:171-199). */
size_t smoe_expert_bytes(int32_t gu_type, int32_t d_type, int64_t n_embd, int64_t n_ff); /* 0 when refused */
size_t smoe_expert_scratch_bytes(int64_t n_embd, int64_t n_ff, int64_t n_tok);
smoe_status smoe_expert(const void* blob, size_t blob_bytes, const uint8_t* x_q8, int32_t gu_type, int32_t d_type,
                        int64_t n_embd, int64_t n_ff, int64_t n_tok, float* y, void* scratch, size_t scratch_bytes,
                        void* hip_stream);

/* ids [n_tokens][k] -> counts [E], offsets [E+1], perm [T*k], slot [T*k]: the canonical stable dispatch
 * (ascending pair index within an expert).  Replaces prefill::fused::group
 * (include/strata/prefill/moe_fused.hpp:46-51) with a fixed in-expert order. */
smoe_status smoe_dispatch(const int32_t* ids, int32_t n_tokens, int32_t k, int32_t n_expert, int32_t* counts,
                          int32_t* offsets, int32_t* perm, int32_t* slot, void* hip_stream);

/* out[t] = RMSNorm(x[t] + r[t]) with unit weight for n_rows rows of n <= 4096 f32 (r may be NULL; out may
 * alias x): the layer junction of the stacked benchmark configuration, x_{l+1} = RMSNorm(x_l + MoE_l(x_l)),
 * eps 1e-6 there.  No counterpart in the reference's MoE block (its layer walk normalises in the
 * hyper-connection read, out of this block's scope); the row sum's order is fixed and restated by the test
 * oracle. */
smoe_status smoe_residual_rmsnorm(const float* x, const float* r, int32_t n_rows, int32_t n, float eps, float* out,
                                  void* hip_stream);

/* ---------------------------------------------------------------------------------------------- synthetic inputs
 * No counterpart in the reference: the seeded generators of the benchmark configurations (counter-based
 * SplitMix64; normals by Box-Muller).  Bitwise equal to the host generators of the test oracle. */
smoe_status smoe_synth_blocks(int32_t type, uint64_t seed, uint64_t stream_id, int64_t n_values, float sigma,
                              void* out, void* hip_stream);
smoe_status smoe_synth_bf16(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, uint16_t* out,
                            void* hip_stream);
smoe_status smoe_synth_normal(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, float* out,
                              void* hip_stream);

/* ---------------------------------------------------------------------------------------------- misc */
const char* smoe_status_str(smoe_status s);
/* Why the last call on this thread was refused ("" after a successful call).  Owned by the library. */
const char* smoe_last_error(void);
/* Version of this ABI (major * 100 + minor). */
int32_t smoe_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
