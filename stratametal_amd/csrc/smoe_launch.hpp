// stratametal_amd/csrc/smoe_launch.hpp - host launchers of the MoE kernels (internal to libsmoe.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace smoe {

// Where the gate/up kernels of a traced call write the expert stages (smoe_trace's hq, egate, eup, sgu, shq; any
// may be NULL).  Row r < P of the pair rows is the routed pair at dispatch position r, row P + t the shared expert's
// token t (t < T).
struct StageOut {
    uint8_t* hq;     // [P][F/32] q8_1 blocks of h
    float* egate;    // [P][F] gate dots
    float* eup;      // [P][F] up dots
    float* sgu;      // [2][T][Fs]: the shared expert's gate dots, then its up dots
    uint8_t* shq;    // [T][Fs/32] q8_1 blocks of the shared expert's h
    int P, T;
    __host__ __device__ bool any() const { return hq || egate || eup || sgu || shq; }
};

bool gemv_shape_ok(int n_in);           // a row length the GEMV kernels tile (n_in % 128 == 0, <= 8 units per lane)
bool down_shapes_match(int F, int Fs);   // routed and shared down rows share one launch shape
size_t img_bytes(int64_t n_blocks);      // bytes of n_blocks q8_1 images

hipError_t launch_prep(const float* x, int64_t n, uint8_t* xq, uint16_t* xb, hipStream_t s);
hipError_t launch_router(const float* xf, const uint16_t* xb, const void* W, const uint16_t* w_inp,
                         const float* bias, int H, int E, int rows_total, int T, float* logits, int ld_logits, float* sg,
                         uint32_t* ximg, int tile_rows, int img_natural, hipStream_t s, const float* rprev = nullptr,
                         float eps = 0.0f, float* xout = nullptr, uint4* clear = nullptr, int clear_n16 = 0,
                         int w_f32 = 0);
// (tile_rows: many tokens, bf16 xb and W on the matrix cores (launch_router_mfma); img_natural: write ximg in the IQ2_S
// kernels' natural order; rprev: the fused stack junction, x = RMSNorm(xf + rprev) written to xout; clear: 16-byte
// units zeroed for the exchange of the k_q2_moe_small launch after it; w_f32: W is f32 (router_dtype 1), x from xf)
// the prefill path's router on the matrix cores (bf16 x and W; row E is w_inp, into sg): f32 sums in the MFMA's order
hipError_t launch_router_mfma(const uint16_t* xb, const uint16_t* W, const uint16_t* w_inp, const float* bias, int H,
                              int E, int rows_total, int T, float* logits, int ld_logits, float* sg, hipStream_t s);
hipError_t launch_topk(const float* logits, int ld_logits, int T, int E, int k, int32_t* ids, float* wts, hipStream_t s);
hipError_t launch_router_margin(const float* logits, int T, int E, int k, float* stats, int32_t* ids, hipStream_t s);
hipError_t launch_dispatch(const int32_t* ids, int P, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                           int32_t* slot, int32_t* elist, int32_t* n_list, int4* items, int max_items, int T, int k,
                           int has_shared, int chunk, int sh_chunk, hipStream_t s);
// the same dispatch in three launches for many pairs (chunk histograms, one scan, chunk ranks); `work` holds
// dispatch_work_bytes(P, E)
size_t dispatch_work_bytes(int64_t P, int E);
hipError_t launch_dispatch_multi(const int32_t* ids, int P, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                                 int32_t* slot, int32_t* elist, int32_t* n_list, int4* items, int max_items, int T,
                                 int k, int has_shared, int chunk, int sh_chunk, int32_t* work, hipStream_t s);
hipError_t launch_topk_dispatch(const float* logits, int T, int E, int k, int32_t* ids, float* wts, int32_t* counts,
                                int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                                int4* items, int max_items, int has_shared, int chunk, int sh_chunk, hipStream_t s);
int shared_items(int T);  // shared-expert work items for T tokens (GEMV path)
int gemv_shared_chunk();   // shared-expert tokens per GEMV work item
hipError_t launch_q2_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint32_t* ximg, const int4* items, const int32_t* perm, int k, int H, int F, int Fs,
                        int has_shared, int max_items, uint32_t* himg, int h_blocks, hipStream_t s,
                        const StageOut* so = nullptr, const uint64_t* eptr = nullptr);
hipError_t launch_q2_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                          const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                          hipStream_t s, const uint64_t* eptr = nullptr, const int32_t* dmap = nullptr);
// (so: the expert stages of a traced call.  eptr: the expert table of the grouped calls -- routed item e
// reads the blob at eptr[e], [gate rows | up rows | down rows], instead of the planes; dmap: routed column row
// first + c of the down kernels is written to Y row dmap[first + c])
// batches of at most 4 tokens: gate/up that routes the batch itself (no route kernel before it), and down rows
// with the combine (no combine kernel after it) when the batch's h images fit in LDS
hipError_t launch_q2_gu_route(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh,
                              const uint8_t* up_sh, const uint32_t* ximg, const float* logits, int T, int E, int k, int H,
                              int F, int Fs, int has_shared, int32_t* ids, float* wts, int32_t* counts,
                              int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                              int4* items, int max_items, uint32_t* himg, int h_blocks, hipStream_t s);
bool down_combine_ok(int T, int k, int h_blocks);
hipError_t launch_q2_down_combine(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                                  const float* sg, const int4* items, int n_items, int H, int F, int Fs,
                                  const int32_t* slot, const float* wts, int T, int k, int add_shared, float* y,
                                  hipStream_t s);
// the two above in one launch (k_q2_moe_small): gate/up work-groups hand their h images to down-and-combine
// work-groups through `xchg` (moe_small_xchg_bytes, cleared by the router launch before it)
bool moe_small_ok(int T, int k, int H, int F, int Fs, int has_shared, int h_blocks);
size_t moe_small_xchg_bytes(int T, int k, int max_items, int h_blocks);
hipError_t launch_q2_moe_small(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh,
                               const uint8_t* up_sh, const uint8_t* down_exps, const uint8_t* down_sh,
                               const uint32_t* ximg, const float* logits, const float* sg, int T, int E, int k, int H,
                               int F, int Fs, int has_shared, int32_t* ids, float* wts, int32_t* counts,
                               int32_t* offsets, int32_t* perm, int32_t* slot, int32_t* elist, int32_t* n_list,
                               int4* items, int max_items, int h_blocks, uint8_t* xchg, int add_shared, float* y,
                               int32_t* status, hipStream_t s);
int fused_status_words(int H);  // wait flags of k_q2_moe_small, one per down work-group
int wait_limit();                 // the bounded waits' poll limit (default_wait_limit(), or the host's switch)
void set_wait_limit(int limit);   // (below zero: every wait gives up at once)
int default_wait_limit();
hipError_t launch_residual_rmsnorm(const float* x, const float* r, int n_rows, int n, float eps, float* out,
                                   hipStream_t s);
// nt: Y is read and y written with streaming (nontemporal) accesses, for a Y larger than the caches
hipError_t launch_combine(const float* Y, const int32_t* slot, const float* wts, int k, int H, int P, int T,
                          int add_shared, float* y, hipStream_t s, int nt = 0);
hipError_t launch_combine_parts(const float* parts, const float* wts, const float* shared, int k, int n, float* y,
                                hipStream_t s);
hipError_t launch_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y, hipStream_t s);
// the other native GGUF types (smoe_native.hip): Q8_0 8, Q4_0 2, Q5_0 6, IQ4_NL 20, IQ4_XS 23, Q3_K 11, Q4_K 12,
// Q5_K 13, Q6_K 14; y[c * ldy + r], times sigmoid(sg[c]) when sg is given
bool native_type(int type);
int native_block_values(int type);
int64_t native_row_bytes(int type, int64_t n);  // -1: not native, or n not a whole number of blocks
hipError_t launch_mmvq_native(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y,
                              int ldy, const float* sg, hipStream_t s);
hipError_t launch_sigmoid_rows(float* y, int T, int n, const float* sg, hipStream_t s);  // y[t][.] *= sigmoid(sg[t])
hipError_t launch_add_rows(float* y, const float* r, int T, int n, hipStream_t s);       // y[t][.] += r[t][.]
hipError_t launch_q2_mmvq(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y, hipStream_t s);

// IQ2_S (decode contract)
bool iq2_shape_ok(int n_in);  // n_in = 256 nb, nb in {2, 4, 8}
hipError_t launch_iq2_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                         const uint32_t* ximg, const int4* items, const int32_t* perm, int k, int H, int F, int Fs,
                         int has_shared, int max_items, uint32_t* himg, int h_blocks, hipStream_t s,
                         const StageOut* so = nullptr, const uint64_t* eptr = nullptr);
hipError_t launch_iq2_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* himg, int h_blocks,
                           const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                           hipStream_t s, const uint64_t* eptr = nullptr, const int32_t* dmap = nullptr);
hipError_t launch_iq2_mmvq(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y, hipStream_t s);

// prefill contract (bf16 MFMA)
int mfma_chunk();                        // tokens per MFMA work item
size_t act_rec_bytes(int64_t n_rec);     // bytes of n_rec 64-value activation records
// flags (or NULL): one int32 per work-group, 1 when one of its values is beyond the fp16 operands (65520 or more);
// act_records_blocks(n_rec) words for k_act_records, n_rows for k_junction_records, (Fmax / 128) * max_items for
// k_mm_gu; launch_flags_mask folds them into the trace's overflow mask
hipError_t launch_junction_records(const float* x, const float* r, int n_rows, int n, float eps, float* out,
                                   uint32_t* rec, uint16_t* xb, hipStream_t s, int32_t* flags = nullptr);
int64_t act_records_blocks(int64_t n_rec);
hipError_t launch_act_records(const float* x, int64_t n_rec, uint32_t* rec, uint16_t* xb, hipStream_t s,
                              int32_t* flags = nullptr);  // xb: bf16 copy or NULL
hipError_t launch_mm_gu(const uint8_t* gate_exps, const uint8_t* up_exps, const uint8_t* gate_sh, const uint8_t* up_sh,
                        const uint32_t* xrec, int64_t n_xrec, const int4* items, const int32_t* perm, int k, int H,
                        int F, int Fs, int has_shared, int max_items, uint32_t* hrec, int h_rec, hipStream_t s,
                        int32_t* flags, int n_expert);  // n_expert: picks where the thin items run
// dst[i] = src[i] for n floats (trace copies)
hipError_t launch_copy_f32(const float* src, int64_t n, float* dst, hipStream_t s);
hipError_t launch_flags_mask(const int32_t* fx, int64_t nx, const int32_t* fh, int64_t nh, int32_t* out,
                             hipStream_t s, const int32_t* fw = nullptr, int64_t nw = 0);
hipError_t launch_mm_down(const uint8_t* down_exps, const uint8_t* down_sh, const uint32_t* hrec, int64_t n_hrec,
                          int h_rec, const float* sg, const int4* items, int H, int F, int Fs, int max_items, float* Y,
                          int nt, hipStream_t s);  // nt: streaming stores of Y

// the hyper-connection ends (smoe_hc.hip): gr_read (two launches; proj [T][hc_lr] and rs [T][hc] are scratch; with
// rprev, R = rprev + yprev * 2 sigmoid(injprev / hc) is formed and stored first) and gr_write
bool hc_shape_ok(int n, int hc, int hc_lr);
hipError_t launch_hc_read(float* R, const float* norm, const uint16_t* down, const uint16_t* up, const uint16_t* inj,
                          int n_tok, int n, int hc, int hc_lr, float eps, float* proj, float* rs, float* mixed,
                          float* inject, const float* rprev, const float* yprev, const float* injprev, hipStream_t s);
hipError_t launch_hc_write(const float* R, const float* y, const float* inject, int n_tok, int n, int hc, float* out,
                           hipStream_t s);

// the expert tier (smoe_cache.hip): routed entries grouped by a table of one blob pointer per expert (at most
// kMaxGroupExperts experts and kMaxGroupEntries entries), with the expert kernels' item table (group g = item g,
// then n_sh_items shared chunks) and the identity slots of the rows' combine when asked; caller-made lists checked
// into an item table; q8_1 blocks into activation images
constexpr int kMaxGroupExperts = 1024;
constexpr int kMaxGroupEntries = 4096;
hipError_t launch_expert_group(const int32_t* ids, int n, int kpt, int E, const uint64_t* eptr, uint64_t* grp_ptr,
                               int32_t* grp_start, int32_t* grp_expert, int32_t* ent_dst, int32_t* ent_tok,
                               int32_t* miss_dst, int32_t* counts, int4* items, int cap_groups, int n_sh_items, int P,
                               int T, int32_t* slot_id, hipStream_t s);
hipError_t launch_group_items(const uint64_t* grp_ptr, const int32_t* grp_start, const int32_t* ent_tok,
                              const int32_t* ent_dst, const int32_t* counts, int cap_groups, int cap_entries, int n_tok,
                              int n_rows, int4* items, int32_t* etok, int32_t* edst, hipStream_t s);
hipError_t launch_q8_images(const uint8_t* xq, int64_t n_blocks, int natural, uint32_t* img, hipStream_t s);
hipError_t launch_iota(int32_t* p, int n, hipStream_t s);

hipError_t launch_synth_blocks(int type, uint64_t seed, uint64_t stream_id, int64_t n_blocks, float sigma, uint8_t* out,
                               hipStream_t s);
hipError_t launch_synth_bf16(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, uint16_t* out, hipStream_t s);
hipError_t launch_synth_normal(uint64_t seed, uint64_t stream_id, int64_t n, float sigma, float* out, hipStream_t s);

}  // namespace smoe
