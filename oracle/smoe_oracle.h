/* oracle/smoe_oracle.h - CPU restatement of StrataMetal's quantized MoE block.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline.  The product path
 * (stratametal_amd, libsmoe.so) never links or calls it.
 *
 * Two families of functions live here:
 *   *_dev  : the arithmetic of the HIP kernels, in the kernels' own documented operation order, so a
 *            device result can be compared BITWISE.  Every order is stated next to the function.
 *   *_ref  : the reference's host references, in the reference's order (32-lane partial order,
 *            double sums), for the tolerance checks the reference itself makes (1e-5 / 1e-6 / 1e-3).
 *
 * Functions whose parity is pinned only by the device restatement and not by an independent
 * check are marked "parity unpinned" in their comment.  (None are at present; see tests/.)
 */
#ifndef SMOE_ORACLE_H
#define SMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- A1: fp16 / bf16 bit conversions (include/strata/kernels/f16_bits.hpp:37-101,
 *      include/strata/kernels/bf16_bits.hpp:37-59) */
uint16_t or_f16_from_f32(float f);
float or_f32_from_f16(uint16_t h);
uint16_t or_bf16_from_f32(float f);
float or_f32_from_bf16(uint16_t h);
void or_f16_from_f32_n(const float* x, int64_t n, uint16_t* y);
void or_f32_from_f16_n(const uint16_t* x, int64_t n, float* y);
void or_bf16_from_f32_n(const float* x, int64_t n, uint16_t* y);

/* ---- elementary functions written from the mathematics (no libm), shared contract with the device */
float or_expf(float x);
float or_logf(float x);
float or_cos2pi(float v);

/* ---- synthetic inputs: counter-based SplitMix64 (one 64-bit hash per index) */
uint64_t or_hash(uint64_t seed, uint64_t stream, uint64_t i);
float or_uniform(uint64_t seed, uint64_t stream, uint64_t i);      /* (0,1), 24-bit */
float or_normal(uint64_t seed, uint64_t stream, uint64_t i);       /* Box-Muller on indices 2i, 2i+1 */
void or_gen_normal(uint64_t seed, uint64_t stream, int64_t n, float sigma, float* out);
void or_gen_bf16(uint64_t seed, uint64_t stream, int64_t n, float sigma, uint16_t* out);
void or_gen_q2_0(uint64_t seed, uint64_t stream, int64_t n_blocks, float sigma, uint8_t* out);
void or_gen_iq2_s(uint64_t seed, uint64_t stream, int64_t n_blocks, float sigma, uint8_t* out);

/* ---- A2: Q2_0 block decode (include/strata/artifact/dequant.hpp:69-78) */
void or_dequant_q2_0(const uint8_t* blocks, int64_t n_blocks, float* out);

/* ---- A3: q8_1 quantizer (metal/shaders/iq.metal:597-627, metal/src/iq_parity.cpp:350-382) */
void or_quant_q8_1(const float* x, int64_t n, uint8_t* y);

/* ---- A4: Q2_0 x q8_1 row products */
/* device order: double-block lane parts, rows summed sequentially (see smoe_oracle.c) */
void or_q2_0_gemv_dev(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y);
/* reference order: metal/src/iq_parity.cpp:275-291 (32-lane partials + xor butterfly) */
void or_q2_0_gemv_ref(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y);
/* brute force: every weight decoded, int64-exact per half block, double sum */
void or_q2_0_gemv_exact(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, double* y);
/* trap variant for tests: the code without the -1 (metal/src/iq_parity.cpp:231-251) */
void or_q2_0_gemv_no_minus_one(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y);

/* ---- A8: IQ2_S x q8_1 */
void or_iq2s_grid(uint64_t* grid1024);
void or_iq2_s_gemv_dev(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y);
void or_iq2_s_gemv_ref(const uint8_t* w, const uint8_t* xq, int n_in, int n_out, float* y);

/* ---- A5: router GEMV and top-k */
void or_bf16_gemv_dev(const uint16_t* xb, const uint16_t* w, int n_in, int n_out, float* y);
void or_bf16_gemv_double(const uint16_t* xb, const uint16_t* w, int n_in, int n_out, float* y);
void or_f32_gemv_dev(const float* x, const float* w, int n_in, int n_out, float* y);
void or_f32_gemv_double(const float* x, const float* w, int n_in, int n_out, float* y);
void or_route_dev(const float* logits, int n_tok, int n_expert, int k, int32_t* ids, float* w);
int or_router_margin_dev(const float* logits, int n_tok, int n_expert, int k, float* stats, int32_t* ids);
void or_route_ref(const float* logits, int n_tok, int n_expert, int k, int32_t* ids, float* w);

/* ---- A6: SwiGLU + q8_1 requant */
void or_swiglu_q8(const float* gate, const float* up, int64_t n, uint8_t* y);
float or_silu_mul(float g, float u);
float or_sigmoid(float z);

/* ---- A9: combine */
void or_residual_rmsnorm_dev(const float* x, const float* r, int n_rows, int n, float eps, float* out);
void or_combine_dev(const float* parts, const float* w, const float* shared, int n_embd, int k, float* y);
void or_combine_double(const float* parts, const float* w, const float* shared, int n_embd, int k, float* y);

/* ---- the other native GGUF types (oracle/smoe_native.c): 8 Q8_0, 2 Q4_0, 6 Q5_0, 20 IQ4_NL, 23 IQ4_XS,
 * 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K */
int or_native_type(int type);
int64_t or_native_row_bytes(int type, int64_t n); /* -1: not a native type or n not a whole number of blocks */
int or_native_dequant(int type, const uint8_t* blocks, int64_t n_values, float* out);
float or_native_part(int type, const uint8_t* blk, const uint8_t* x0, int iqs);
int or_native_gemv(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y);
int or_native_gemv_double(int type, const uint8_t* w, const uint8_t* xq, int n_in, int n_out, int n_col, float* y);

/* ---- A10: canonical dispatch */
void or_dispatch(const int32_t* ids, int n_tok, int k, int n_expert, int32_t* counts, int32_t* offsets,
                 int32_t* perm, int32_t* slot);

/* ---- the expert tier (smoe_cache.c): the hit/miss split and grouping; one routed expert on a blob
 * [gate rows | up rows | down rows] under the decode contract */
int or_expert_group(const int32_t* ids, int n, int kpt, int n_expert, const uint8_t* resident, int32_t* grp_expert,
                    int32_t* grp_start, int32_t* ent_dst, int32_t* ent_tok, int32_t* miss_dst, int32_t* counts);
int or_expert_dev(int type, const uint8_t* blob, int H, int F, const uint8_t* xq, float* out);

/* ---- the whole block */
typedef struct {
    int32_t n_embd, n_ff, n_ff_shared, n_expert, top_k;
    int32_t w_type;  /* 42 = Q2_0, 22 = IQ2_S (routed experts) */
    int32_t sh_type; /* 42 / 22, or -1 = no shared expert */
    int32_t router_dtype;
    /* the shared expert's projections in their own native types (0: sh_type); any type other than the routed one
     * makes the shared expert a native one, run on the q8_1 GEMV contract of smoe_native.c in both paths */
    int32_t sh_gate_type, sh_up_type, sh_down_type;
} or_geom;

typedef struct {
    const uint8_t *gate_exps, *up_exps, *down_exps;
    const uint16_t* router; /* [E][H] bf16, or f32 when router_dtype is 1 */
    const uint8_t *gate_sh, *up_sh, *down_sh;
    const uint16_t* gate_inp_sh;
    const float* logit_bias;
} or_weights;

/* Optional per-stage outputs (NULL to skip): logits [T][E], ids/weights [T][k], counts [E], offsets [E+1],
 * perm/slot [T*k], xq [T][H/32*36], hq [T*k][FF/32*36] by slot, parts [T*k][H] by slot, shared [T][H],
 * sgate [T] (the shared gate's dot, before the sigmoid). */
typedef struct {
    float* logits;
    int32_t* ids;
    float* weights;
    int32_t *counts, *offsets, *perm, *slot;
    uint8_t* xq;
    uint8_t* hq;
    float* parts;
    float* shared;
    float* sgate;
} or_trace;

/* Decode contract (q8_1 activations), device order.  n_threads <= 0 uses one thread. */
int or_moe_decode_dev(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                      const or_trace* tr, int n_threads);
/* Decode contract in the reference's host order (FfnExec::run chain with the parity files' host refs). */
int or_moe_decode_ref(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                      int n_threads);
/* Prefill contract (bf16 activations, exact per-block weight scale), double accumulation. */
int or_moe_prefill(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                   const or_trace* tr, int n_threads);
/* The same with the router's logits [T][E] (bias included) and the shared gate dots [T] given (NULL: computed). */
int or_moe_prefill_logits(const or_geom* g, const or_weights* w, const float* x, int n_tok, const float* logits,
                          const float* sgate, float* y, int add_shared, const or_trace* tr, int n_threads);

/* The decode contract again, bitwise equal to or_moe_decode_dev, organised as the reference CPU path's pool
 * (flat (expert, row-range) job batches, each weight row decoded once for all of its expert's tokens): the timed
 * CPU baseline (oracle/smoe_cpu_pool.c).  n_threads <= 0 keeps the OpenMP default. */
int or_moe_decode_pool(const or_geom* g, const or_weights* w, const float* x, int n_tok, float* y, int add_shared,
                       int n_threads);

/* The hyper-connection ends (gr_read / gr_write, one token each; R is [n_tok][hc][n]).  `inject` may be NULL. */
int or_hc_read_dev(const float* R, int n_tok, int n, int hc, int hc_lr, float eps, const float* norm,
                   const uint16_t* down, const uint16_t* up, const uint16_t* inj, float* mixed, float* inject);
int or_hc_read_ref(const float* R, int n_tok, int n, int hc, int hc_lr, float eps, const float* norm,
                   const uint16_t* down, const uint16_t* up, const uint16_t* inj, int round_act, float* mixed,
                   float* inject);
void or_hc_write_dev(const float* R, const float* y, const float* inject, int n_tok, int n, int hc, float* out);

/* Byte sizes */
int64_t or_row_bytes(int type, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
