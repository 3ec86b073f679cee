/* q27o.h -- CPU oracle for the chained-MTP verify path. TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference engine's arithmetic for the speculative verify step
 * (bespokeontology/qwen3.8-27b-mi50-cpp-engine; citations are file:line into that tree). It is
 * the checker the GPU path is compared against, and the CPU baseline's integer loop. Nothing in
 * the product links, loads or calls it: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg do.
 *
 * Fixed reduction orders. Every floating-point sum is restated in one fixed order so that the
 * GPU kernels (which use the same order) match bit for bit:
 *   lane-slab order (W8A8 projection, src/q27_fp8.hip:3826-3861): slab s of 16 elements belongs
 *     to lane s%64 at step s/64; each lane accumulates its slabs in ascending step order with
 *     fmaf((float)dot, ws*xs, acc); the 64 lane sums are combined by the shfl_down tree
 *     (offsets 32,16,8,4,2,1).
 *   bf16 GEMV: the same with chunks of 8 bf16 (lane c%64, step c/64), fmaf per element.
 *   row sum of squares (hidden rows, n % 1024 == 0): thread t of 256 accumulates elements
 *     1024i + 4t + e; four wave trees; ((w0 + w1) + w2) + w3.
 *   head sums (128 dims): tree(elements 0..63) + tree(elements 64..127).
 * Transcendentals (exp, exp2, log1p) are the portable routines below (range reduction + fixed
 * polynomial, basic IEEE operations only), used identically on the device, so that greedy token
 * sequences are reproducible bit for bit. Their accuracy against libm is pinned by tests.
 *
 * parity pinning: see tests/test_oracle_*.py (closed forms, fp64 brute force, invariants). The
 * MTP draft layer's composition (src/q27_main.cpp:2551-2618: fc halves, the decoder layer on its
 * own KV cache, the four bf16-rounded down slices, mtp.norm + lm_head) is pinned against a float64
 * forward written from its definition, with planted composition mistakes shown to fail
 * (tests/test_oracle_mtp.py); the draft hand-off by spec == plain greedy under forced drafts with
 * planted wrong tokens (tests/test_oracle_model.py). The trunk's composition (verify(); the
 * reference's run_layer_tp_nr, src/q27_main.cpp:2271-2489, head 2457-2481: input norm, mixer,
 * out_proj / o_proj + residual, post norm from the fp32 r1, MLP + residual on bf16(r1), the head's
 * bf16(bf16(r1) + r2), final norm, lm_head) is pinned against float64 forwards written from its
 * definition: the ideal forward end to end within the quantization error, and a storage-faithful
 * forward stage by stage from the oracle's own traced inputs (r1, the post-norm codes, r2, the
 * final residual bits, the logits); planted composition and storage-point mistakes fail both
 * (tests/test_oracle_trunk.py).
 */
#ifndef Q27O_H
#define Q27O_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---- */
uint16_t q27o_f2bf(float f);            /* RNE, include/q27.h:136-139 */
float    q27o_bf2f(uint16_t b);         /* include/q27.h:133-135 */
float    q27o_exp(float x);
float    q27o_exp2(float x);
float    q27o_log1p(float x);
float    q27o_sigmoid(float x);          /* 1/(1+e^-x), src/q27_gdn.hip:114-116 */
float    q27o_silu(float x);             /* x/(1+e^-x), src/q27_gdn.hip:117-119 */
float    q27o_softplus(float x);         /* x > 20 ? x : log1p(e^x), src/q27_gdn.hip:317 */
void     q27o_math_vec(const float* x, float* y, int n, int op);

/* ---- seeded synthetic generator (shared definition with the device generator) ---- */
uint64_t q27o_hash(uint64_t seed, uint64_t tensor, uint64_t idx);
float    q27o_normal(uint64_t seed, uint64_t tensor, uint64_t idx);   /* ~N(0,1), Irwin-Hall(4) */
float    q27o_uniform(uint64_t seed, uint64_t tensor, uint64_t idx);  /* [0,1), 24-bit */

/* ---- R5 / R8 / R16 quantizers ---- */
void q27o_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs,
                     int sstride, int n, float in_scale, int nrows);
void q27o_quant_f32(const float* v, int n, int group, int8_t* q, float* s);
void q27o_quant_weights_i8g64(const float* w, int rows, int K, int8_t* wq, float* ws);
void q27o_swiglu_quant_rows(const float* gate, const float* up, int stride, int8_t* xq,
                            float* xs, int n, float in_scale, int nr);

/* ---- R7 projection (pre-epilogue value acc*alpha) and its int32 slab partials ---- */
void q27o_proj_rows(const int8_t* W, const float* WS, float alpha, int rows, int K,
                    const int8_t* xq, int xstride, const float* xs, float* y, int ystride,
                    int nr);
void q27o_proj_partials(const int8_t* W, int rows, int K, const int8_t* xq, int xstride,
                        int32_t* part, int nr);
/* the kernel-tier epilogue of q27x_proj_rows */
void q27o_proj_rows_epi(const int8_t* W, const float* WS, float alpha, int rows, int K,
                        const int8_t* xq, int xstride, const float* xs, void* y, int ystride,
                        int out_bf16, const void* res, int res_bf16, int rstride, float rs,
                        int nr);

/* ---- bf16 GEMV (R9, lm_head) ---- */
void q27o_bf16_gemv_rows(const uint16_t* W, int rows, int K, const uint16_t* x, int xstride,
                         float* y, int ystride, int nr);

/* ---- R22 norms ---- */
float q27o_rowsumsq(const float* x, int n);
float q27o_headsum(const float* a, const float* b, int n);  /* sum a*b over n (n%64==0) */
void  q27o_rmsnorm_quant_rows(const void* x, int x_bf16, int xstride, const uint16_t* w,
                              float plus, float eps, int n, uint16_t* hcopy, uint16_t* y,
                              int ystride, int8_t* xq, float* xs, int quant_bf16,
                              float in_scale, int nr);

void  q27o_rmsnorm_f32_rows(const void* x, int x_bf16, int xstride, const uint16_t* w, float plus,
                            float eps, int n, uint16_t* hcopy, uint16_t* y, int ystride, float* yf,
                            int yfstride, int round_bf16, int nr);

void  q27o_quant_tok_groups_g(const float* x, int xstride, int M, int K, int gs, float g, int8_t* xq,
                              float* xs);

/* ---- checkpoint formats (src/q27_nvfp4.hip:4166-4311; include/q27.h:95-114) ---- */
float q27o_e4m3(uint8_t b);
void  q27o_fp8_to_i8g64(const uint8_t* f8, int rows, int K, int ld, int8_t* w8, float* s64);
void  q27o_nvfp4_to_i8g64(const uint8_t* w, const uint8_t* gs, int rows, int K, int8_t* w8, float* s64);
void  q27o_nvfp4_to_bf16(const uint8_t* w, const uint8_t* gs, float ws2, int rows, int K, uint16_t* out);
void  q27o_bf16_to_i8g64(const uint16_t* x, int rows, int K, int ld, int8_t* w8, float* s64);

/* ---- R10/R11/R12 GDN verify with deferred commit ---- */
size_t q27o_gdn_pend_bytes(int kh, int vh, int d, int max_rows);
void q27o_gdn_verify(const uint16_t* qkv_raw, int qkv_stride, const uint16_t* z, int z_stride,
                     const float* a, const float* b, int ab_stride, const uint16_t* A_log,
                     const uint16_t* dt_bias, const uint16_t* norm_w, const uint16_t* conv_w,
                     float* S, uint16_t* conv_hist, void* pend, int npend, int kh, int vh,
                     int d, float eps, uint16_t* out, int out_stride, int8_t* xq, float* xs,
                     int nr);

/* ---- R14/R15 attention ---- */
void q27o_rope_table(int ctx, int rot, double theta, float* cosv, float* sinv);
void q27o_attn_prep_rows(const uint16_t* qkv, int qkv_stride, const uint16_t* q_norm_w,
                         const uint16_t* k_norm_w, const float* rope_cos,
                         const float* rope_sin, int rot, int8_t* kc, float* ks, int8_t* vc,
                         float* vs, int kv_group, uint16_t* qh, int nq, int nkv, int hd,
                         int gate, float eps, int pos0, int nr);
void q27o_attn_rows(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride,
                    const int8_t* kc, const float* ks, const int8_t* vc, const float* vs,
                    int kv_group, int nq, int nkv, int hd, int gate, int pos0, int nr,
                    uint16_t* out, int8_t* xq, float* xs);

/* ---- prefill GEMM, per-(row, group) int8 (src/q27_rb.cpp:43-55, src/q27_epi.hip:14-75, 189-243) ---- */
void q27o_i8g64_to_grp(const int8_t* w, const float* s64, int rows, int K, int gs, int8_t* wg, float* sg);
void q27o_quant_tok_groups(const float* x, int xstride, int M, int K, int gs, int8_t* xq, float* xs);
void q27o_gemm_i8g_partials(const int8_t* w, int N, int K, int gs, const int8_t* x, int M, int32_t* part);
void q27o_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                   const float* sx, int M, float* y, int ldy, const float* res, int ldr, float rs);

/* ---- R18 / R20 ---- */
void q27o_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val);
int  q27o_accept(const int32_t* nx, const int32_t* dt, int k, int32_t* committed);

/* ---- whole model (R1-R4, R17-R21) ---- */
typedef struct q27o_cfg {
    int hidden, inter, vocab, n_layers, attn_period;
    int gdn_kh, gdn_vh, gdn_d;
    int n_q, n_kv, head_dim, attn_gate, rot_dims;
    double rope_theta;
    int kv_group;
    float rms_eps;
    int head_double_residual, mtp_swap, mtp_plus_one;
    int spec_k, ctx;
    int pf_gs;           /* prefill GEMM K-group: 0 = the whole K, or 1024 (the reference's Q27_Q8_GS) */
} q27o_cfg;

typedef struct q27o_model q27o_model;
q27o_model* q27o_model_create(const q27o_cfg* c, uint64_t seed);   /* generates the weights */
void q27o_model_destroy(q27o_model* m);
void q27o_model_reset(q27o_model* m);
int  q27o_model_prefill(q27o_model* m, const int32_t* ids, int n);          /* returns token */
int  q27o_model_decode_step(q27o_model* m);                                 /* returns token */
int  q27o_model_spec_round(q27o_model* m, int32_t* out, const int32_t* forced); /* ncommit */
int  q27o_model_verify_rows(q27o_model* m, int nr, const int32_t* toks, int32_t* nx);
int  q27o_model_set_pos(q27o_model* m, int pos);   /* benchmark set-up: next verify at pos */
int  q27o_model_verify_logits(q27o_model* m, int nr, const int32_t* toks, int32_t* nx, float* logits, int advance);
/* The same pass recording, per layer, r1 and r2 (fp32 [n_layers][nr][H]) and the post norm's codes
 * and per-16 scales ([n_layers][nr][H], [n_layers][nr][H/16]); any of them may be NULL. */
int  q27o_model_verify_trace(q27o_model* m, int nr, const int32_t* toks, int32_t* nx, float* logits, int advance,
                             float* r1, float* r2, int8_t* pq, float* ps);
/* Layer-major prefill on the GEMM representation (chunks of `chunk` tokens): every projection as
 * the per-(row, group) x per-(token, group) int8 GEMM (group 1024, or the whole K when 1024 does
 * not divide it), everything else in the decode path's arithmetic; the MTP prompt pass computes
 * only the draft KV cache (fc, input norm, k|v). Leaves the state fully committed; returns the
 * first generated token. */
int  q27o_model_prefill_gemm(q27o_model* m, const int32_t* ids, int n, int chunk);
void q27o_debug_plant(int code);   /* tests only: plants a prefill composition mistake */
/* A layer's checkpoint scales (all 1 after create): v = { alpha of q|in_qkv, k|in_z, v, o|out_proj,
 * gate, up, down; input_scale of the input norm, post norm, SwiGLU output, mixer output } */
void q27o_model_set_scales(q27o_model* m, int layer, const float* v);
/* one MTP pass (mtp_pass_nr, src/q27_main.cpp:2551-2618) over nr rows at draft positions dpos0..;
 * res [nr][H] bf16 out, logits [vocab] of head_row (may be NULL); returns the head row's argmax */
int  q27o_model_mtp_pass(q27o_model* m, int nr, const uint16_t* hrows, const int32_t* toks, int dpos0,
                         int head_row, uint16_t* res, float* logits);
double q27o_model_weight_bytes(const q27o_model* m);
/* access to named tensors / buffers for the tests */
void* q27o_model_tensor(q27o_model* m, const char* name, int layer, size_t* bytes);

#ifdef __cplusplus
}
#endif
#endif
