/* q27x.h -- C ABI of the MI355X (gfx950) chained-MTP speculative decode step.
 *
 * Two tiers, mirroring the reference engine's own boundary:
 *   kernel tier  : stream-ordered launchers on caller-owned device buffers (reference:
 *                  include/q27.h:208-477, include/q27_nr.h:6-79). They never allocate and never
 *                  synchronise. Return Q27X_OK or a negative Q27X_E_* (the reference returns 1/0
 *                  "ran / shape declined"; a declined shape here is Q27X_E_SHAPE, never a silent
 *                  fallback).
 *   engine tier  : a context that owns weights, KV cache, recurrent state and scratch, with the
 *                  reference's load / decode / speculative-round entry points (reference:
 *                  include/q27_load.h:146-243 for load, src/q27_main.cpp:1704 run_layer_tp for the
 *                  plain step, src/q27_main.cpp:2702 spec_round for the speculative round).
 *
 * Plain C types only: pointers, sizes, ints, floats. Streams are hipStream_t passed as void*.
 * bf16 values are uint16_t bit patterns (round-to-nearest-even, include/q27.h:133-139).
 * Threading: one context per host thread; launchers are stream-ordered; calls that share a
 * context or the module scratch of a launcher must not run concurrently on different streams
 * (the same contract as the reference, include/q27_nr.h + src/q27_elem.hip:218-220).
 */
#ifndef Q27X_H
#define Q27X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* q27x_stream_t; /* hipStream_t; NULL = the null stream */

/* ---- status codes (the reference loader's Q27_OK / Q27_E_*, include/q27_load.h:70-78) ---- */
#define Q27X_OK        0
#define Q27X_E_ARG    -1   /* null pointer, bad count, bad flag                  */
#define Q27X_E_SHAPE  -2   /* geometry this build has no kernel for              */
#define Q27X_E_HIP    -3   /* a HIP runtime call failed                          */
#define Q27X_E_NOMEM  -4   /* device or host allocation failed                   */
#define Q27X_E_STATE  -5   /* call out of order (no weights, no prefill, ...)   */
#define Q27X_E_RANGE  -6   /* position / context / row count out of range        */
#define Q27X_E_DEVICE -7   /* a kernel raised its device-side error flag         */
#define Q27X_E_IO     -8   /* checkpoint open / stat / mmap failed               */
#define Q27X_E_FORMAT -9   /* checkpoint header malformed or census mismatch     */
#define Q27X_E_MISSING -10 /* a tensor the plan needs is absent                  */

/* Last error message of the calling thread (never NULL). */
const char* q27x_last_error(void);
const char* q27x_version(void);

/* ======================================================================================
 * Device plumbing (no reference counterpart: the reference calls HIP directly). Lets tests and
 * benches drive the kernel tier without any framework.
 * ====================================================================================== */
int q27x_device_count(int* n);
int q27x_set_device(int dev);
int q27x_device_name(int dev, char* buf, int len);
int q27x_device_cus(int dev, int* n_cu);
int q27x_malloc(void** p, size_t bytes);
int q27x_free(void* p);
int q27x_host_malloc(void** p, size_t bytes);   /* pinned host memory */
int q27x_host_free(void* p);
int q27x_memcpy_h2d(void* dst, const void* src, size_t bytes, q27x_stream_t s);
int q27x_memcpy_d2h(void* dst, const void* src, size_t bytes, q27x_stream_t s);
int q27x_memcpy_d2d(void* dst, const void* src, size_t bytes, q27x_stream_t s);
int q27x_memset(void* p, int value, size_t bytes, q27x_stream_t s);
int q27x_stream_create(q27x_stream_t* s);
int q27x_stream_destroy(q27x_stream_t s);
int q27x_stream_sync(q27x_stream_t s);
int q27x_device_sync(void);
int q27x_event_create(void** e);
int q27x_event_destroy(void* e);
int q27x_event_record(void* e, q27x_stream_t s);
int q27x_event_elapsed_ms(void* start, void* stop, float* ms);

/* ======================================================================================
 * Kernel tier
 * ====================================================================================== */

/* INT8 per-64-group weight handle. Replaces q27_i8g_t (include/q27.h:158-163); same fields,
 * same meaning: w [rows][K] int8 natural K order, s [rows][K/64] fp32 group scales, alpha the
 * per-tensor multiplier applied once per output. */
typedef struct q27x_i8g {
    const int8_t* w;
    const float*  s;
    float alpha;
    int rows, K;
} q27x_i8g_t;

/* R5 activation quantizer, natural order, per-16 absmax (replaces q27_quant_fp8_b,
 * include/q27_nr.h:73-74; math at src/q27_fp8.hip:373-425):
 *   g = 1/in_scale; per 16: mx = max|x|; s = mx*g*(1/127); inv = s>0 ? g/s : 0;
 *   q = clamp(rint(x*inv), -127, 127); xs = s.
 * Row r of x starts at x + r*xstride (bf16 elements), of xq at xq + r*qstride, of xs at
 * xs + r*sstride. n % 16 == 0. */
int q27x_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs,
                    int sstride, int n, float in_scale, int nrows, q27x_stream_t s);

/* R8 weight mirror rule, per 64 (replaces q27_fp8_to_i8g64_conv, include/q27.h:397; math at
 * src/q27_nvfp4.hip:4259-4289): sc = mx*(1/127); inv = sc>0 ? 1/sc : 0; q = clamp(rint(v*inv)).
 * w fp32 [rows][K] -> wq int8 [rows][K] + ws fp32 [rows][K/64]. K % 64 == 0. */
int q27x_quant_weights_i8g64(const float* w, int rows, int K, int8_t* wq, float* ws,
                             q27x_stream_t s);

/* R7 W8A8 projection of nr rows (1..8) through one pass over the weights (replaces
 * q27_proj_i8g_rows via q27_df2_gemm, include/q27_nr.h:57-58, and the NR launchers
 * q27_proj_fp8_bf16_nr / q27_proj_fp8_res_nr, include/q27_nr.h:7-11; math at
 * src/q27_fp8.hip:3814-3871):
 *   y[n][r] = alpha * sum over 16-slabs s of (float)(int32 dot of the slab) * (ws64*xs16)
 *             (+ rs * res[n][r])
 * xq row n at xq + n*xstride, xs row n at xs + n*(xstride/16). out_bf16: 1 = bf16 (RNE) output,
 * 0 = fp32 output. res may be NULL; res_bf16 selects its element type (bf16 / fp32); row n of res
 * at res + n*rstride. K in {1024*k} or any K % 64 == 0 up to 20480. */
int q27x_proj_rows(const q27x_i8g_t* w, const int8_t* xq, int xstride, const float* xs,
                   void* y, int ystride, int out_bf16, const void* res, int res_bf16,
                   int rstride, float rs, int nr, q27x_stream_t s);

/* Debug export for the bit-exactness gate: the exact int32 dot of every 16-element slab,
 * part[n][r][slab] (slab = k/16), for nr rows. */
int q27x_proj_partials(const q27x_i8g_t* w, const int8_t* xq, int xstride, int32_t* part,
                       int nr, q27x_stream_t s);

/* ---- Prefill ingest GEMM on int8 MFMA (per-(row, group) scales) ----
 * The reference's layer-split prefill quantizes per K group of gs = 1024 columns (or the whole K)
 * and runs one rocBLAS int8 gemm_ex per group into int32 slabs, then sums the slabs in fp32
 * (src/q27_epi.hip:1-8). These three entry points are that data path on gfx950 MFMA. */

/* Weights, per-64 mirror -> per-(row, group) (replaces q27_i8g64_to_row_conv,
 * src/q27_epi.hip:36-47; math at 14-35): sg = max of the group's gs/64 per-64 scales;
 * inv = sg>0 ? 1/sg : 0; code = clamp(rint((w*s64)*inv), -127, 127). w, s64 [rows][K], [rows][K/64]
 * -> wg [rows][K], sg [rows][K/gs]; wg may be w (in place, as the reference). gs % 64 == 0, K % gs == 0. */
int q27x_i8g64_to_grp(const int8_t* w, const float* s64, int rows, int K, int gs, int8_t* wg,
                      float* sg, q27x_stream_t s);

/* Activations per (token, group) (the quantizer q27_quant_group, src/q27_epi.hip:64-75, that the
 * reference fuses into its prefill norms and requant kernels, src/q27_epi.hip:80-186), here on fp32
 * rows: sc = max|v|*(1/127); qi = sc>0 ? 1/sc : 0; code = clamp(rint(v*qi), -127, 127).
 * x [M] rows of xstride floats (16-byte aligned) -> xq [M][K], xs [M][K/gs]. K % gs == 0. */
int q27x_quant_tok_groups(const float* x, int xstride, int M, int K, int gs, int8_t* xq, float* xs,
                          q27x_stream_t s);

/* y[t][n] = alpha * sum over groups g (ascending) of fmaf((float)acc_g[t][n], sw[n][g]*sx[t][g], .)
 *           (+ rs * res[t][n]),  acc_g = the exact int32 dot of group g.
 * Replaces q27_rb_gemm_i8g (src/q27_rb.cpp:43-55) together with its fp32 slab epilogue
 * q27_epi_f32r (src/q27_epi.hip:189-203, 235-243, 257-262), without the int32 slabs in memory.
 * w [N][K] + sw [N][K/gs]; x [M][K] + sx [M][K/gs]; y rows of ldy floats; res may be NULL (rows of
 * ldr floats). Kernel geometry: N % 128 == 0, K % 64 == 0, gs % 64 == 0, K/gs <= 20, w and x
 * 16-byte aligned; any M >= 1. Other shapes return Q27X_E_SHAPE. */
int q27x_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha,
                  const int8_t* x, const float* sx, int M, float* y, int ldy, const float* res,
                  int ldr, float rs, q27x_stream_t s);

/* R9 / lm_head bf16 GEMV of nr rows (replaces q27_bf16_gemv2_tile, include/q27_nr.h:75-76):
 *   y[n][r] = sum_k bf16(W[r][k]) * bf16(x[n][k]) in fp32; out_bf16 selects bf16 / fp32 out.
 * K % 8 == 0. */
int q27x_bf16_gemv_rows(const uint16_t* w, int rows, int K, const uint16_t* x, int xstride,
                        void* y, int ystride, int out_bf16, int nr, q27x_stream_t s);

/* R22 + R5 RMSNorm + quantize of nr rows (replaces q27_rmsnorm_quant_fp8, include/q27.h:321-323,
 * and q27_rmsnorm_hostss_fp8_b, include/q27_nr.h:33-35; math at src/q27_elem.hip:453-613,
 * 835-910):
 *   inv = 1/sqrt(sum x^2 / n + eps); nrm = x*inv*(plus + w)
 *   hcopy = bf16(x) (optional), y = bf16(nrm) (optional), xq/xs = quantize(quant_bf16 ? y : nrm)
 * x is fp32 (x_bf16 = 0) or bf16 (x_bf16 = 1). n % 1024 == 0. */
int q27x_rmsnorm_quant_rows(const void* x, int x_bf16, int xstride, const uint16_t* w,
                            float plus, float eps, int n, uint16_t* hcopy, uint16_t* y,
                            int ystride, int8_t* xq, float* xs, int quant_bf16,
                            float in_scale, int nr, q27x_stream_t s);

/* R16 SwiGLU + per-16 quantize (replaces q27_swiglu_quant_b, include/q27_nr.h:71-72; math at
 * src/q27_nvfp4.hip:3984-4031, natural order):
 *   v = (g/(1+e^-g)) * u * (1/in_scale); per 16: s = mx/127; q = clamp(rint(v/s)). */
int q27x_swiglu_quant_rows(const float* gate, const float* up, int stride, int8_t* xq,
                           float* xs, int n, float in_scale, int nr, q27x_stream_t s);

/* R10 + R11 + R12 gated-delta-rule verify of nr rows for one layer (replaces
 * q27_gdn_conv_tp_tile2 + q27_gdn_scan_tp_snap + the snapshot-bank restore, include/q27_nr.h:
 * 77-83, src/q27_main.cpp:2933-2941; math at src/q27_gdn.hip:206-372, 411-592).
 * Deferred commit replaces the snapshot banks: the state S in HBM is the state after the last
 * COMMITTED position minus `npend` pending rows whose (k^, delta, decay) vectors and raw conv
 * inputs the previous call left in `pend`. The call first applies those npend rows (the exact
 * update the rows already received), writes the committed state back, then runs the nr new rows
 * and leaves their update vectors in `pend` for the next call. Rolling back to an accepted prefix
 * of a rows is therefore just calling again with npend = a.
 *   qkv_raw  [nr][nqkv] bf16  projection output before conv (q | k | v, nqkv = (2*KH+VH)*D)
 *   z        [nr][VH*D] bf16, a/b logits [nr][VH] fp32 (already a = in_proj_a.x, b = in_proj_b.x)
 *   A_log, dt_bias [VH] bf16; norm_w [D] bf16 (raw weight, no +1); conv_w [nqkv][4] bf16
 *   S [VH][D][D] fp32 key-major; conv_hist [nqkv][3] bf16 (oldest first)
 *   pend: opaque buffer of q27x_gdn_pend_bytes(KH, VH, D, 8) bytes
 *   out [nr][VH*D] bf16 gated-normed output, xq/xs its per-16 quantization (nullable). */
size_t q27x_gdn_pend_bytes(int kh, int vh, int d, int max_rows);
int q27x_gdn_verify(const uint16_t* qkv_raw, int qkv_stride, const uint16_t* z, int z_stride,
                    const float* a, const float* b, int ab_stride, const uint16_t* A_log,
                    const uint16_t* dt_bias, const uint16_t* norm_w, const uint16_t* conv_w,
                    float* S, uint16_t* conv_hist, void* pend, int npend, int kh, int vh,
                    int d, uint16_t* out, int out_stride, int8_t* xq, float* xs,
                    int nr, q27x_stream_t s);

/* R12 commit without new rows: apply the npend pending rows that the last q27x_gdn_verify call
 * left in `pend` (the accepted prefix) to S and conv_hist, leaving nothing pending (the next
 * q27x_gdn_verify passes npend = 0). Replaces the snapshot-bank restore of the reference's round
 * tail (src/q27_main.cpp:2933-2941) for callers that need the committed state materialised. */
int q27x_gdn_commit(float* S, uint16_t* conv_hist, void* pend, int npend, int kh, int vh, int d,
                    q27x_stream_t s);

/* R14 attention prep for nr consecutive positions pos0..pos0+nr-1 (replaces
 * q27_attn_prep_tp_nr, include/q27_nr.h:84-86; math at src/q27_attn.hip:156-253):
 * per head RMSNorm(1+w) over head_dim, rotate-half RoPE on the first rot dims using the
 * [pos][rot/2] cos/sin tables, q -> bf16 qh [nr][nq*hd]; K (normed, roped) and V (raw) ->
 * int8 KV cache [pos][nkv*hd] with fp32 per-`kv_group` scales [pos][nkv*hd/kv_group].
 * qkv row layout: q block (nq heads x (gate ? 2*hd : hd), query dims first) | k | v. */
int q27x_attn_prep_rows(const uint16_t* qkv, int qkv_stride, const uint16_t* q_norm_w,
                        const uint16_t* k_norm_w, const float* rope_cos, const float* rope_sin,
                        int rot, int8_t* kc, float* ks, int8_t* vc, float* vs, int kv_group,
                        uint16_t* qh, int nq, int nkv, int hd, int gate, float eps, int pos0,
                        int nr, q27x_stream_t s);

/* R15 causal GQA attention of nr verify rows over the int8 KV cache (replaces
 * q27_attn_decode_tp_nr, include/q27_nr.h:87-89; math at src/q27_attn.hip:258-463):
 * row r attends keys 0..pos0+r; fixed 64-key splits; out = bf16(softmax(q.k/sqrt(hd)) v *
 * sigmoid(gate)) [nr][nq*hd]; xq/xs its per-16 quantization (nullable). `work` is scratch of
 * q27x_attn_work_bytes(nq, hd, ctx, nr) bytes. */
size_t q27x_attn_work_bytes(int nq, int hd, int ctx, int nr);
int q27x_attn_rows(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride,
                   const int8_t* kc, const float* ks, const int8_t* vc, const float* vs,
                   int kv_group, int nq, int nkv, int hd, int gate, int pos0, int nr,
                   void* work, uint16_t* out, int8_t* xq, float* xs, q27x_stream_t s);

/* q27x_attn_rows without the `work` argument and without any allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The split partials live in one file-scope
 * device array of 32.5 MiB per GPU (held until the process ends), so nr x nq x ceil((pos0+nr)/64)
 * may be at most 65536 (e.g. 8 rows x 32 query heads at 16384 positions); larger calls return
 * Q27X_E_RANGE. Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race. Same kernels and the same bits as q27x_attn_rows. */
int q27x_attn_rows_noalloc(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride,
                           const int8_t* kc, const float* ks, const int8_t* vc, const float* vs,
                           int kv_group, int nq, int nkv, int hd, int gate, int pos0, int nr,
                           uint16_t* out, int8_t* xq, float* xs, q27x_stream_t s);

/* R18 argmax of nr rows of n logits: non-finite filtered, ties -> lowest index, all non-finite
 * -> index 0 / value -inf (replaces q27_argmax_val, include/q27.h:348; src/q27_elem.hip:216-322). */
int q27x_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val,
                     q27x_stream_t s);

/* R20 greedy acceptance on the device: nacc = longest prefix with nx[j] == dt[j] (j < k),
 * ncommit = nacc + 1, committed = nx[0..nacc] (src/q27_main.cpp:2811-2812, 2929-2932). */
int q27x_accept(const int32_t* nx, const int32_t* dt, int k, int32_t* nacc_ncommit,
                int32_t* committed, q27x_stream_t s);

/* Test hook: the device's elementwise math (exp, exp2, log1p, sigmoid, SiLU, softplus) on n
 * values, op = 0..5, so the bit-exact host restatement can be checked against it. */
int q27x_math_test(const float* x, float* y, int n, int op, q27x_stream_t s);

/* ======================================================================================
 * Engine tier: the reference's load / decode / speculative-round entry points
 * ====================================================================================== */

/* Model geometry and semantic switches. All dimensions are runtime values. */
typedef struct q27x_config {
    int hidden;          /* 5120 */
    int inter;           /* 17408 (SwiGLU intermediate) */
    int vocab;           /* 62080 (untied bf16 lm_head rows) */
    int n_layers;        /* 64 */
    int attn_period;     /* 4: layer L is full attention when L % attn_period == attn_period-1 */
    int gdn_kh, gdn_vh, gdn_d;      /* 16, 48, 128 */
    int n_q, n_kv, head_dim;        /* 32, 8, 128 */
    int attn_gate;       /* 1: q_proj emits an output gate per head (trunk semantics) */
    int rot_dims;        /* rotary dims of a head (32 = partial factor 0.25 of 128) */
    double rope_theta;   /* 1e7 */
    int kv_group;        /* 32: fp32 scale per 32 KV elements */
    float rms_eps;       /* 1e-6 */
    int head_double_residual; /* 1: final-norm input bf16(bf16(r1)+r2) as the reference */
    int mtp_swap;        /* Q27_MTP_SWAP (1, the reference default, src/q27_main.cpp:3367: the
                            embedding half first, src/q27_mtp_defs.h:94-95; 0: the hidden half first) */
    int mtp_plus_one;    /* Q27_MTP_PO (1) */
    int spec;            /* Q27_SPEC: 1 = speculative decode */
    int spec_k;          /* Q27_SPEC_K: drafts per round, [1, 7] */
    int ctx;             /* context capacity in positions */
    int pf_gs;           /* Q27_Q8_GS: K-group size of the prefill GEMM's per-(row, group) weight
                            and per-(token, group) activation scales: 0 = the whole K (the
                            reference default, src/q27_load.cpp:1622-1623, src/q27_main.cpp:4020),
                            or 1024. The MTP prompt pass always uses the whole K
                            (src/q27_main.cpp:2625-2628, 2665-2668). */
    int eos_id;          /* stop tokens of q27x_generate (q27_is_eos, src/q27_main.cpp:709-710, */
    int eos_id2;         /* applied as at 6680-6683): a request ends after the first committed
                            token equal to either; -1 = none. Defaults 248044 and -1; eos_id2 is
                            248046 when Q27_EOS_IM_END is set (src/q27_main.cpp:3111). The
                            single-step entries (q27x_spec_round, q27x_decode_step,
                            q27x_run_rounds) never stop on them. */
} q27x_config;

/* Statistics of a decode run (the reference's Q27_SPEC / Q27_SPEC_T lines,
 * src/q27_main.cpp:6725-6733). */
typedef struct q27x_stats {
    long long rounds;
    long long committed;
    long long accepted;        /* sum of nacc */
    long long acc_hist[9];     /* rounds with >= j accepted drafts, j = 0..8 */
    double decode_ms;          /* wall clock of the decode loop (no load, no prefill) */
    double prefill_ms;
    /* per-round phases summed over the rounds (Q27_SPEC_T, src/q27_main.cpp:6731-6733), from
     * device clock stamps: draft (round start to the last draft's argmax), verify layers (to the
     * head norm), head (final norm, lm_head, argmax), tail (acceptance, rollback, hand-off) */
    double draft_ms, verify_ms, head_ms, tail_ms;
} q27x_stats;

typedef struct q27x_ctx q27x_ctx;

/* The benchmark config-3 geometry (64 layers: 48 GDN + 16 attention). */
int q27x_config_default(q27x_config* c);
/* A tiny geometry with the same structure for CPU-checkable parity runs. */
int q27x_config_tiny(q27x_config* c);
/* Q27_SPEC (bool, default 1) / Q27_SPEC_K (int, default 1, clamped to [1,7]) with the reference's
 * fail-closed parsing (include/q27.h:189-206, src/q27_main.cpp:3360-3361): an unparseable value
 * prints FATAL and aborts. Host-only. */
int q27x_spec_config_from_env(q27x_config* c);

int q27x_ctx_create(int device, const q27x_config* c, q27x_ctx** out);
int q27x_ctx_destroy(q27x_ctx* ctx);
/* ---- checkpoint catalog (q27_open / q27_close / q27_host_ptr / q27_catalog_*,
 * include/q27_load.h:146-165; src/q27_load.cpp:428-494). Host only: nothing touches the GPU.
 * The shards model-XXXXX-of-NNNNN.safetensors (numbered from 0 or 1) are mapped read-only; every
 * tensor needs a known dtype, offsets inside its shard's payload, a byte count equal to its
 * shape's and a unique name, and the census (tensor count, payload bytes) must match: any
 * mismatch returns NULL with the reason in err (Q27X_E_IO / _FORMAT / _SHAPE). */
#define Q27X_CKPT_SHARDS         3              /* the reference checkpoint (include/q27_load.h:52-54) */
#define Q27X_CKPT_TENSORS        2194
#define Q27X_CKPT_PAYLOAD_BYTES  21921428072LL
#define Q27X_MAX_DIMS            8
enum {                                          /* dtype codes, include/q27_load.h:60-66 */
    Q27X_DT_UNKNOWN = 0,
    Q27X_DT_BF16, Q27X_DT_F16, Q27X_DT_F32, Q27X_DT_F64,
    Q27X_DT_F8_E4M3, Q27X_DT_F8_E5M2,
    Q27X_DT_U8, Q27X_DT_I8, Q27X_DT_U16, Q27X_DT_I16,
    Q27X_DT_U32, Q27X_DT_I32, Q27X_DT_U64, Q27X_DT_I64, Q27X_DT_BOOL
};
typedef struct q27x_ckpt q27x_ckpt;
/* the reference checkpoint's census (3 shards, 2194 tensors, 21,921,428,072 payload bytes) */
q27x_ckpt* q27x_ckpt_open(const char* dir, char* err, size_t errcap);
/* any other census; a negative expectation is not checked */
q27x_ckpt* q27x_ckpt_open_census(const char* dir, int nshards, long long expect_tensors,
                                 long long expect_bytes, char* err, size_t errcap);
void        q27x_ckpt_close(q27x_ckpt* ck);
int         q27x_ckpt_tensor_count(const q27x_ckpt* ck);
long long   q27x_ckpt_payload_bytes(const q27x_ckpt* ck);
/* host pointer into the mapping for a named tensor, or NULL; shape has room for Q27X_MAX_DIMS */
const void* q27x_ckpt_host_ptr(const q27x_ckpt* ck, const char* name, size_t* nbytes, int* dtype,
                               int* ndim, long long* shape);
const char* q27x_ckpt_name(const q27x_ckpt* ck, int i);
int         q27x_ckpt_info(const q27x_ckpt* ck, int i, int* shard, int* dtype, long long* offset,
                           size_t* nbytes, int* ndim, long long* shape);

/* Seeded random-init weights (replaces q27_open + q27_upload_*, include/q27_load.h:146-243,
 * for a synthetic checkpoint): int8 per-64 projections from N(0, 0.02) draws, bf16 lm_head,
 * embeddings, norms and GDN parameters; deterministic in (seed, tensor, index). */
int q27x_load_synthetic(q27x_ctx* ctx, uint64_t seed);
/* The checkpoint's tensors against this geometry's plan (names, dtypes, shapes, scales), host
 * only: Q27X_E_MISSING / Q27X_E_SHAPE with the first problem in err. */
int q27x_ckpt_check(const q27x_ckpt* ck, const q27x_config* cfg, char* err, size_t errcap);
/* Upload a checkpoint in the reference's naming and formats (replaces q27_upload_*,
 * include/q27_load.h:167-243; tensor plan src/q27_load.cpp:1139-1235, MTP head
 * src/q27_main.cpp:7134-7152): fp8 and NVFP4 matrices become int8 per 64 by the reference's
 * mirror rule (src/q27_nvfp4.hip:4166-4311) with alpha = input_scale x weight_scale applied per
 * output and each projection's input quantized with its input_scale; lm_head becomes bf16
 * (e2m1 x e4m3 x weight_scale_2); the bf16 MTP head is quantized per 64 from its values (alpha 1,
 * input_scale 1). Checks the plan first (q27x_ckpt_check); then resets the state. */
int q27x_load_checkpoint(q27x_ctx* ctx, const q27x_ckpt* ck, char* err, size_t errcap);
/* Bytes of weights resident on the device. */
int q27x_weight_bytes(q27x_ctx* ctx, size_t* bytes);
/* Reset positions, KV, recurrent state and speculation state (a new request). */
int q27x_reset(q27x_ctx* ctx);
/* Ingest a prompt (positions 0..n-1), produce the first decode token, and prompt-condition the
 * MTP layer (reference: prefill sweep + mtp_prompt_pass, src/q27_main.cpp:2649-2692, 5131-5136). */
int q27x_prefill(q27x_ctx* ctx, const int32_t* ids, int n, int32_t* first_token);
/* The same ingest on the layer-major GEMM path (the reference's Q27_LS_Q8 prefill graph,
 * ls_q8_layer, src/q27_main.cpp:4076-4316, and mtp_prompt_pass, 2647-2688): the prompt in chunks
 * of up to 2048 rows (Q27X_PF_CHUNK overrides), each chunk through every layer; every projection is
 * the int8 MFMA GEMM of per-(row, 1024) weights and per-(token, 1024) activations (whole-K groups
 * where 1024 does not divide K); norms, GDN conv / scan, attention, SwiGLU and residual adds keep
 * the decode path's arithmetic; the MTP prompt pass computes only the draft KV cache. Leaves the
 * state fully committed. Its results differ from q27x_prefill's by the quantization granularity. */
int q27x_prefill_gemm(q27x_ctx* ctx, const int32_t* ids, int n, int32_t* first_token);
/* One plain greedy step (Q27_SPEC=0 semantics): consumes the current token, returns the next. */
int q27x_decode_step(q27x_ctx* ctx, int32_t* out_token);
/* One chained-MTP speculative round (spec_round, src/q27_main.cpp:2702-2958): K drafts, an
 * NR = K+1 row verify, greedy acceptance, rollback and hand-off, all on the device. Returns the
 * committed tokens (ncommit = nacc+1 <= K+1). As in the reference's decode loop (6391), a round runs
 * only while pos + K < ctx; closer to the end of the context this call takes one plain step
 * (ncommit = 1), and at pos == ctx it returns Q27X_E_RANGE. */
int q27x_spec_round(q27x_ctx* ctx, int32_t* out_tokens, int* ncommit);
/* R2 MTP draft layer on its own (mtp_pass_nr, src/q27_main.cpp:2551-2618; single-row twin
 * mtp_draft_step 7346-7411): nr (1..8) rows of (hidden row, token) at draft positions
 * dpos0 .. dpos0+nr-1 of the MTP layer's own KV cache (written by the call): fc over
 * [norm(emb) | norm(h)], the full-attention decoder layer, and for head_row >= 0 mtp.norm + the
 * shared lm_head + argmax of that row. Device buffers: hrows [nr][hidden] bf16, toks [nr] int32;
 * res [nr][hidden] bf16 receives the layer's residual rows (nullable), token one int32 (nullable).
 * Ordered after prior work on stream s, and later work on s waits for it. Uses the context's
 * scratch: not concurrent with other calls on the same context. */
int q27x_mtp_draft(q27x_ctx* ctx, const uint16_t* hrows, const int32_t* toks, int nr, int dpos0,
                   int head_row, uint16_t* res, int32_t* token, q27x_stream_t s);
/* Forced-acceptance mode: drafts are taken from this token stream (the trunk's own greedy
 * continuation, positions after the prompt) instead of the MTP argmax; the draft and verify work
 * is unchanged. n = 0 switches it off. */
int q27x_set_forced_drafts(q27x_ctx* ctx, const int32_t* toks, int n);
/* Decode loop (src/q27_main.cpp:6382-6696): after q27x_prefill, generate until max_new tokens
 * are committed (including the first token from prefill) or the context is full. spec = 1 runs
 * speculative rounds (with the device-side graph and a one-round-lagged host mailbox) while
 * pos + K < ctx and plain steps after that (6391); spec = 0 plain steps. out receives the first
 * min(committed, max_new) tokens of the request (a round may commit past max_new; those tokens
 * are kept and a later call continues after them). */
int q27x_generate(q27x_ctx* ctx, int max_new, int spec, int32_t* out, int* n_out,
                  q27x_stats* st);
/* Exactly n speculative rounds (spec = 1) or plain steps (spec = 0) from the current state, launched
 * back to back; stats cover those n. */
int q27x_run_rounds(q27x_ctx* ctx, int n, int spec, q27x_stats* st);
/* Time of one verify pass (64 layers + head, nr rows) averaged over iters, device events. Clears
 * the stop flag a finished request leaves, so the kernels do their work. */
int q27x_bench_verify(q27x_ctx* ctx, int nr, int iters, float* ms_per_verify);
/* Time one projection launch of layer `layer` as the verify pass runs it (which: 0 in_qkv|in_z with
 * its input-norm prologue, 1 gate|up with its post-norm prologue and SwiGLU epilogue, 2 down +
 * residual, 3 out_proj + residual, 4 lm_head + argmax partials; 5 and 6 are 0 and 1 fed with
 * already-quantized rows, no prologue, for comparison) over iters launches with device
 * events on the context's stream, cycling through the layers so no launch finds its weights in the
 * Infinity Cache; reports ms per launch and its algorithmic bytes (weights + scales + input rows +
 * outputs). Overwrites the context's activation scratch and clears the stop flag. */
int q27x_bench_kernel(q27x_ctx* ctx, int layer, int which, int nr, int iters, float* ms, double* bytes);
/* Benchmark configs 1 and 2 on the engine's own kernels: the mixer half of one layer (attn = 0:
 * GDN -- in_qkv|in_z with the input-norm prologue, the GDN kernel, out_proj + residual; attn = 1:
 * q|k|v with the prologue, attention over positions 0..pos+nr-1, o_proj + residual) for nr rows at
 * position pos, averaged over iters launches that cycle through the layers of that kind; reports
 * ms per layer and its algorithmic bytes. Overwrites the recurrent state, the KV cache and the
 * activation scratch (prefill again before decoding). */
int q27x_bench_mixer(q27x_ctx* ctx, int attn, int pos, int nr, int iters, float* ms, double* bytes);
/* HBM calibration (no reference counterpart): a streaming read (mode 0) or plain copy (mode 1) of
 * `bytes` per launch, cycling through 1 GiB so no launch hits the 256 MB Infinity Cache; grid =
 * CUs x blocks_per_cu blocks of 256 threads, `unroll` (1, 2, 4, 8) 16-byte loads in flight per
 * thread. Reports ms per launch over iters launches (device events, null stream). Allocates and
 * frees its own buffers. */
int q27x_bench_stream(int mode, size_t bytes, int blocks_per_cu, int unroll, int iters, float* ms);
/* Raw access for tests: copy a device tensor of the context to the host by name. The name
 * "pf_allocs" instead gives (int32) the number of device allocations held for the prefill GEMM's
 * weight copies, which a weight reload releases. */
int q27x_debug_read(q27x_ctx* ctx, const char* name, int layer, void* dst, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* Q27X_H */
