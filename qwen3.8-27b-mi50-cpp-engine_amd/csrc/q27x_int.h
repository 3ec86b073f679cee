// q27x_int.h -- internal launcher interface between the kernel files and the engine.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/q27x.h"

namespace q27x {

// thread-local error text behind q27x_last_error()
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
#define Q27X_HIP(call)                                                   \
    do {                                                                 \
        hipError_t e_ = (call);                                          \
        if (e_ != hipSuccess) return ::q27x::hip_fail(e_, #call);        \
    } while (0)

constexpr int kMaxRows = 8;      // verify rows (K <= 7) and prefill chunk
constexpr int kSplit = 64;       // attention keys per split (fixed: results independent of NR)

// ---------------------------------------------------------------- norms
struct NormArgs {
    const void* x; int x_bf16; int xstride;      // input rows
    const uint16_t* emb; const int* tok;          // embedding mode: x = emb[tok[r]]
    const uint16_t* hadd;                         // head mode: x = bf16(bf16(hadd) + x) (fp32 x)
    uint16_t* hout;                               // head mode: writes the combined bf16 rows
    const uint16_t* w; float plus; float eps; int n;
    uint16_t* hcopy;                              // bf16(x)
    uint16_t* y; int ystride;                     // bf16 normed
    int8_t* xq; float* xs; int quant_bf16; float in_scale;
    const int* stop;
    const int* row_sel;                           // optional: process only row *row_sel (into row 0)
    unsigned long long* stamp;                    // optional: block 0 stores the wall clock at its start
    float* yf; int yfstride;                      // optional: the values xq would quantize, as fp32
};
// ---------------------------------------------------------------- projection
enum ProjEpi { EPI_STORE = 0, EPI_SWIGLU = 2, EPI_CONV = 3 };
// Per-output scale of a stacked matrix (the reference's alpha = input_scale x weight_scale, applied
// once per output, one per source tensor): rows [0, split_b) take alpha, [split_b, split_c) alpha_b,
// [split_c, rows) alpha_c (a split <= 0 is absent); alpha_gu: the SwiGLU layout of 32-row units,
// gate rows (row & 16 == 0) alpha, up rows alpha_b.
struct AlphaSel {
    float alpha_b, alpha_c; int split_b, split_c, alpha_gu;
};
__host__ __device__ inline float alpha_of(float alpha, const AlphaSel& s, int row) {
    if (s.alpha_gu) return (row & 16) ? s.alpha_b : alpha;
    float a = alpha;
    if (s.split_b > 0 && row >= s.split_b) a = s.alpha_b;
    if (s.split_c > 0 && row >= s.split_c) a = s.alpha_c;
    return a;
}
struct ProjArgs {
    const int8_t* W; const float* WS; int rows; int K; float alpha; AlphaSel asel;
    const int8_t* xq; int xst; const float* xs;
    // EPI_STORE: y = v (+ rs*res); res_round rounds v through bf16 before the add
    void* y; int ystride; int out_bf16;
    const void* res; int res_bf16; int rstride; float rs; int res_round;
    // EPI_SWIGLU: the weight rows interleave 16 gate rows and 16 up rows per block of 32.
    // sw_part / sw_cnt: scratch for units split over blocks (kSwMaxSplit units of 16 x kMaxRows
    // floats, kSwMaxSplit counters that start at zero and are left at zero)
    int8_t* act_q; float* act_s; int act_stride; float gscale;
    float* sw_part; unsigned* sw_cnt;
    // EPI_CONV (the GDN in_qkv|in_z projection, bf16 out): rows < nconv are the q|k|v channels,
    // each convolved by the wave that computes it -- causal depthwise conv of 4 taps over
    // (committed history, the call's rows), SiLU, bf16 -- with the history's deferred commit:
    // conv_st[row] is a 16 x bf16 record (committed history h0 h1 h2, pad, the last call's raw
    // inputs r0..r7, pad); the first *npend_ptr of those are committed before the call's rows.
    // Rows >= nconv are stored as EPI_STORE.
    const uint16_t* conv_w; uint16_t* conv_st; int nconv; const int* npend_ptr;
    // EPI_CONV also prepares the GDN row scalars: wave 0 of block b < 2 ab_vh takes, before its
    // rows, the bf16 dot product of weight row b/2 of in_a (b even) or in_b (b odd) with each bf16
    // normalized input row (lane-chunk order of the bf16 GEMV), rounds it to bf16 and stores
    // decay = exp(-exp(A_log) softplus(a + dt_bias)) or beta = sigmoid(b) into
    // ab_out [2][kMaxRows][ab_vh] (decay rows, then beta rows). ab_vh = 0: none.
    const uint16_t* in_a; const uint16_t* in_b; const uint16_t* A_log; const uint16_t* dt_bias;
    int ab_vh; float* ab_out;
    const int* stop;             // early exit when *stop != 0
    // norm prologue: instead of xq/xs, every block stages the RMSNorm + quantize of the raw rows
    // described by `pre` (K = pre.n); block 0 also writes pre's side outputs (hcopy, y, xq/xs)
    int has_pre; NormArgs pre;
};
constexpr int kSwMaxSplit = 256;
int launch_proj(const ProjArgs& a, int epi, int nr, hipStream_t s);
// The MTP layer's down as four column slices of K4 = K/4 (W[j], WS[j]: [rows][K4] codes and
// per-64 scales), each slice's projection times alpha[j] added into the bf16 rows y in slice order
// with its own bf16 rounding; xq/xs: the rows' codes and per-16 scales for the whole K (stride xst).
struct Down4Args {
    const int8_t* W[4]; const float* WS[4]; float alpha[4];
    int rows; int K4;
    const int8_t* xq; int xst; const float* xs;
    uint16_t* y; int ystride;
    const int* stop;
};
bool down4_supported(int K4, int nr);
int launch_down4(const Down4Args& a, int nr, hipStream_t s);
// whether the projection kernels have an instance for a plain (stored, no norm prologue) K
bool proj_k_supported(int K);

// bf16 GEMV: y = W x (fp32 / bf16 out) or, argmax mode, per-block (val, idx) partials
struct GemvArgs {
    const uint16_t* W; int rows; int K;
    const uint16_t* x; int xst;
    void* y; int ystride; int out_bf16;
    float* pval; uint32_t* pidx; int pstride;   // argmax partials [n][pstride]
    const int* stop;
};
int launch_gemv(const GemvArgs& a, int argmax_mode, int nr, int* nblocks_out, hipStream_t s);
int launch_argmax_final(const float* pval, const uint32_t* pidx, int pstride, int nblocks,
                        int nr, int32_t* idx, float* val, const int* stop, hipStream_t s);
int argmax_scratch(float** pv, uint32_t** pi);
int launch_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val,
                       float* pval, uint32_t* pidx, hipStream_t s);

int launch_norm(const NormArgs& a, int nr, hipStream_t s);
int launch_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs,
                      int sstride, int n, float in_scale, int nrows, hipStream_t s);
int launch_swiglu(const float* g, const float* u, int stride, int8_t* xq, float* xs, int n,
                  float in_scale, int nr, hipStream_t s);

// ---------------------------------------------------------------- GDN
struct GdnArgs {
    const uint16_t* qkv; int qkv_stride;          // convolved q|k|v rows (bf16)
    const uint16_t* z; int z_stride;
    const float* rowsc;                            // prepared row scalars [2][kMaxRows][vh]: decay, beta; or
    const float* a; const float* b; int ab_stride; // the a/b logits (fp32) with A_log and dt_bias
    const uint16_t* A_log; const uint16_t* dt_bias; const uint16_t* norm_w;
    float* S; void* pend; const int* npend_ptr; int npend_imm;
    int kh, vh, d; float eps;
    uint16_t* out; int out_stride; int8_t* xq; float* xs;
    const int* stop;
    float in_scale;                                // the quantized output's input_scale (0 = 1)
};
int launch_gdn(const GdnArgs& a, int nr, hipStream_t s);
// prefill: nrows rows (any count) with the row scalars prepared in rowsc [2][nrows][vh], the state
// committed through the last row, bf16 output only; scratch: qk [nrows][kh][256] and kq
// [nrows][kh] (the rows' normed q^|k^ and k^.q^), mix [nrows][vh*128], all fp32
int launch_gdn_scan(const GdnArgs& a, int nrows, float* qk, float* kq, float* mix, hipStream_t s);
int gdn_set_lds_limit();
// conv + SiLU with deferred commit as a standalone kernel (kernel-tier entry)
int launch_gdn_conv(const uint16_t* raw, int raw_stride, uint16_t* out, int out_stride,
                    int nconv, const uint16_t* conv_w, uint16_t* conv_hist, uint16_t* pend_raw,
                    const int* npend_ptr, int npend_imm, int nr, hipStream_t s);
size_t gdn_pend_bytes(int kh, int vh, int d);
size_t gdn_pend_raw_offset(int kh, int vh, int d);

// ---------------------------------------------------------------- attention
struct AttnArgs {
    const uint16_t* qkv; int qkv_stride;          // projection rows q(+gate) | k | v
    const uint16_t* q_norm_w; const uint16_t* k_norm_w;
    const float* rope_cos; const float* rope_sin; int rot;
    int8_t* kc; float* ks; int8_t* vc; float* vs; int kv_group;
    uint16_t* qh;                                 // [nr][nq*hd]
    int nq, nkv, hd, gate; float eps;
    const int* pos0_ptr; int pos0_imm;
    const int* nact_ptr;                          // active rows (MTP), null = nr
    float* work; int max_splits;                  // split partials
    float sl2e;                                   // (float)(log2(e) / sqrt(hd))
    uint16_t* out; int8_t* xq; float* xs;
    const int* stop;
    // prefill: the rows come in tiles of zrows (grid.z = tile) out of ztotal rows; tile z holds rows
    // z zrows .. at positions pos0 + z zrows .., its own work region; 0 = no tiles
    int zrows, ztotal;
    int prep_kv_only;                             // prep writes K/V only (the MTP prompt pass)
    float in_scale;                               // the quantized output's input_scale (0 = 1)
};
int launch_attn_prep(const AttnArgs& a, int nr, hipStream_t s);
int launch_attn_prep_rows(const AttnArgs& a, int nrows, hipStream_t s);   // any row count (prefill)
// prep_fused: the split kernel also norms/ropes the rows and writes the new K/V (no prep launch)
int launch_attn(const AttnArgs& a, int nr, hipStream_t s, bool prep_fused = false);
size_t attn_work_floats(int nq, int hd, int max_splits, int nr);

// ---------------------------------------------------------------- prefill GEMM (int8 MFMA)
// y = GEMM of per-(row, group) weights and per-(token, group) activations (k_gemm.hip), y bf16 when
// out_bf16, the residual bf16 when res_bf16
int launch_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                    const float* sx, int M, void* y, int ldy, int out_bf16, const void* res, int ldr, int res_bf16,
                    float rs, hipStream_t s, const AlphaSel* asel = nullptr);

// ---------------------------------------------------------------- prefill element kernels (k_prefill.hip)
int launch_pf_quant_bf16(const uint16_t* x, int ld, int M, int K, int gs, float in_scale, int8_t* xq, float* xs,
                         hipStream_t s);
int launch_quant_tok_grp(const float* x, int xstride, int M, int K, int gs, float in_scale, int8_t* xq, float* xs,
                         hipStream_t s);
int launch_pf_conv(const uint16_t* buf, int ld, int C, int nconv, const uint16_t* conv_w, uint16_t* rec, int npend,
                   uint16_t* out, int ldo, hipStream_t s);
int launch_pf_ab(const uint16_t* in_a, const uint16_t* in_b, const uint16_t* A_log, const uint16_t* dt_bias,
                 const uint16_t* y, int ystride, int K, int vh, int C, float* out, hipStream_t s);
int launch_pf_swiglu_quant(const float* gu, int I, int gs, float gscale, int C, int8_t* xq, float* xs,
                           hipStream_t s);

// ---------------------------------------------------------------- checkpoint (ckpt.hip)
struct CkTensor { int dtype, ndim; long long shape[Q27X_MAX_DIMS]; const void* host; size_t nbytes; };
int ckpt_get(const q27x_ckpt* ck, const char* name, CkTensor* out);   // Q27X_E_MISSING if absent
// kind 0 fp8 E4M3, 1 NVFP4 (gsc = its E4M3 per-16 scales), 2 bf16 -> int8 per-64 (row_mode 1 / 2:
// gate / up rows into the fused gate|up layout)
int launch_to_i8g64(int kind, const void* src, const void* gsc, int rows, int K, int src_ld, int8_t* w8, float* s64,
                    int row_mode, hipStream_t s);
int launch_nvfp4_to_bf16(const void* src, const void* gsc, float ws2, int rows, int K, uint16_t* out, hipStream_t s);

// ---------------------------------------------------------------- synthetic weights
int launch_gen_i8(int8_t* W, float* WS, int rows, int K, uint64_t key, int layout_gu, int is_up,
                  hipStream_t s);
int launch_gen_bf16(uint16_t* p, size_t n, uint64_t key, float stdv, float mean, int uniform,
                    hipStream_t s);
int launch_quant_w(const float* w, int rows, int K, int8_t* wq, float* ws, hipStream_t s);
int launch_math_test(const float* x, float* y, int n, int op, hipStream_t s);

}  // namespace q27x
