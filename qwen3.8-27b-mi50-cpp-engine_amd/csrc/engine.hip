// engine.hip -- the chained-MTP speculative decode step on one MI355X.
//
// Host side of the reference's spec_round (src/q27_main.cpp:2702-2958) and its verify layer
// run_layer_tp_nr (2271-2489), re-planned for one GPU:
//   * no tensor parallelism: every projection is unsharded and the residual share is 1;
//   * the round never returns to the host: drafts, verify-row tokens, acceptance, rollback and
//     hand-off live in a device control block (Dctl) that small control kernels update, so one
//     round is a fixed kernel sequence captured once in a HIP graph and replayed;
//   * rollback is the GDN kernel's deferred commit (no snapshot banks); KV needs none (R13);
//   * only the round's (ncommit, tokens) reach the host, through a pinned mailbox.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

// tensor ids shared with the host restatement: ((layer code) << 8) | kind
enum {
    T_IN_NORM = 1, T_POST_NORM = 2,
    T_IN_QKV = 10, T_IN_Z = 11, T_IN_A = 12, T_IN_B = 13, T_A_LOG = 14, T_DT_BIAS = 15,
    T_GDN_NORM = 16, T_CONV_W = 17, T_OUT_PROJ = 18,
    T_Q = 20, T_K = 21, T_V = 22, T_Q_NORM = 23, T_K_NORM = 24, T_O = 25,
    T_GATE = 30, T_UP = 31, T_DOWN = 32, T_DOWN_S0 = 33,   // MTP down slices: 33..36
    T_EMB = 40, T_FINAL_NORM = 41, T_LM_HEAD = 42,
    T_PRE_EMB = 50, T_PRE_HID = 51, T_FC0 = 52, T_FC1 = 53, T_MTP_NORM = 54
};
static uint64_t tid(int code, int kind) { return ((uint64_t)code << 8) | (uint64_t)kind; }

struct Mat {
    int8_t* w = nullptr; float* s = nullptr; int rows = 0, K = 0;
    // per-output scale of the stacked source tensors (alpha = input_scale x weight_scale; 1 for
    // weights made from their values, as the synthetic ones)
    float alpha = 1.0f; AlphaSel asel{};
    // the prefill GEMM's representation of the same matrix (per-(row, group) codes and scales,
    // groups of pgs columns), made on the first GEMM prefill after a load
    int8_t* pw = nullptr; float* ps = nullptr; int pgs = 0;
};

struct LayerDev {
    int is_attn = 0;
    uint16_t *in_norm = nullptr, *post_norm = nullptr;
    Mat qkvz; uint16_t *in_a = nullptr, *in_b = nullptr, *A_log = nullptr, *dt_bias = nullptr;
    uint16_t *gdn_norm = nullptr, *conv_w = nullptr; Mat out_proj;
    Mat qkv; uint16_t *q_norm = nullptr, *k_norm = nullptr; Mat o;
    Mat gu, down;
    Mat down4[4];   // MTP layer: down as four column slices of I/4 (src/q27_main.cpp:2605-2612)
    int8_t *kc = nullptr, *vc = nullptr; float *ks = nullptr, *vs = nullptr;
    float* S = nullptr; void* pend = nullptr;
    uint16_t* conv_st = nullptr;   // per q|k|v channel: committed conv history + pending raw inputs (16 bf16)
    // input_scale of the quantized activations each projection consumes (the input norm's for
    // in_qkv / q_proj, the post norm's for gate|up, the SwiGLU output's for down, the mixer
    // output's for out_proj / o_proj)
    float in_s_in = 1.0f, in_s_post = 1.0f, in_s_down = 1.0f, in_s_out = 1.0f;
};

// device control block (the Dev NR fields of src/q27_main.cpp:360-379 plus the round's tokens)
struct Dctl {
    int pos, tok, ncatch, gdn_npend;
    int catch_tok[8];
    int dt[8], nx[8];
    float nxval[8];
    int dt_raw[8];      // the MTP argmax of each draft, before a forced replacement
    int vtok[8];
    int mtp_nact, mtp_dpos0, mtp_head, mtp_out;
    int mtp_tok[8];
    int committed, max_new, stop, rounds;
    int forced_on, forced_n, forced_base, ctx;
    int nacc_last, ncommit_last, err, pad0;
    // q27x_generate's stop tokens (-1: none) and the output length through the first of them (0: none seen)
    int eos0, eos1, emit_end, pad1;
    long long acc_hist[9];
    long long accepted;
    // per-round phase timing (the reference's Q27_SPEC_T buckets, src/q27_main.cpp:2705-2707,
    // 6731-6733), in device wall-clock ticks: stamps of the current round and running sums of
    // draft (round start -> last draft's argmax), verify layers (-> head norm), head (-> acceptance)
    // and tail (acceptance, rollback and hand-off)
    unsigned long long t_begin, t_draft, t_verify, t_pad;
    unsigned long long sp_t[4];
};

struct Mailbox { volatile int round; volatile int committed; volatile int ncommit; volatile int stop; volatile int tok[8]; };

}  // namespace q27x

using namespace q27x;

// Buffers of the layer-major prefill (allocated on its first use, sized for a chunk of `cap` rows).
struct PfBuf {
    int cap = 0;
    float* x = nullptr;          // [cap][H] fp32 residual
    uint16_t* h = nullptr;       // [cap][H] bf16 residual copy (the next add's residual)
    uint16_t* y = nullptr;       // [cap][H] bf16 normed rows (GDN a/b)
    float* yf = nullptr;         // [cap][H] normed values to quantize; the GDN scan's q^|k^ ([cap][kh][256])
    int8_t* xq = nullptr; float* xs = nullptr;     // [cap][kmax] codes, [cap][32] group scales
    int8_t* xq2 = nullptr; float* xs2 = nullptr;   // [cap][H], [cap][32]: the MTP pass's second fc input
    uint16_t* pb = nullptr;      // [cap][wmax] projection rows
    uint16_t* qh = nullptr;      // [cap][att] normed, roped queries
    float* gu = nullptr;         // [cap][max(2I, nz)] gate|up GEMM output (GDN scan's mixed rows before)
    uint16_t* mix = nullptr;     // [cap][max(nz, att)] mixer output
    float* rowsc = nullptr;      // [3][cap][vh] GDN decay, beta; the scan's k^.q^ ([cap][kh])
    float* work = nullptr;       // attention split partials of one launch (pf_attn_work_rows rows)
    uint16_t* cv = nullptr;      // [cap][nqkv] convolved q|k|v rows
    std::vector<void*> allocs;
};

struct q27x_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    q27x_config c{};
    int H = 0, I = 0, V = 0, D = 128, nqkv = 0, nz = 0, qr = 0, kvr = 0, att = 0;
    char* warena = nullptr; size_t wcap = 0, woff = 0;
    char* sarena = nullptr; size_t scap = 0, soff = 0;
    std::vector<LayerDev> L;
    LayerDev mtp;
    uint16_t *pre_emb = nullptr, *pre_hid = nullptr, *mtp_norm = nullptr;
    Mat fc0, fc1;
    uint16_t *emb = nullptr, *final_norm = nullptr, *lm_head = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    size_t weight_bytes = 0;
    // scratch
    Dctl* dctl = nullptr;
    uint16_t *hid = nullptr, *ynorm = nullptr, *hfinal = nullptr, *hall = nullptr;
    float* xres = nullptr;
    // activation codes / per-16 scales: region A (the step's input), B (the second MTP fc half),
    // ACT (SwiGLU output), each kMaxRows rows; offsets in elements
    int8_t* xq = nullptr; float* xs = nullptr;
    size_t xb_off = 0, act_off = 0;
    uint16_t *pb = nullptr, *qh = nullptr, *ao = nullptr, *gout = nullptr;
    uint16_t *cat = nullptr, *mtp_hin = nullptr, *mtp_res = nullptr, *hprev = nullptr, *hcatch = nullptr;
    float* attn_work = nullptr; int max_splits = 0;
    float* sw_part = nullptr; unsigned* sw_cnt = nullptr;   // SwiGLU units split over blocks
    float* gab = nullptr;          // GDN row scalars of the current layer: [2][kMaxRows][vh] decay, beta
    float* pval = nullptr; uint32_t* pidx = nullptr; int pstride = 4096;
    int32_t* out_ring = nullptr; int ring_cap = 0;
    int32_t* forced = nullptr; int forced_cap = 0;
    int32_t* prompt_dev = nullptr; int prompt_cap = 0;
    Mailbox* mbox = nullptr;   // pinned host memory, mapped
    Mailbox* mbox_dev = nullptr;
    int loaded = 0, prefilled = 0, s_fail = 0;
    int n_prompt = 0;
    hipGraphExec_t g_spec = nullptr, g_plain = nullptr;
    int g_spec_k = 0;
    int wclk_khz = 0;      // device wall clock (s_memrealtime) rate
    float sl2e = 0.0f;
    PfBuf* pf = nullptr;
    std::vector<void*> pf_walloc;   // the GEMM representations of the weights
    int pf_wready = 0;
    // chunk pipeline of the prefill: the further chunk buffer sets and their streams (set 0 is pf
    // on the context's stream), and per buffer set one event per layer (+ the MTP pass, + the end)
    PfBuf* pfx[2] = { nullptr, nullptr };
    hipStream_t pf_stream[2] = { nullptr, nullptr };
    std::vector<hipEvent_t> pf_ev;
    PfBuf* pfc = nullptr;         // the chunk being enqueued: its buffers and stream
    hipStream_t pfs = nullptr;
};

namespace q27x {

static void* walloc(q27x_ctx* x, size_t bytes) {
    const size_t off = (x->woff + 255) & ~(size_t)255;
    if (off + bytes > x->wcap) return nullptr;
    x->woff = off + bytes;
    return x->warena + off;
}
static void* salloc(q27x_ctx* x, size_t bytes) {
    const size_t off = (x->soff + 255) & ~(size_t)255;
    if (x->s_fail || off + bytes > x->scap) { x->s_fail = 1; return nullptr; }
    x->soff = off + bytes;
    return x->sarena + off;
}
static int is_attn_layer(const q27x_config& c, int L) { return (L % c.attn_period) == c.attn_period - 1; }

// ---------------------------------------------------------------- control kernels
// Small single-block kernels that move the round's bookkeeping on the device.
__global__ void k_set_ints(int* base, int n, int o0, int v0, int o1, int v1, int o2, int v2, int o3, int v3) {
    if (threadIdx.x != 0) return;
    const int offs[4] = { o0, o1, o2, o3 }, vals[4] = { v0, v1, v2, v3 };
    for (int i = 0; i < n && i < 4; ++i) base[offs[i]] = vals[i];
}
__device__ __forceinline__ void copy_row(uint16_t* dst, const uint16_t* src, int H) {
    for (int i = threadIdx.x * 8; i < H; i += blockDim.x * 8) *(uint4*)(dst + i) = *(const uint4*)(src + i);
}
// draft 0 rows: the catch-up rows then (h_prev, tok) (src/q27_main.cpp:2737-2744)
// A round writes positions pos .. pos + K: it needs pos + K < ctx, the reference's condition for a
// speculative round (src/q27_main.cpp:6391). The host never launches one past it; if it happens
// anyway the round raises the device error, stops, and tells the host through the mailbox.
__device__ __forceinline__ void raise_range(Dctl* d, Mailbox* mb) {
    d->err = 6;
    d->stop = 1;
    if (mb) {
        mb->stop = 1;
        __threadfence_system();
        mb->round = d->rounds + 1;
    }
}
__global__ __launch_bounds__(256) void k_round_begin(Dctl* d, uint16_t* mtp_hin, const uint16_t* hcatch,
                                                     const uint16_t* hprev, Mailbox* mb, int H, int K) {
    if (d->stop) return;
    if (d->pos + K >= d->ctx) {
        if (threadIdx.x == 0) raise_range(d, mb);
        return;
    }
    if (threadIdx.x == 0) d->t_begin = __builtin_amdgcn_s_memrealtime();
    const int nc = d->ncatch;
    for (int r = 0; r < nc; ++r) copy_row(mtp_hin + (size_t)r * H, hcatch + (size_t)r * H, H);
    copy_row(mtp_hin + (size_t)nc * H, hprev, H);
    if (threadIdx.x == 0) {
        for (int r = 0; r < nc; ++r) d->mtp_tok[r] = d->catch_tok[r];
        d->mtp_tok[nc] = d->tok;
        for (int r = nc + 1; r < 8; ++r) d->mtp_tok[r] = 0;
        d->mtp_nact = nc + 1;
        d->mtp_dpos0 = d->pos - 1 - nc;
        d->mtp_head = nc;
    }
}
// after draft j: record dt[j] (the MTP argmax, or the forced token), chain the layer's own
// residual into the next draft (src/q27_main.cpp:2745-2750), or set the verify rows after the
// last draft
__global__ __launch_bounds__(256) void k_draft_post(Dctl* d, uint16_t* mtp_hin, const uint16_t* mtp_res,
                                                    const int32_t* forced, int H, int j, int K) {
    if (d->stop) return;
    __shared__ int s_tok;
    if (threadIdx.x == 0) {
        if (j + 1 == K) d->t_draft = __builtin_amdgcn_s_memrealtime();
        int t = d->mtp_out;
        d->dt_raw[j] = t;
        if (d->forced_on) {
            const int fi = d->pos - d->forced_base + 1 + j;
            if (fi >= 0 && fi < d->forced_n) t = forced[fi];
        }
        d->dt[j] = t;
        s_tok = t;
    }
    __syncthreads();
    if (j + 1 < K) {
        copy_row(mtp_hin, mtp_res + (size_t)d->mtp_head * H, H);
        __syncthreads();
        if (threadIdx.x == 0) {
            d->mtp_tok[0] = s_tok;
            d->mtp_nact = 1;
            d->mtp_dpos0 = d->pos + j;      // pos - 1 + (j + 1)
            d->mtp_head = 0;
        }
    } else if (threadIdx.x == 0) {
        d->vtok[0] = d->tok;
        for (int r = 1; r <= K; ++r) d->vtok[r] = d->dt[r - 1];
        d->ncatch = 0;
    }
}
// [3] greedy acceptance, [4] rollback (= how many rows the next GDN call commits) and hand-off
// (src/q27_main.cpp:2811-2812, 2929-2950); one-round-lagged mailbox to the host. The round's
// tokens and counters are read into registers up front, all loads in one round trip: stores to
// the ring and the mailbox may alias the control block as far as the compiler knows, so reading
// the block between them would wait for a load after each store.
__global__ __launch_bounds__(256) void k_accept(Dctl* d, const uint16_t* hfinal, uint16_t* hcatch, uint16_t* hprev,
                                                int32_t* ring, int ring_cap, Mailbox* mb, int H, int K) {
    if (d->stop) return;
    __shared__ int s_nacc;
    __shared__ unsigned long long s_t0;
    int nx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) nx[j] = d->nx[j];
    if (threadIdx.x == 0) {
        s_t0 = __builtin_amdgcn_s_memrealtime();
        int dt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) dt[j] = d->dt[j];
        int nacc = 0;
        bool run = true;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            run = run && j < K && nx[j] == dt[j];
            nacc += run ? 1 : 0;
        }
        s_nacc = nacc;
    }
    __syncthreads();
    const int nacc = s_nacc;
    for (int j = 0; j < nacc; ++j) copy_row(hcatch + (size_t)j * H, hfinal + (size_t)j * H, H);
    copy_row(hprev, hfinal + (size_t)nacc * H, H);
    if (threadIdx.x == 0) {
        const int eos0 = d->eos0, eos1 = d->eos1, max_new = d->max_new;
        const int c0 = d->committed, rounds = d->rounds + 1;
        int emit_end = d->emit_end, stop = d->stop;
        const long long accepted = d->accepted;
        const unsigned long long t_begin = d->t_begin, t_draft = d->t_draft, t_verify = d->t_verify;
        const int pos = d->pos;
        // every committed token goes to the ring (a round that passes max_new still advanced the
        // state by ncommit positions; a later call continues after them)
        const int ncommit = nacc + 1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < ncommit) {
                const int c = c0 + j;
                if (c < ring_cap) ring[c] = nx[j];
                // q27x_generate's stop tokens: the request's output ends after the first one
                if (emit_end == 0 && (nx[j] == eos0 || nx[j] == eos1)) emit_end = c + 1;
            }
        }
        const int c = c0 + ncommit;
        int tok = nx[0];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < nacc) d->catch_tok[j] = nx[j];
            if (j == nacc) tok = nx[j];
        }
        d->ncatch = nacc;
        d->tok = tok;
        d->pos = pos + ncommit;
        d->gdn_npend = ncommit;
        d->committed = c;
        d->rounds = rounds;
        d->accepted = accepted + nacc;
        for (int j = 0; j <= nacc && j < 9; ++j) d->acc_hist[j] += 1;
        d->nacc_last = nacc;
        d->ncommit_last = ncommit;
        d->emit_end = emit_end;
        if (c >= max_new || emit_end > 0) stop = 1;
        d->stop = stop;
        if (mb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) mb->tok[j] = j < ncommit ? nx[j] : -1;
            mb->ncommit = ncommit;
            mb->committed = c;
            mb->stop = stop;
            __threadfence_system();
            mb->round = rounds;
        }
        d->sp_t[0] += t_draft - t_begin;
        d->sp_t[1] += t_verify - t_draft;
        d->sp_t[2] += s_t0 - t_verify;
        d->sp_t[3] += __builtin_amdgcn_s_memrealtime() - s_t0;
    }
}
// plain greedy step bookkeeping (src/q27_main.cpp:6462-6466, 6680-6695)
__global__ void k_plain_pre(Dctl* d, Mailbox* mb) {
    if (d->stop || threadIdx.x) return;
    if (d->pos >= d->ctx) { raise_range(d, mb); return; }
    d->vtok[0] = d->tok;
}
__global__ __launch_bounds__(256) void k_plain_post(Dctl* d, const uint16_t* hfinal, uint16_t* hprev, int32_t* ring,
                                                    int ring_cap, Mailbox* mb, int H) {
    if (d->stop) return;
    copy_row(hprev, hfinal, H);
    if (threadIdx.x == 0) {
        const int c = d->committed;
        if (c < ring_cap) ring[c] = d->nx[0];
        if (d->emit_end == 0 && (d->nx[0] == d->eos0 || d->nx[0] == d->eos1)) d->emit_end = c + 1;
        d->committed = c + 1;
        d->tok = d->nx[0];
        d->pos += 1;
        d->gdn_npend = 1;
        d->ncatch = 0;
        d->rounds += 1;
        if (d->committed >= d->max_new || d->emit_end > 0) d->stop = 1;
        if (mb) {
            mb->tok[0] = d->nx[0];
            mb->ncommit = 1;
            mb->committed = d->committed;
            mb->stop = d->stop;
            __threadfence_system();
            mb->round = d->rounds;
        }
    }
}
__global__ void k_accept_rows(const int32_t* nx, const int32_t* dt, int k, int32_t* out2, int32_t* committed) {
    if (threadIdx.x) return;
    int nacc = 0;
    while (nacc < k && nx[nacc] == dt[nacc]) ++nacc;
    for (int j = 0; j <= nacc; ++j) committed[j] = nx[j];
    out2[0] = nacc;
    out2[1] = nacc + 1;
}

// ---------------------------------------------------------------- the verify pass
// Norms: each RMSNorm + quantize of the step's rows runs as the prologue of the projection that
// consumes it (every block normalizes the rows into its own LDS stage; block 0 writes the bf16
// side outputs), so no norm is a launch of its own except the head's. norm_of() describes one.
static NormArgs norm_of(q27x_ctx* x, const void* src, int src_bf16, const uint16_t* w, float plus, int quant_bf16,
                        uint16_t* hcopy, uint16_t* y) {
    NormArgs n{};
    n.x = src; n.x_bf16 = src_bf16; n.xstride = x->H; n.w = w; n.plus = plus; n.eps = x->c.rms_eps; n.n = x->H;
    n.hcopy = hcopy; n.y = y; n.ystride = x->H; n.quant_bf16 = quant_bf16; n.in_scale = 1.0f;
    n.stop = &x->dctl->stop;
    return n;
}
static void set_pre(ProjArgs& p, const NormArgs& n) { p.has_pre = 1; p.pre = n; }

// One layer of the verify pass (run_layer_tp_nr, src/q27_main.cpp:2271-2489) for nr rows; mlp = 0
// stops after the mixer half (attention or GDN, then o_proj / out_proj + residual).
static int layer_pass(q27x_ctx* x, int l, int nr, int mlp) {
    const q27x_config& c = x->c;
    hipStream_t s = x->stream;
    Dctl* d = x->dctl;
    const int H = x->H, I = x->I;
    int8_t* xa = x->xq;  float* sa = x->xs;
    int8_t* xact = x->xq + x->act_off;  float* sact = x->xs + x->act_off / 16;
    int rc;
    {
        LayerDev& Y = x->L[l];
        // input norm. Layer 0: the bf16 embedding rows, quantizing the bf16 normed rows
        // (q27_rmsnorm_quant_fp8); later layers: the fp32 residual r2, quantizing the fp32 normed
        // rows (q27_rmsnorm_hostss_fp8_b). Side outputs h = bf16(x), y = bf16(normed) (GDN a/b).
        NormArgs nin;
        if (l == 0) {
            nin = norm_of(x, nullptr, 1, Y.in_norm, 1.0f, 1, x->hid, nullptr);
            nin.emb = x->emb; nin.tok = d->vtok;
        } else {
            nin = norm_of(x, x->xres, 0, Y.in_norm, 1.0f, 0, x->hid, nullptr);
        }
        nin.in_scale = Y.in_s_in;
        ProjArgs o{};
        o.y = x->xres; o.ystride = H; o.out_bf16 = 0;
        o.res = x->hid; o.res_bf16 = 1; o.rstride = H; o.rs = 1.0f; o.stop = &d->stop;
        if (Y.is_attn) {
            ProjArgs p{};
            p.alpha = Y.qkv.alpha; p.asel = Y.qkv.asel; p.stop = &d->stop;
            p.W = Y.qkv.w; p.WS = Y.qkv.s; p.rows = Y.qkv.rows; p.K = H;
            p.y = x->pb; p.ystride = Y.qkv.rows; p.out_bf16 = 1;
            set_pre(p, nin);
            if ((rc = launch_proj(p, EPI_STORE, nr, s))) return rc;
            AttnArgs a{};
            a.qkv = x->pb; a.qkv_stride = Y.qkv.rows; a.q_norm_w = Y.q_norm; a.k_norm_w = Y.k_norm;
            a.rope_cos = x->rope_cos; a.rope_sin = x->rope_sin; a.rot = c.rot_dims;
            a.kc = Y.kc; a.ks = Y.ks; a.vc = Y.vc; a.vs = Y.vs; a.kv_group = c.kv_group; a.qh = x->qh;
            a.nq = c.n_q; a.nkv = c.n_kv; a.hd = c.head_dim; a.gate = c.attn_gate; a.eps = c.rms_eps;
            a.pos0_ptr = &d->pos; a.work = x->attn_work; a.max_splits = x->max_splits; a.sl2e = x->sl2e;
            a.out = x->ao; a.xq = xa; a.xs = sa; a.stop = &d->stop; a.in_scale = Y.in_s_out;
            if ((rc = launch_attn(a, nr, s, true))) return rc;
            o.W = Y.o.w; o.WS = Y.o.s; o.rows = H; o.K = x->att; o.xq = xa; o.xst = x->att; o.xs = sa;
            o.alpha = Y.o.alpha; o.asel = Y.o.asel;
        } else {
            // in_qkv | in_z (raw bf16 rows; the conv runs inside the GDN kernel)
            const int rows = Y.qkvz.rows;
            // the q|k|v channels are convolved in the projection's epilogue (with the deferred
            // commit of their history), the z rows stored raw
            ProjArgs p{};
            p.alpha = Y.qkvz.alpha; p.asel = Y.qkvz.asel; p.stop = &d->stop;
            p.W = Y.qkvz.w; p.WS = Y.qkvz.s; p.rows = rows; p.K = H;
            p.y = x->pb; p.ystride = rows; p.out_bf16 = 1;
            p.conv_w = Y.conv_w; p.conv_st = Y.conv_st; p.nconv = x->nqkv; p.npend_ptr = &d->gdn_npend;
            // ... and the rows' (decay, beta) from the in_a / in_b dot products
            p.in_a = Y.in_a; p.in_b = Y.in_b; p.A_log = Y.A_log; p.dt_bias = Y.dt_bias; p.ab_vh = c.gdn_vh;
            p.ab_out = x->gab;
            set_pre(p, nin);
            if ((rc = launch_proj(p, EPI_CONV, nr, s))) return rc;
            GdnArgs g{};
            g.qkv = x->pb; g.qkv_stride = rows; g.z = x->pb + x->nqkv; g.z_stride = rows;
            g.rowsc = x->gab; g.norm_w = Y.gdn_norm;
            g.S = Y.S; g.pend = Y.pend; g.npend_ptr = &d->gdn_npend;
            g.kh = c.gdn_kh; g.vh = c.gdn_vh; g.d = x->D; g.eps = c.rms_eps;
            g.out = x->gout; g.out_stride = x->nz; g.xq = xa; g.xs = sa; g.stop = &d->stop; g.in_scale = Y.in_s_out;
            if ((rc = launch_gdn(g, nr, s))) return rc;
            o.W = Y.out_proj.w; o.WS = Y.out_proj.s; o.rows = H; o.K = x->nz; o.xq = xa; o.xst = x->nz; o.xs = sa;
            o.alpha = Y.out_proj.alpha; o.asel = Y.out_proj.asel;
        }
        if ((rc = launch_proj(o, EPI_STORE, nr, s))) return rc;
        if (!mlp) return Q27X_OK;
        // post norm of r1 (fp32, quantize the fp32 normed rows, h = bf16(r1)): gate|up prologue
        ProjArgs gu{};
        gu.W = Y.gu.w; gu.WS = Y.gu.s; gu.rows = 2 * I; gu.K = H; gu.alpha = Y.gu.alpha; gu.asel = Y.gu.asel;
        gu.act_q = xact; gu.act_s = sact; gu.act_stride = I; gu.gscale = 1.0f / Y.in_s_down; gu.stop = &d->stop;
        gu.sw_part = x->sw_part; gu.sw_cnt = x->sw_cnt;
        NormArgs npost = norm_of(x, x->xres, 0, Y.post_norm, 1.0f, 0, x->hid, nullptr);
        npost.in_scale = Y.in_s_post;
        set_pre(gu, npost);
        if ((rc = launch_proj(gu, EPI_SWIGLU, nr, s))) return rc;
        ProjArgs dn{};
        dn.W = Y.down.w; dn.WS = Y.down.s; dn.rows = H; dn.K = I; dn.alpha = Y.down.alpha; dn.asel = Y.down.asel;
        dn.xq = xact; dn.xst = I; dn.xs = sact;
        dn.y = x->xres; dn.ystride = H; dn.out_bf16 = 0;
        dn.res = x->hid; dn.res_bf16 = 1; dn.rstride = H; dn.rs = 1.0f; dn.stop = &d->stop;
        if ((rc = launch_proj(dn, EPI_STORE, nr, s))) return rc;
    }
    return Q27X_OK;
}

// run_layer_tp_nr on one card for nr rows: tokens d->vtok, positions d->pos.., GDN commits
// d->gdn_npend pending rows. head: 0 = final residual rows only, 1 = + final norm, lm_head and
// argmax into d->nx. hout: where the final residual rows go (default ctx->hfinal).
static int verify_pass(q27x_ctx* x, int nr, int head, uint16_t* hout) {
    const q27x_config& c = x->c;
    hipStream_t s = x->stream;
    Dctl* d = x->dctl;
    const int H = x->H;
    int rc;
    for (int l = 0; l < c.n_layers; ++l)
        if ((rc = layer_pass(x, l, nr, 1))) return rc;
    // head (src/q27_main.cpp:2457-2481): final residual rows, final norm, lm_head, argmax
    NormArgs hn{};
    hn.x = x->xres; hn.x_bf16 = 0; hn.xstride = H; hn.hadd = c.head_double_residual ? x->hid : nullptr;
    hn.hout = hout ? hout : x->hfinal; hn.w = x->final_norm; hn.plus = 1.0f; hn.eps = c.rms_eps; hn.n = H;
    hn.y = head ? x->ynorm : nullptr; hn.ystride = H; hn.in_scale = 1.0f; hn.stop = &d->stop;
    hn.stamp = &d->t_verify;
    if ((rc = launch_norm(hn, nr, s))) return rc;
    if (head) {
        GemvArgs ga{};
        ga.W = x->lm_head; ga.rows = x->V; ga.K = H; ga.x = x->ynorm; ga.xst = H;
        ga.pval = x->pval; ga.pidx = x->pidx; ga.pstride = x->pstride; ga.stop = &d->stop;
        int nb = 0;
        if ((rc = launch_gemv(ga, 1, nr, &nb, s))) return rc;
        if ((rc = launch_argmax_final(x->pval, x->pidx, x->pstride, nb, nr, d->nx, d->nxval, &d->stop, s))) return rc;
    }
    return Q27X_OK;
}

// ---------------------------------------------------------------- the MTP pass
// mtp_pass_nr (src/q27_main.cpp:2551-2618) over nr row slots (d->mtp_nact active): hidden rows
// ctx->mtp_hin, tokens d->mtp_tok, draft positions d->mtp_dpos0.. on the layer's own KV cache.
// kv_only stops after the K/V write (prompt conditioning, 2649-2692). head: mtp.norm + lm_head +
// argmax of row d->mtp_head into d->mtp_out.
static int mtp_pass(q27x_ctx* x, int nr, int head, int kv_only) {
    const q27x_config& c = x->c;
    hipStream_t s = x->stream;
    Dctl* d = x->dctl;
    LayerDev& Y = x->mtp;
    const int H = x->H, I = x->I;
    const float po = c.mtp_plus_one ? 1.0f : 0.0f;
    int8_t* xa = x->xq;  float* sa = x->xs;
    int8_t* xact = x->xq + x->act_off;  float* sact = x->xs + x->act_off / 16;
    int rc;
    // fc over [norm(emb) | norm(h)] (order by mtp_swap, src/q27_mtp_defs.h:108-109) as two K = H
    // halves (per-16 groups never straddle halves); each half's norm (quantizing the bf16 normed
    // rows) is the prologue of its fc projection
    NormArgs ne = norm_of(x, nullptr, 1, x->pre_emb, po, 1, nullptr, nullptr);
    ne.emb = x->emb; ne.tok = d->mtp_tok;
    NormArgs nh = norm_of(x, x->mtp_hin, 1, x->pre_hid, po, 1, nullptr, nullptr);
    const NormArgs& n0 = c.mtp_swap ? ne : nh;
    const NormArgs& n1 = c.mtp_swap ? nh : ne;
    ProjArgs f0{};
    f0.W = x->fc0.w; f0.WS = x->fc0.s; f0.rows = H; f0.K = H; f0.alpha = 1.0f;
    f0.y = x->mtp_res; f0.ystride = H; f0.out_bf16 = 1; f0.stop = &d->stop;
    set_pre(f0, n0);
    if ((rc = launch_proj(f0, EPI_STORE, nr, s))) return rc;
    ProjArgs f1{};
    f1.W = x->fc1.w; f1.WS = x->fc1.s; f1.rows = H; f1.K = H; f1.alpha = 1.0f;
    f1.y = x->mtp_res; f1.ystride = H; f1.out_bf16 = 1; f1.res = x->mtp_res; f1.res_bf16 = 1; f1.rstride = H;
    f1.rs = 1.0f; f1.stop = &d->stop;
    set_pre(f1, n1);
    if ((rc = launch_proj(f1, EPI_STORE, nr, s))) return rc;
    // input norm (bf16 residual, quantize the bf16 normed rows): q|k|v prologue
    ProjArgs q{};
    q.W = Y.qkv.w; q.WS = Y.qkv.s; q.rows = Y.qkv.rows; q.K = H; q.alpha = 1.0f;
    q.y = x->pb; q.ystride = Y.qkv.rows; q.out_bf16 = 1; q.stop = &d->stop;
    set_pre(q, norm_of(x, x->mtp_res, 1, Y.in_norm, po, 1, nullptr, nullptr));
    if ((rc = launch_proj(q, EPI_STORE, nr, s))) return rc;
    AttnArgs a{};
    a.qkv = x->pb; a.qkv_stride = Y.qkv.rows; a.q_norm_w = Y.q_norm; a.k_norm_w = Y.k_norm;
    a.rope_cos = x->rope_cos; a.rope_sin = x->rope_sin; a.rot = c.rot_dims;
    a.kc = Y.kc; a.ks = Y.ks; a.vc = Y.vc; a.vs = Y.vs; a.kv_group = c.kv_group; a.qh = x->qh;
    a.nq = c.n_q; a.nkv = c.n_kv; a.hd = c.head_dim; a.gate = c.attn_gate; a.eps = c.rms_eps;
    a.pos0_ptr = &d->mtp_dpos0; a.nact_ptr = &d->mtp_nact; a.work = x->attn_work; a.max_splits = x->max_splits;
    a.sl2e = x->sl2e; a.out = x->ao; a.xq = xa; a.xs = sa; a.stop = &d->stop;
    if (kv_only) return launch_attn_prep(a, nr, s);
    if ((rc = launch_attn(a, nr, s, true))) return rc;
    // o-proj rounded to bf16 before the residual add
    ProjArgs o{};
    o.W = Y.o.w; o.WS = Y.o.s; o.rows = H; o.K = x->att; o.alpha = 1.0f; o.xq = xa; o.xst = x->att; o.xs = sa;
    o.y = x->mtp_res; o.ystride = H; o.out_bf16 = 1; o.res = x->mtp_res; o.res_bf16 = 1; o.rstride = H; o.rs = 1.0f;
    o.res_round = 1; o.stop = &d->stop;
    if ((rc = launch_proj(o, EPI_STORE, nr, s))) return rc;
    // post norm (bf16 residual, quantize the bf16 normed rows): gate|up prologue
    ProjArgs gu{};
    gu.W = Y.gu.w; gu.WS = Y.gu.s; gu.rows = 2 * I; gu.K = H; gu.alpha = 1.0f;
    gu.act_q = xact; gu.act_s = sact; gu.act_stride = I; gu.gscale = 1.0f; gu.stop = &d->stop;
    gu.sw_part = x->sw_part; gu.sw_cnt = x->sw_cnt;
    set_pre(gu, norm_of(x, x->mtp_res, 1, Y.post_norm, po, 1, nullptr, nullptr));
    if ((rc = launch_proj(gu, EPI_SWIGLU, nr, s))) return rc;
    // down as four K = I/4 column slices, each added into the bf16 residual with its own bf16
    // rounding (src/q27_main.cpp:2605-2612: one fp32 slice projection, then q27_add_inplace)
    const int I4 = I / 4;
    const bool one = down4_supported(I4, nr);          // one launch (same bits as the four below)
    if (one) {
        Down4Args d4{};
        for (int j = 0; j < 4; ++j) { d4.W[j] = Y.down4[j].w; d4.WS[j] = Y.down4[j].s; d4.alpha[j] = 1.0f; }
        d4.rows = H; d4.K4 = I4; d4.xq = xact; d4.xst = I; d4.xs = sact;
        d4.y = x->mtp_res; d4.ystride = H; d4.stop = &d->stop;
        if ((rc = launch_down4(d4, nr, s))) return rc;
    }
    for (int j = 0; j < 4 && !one; ++j) {
        ProjArgs dn{};
        dn.W = Y.down4[j].w; dn.WS = Y.down4[j].s; dn.rows = H; dn.K = I4; dn.alpha = 1.0f;
        dn.xq = xact + (size_t)j * I4; dn.xst = I; dn.xs = sact + (size_t)j * (I4 / 16);
        dn.y = x->mtp_res; dn.ystride = H; dn.out_bf16 = 1; dn.res = x->mtp_res; dn.res_bf16 = 1;
        dn.rstride = H; dn.rs = 1.0f; dn.stop = &d->stop;
        if ((rc = launch_proj(dn, EPI_STORE, nr, s))) return rc;
    }
    if (head) {
        NormArgs hn{};
        hn.x = x->mtp_res; hn.x_bf16 = 1; hn.xstride = H; hn.w = x->mtp_norm; hn.plus = 1.0f; hn.eps = c.rms_eps;
        hn.n = H; hn.y = x->ynorm; hn.ystride = H; hn.in_scale = 1.0f; hn.row_sel = &d->mtp_head; hn.stop = &d->stop;
        if ((rc = launch_norm(hn, 1, s))) return rc;
        GemvArgs ga{};
        ga.W = x->lm_head; ga.rows = x->V; ga.K = H; ga.x = x->ynorm; ga.xst = H;
        ga.pval = x->pval; ga.pidx = x->pidx; ga.pstride = x->pstride; ga.stop = &d->stop;
        int nb = 0;
        if ((rc = launch_gemv(ga, 1, 1, &nb, s))) return rc;
        if ((rc = launch_argmax_final(x->pval, x->pidx, x->pstride, nb, 1, &d->mtp_out, nullptr, &d->stop, s))) return rc;
    }
    return Q27X_OK;
}

static int set_ints(q27x_ctx* x, int n, int o0, int v0, int o1 = 0, int v1 = 0, int o2 = 0, int v2 = 0, int o3 = 0,
                    int v3 = 0) {
    hipLaunchKernelGGL(k_set_ints, dim3(1), dim3(64), 0, x->stream, (int*)x->dctl, n, o0, v0, o1, v1, o2, v2, o3, v3);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
#define DOFF(f) ((int)(offsetof(Dctl, f) / sizeof(int)))

// one speculative round as a fixed kernel sequence (captured into a graph)
static int enqueue_spec_round(q27x_ctx* x) {
    const int K = x->c.spec_k, H = x->H;
    Dctl* d = x->dctl;
    int rc;
    hipLaunchKernelGGL(k_round_begin, dim3(1), dim3(256), 0, x->stream, d, x->mtp_hin, x->hcatch, x->hprev, x->mbox_dev,
                       H, K);
    Q27X_HIP(hipGetLastError());
    for (int j = 0; j < K; ++j) {
        if ((rc = mtp_pass(x, j == 0 ? K + 1 : 1, 1, 0))) return rc;
        hipLaunchKernelGGL(k_draft_post, dim3(1), dim3(256), 0, x->stream, d, x->mtp_hin, x->mtp_res, x->forced, H, j, K);
        Q27X_HIP(hipGetLastError());
    }
    if ((rc = verify_pass(x, K + 1, 1, nullptr))) return rc;
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(256), 0, x->stream, d, x->hfinal, x->hcatch, x->hprev, x->out_ring,
                       x->ring_cap, x->mbox_dev, H, K);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
static int enqueue_plain_step(q27x_ctx* x) {
    hipLaunchKernelGGL(k_plain_pre, dim3(1), dim3(64), 0, x->stream, x->dctl, x->mbox_dev);
    Q27X_HIP(hipGetLastError());
    int rc = verify_pass(x, 1, 1, nullptr);
    if (rc) return rc;
    hipLaunchKernelGGL(k_plain_post, dim3(1), dim3(256), 0, x->stream, x->dctl, x->hfinal, x->hprev, x->out_ring,
                       x->ring_cap, x->mbox_dev, x->H);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
static int build_graph(q27x_ctx* x, int spec, hipGraphExec_t* out) {
    hipGraph_t g = nullptr;
    Q27X_HIP(hipStreamBeginCapture(x->stream, hipStreamCaptureModeThreadLocal));
    int rc = spec ? enqueue_spec_round(x) : enqueue_plain_step(x);
    hipError_t e = hipStreamEndCapture(x->stream, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    return Q27X_OK;
}
static int use_graphs() {
    const char* v = getenv("Q27X_GRAPH");
    return !(v && v[0] == '0');
}
static int check_device_err(q27x_ctx* x) {
    int err = 0;
    Q27X_HIP(hipMemcpy(&err, &x->dctl->err, 4, hipMemcpyDeviceToHost));
    if (err == 6) { set_error("context capacity exhausted (ctx=%d)", x->c.ctx); return Q27X_E_RANGE; }
    if (err) { set_error("device error flag %d", err); return Q27X_E_DEVICE; }
    return Q27X_OK;
}

}  // namespace q27x

// ================================================================ C ABI: engine tier
extern "C" {

int q27x_config_default(q27x_config* c) {
    if (!c) return Q27X_E_ARG;
    memset(c, 0, sizeof *c);
    c->hidden = 5120; c->inter = 17408; c->vocab = 62080; c->n_layers = 64; c->attn_period = 4;
    c->gdn_kh = 16; c->gdn_vh = 48; c->gdn_d = 128;
    c->n_q = 32; c->n_kv = 8; c->head_dim = 128; c->attn_gate = 1; c->rot_dims = 32; c->rope_theta = 1e7;
    c->kv_group = 32; c->rms_eps = 1e-6f; c->head_double_residual = 1; c->mtp_swap = 1; c->mtp_plus_one = 1;
    c->spec = 1; c->spec_k = 2; c->ctx = 2048; c->pf_gs = 0;
    c->eos_id = 248044; c->eos_id2 = -1;
    return Q27X_OK;
}
int q27x_config_tiny(q27x_config* c) {
    if (!c) return Q27X_E_ARG;
    q27x_config_default(c);
    c->hidden = 1024; c->inter = 2048; c->vocab = 4096; c->n_layers = 8;
    c->gdn_kh = 2; c->gdn_vh = 6; c->n_q = 4; c->n_kv = 1; c->ctx = 512;
    return Q27X_OK;
}

// fail-closed parsing (include/q27.h:189-206)
static int env_flag(const char* name, int def) {
    const char* v = getenv(name);
    if (!v || !*v) return def;
    if (!strcmp(v, "0") || !strcmp(v, "false") || !strcmp(v, "no") || !strcmp(v, "off")) return 0;
    if (!strcmp(v, "1") || !strcmp(v, "true") || !strcmp(v, "yes") || !strcmp(v, "on")) return 1;
    fprintf(stderr, "FATAL %s=\"%s\" is not a boolean (use 0/1, false/true, no/yes, off/on). "
                    "Refusing to guess which arm you meant.\n", name, v);
    abort();
}
static int env_int(const char* name, int def) {
    const char* v = getenv(name);
    if (!v || !*v) return def;
    char* end = nullptr;
    const long x = strtol(v, &end, 10);
    if (end == v || *end) { fprintf(stderr, "FATAL %s=\"%s\" is not an integer.\n", name, v); abort(); }
    return (int)x;
}
// src/q27_main.cpp:3360-3361: Q27_SPEC default on; Q27_SPEC_K default 1, clamped to [1, 7]
int q27x_spec_config_from_env(q27x_config* c) {
    if (!c) return Q27X_E_ARG;
    c->spec = env_flag("Q27_SPEC", 1);
    int k = env_int("Q27_SPEC_K", 1);
    if (k < 1) k = 1;
    if (k > 7) k = 7;
    c->spec_k = k;
    c->mtp_swap = env_flag("Q27_MTP_SWAP", c->mtp_swap);
    c->mtp_plus_one = env_int("Q27_MTP_PO", c->mtp_plus_one);
    // src/q27_load.cpp:1623, src/q27_main.cpp:4020: Q27_Q8_GS, default 0 (the whole K); the only
    // other group the reference's prefill runs is 1024
    const int gs = env_int("Q27_Q8_GS", 0);
    if (gs != 0 && gs != 1024) {
        fprintf(stderr, "FATAL Q27_Q8_GS=%d: the prefill groups are 0 (the whole K) or 1024.\n", gs);
        abort();
    }
    c->pf_gs = gs;
    // src/q27_main.cpp:709-710, 3111: <|im_end|> stops a request when Q27_EOS_IM_END is set (the
    // reference defaults it to its serve mode, which this library does not have)
    c->eos_id2 = env_flag("Q27_EOS_IM_END", 0) ? 248046 : -1;
    return Q27X_OK;
}

int q27x_ctx_create(int device, const q27x_config* cfg, q27x_ctx** out) {
    if (!cfg || !out) { set_error("q27x_ctx_create: null argument"); return Q27X_E_ARG; }
    *out = nullptr;
    const q27x_config& c = *cfg;
    const bool rot_ok = c.rot_dims >= 2 && (c.rot_dims & (c.rot_dims - 1)) == 0 &&
                        (c.rot_dims <= 64 || (c.rot_dims == 128 && c.head_dim == 128));
    if ((c.hidden != 1024 && c.hidden != 5120) || c.inter % 1024 || c.gdn_d != 128 ||
        (c.head_dim != 128 && c.head_dim != 256) || !rot_ok ||
        c.n_layers < 1 || c.attn_period < 1 || c.spec_k < 1 || c.spec_k > 7 || c.ctx < 16 || c.vocab < 16 ||
        c.gdn_vh % c.gdn_kh || c.n_q % c.n_kv || (c.n_q / c.n_kv) * 8 > 64 || c.kv_group < 16 ||
        (c.pf_gs != 0 && c.pf_gs != 1024)) {
        set_error("q27x_ctx_create: unsupported geometry");
        return Q27X_E_SHAPE;
    }
    // the stored projections' input widths: down (inter), out_proj (value heads x 128), o_proj
    for (const int K : { c.inter, c.gdn_vh * 128, c.n_q * c.head_dim })
        if (!proj_k_supported(K)) {
            set_error("q27x_ctx_create: no projection kernel for an input width of %d", K);
            return Q27X_E_SHAPE;
        }
    q27x_ctx* x = new q27x_ctx();
    x->device = device; x->c = c;
    x->H = c.hidden; x->I = c.inter; x->V = c.vocab; x->D = c.gdn_d;
    x->nqkv = (2 * c.gdn_kh + c.gdn_vh) * c.gdn_d; x->nz = c.gdn_vh * c.gdn_d;
    x->qr = c.n_q * (c.attn_gate ? 2 * c.head_dim : c.head_dim); x->kvr = c.n_kv * c.head_dim;
    x->att = c.n_q * c.head_dim;
    x->sl2e = (float)((1.0 / sqrt((double)c.head_dim)) * 1.4426950408889634);
    auto fail = [&](int rc) { q27x_ctx_destroy(x); return rc; };
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return fail(hip_fail(e, "hipSetDevice"));
    if ((e = hipStreamCreateWithFlags(&x->stream, hipStreamNonBlocking)) != hipSuccess) return fail(hip_fail(e, "hipStreamCreate"));
    if ((e = hipDeviceGetAttribute(&x->wclk_khz, hipDeviceAttributeWallClockRate, device)) != hipSuccess) return fail(hip_fail(e, "hipDeviceGetAttribute"));
    if (int rc0 = gdn_set_lds_limit()) return fail(rc0);
    // weight arena
    const size_t H = x->H, I = x->I, V = x->V;
    auto i8b = [](size_t r, size_t k) { return r * k + r * (k / 64) * 4 + 512; };
    size_t wb = 0;
    int n_attn = 0;
    for (int l = 0; l < c.n_layers; ++l) {
        wb += 2 * H * 2 + 512 + i8b(2 * I, H) + i8b(H, I);
        if (is_attn_layer(c, l)) { wb += i8b(x->qr + 2 * x->kvr, H) + i8b(H, x->att) + 2 * (size_t)c.head_dim * 2 + 1024; ++n_attn; }
        else wb += i8b(x->nqkv + x->nz, H) + 2 * (size_t)c.gdn_vh * H * 2 + (size_t)x->nqkv * 4 * 2 + i8b(H, x->nz) + 4096;
    }
    wb += 2 * H * 2 + i8b(2 * I, H) + 4 * i8b(H, I / 4) + i8b(x->qr + 2 * x->kvr, H) + i8b(H, x->att) + 4096;   // MTP
    wb += 3 * H * 2 + 2 * i8b(H, H) + 2 * V * H * 2 + H * 2 + 8192;
    x->wcap = wb;
    if ((e = hipMalloc((void**)&x->warena, wb)) != hipSuccess) return fail(hip_fail(e, "hipMalloc(weights)"));
    // state + scratch arena
    const size_t kvn = (size_t)c.ctx * x->kvr;
    const size_t n_gdn = (size_t)(c.n_layers - n_attn);
    x->max_splits = (c.ctx + kSplit - 1) / kSplit;
    size_t sb = (n_attn + 1) * (2 * kvn + 2 * kvn / c.kv_group * 4 + 1024);
    sb += n_gdn * ((size_t)c.gdn_vh * 128 * 128 * 4 + (size_t)x->nqkv * 32 + gdn_pend_bytes(c.gdn_kh, c.gdn_vh, 128) + 1024);
    const size_t R = kMaxRows;
    size_t maxk = (size_t)H;
    if ((size_t)x->nz > maxk) maxk = x->nz;
    if ((size_t)x->att > maxk) maxk = x->att;
    const size_t xqn = R * (2 * maxk + I);
    const size_t pbn = R * (size_t)((x->qr + 2 * x->kvr) > (x->nqkv + x->nz) ? (x->qr + 2 * x->kvr) : (x->nqkv + x->nz));
    sb += sizeof(Dctl) + R * H * 2 * 4 + R * H * 4 + xqn + xqn / 16 * 4 + R * (size_t)x->nz * 2 + 256;
    sb += (size_t)kSwMaxSplit * 16 * R * 4 + kSwMaxSplit * 4 + 512 + 2 * R * (size_t)c.gdn_vh * 4 + 256;
    sb += pbn * 2 + 2 * R * (size_t)x->att * 2 + R * 2 * H * 2 + R * H * 2 * 3 + H * 2;
    sb += attn_work_floats(c.n_q, c.head_dim, x->max_splits, kMaxRows) * 4 + R * (size_t)x->pstride * 8;
    x->ring_cap = c.ctx + 64; x->forced_cap = c.ctx + 64; x->prompt_cap = c.ctx + 64;
    sb += (size_t)(x->ring_cap + x->forced_cap + x->prompt_cap) * 4 + (size_t)c.ctx * H * 2;
    sb += (size_t)c.ctx * (c.rot_dims / 2) * 4 * 2 + 64 * 256;
    x->scap = sb;
    if ((e = hipMalloc((void**)&x->sarena, sb)) != hipSuccess) return fail(hip_fail(e, "hipMalloc(state)"));
    if ((e = hipMemset(x->sarena, 0, sb)) != hipSuccess) return fail(hip_fail(e, "hipMemset(state)"));
    x->L.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        LayerDev& Y = x->L[l];
        Y.is_attn = is_attn_layer(c, l);
        if (Y.is_attn) {
            Y.kc = (int8_t*)salloc(x, kvn); Y.vc = (int8_t*)salloc(x, kvn);
            Y.ks = (float*)salloc(x, kvn / c.kv_group * 4); Y.vs = (float*)salloc(x, kvn / c.kv_group * 4);
        } else {
            Y.S = (float*)salloc(x, (size_t)c.gdn_vh * 128 * 128 * 4);
            Y.conv_st = (uint16_t*)salloc(x, (size_t)x->nqkv * 32);
            Y.pend = salloc(x, gdn_pend_bytes(c.gdn_kh, c.gdn_vh, 128));
        }
    }
    x->mtp.is_attn = 1;
    x->mtp.kc = (int8_t*)salloc(x, kvn); x->mtp.vc = (int8_t*)salloc(x, kvn);
    x->mtp.ks = (float*)salloc(x, kvn / c.kv_group * 4); x->mtp.vs = (float*)salloc(x, kvn / c.kv_group * 4);
    x->dctl = (Dctl*)salloc(x, sizeof(Dctl));
    x->hid = (uint16_t*)salloc(x, R * H * 2);
    x->ynorm = (uint16_t*)salloc(x, R * H * 2);
    x->hfinal = (uint16_t*)salloc(x, R * H * 2);
    x->xres = (float*)salloc(x, R * H * 4);
    x->xq = (int8_t*)salloc(x, xqn);
    x->xs = (float*)salloc(x, xqn / 16 * 4);
    x->xb_off = R * maxk;
    x->act_off = 2 * R * maxk;
    x->gout = (uint16_t*)salloc(x, R * (size_t)x->nz * 2);
    x->pb = (uint16_t*)salloc(x, pbn * 2);
    x->qh = (uint16_t*)salloc(x, R * (size_t)x->att * 2);
    x->ao = (uint16_t*)salloc(x, R * (size_t)x->att * 2);
    x->cat = (uint16_t*)salloc(x, R * 2 * H * 2);
    x->mtp_hin = (uint16_t*)salloc(x, R * H * 2);
    x->mtp_res = (uint16_t*)salloc(x, R * H * 2);
    x->hcatch = (uint16_t*)salloc(x, R * H * 2);
    x->hprev = (uint16_t*)salloc(x, H * 2);
    x->attn_work = (float*)salloc(x, attn_work_floats(c.n_q, c.head_dim, x->max_splits, kMaxRows) * 4);
    x->sw_part = (float*)salloc(x, (size_t)kSwMaxSplit * 16 * R * 4);
    x->sw_cnt = (unsigned*)salloc(x, kSwMaxSplit * 4);
    x->gab = (float*)salloc(x, (size_t)2 * kMaxRows * c.gdn_vh * 4);
    x->pval = (float*)salloc(x, R * (size_t)x->pstride * 4);
    x->pidx = (uint32_t*)salloc(x, R * (size_t)x->pstride * 4);
    x->out_ring = (int32_t*)salloc(x, (size_t)x->ring_cap * 4);
    x->forced = (int32_t*)salloc(x, (size_t)x->forced_cap * 4);
    x->prompt_dev = (int32_t*)salloc(x, (size_t)x->prompt_cap * 4);
    x->hall = (uint16_t*)salloc(x, (size_t)c.ctx * H * 2);
    x->rope_cos = (float*)salloc(x, (size_t)c.ctx * (c.rot_dims / 2) * 4);
    x->rope_sin = (float*)salloc(x, (size_t)c.ctx * (c.rot_dims / 2) * 4);
    if (x->s_fail || !x->rope_sin) { set_error("q27x_ctx_create: state arena sizing"); return fail(Q27X_E_NOMEM); }
    // RoPE tables (src/q27_attn.hip:239-247): double inv_freq and angle, rounded to float
    {
        const int half = c.rot_dims / 2;
        std::vector<float> cs((size_t)c.ctx * half), sn((size_t)c.ctx * half);
        const double l2t = log2(c.rope_theta);
        for (int p = 0; p < c.ctx; ++p)
            for (int f = 0; f < half; ++f) {
                const double ifq = exp2(-((double)(2 * f) / (double)c.rot_dims) * l2t);
                const double ang = (double)p * ifq;
                cs[(size_t)p * half + f] = (float)cos(ang);
                sn[(size_t)p * half + f] = (float)sin(ang);
            }
        if ((e = hipMemcpy(x->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) return fail(hip_fail(e, "rope"));
        if ((e = hipMemcpy(x->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) return fail(hip_fail(e, "rope"));
    }
    if ((e = hipHostMalloc((void**)&x->mbox, sizeof(Mailbox), hipHostMallocMapped)) != hipSuccess) return fail(hip_fail(e, "hipHostMalloc"));
    memset((void*)x->mbox, 0, sizeof(Mailbox));
    if ((e = hipHostGetDevicePointer((void**)&x->mbox_dev, (void*)x->mbox, 0)) != hipSuccess) return fail(hip_fail(e, "hipHostGetDevicePointer"));
    *out = x;
    return Q27X_OK;
}

int q27x_ctx_destroy(q27x_ctx* x) {
    if (!x) return Q27X_OK;
    (void)hipSetDevice(x->device);
    if (x->stream) (void)hipStreamSynchronize(x->stream);
    if (x->g_spec) (void)hipGraphExecDestroy(x->g_spec);
    if (x->g_plain) (void)hipGraphExecDestroy(x->g_plain);
    if (x->mbox) (void)hipHostFree((void*)x->mbox);
    for (PfBuf* b : { x->pf, x->pfx[0], x->pfx[1] })
        if (b) {
            for (void* p : b->allocs) (void)hipFree(p);
            delete b;
        }
    for (hipEvent_t e : x->pf_ev) (void)hipEventDestroy(e);
    for (hipStream_t ps : x->pf_stream) if (ps) (void)hipStreamDestroy(ps);
    for (void* p : x->pf_walloc) (void)hipFree(p);
    if (x->warena) (void)hipFree(x->warena);
    if (x->sarena) (void)hipFree(x->sarena);
    if (x->stream) (void)hipStreamDestroy(x->stream);
    delete x;
    return Q27X_OK;
}

static int gen_i8m(q27x_ctx* x, Mat& m, int rows, int K) {
    m.rows = rows; m.K = K;
    m.w = (int8_t*)walloc(x, (size_t)rows * K);
    m.s = (float*)walloc(x, (size_t)rows * (K / 64) * 4);
    if (!m.s) { set_error("weight arena sizing"); return Q27X_E_NOMEM; }
    x->weight_bytes += (size_t)rows * K + (size_t)rows * (K / 64) * 4;
    return Q27X_OK;
}
// Everything made from the current weights that a reload must not reuse: the captured round and
// plain-step graphs (their kernel arguments hold weight pointers, alphas, alpha selectors and input
// scales by value) and the prefill GEMM copies of the matrices. Both loaders call this before
// they touch the weight arena; nothing may still be running on the context's streams.
static int drop_weight_derived(q27x_ctx* x) {
    Q27X_HIP(hipSetDevice(x->device));
    Q27X_HIP(hipStreamSynchronize(x->stream));
    for (hipStream_t ps : x->pf_stream) if (ps) Q27X_HIP(hipStreamSynchronize(ps));
    if (x->g_spec) (void)hipGraphExecDestroy(x->g_spec);
    if (x->g_plain) (void)hipGraphExecDestroy(x->g_plain);
    x->g_spec = x->g_plain = nullptr;
    x->g_spec_k = 0;
    for (void* p : x->pf_walloc) (void)hipFree(p);
    x->pf_walloc.clear();
    x->pf_wready = 0;
    return Q27X_OK;
}
static uint16_t* gen_vec(q27x_ctx* x, uint64_t seed, uint64_t t, size_t n, float stdv, float mean, int uni) {
    uint16_t* p = (uint16_t*)walloc(x, n * 2);
    if (!p) return nullptr;
    x->weight_bytes += n * 2;
    if (launch_gen_bf16(p, n, tensor_key(seed, t), stdv, mean, uni, x->stream)) return nullptr;
    return p;
}

int q27x_load_synthetic(q27x_ctx* x, uint64_t seed) {
    if (!x) return Q27X_E_ARG;
    const q27x_config& c = x->c;
    const int H = x->H, I = x->I;
    hipStream_t s = x->stream;
    int rc = drop_weight_derived(x);
    if (rc) return rc;
    x->loaded = 0;
    x->woff = 0; x->weight_bytes = 0;
    // (a checkpoint loaded before may have left per-tensor scales: generated weights have none)
    for (LayerDev& Y : x->L) {
        Y.qkvz = Y.out_proj = Y.qkv = Y.o = Y.gu = Y.down = Mat{};
        Y.in_s_in = Y.in_s_post = Y.in_s_down = Y.in_s_out = 1.0f;
    }
    x->mtp.qkv = x->mtp.o = x->mtp.gu = Mat{};
    for (Mat& m : x->mtp.down4) m = Mat{};
    x->fc0 = x->fc1 = Mat{};
#define GEN(m, rows, K) if ((rc = gen_i8m(x, m, rows, K))) return rc
#define VEC(dst, t, n, sd, mn, uni) if (!((dst) = gen_vec(x, seed, t, n, sd, mn, uni))) { set_error("weight generation"); return Q27X_E_NOMEM; }
    // slices: 0 = one down matrix (trunk layers), 4 = four [H][I/4] column slices (the MTP layer)
    auto mlp = [&](LayerDev& Y, int code, int slices) -> int {
        int r2;
        VEC(Y.in_norm, tid(code, T_IN_NORM), H, 0.02f, 0.0f, 0);
        VEC(Y.post_norm, tid(code, T_POST_NORM), H, 0.02f, 0.0f, 0);
        if ((r2 = gen_i8m(x, Y.gu, 2 * I, H))) return r2;
        if ((r2 = launch_gen_i8(Y.gu.w, Y.gu.s, I, H, tensor_key(seed, tid(code, T_GATE)), 1, 0, s))) return r2;
        if ((r2 = launch_gen_i8(Y.gu.w, Y.gu.s, I, H, tensor_key(seed, tid(code, T_UP)), 1, 1, s))) return r2;
        if (slices) {
            for (int j = 0; j < 4; ++j) {
                if ((r2 = gen_i8m(x, Y.down4[j], H, I / 4))) return r2;
                if ((r2 = launch_gen_i8(Y.down4[j].w, Y.down4[j].s, H, I / 4, tensor_key(seed, tid(code, T_DOWN_S0 + j)),
                                        0, 0, s))) return r2;
            }
            return Q27X_OK;
        }
        if ((r2 = gen_i8m(x, Y.down, H, I))) return r2;
        if ((r2 = launch_gen_i8(Y.down.w, Y.down.s, H, I, tensor_key(seed, tid(code, T_DOWN)), 0, 0, s))) return r2;
        return Q27X_OK;
    };
    auto attn = [&](LayerDev& Y, int code) -> int {
        int r2;
        if ((r2 = gen_i8m(x, Y.qkv, x->qr + 2 * x->kvr, H))) return r2;
        if ((r2 = launch_gen_i8(Y.qkv.w, Y.qkv.s, x->qr, H, tensor_key(seed, tid(code, T_Q)), 0, 0, s))) return r2;
        if ((r2 = launch_gen_i8(Y.qkv.w + (size_t)x->qr * H, Y.qkv.s + (size_t)x->qr * (H / 64), x->kvr, H,
                                tensor_key(seed, tid(code, T_K)), 0, 0, s))) return r2;
        if ((r2 = launch_gen_i8(Y.qkv.w + (size_t)(x->qr + x->kvr) * H, Y.qkv.s + (size_t)(x->qr + x->kvr) * (H / 64),
                                x->kvr, H, tensor_key(seed, tid(code, T_V)), 0, 0, s))) return r2;
        VEC(Y.q_norm, tid(code, T_Q_NORM), c.head_dim, 0.02f, 0.0f, 0);
        VEC(Y.k_norm, tid(code, T_K_NORM), c.head_dim, 0.02f, 0.0f, 0);
        if ((r2 = gen_i8m(x, Y.o, H, x->att))) return r2;
        if ((r2 = launch_gen_i8(Y.o.w, Y.o.s, H, x->att, tensor_key(seed, tid(code, T_O)), 0, 0, s))) return r2;
        return Q27X_OK;
    };
    for (int l = 0; l < c.n_layers; ++l) {
        LayerDev& Y = x->L[l];
        const int code = l + 1;
        if ((rc = mlp(Y, code, 0))) return rc;
        if (Y.is_attn) { if ((rc = attn(Y, code))) return rc; continue; }
        GEN(Y.qkvz, x->nqkv + x->nz, H);
        if ((rc = launch_gen_i8(Y.qkvz.w, Y.qkvz.s, x->nqkv, H, tensor_key(seed, tid(code, T_IN_QKV)), 0, 0, s))) return rc;
        if ((rc = launch_gen_i8(Y.qkvz.w + (size_t)x->nqkv * H, Y.qkvz.s + (size_t)x->nqkv * (H / 64), x->nz, H,
                                tensor_key(seed, tid(code, T_IN_Z)), 0, 0, s))) return rc;
        VEC(Y.in_a, tid(code, T_IN_A), (size_t)c.gdn_vh * H, 0.02f, 0.0f, 0);
        VEC(Y.in_b, tid(code, T_IN_B), (size_t)c.gdn_vh * H, 0.02f, 0.0f, 0);
        VEC(Y.A_log, tid(code, T_A_LOG), c.gdn_vh, 2.7f, 0.0f, 1);
        VEC(Y.dt_bias, tid(code, T_DT_BIAS), c.gdn_vh, 0.1f, 0.0f, 0);
        VEC(Y.gdn_norm, tid(code, T_GDN_NORM), 128, 0.02f, 1.0f, 0);
        VEC(Y.conv_w, tid(code, T_CONV_W), (size_t)x->nqkv * 4, 0.3f, 0.0f, 0);
        GEN(Y.out_proj, H, x->nz);
        if ((rc = launch_gen_i8(Y.out_proj.w, Y.out_proj.s, H, x->nz, tensor_key(seed, tid(code, T_OUT_PROJ)), 0, 0, s))) return rc;
    }
    if ((rc = mlp(x->mtp, 1000, 4))) return rc;
    if ((rc = attn(x->mtp, 1000))) return rc;
    VEC(x->pre_emb, tid(1000, T_PRE_EMB), H, 0.02f, 0.0f, 0);
    VEC(x->pre_hid, tid(1000, T_PRE_HID), H, 0.02f, 0.0f, 0);
    VEC(x->mtp_norm, tid(1000, T_MTP_NORM), H, 0.02f, 0.0f, 0);
    GEN(x->fc0, H, H);
    if ((rc = launch_gen_i8(x->fc0.w, x->fc0.s, H, H, tensor_key(seed, tid(1000, T_FC0)), 0, 0, s))) return rc;
    GEN(x->fc1, H, H);
    if ((rc = launch_gen_i8(x->fc1.w, x->fc1.s, H, H, tensor_key(seed, tid(1000, T_FC1)), 0, 0, s))) return rc;
    VEC(x->emb, tid(0, T_EMB), (size_t)x->V * H, 1.0f, 0.0f, 0);
    VEC(x->final_norm, tid(0, T_FINAL_NORM), H, 0.02f, 0.0f, 0);
    VEC(x->lm_head, tid(0, T_LM_HEAD), (size_t)x->V * H, 0.02f, 0.0f, 0);
#undef GEN
#undef VEC
    Q27X_HIP(hipStreamSynchronize(s));
    x->loaded = 1;
    x->pf_wready = 0;   // the GEMM representations are remade from these weights
    return q27x_reset(x);
}

// ---------------------------------------------------------------- checkpoint plan and upload
// The tensors of a checkpoint in the reference's naming and formats (tp_plan / the group
// loaders, src/q27_load.cpp:690-815; the MTP head, src/q27_main.cpp:7134-7152) for this context's
// geometry. Trunk: MLP NVFP4 (weight U8 [R][K/2], weight_scale E4M3 [R][K/16], weight_scale_2,
// input_scale F32 scalars), attention and GDN projections fp8 E4M3 [R][K] with weight_scale and
// input_scale, norms / a / b / conv1d / A_log / dt_bias bf16; lm_head NVFP4; the MTP head bf16.
// Every matrix becomes the engine's int8 per-64 form (the reference's load-time mirror rule) with
// alpha = input_scale x weight_scale per source tensor; each projection's input is quantized with
// its input_scale; lm_head becomes bf16 (e2m1 x e4m3 x weight_scale_2), the MTP weights are
// quantized from their bf16 values (alpha 1, input_scale 1). Fail closed: a missing tensor is
// Q27X_E_MISSING, a wrong dtype or shape, a non-positive scale or gate/up (q/k/v) input scales
// that differ are Q27X_E_SHAPE.
namespace {
struct CkPlan {
    q27x_ctx* x;                  // null: check only
    const q27x_ckpt* ck;
    const q27x_config& c;
    char* err; size_t cap;
    int rc = Q27X_OK;
    void* stage = nullptr; size_t stage_cap = 0;
    int fail(int code, const char* fmt, ...) {
        if (rc) return rc;
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        if (err && cap) { strncpy(err, buf, cap - 1); err[cap - 1] = 0; }
        set_error("%s", buf);
        rc = code;
        return rc;
    }
    // the tensor, checked for dtype and element count (shape product; dims as given)
    bool get(const char* name, int dtype, long long n0, long long n1, CkTensor& T) {
        if (rc) return false;
        if (ckpt_get(ck, name, &T)) { fail(Q27X_E_MISSING, "checkpoint: '%s' missing", name); return false; }
        long long n = 1;
        for (int i = 0; i < T.ndim; ++i) n *= T.shape[i];
        const bool shape_ok = (n1 < 0) ? (n == n0) : (T.ndim == 2 && T.shape[0] == n0 && T.shape[1] == n1);
        if (T.dtype != dtype || !shape_ok) {
            fail(Q27X_E_SHAPE, "checkpoint: '%s' has dtype %d and %d dims (%lld x %lld), expected dtype %d, %lld x %lld",
                 name, T.dtype, T.ndim, T.ndim > 0 ? T.shape[0] : 0, T.ndim > 1 ? T.shape[1] : 0, dtype, n0, n1);
            return false;
        }
        return true;
    }
    float scalar(const char* name) {
        CkTensor T;
        if (!get(name, Q27X_DT_F32, 1, -1, T)) return 0.0f;
        float v;
        memcpy(&v, T.host, 4);
        if (!(v > 0.0f) || !(v < 1e30f)) { fail(Q27X_E_SHAPE, "checkpoint: '%s' = %g is not a positive scale", name, (double)v); return 0.0f; }
        return v;
    }
    void* staged(const CkTensor& T) {      // a device copy of the tensor's bytes (upload mode)
        if (!staged_resize(T.nbytes)) return nullptr;
        const hipError_t e = hipMemcpy(stage, T.host, T.nbytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { rc = hip_fail(e, "hipMemcpy (checkpoint)"); return nullptr; }
        return stage;
    }
    // bf16 vector / matrix of n elements into the weight arena
    void vec(const char* name, long long n, uint16_t** dst) {
        CkTensor T;
        if (!get(name, Q27X_DT_BF16, n, -1, T) || !x) return;
        *dst = (uint16_t*)walloc(x, (size_t)n * 2);
        if (!*dst) { fail(Q27X_E_NOMEM, "weight arena sizing"); return; }
        x->weight_bytes += (size_t)n * 2;
        const hipError_t e = hipMemcpy(*dst, T.host, (size_t)n * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpy (checkpoint)");
    }
    bool mat_alloc(Mat& m, int rows, int K) {
        if (!x || rc) return false;
        if (!m.w) {
            m.rows = rows; m.K = K;
            m.w = (int8_t*)walloc(x, (size_t)rows * K);
            m.s = (float*)walloc(x, (size_t)rows * (K / 64) * 4);
            if (!m.s) { fail(Q27X_E_NOMEM, "weight arena sizing"); return false; }
            x->weight_bytes += (size_t)rows * K + (size_t)rows * (K / 64) * 4;
        }
        return true;
    }
    // fp8 projection base.{weight, weight_scale, input_scale} [rows][K] -> rows row0.. of m;
    // returns alpha = input_scale x weight_scale
    float fp8(const char* base, int rows, int K, Mat& m, int mrows, int row0, float* in_scale) {
        char n[256];
        CkTensor T;
        snprintf(n, sizeof n, "%s.weight", base);
        const bool ok = get(n, Q27X_DT_F8_E4M3, rows, K, T);
        snprintf(n, sizeof n, "%s.weight_scale", base);
        const float ws = scalar(n);
        snprintf(n, sizeof n, "%s.input_scale", base);
        const float is = scalar(n);
        if (in_scale) *in_scale = is;
        if (ok && mat_alloc(m, mrows, K)) {
            const void* d = staged(T);
            if (d && !rc)
                rc = launch_to_i8g64(0, d, nullptr, rows, K, K, m.w + (size_t)row0 * K, m.s + (size_t)row0 * (K / 64), 0,
                                     x->stream);
            if (!rc) { const hipError_t e = hipStreamSynchronize(x->stream); if (e != hipSuccess) rc = hip_fail(e, "convert"); }
        }
        return is * ws;
    }
    // NVFP4 matrix base.{weight, weight_scale, weight_scale_2, input_scale} -> m (row_mode: 0 rows
    // 0.., 1 / 2 gate / up rows of the fused gate|up layout); returns alpha
    float nvfp4(const char* base, int rows, int K, Mat& m, int mrows, int row_mode, float* in_scale) {
        char n[256];
        CkTensor T, G;
        snprintf(n, sizeof n, "%s.weight", base);
        const bool ok = get(n, Q27X_DT_U8, rows, K / 2, T);
        snprintf(n, sizeof n, "%s.weight_scale", base);
        const bool okg = get(n, Q27X_DT_F8_E4M3, rows, K / 16, G);
        snprintf(n, sizeof n, "%s.weight_scale_2", base);
        const float ws2 = scalar(n);
        snprintf(n, sizeof n, "%s.input_scale", base);
        const float is = scalar(n);
        if (in_scale) *in_scale = is;
        if (ok && okg && mat_alloc(m, mrows, K)) {
            // (weights and group scales staged together)
            if (!staged_resize(T.nbytes + G.nbytes)) return 0.0f;
            hipError_t e = hipMemcpy(stage, T.host, T.nbytes, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy((char*)stage + T.nbytes, G.host, G.nbytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) { rc = hip_fail(e, "hipMemcpy (checkpoint)"); return 0.0f; }
            rc = launch_to_i8g64(1, stage, (char*)stage + T.nbytes, rows, K, K / 2, m.w, m.s, row_mode, x->stream);
            if (!rc) { e = hipStreamSynchronize(x->stream); if (e != hipSuccess) rc = hip_fail(e, "convert"); }
        }
        return is * ws2;
    }
    bool staged_resize(size_t bytes) {
        if (bytes <= stage_cap) return true;
        if (stage) (void)hipFree(stage);
        stage = nullptr; stage_cap = 0;
        const hipError_t e = hipMalloc(&stage, bytes);
        if (e != hipSuccess) { rc = hip_fail(e, "hipMalloc (checkpoint staging)"); return false; }
        stage_cap = bytes;
        return true;
    }
    // bf16 matrix [rows][ld] columns col0 .. col0+K -> rows row0.. of m, quantized per 64
    void bf16m(const char* name, int rows, int ld, int col0, int K, Mat& m, int mrows, int row0, int row_mode) {
        CkTensor T;
        if (!get(name, Q27X_DT_BF16, rows, ld, T) || !mat_alloc(m, mrows, K)) return;
        const void* d = staged(T);
        if (!d || rc) return;
        rc = launch_to_i8g64(2, (const uint16_t*)d + col0, nullptr, rows, K, ld,
                             row_mode ? m.w : m.w + (size_t)row0 * K, row_mode ? m.s : m.s + (size_t)row0 * (K / 64),
                             row_mode, x->stream);
        if (!rc) { const hipError_t e = hipStreamSynchronize(x->stream); if (e != hipSuccess) rc = hip_fail(e, "convert"); }
    }
};

int ckpt_plan(CkPlan& P) {
    q27x_ctx* x = P.x;
    const q27x_config& c = P.c;
    const int H = c.hidden, I = c.inter, hd = c.head_dim, D = c.gdn_d;
    const int qr = c.n_q * (c.attn_gate ? 2 * hd : hd), kvr = c.n_kv * hd, att = c.n_q * hd;
    const int nqkv = (2 * c.gdn_kh + c.gdn_vh) * D, nz = c.gdn_vh * D;
    static Mat scratch_m;                       // (check mode: no allocation)
    LayerDev dummy;
    char n[256], b[256];
    for (int l = 0; l < c.n_layers && !P.rc; ++l) {
        LayerDev& Y = x ? x->L[l] : dummy;
        const bool is_attn = is_attn_layer(c, l);
        snprintf(b, sizeof b, "model.language_model.layers.%d", l);
        snprintf(n, sizeof n, "%s.input_layernorm.weight", b); P.vec(n, H, &Y.in_norm);
        snprintf(n, sizeof n, "%s.post_attention_layernorm.weight", b); P.vec(n, H, &Y.post_norm);
        float gi = 0, ui = 0, di = 0;
        snprintf(n, sizeof n, "%s.mlp.gate_proj", b); const float ag = P.nvfp4(n, I, H, x ? Y.gu : scratch_m, 2 * I, 1, &gi);
        snprintf(n, sizeof n, "%s.mlp.up_proj", b); const float au = P.nvfp4(n, I, H, x ? Y.gu : scratch_m, 2 * I, 2, &ui);
        snprintf(n, sizeof n, "%s.mlp.down_proj", b); const float ad = P.nvfp4(n, H, I, x ? Y.down : scratch_m, H, 0, &di);
        if (!P.rc && gi != ui) return P.fail(Q27X_E_SHAPE, "layer %d: mlp gate input_scale %g != up input_scale %g", l, (double)gi, (double)ui);
        Y.gu.alpha = ag; Y.gu.asel = AlphaSel{}; Y.gu.asel.alpha_gu = 1; Y.gu.asel.alpha_b = au;
        Y.down.alpha = ad; Y.in_s_post = gi; Y.in_s_down = di;
        if (is_attn) {
            float qi = 0, ki = 0, vi = 0, oi = 0;
            snprintf(n, sizeof n, "%s.self_attn.q_proj", b); const float aq = P.fp8(n, qr, H, x ? Y.qkv : scratch_m, qr + 2 * kvr, 0, &qi);
            snprintf(n, sizeof n, "%s.self_attn.k_proj", b); const float ak = P.fp8(n, kvr, H, x ? Y.qkv : scratch_m, qr + 2 * kvr, qr, &ki);
            snprintf(n, sizeof n, "%s.self_attn.v_proj", b); const float av = P.fp8(n, kvr, H, x ? Y.qkv : scratch_m, qr + 2 * kvr, qr + kvr, &vi);
            snprintf(n, sizeof n, "%s.self_attn.o_proj", b); const float ao = P.fp8(n, H, att, x ? Y.o : scratch_m, H, 0, &oi);
            if (!P.rc && !(qi == ki && ki == vi))
                return P.fail(Q27X_E_SHAPE, "layer %d: q/k/v input_scale differ (%g / %g / %g)", l, (double)qi, (double)ki, (double)vi);
            Y.qkv.alpha = aq; Y.qkv.asel = AlphaSel{}; Y.qkv.asel.split_b = qr; Y.qkv.asel.alpha_b = ak;
            Y.qkv.asel.split_c = qr + kvr; Y.qkv.asel.alpha_c = av;
            Y.o.alpha = ao; Y.in_s_in = qi; Y.in_s_out = oi;
            snprintf(n, sizeof n, "%s.self_attn.q_norm.weight", b); P.vec(n, hd, &Y.q_norm);
            snprintf(n, sizeof n, "%s.self_attn.k_norm.weight", b); P.vec(n, hd, &Y.k_norm);
        } else {
            float qi = 0, zi = 0, oi = 0;
            snprintf(n, sizeof n, "%s.linear_attn.in_proj_qkv", b); const float aq = P.fp8(n, nqkv, H, x ? Y.qkvz : scratch_m, nqkv + nz, 0, &qi);
            snprintf(n, sizeof n, "%s.linear_attn.in_proj_z", b); const float az = P.fp8(n, nz, H, x ? Y.qkvz : scratch_m, nqkv + nz, nqkv, &zi);
            snprintf(n, sizeof n, "%s.linear_attn.out_proj", b); const float ao = P.fp8(n, H, nz, x ? Y.out_proj : scratch_m, H, 0, &oi);
            Y.qkvz.alpha = aq; Y.qkvz.asel = AlphaSel{}; Y.qkvz.asel.split_b = nqkv; Y.qkvz.asel.alpha_b = az;
            Y.out_proj.alpha = ao; Y.in_s_in = qi; Y.in_s_out = oi;
            snprintf(n, sizeof n, "%s.linear_attn.in_proj_a.weight", b); P.vec(n, (long long)c.gdn_vh * H, &Y.in_a);
            snprintf(n, sizeof n, "%s.linear_attn.in_proj_b.weight", b); P.vec(n, (long long)c.gdn_vh * H, &Y.in_b);
            snprintf(n, sizeof n, "%s.linear_attn.conv1d.weight", b); P.vec(n, (long long)nqkv * 4, &Y.conv_w);
            snprintf(n, sizeof n, "%s.linear_attn.A_log", b); P.vec(n, c.gdn_vh, &Y.A_log);
            snprintf(n, sizeof n, "%s.linear_attn.dt_bias", b); P.vec(n, c.gdn_vh, &Y.dt_bias);
            snprintf(n, sizeof n, "%s.linear_attn.norm.weight", b); P.vec(n, D, &Y.gdn_norm);
        }
    }
    if (P.rc) return P.rc;
    // globals
    uint16_t* dummy16 = nullptr;
    P.vec("model.language_model.embed_tokens.weight", (long long)c.vocab * H, x ? &x->emb : &dummy16);
    P.vec("model.language_model.norm.weight", H, x ? &x->final_norm : &dummy16);
    {
        CkTensor T, G;
        const bool ok = P.get("lm_head.weight", Q27X_DT_U8, c.vocab, H / 2, T);
        const bool okg = P.get("lm_head.weight_scale", Q27X_DT_F8_E4M3, c.vocab, H / 16, G);
        const float ws2 = P.scalar("lm_head.weight_scale_2");
        if (ok && okg && x && !P.rc) {
            x->lm_head = (uint16_t*)walloc(x, (size_t)c.vocab * H * 2);
            if (!x->lm_head) return P.fail(Q27X_E_NOMEM, "weight arena sizing");
            x->weight_bytes += (size_t)c.vocab * H * 2;
            if (!P.staged_resize(T.nbytes + G.nbytes)) return P.rc;
            hipError_t e = hipMemcpy(P.stage, T.host, T.nbytes, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy((char*)P.stage + T.nbytes, G.host, G.nbytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) return P.rc = hip_fail(e, "hipMemcpy (checkpoint)");
            if ((P.rc = launch_nvfp4_to_bf16(P.stage, (char*)P.stage + T.nbytes, ws2, c.vocab, H, x->lm_head, x->stream)))
                return P.rc;
            if ((e = hipStreamSynchronize(x->stream)) != hipSuccess) return P.rc = hip_fail(e, "convert");
        }
    }
    if (P.rc) return P.rc;
    // the MTP head (bf16; quantized per 64 from its values)
    LayerDev& M = x ? x->mtp : dummy;
    const char* B = "mtp.layers.0";
    snprintf(n, sizeof n, "%s.self_attn.q_proj.weight", B); P.bf16m(n, qr, H, 0, H, x ? M.qkv : scratch_m, qr + 2 * kvr, 0, 0);
    snprintf(n, sizeof n, "%s.self_attn.k_proj.weight", B); P.bf16m(n, kvr, H, 0, H, x ? M.qkv : scratch_m, qr + 2 * kvr, qr, 0);
    snprintf(n, sizeof n, "%s.self_attn.v_proj.weight", B); P.bf16m(n, kvr, H, 0, H, x ? M.qkv : scratch_m, qr + 2 * kvr, qr + kvr, 0);
    snprintf(n, sizeof n, "%s.self_attn.o_proj.weight", B); P.bf16m(n, H, att, 0, att, x ? M.o : scratch_m, H, 0, 0);
    snprintf(n, sizeof n, "%s.mlp.gate_proj.weight", B); P.bf16m(n, I, H, 0, H, x ? M.gu : scratch_m, 2 * I, 0, 1);
    snprintf(n, sizeof n, "%s.mlp.up_proj.weight", B); P.bf16m(n, I, H, 0, H, x ? M.gu : scratch_m, 2 * I, 0, 2);
    snprintf(n, sizeof n, "%s.mlp.down_proj.weight", B);
    for (int j = 0; j < 4; ++j) P.bf16m(n, H, I, j * (I / 4), I / 4, x ? M.down4[j] : scratch_m, H, 0, 0);
    P.bf16m("mtp.fc.weight", H, 2 * H, 0, H, x ? x->fc0 : scratch_m, H, 0, 0);
    P.bf16m("mtp.fc.weight", H, 2 * H, H, H, x ? x->fc1 : scratch_m, H, 0, 0);
    snprintf(n, sizeof n, "%s.input_layernorm.weight", B); P.vec(n, H, &M.in_norm);
    snprintf(n, sizeof n, "%s.post_attention_layernorm.weight", B); P.vec(n, H, &M.post_norm);
    snprintf(n, sizeof n, "%s.self_attn.q_norm.weight", B); P.vec(n, hd, &M.q_norm);
    snprintf(n, sizeof n, "%s.self_attn.k_norm.weight", B); P.vec(n, hd, &M.k_norm);
    P.vec("mtp.norm.weight", H, x ? &x->mtp_norm : &dummy16);
    P.vec("mtp.pre_fc_norm_embedding.weight", H, x ? &x->pre_emb : &dummy16);
    P.vec("mtp.pre_fc_norm_hidden.weight", H, x ? &x->pre_hid : &dummy16);
    return P.rc;
}
}  // namespace

int q27x_ckpt_check(const q27x_ckpt* ck, const q27x_config* cfg, char* err, size_t errcap) {
    if (!ck || !cfg) { set_error("q27x_ckpt_check: null argument"); return Q27X_E_ARG; }
    CkPlan P{nullptr, ck, *cfg, err, errcap};
    return ckpt_plan(P);
}

int q27x_load_checkpoint(q27x_ctx* x, const q27x_ckpt* ck, char* err, size_t errcap) {
    if (!x || !ck) { set_error("q27x_load_checkpoint: null argument"); return Q27X_E_ARG; }
    int rc = q27x_ckpt_check(ck, &x->c, err, errcap);
    if (rc) return rc;
    if ((rc = drop_weight_derived(x))) return rc;
    x->loaded = 0;
    x->woff = 0; x->weight_bytes = 0;
    for (LayerDev& Y : x->L) { Y.qkvz = Y.out_proj = Y.qkv = Y.o = Y.gu = Y.down = Mat{}; }
    x->mtp.qkv = x->mtp.o = x->mtp.gu = Mat{};
    for (Mat& m : x->mtp.down4) m = Mat{};
    x->fc0 = x->fc1 = Mat{};
    Q27X_HIP(hipSetDevice(x->device));
    CkPlan P{x, ck, x->c, err, errcap};
    rc = ckpt_plan(P);
    if (P.stage) (void)hipFree(P.stage);
    if (rc) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    x->loaded = 1;
    x->pf_wready = 0;
    return q27x_reset(x);
}

int q27x_weight_bytes(q27x_ctx* x, size_t* bytes) {
    if (!x || !bytes) return Q27X_E_ARG;
    *bytes = x->weight_bytes;
    return Q27X_OK;
}

int q27x_reset(q27x_ctx* x) {
    if (!x) return Q27X_E_ARG;
    const q27x_config& c = x->c;
    const size_t kvn = (size_t)c.ctx * x->kvr;
    hipStream_t s = x->stream;
    for (auto* Y : { (LayerDev*)nullptr }) (void)Y;
    for (int l = 0; l < c.n_layers; ++l) {
        LayerDev& Y = x->L[l];
        if (Y.is_attn) {
            Q27X_HIP(hipMemsetAsync(Y.kc, 0, kvn, s)); Q27X_HIP(hipMemsetAsync(Y.vc, 0, kvn, s));
            Q27X_HIP(hipMemsetAsync(Y.ks, 0, kvn / c.kv_group * 4, s)); Q27X_HIP(hipMemsetAsync(Y.vs, 0, kvn / c.kv_group * 4, s));
        } else {
            Q27X_HIP(hipMemsetAsync(Y.S, 0, (size_t)c.gdn_vh * 128 * 128 * 4, s));
            Q27X_HIP(hipMemsetAsync(Y.conv_st, 0, (size_t)x->nqkv * 32, s));
            Q27X_HIP(hipMemsetAsync(Y.pend, 0, gdn_pend_bytes(c.gdn_kh, c.gdn_vh, 128), s));
        }
    }
    Q27X_HIP(hipMemsetAsync(x->mtp.kc, 0, kvn, s)); Q27X_HIP(hipMemsetAsync(x->mtp.vc, 0, kvn, s));
    Q27X_HIP(hipMemsetAsync(x->mtp.ks, 0, kvn / c.kv_group * 4, s)); Q27X_HIP(hipMemsetAsync(x->mtp.vs, 0, kvn / c.kv_group * 4, s));
    Dctl h{};
    h.ctx = c.ctx;
    h.max_new = 0x7fffffff;
    h.eos0 = h.eos1 = -1;
    Q27X_HIP(hipMemcpyAsync(x->dctl, &h, sizeof h, hipMemcpyHostToDevice, s));
    Q27X_HIP(hipStreamSynchronize(s));
    memset((void*)x->mbox, 0, sizeof(Mailbox));
    x->prefilled = 0;
    return Q27X_OK;
}

// Prompt ingest through the verify path in chunks of 8 rows, then the MTP prompt conditioning.
int q27x_prefill(q27x_ctx* x, const int32_t* ids, int n, int32_t* first_token) {
    if (!x || !ids || n < 1) { set_error("q27x_prefill: bad arguments"); return Q27X_E_ARG; }
    if (!x->loaded) { set_error("q27x_prefill: no weights"); return Q27X_E_STATE; }
    if (n + x->c.spec_k + 2 > x->c.ctx || n > x->prompt_cap) { set_error("q27x_prefill: prompt of %d exceeds ctx %d", n, x->c.ctx); return Q27X_E_RANGE; }
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= x->V) { set_error("q27x_prefill: token %d out of range", ids[i]); return Q27X_E_RANGE; }
    int rc = q27x_reset(x);
    if (rc) return rc;
    const auto t0 = std::chrono::steady_clock::now();
    hipStream_t s = x->stream;
    const int H = x->H;
    Q27X_HIP(hipMemcpyAsync(x->prompt_dev, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
    int npend = 0;
    for (int c0 = 0; c0 < n; c0 += kMaxRows) {
        const int cn = (n - c0 < kMaxRows) ? n - c0 : kMaxRows;
        const int last = (c0 + cn == n);
        Q27X_HIP(hipMemcpyAsync(x->dctl->vtok, x->prompt_dev + c0, (size_t)cn * 4, hipMemcpyDeviceToDevice, s));
        if ((rc = set_ints(x, 2, DOFF(pos), c0, DOFF(gdn_npend), npend))) return rc;
        if ((rc = verify_pass(x, cn, last, x->hall + (size_t)c0 * H))) return rc;
        npend = cn;
    }
    int32_t first = 0;
    Q27X_HIP(hipMemcpyAsync(&first, &x->dctl->nx[(n - 1) % kMaxRows], 4, hipMemcpyDeviceToHost, s));
    // prompt conditioning: MTP position p pairs the final residual at p with token p+1
    for (int p0 = 0; p0 + 1 < n; p0 += kMaxRows) {
        const int cn = (n - 1 - p0 < kMaxRows) ? n - 1 - p0 : kMaxRows;
        Q27X_HIP(hipMemcpyAsync(x->dctl->mtp_tok, x->prompt_dev + p0 + 1, (size_t)cn * 4, hipMemcpyDeviceToDevice, s));
        Q27X_HIP(hipMemcpyAsync(x->mtp_hin, x->hall + (size_t)p0 * H, (size_t)cn * H * 2, hipMemcpyDeviceToDevice, s));
        if ((rc = set_ints(x, 2, DOFF(mtp_nact), cn, DOFF(mtp_dpos0), p0))) return rc;
        if ((rc = mtp_pass(x, cn, 0, 1))) return rc;
    }
    Q27X_HIP(hipMemcpyAsync(x->hprev, x->hall + (size_t)(n - 1) * H, (size_t)H * 2, hipMemcpyDeviceToDevice, s));
    Q27X_HIP(hipStreamSynchronize(s));
    if ((rc = set_ints(x, 4, DOFF(pos), n, DOFF(tok), first, DOFF(ncatch), 0, DOFF(gdn_npend), npend))) return rc;
    if ((rc = set_ints(x, 4, DOFF(committed), 1, DOFF(rounds), 0, DOFF(stop), 0, DOFF(max_new), 0x7fffffff))) return rc;
    Q27X_HIP(hipMemcpyAsync(x->out_ring, &first, 4, hipMemcpyHostToDevice, s));
    Q27X_HIP(hipStreamSynchronize(s));
    if ((rc = check_device_err(x))) return rc;
    x->prefilled = 1;
    x->n_prompt = n;
    if (first_token) *first_token = first;
    (void)t0;
    return Q27X_OK;
}

// ---------------------------------------------------------------- layer-major prefill (GEMM path)
// The prompt in chunks (pf_chunk), each chunk through every layer (ls_q8_layer's
// stage order, src/q27_main.cpp:4076-4316): every projection is the int8 MFMA GEMM of per-(row,
// group) weights and per-(token, group) activations (group 1024, or the whole K), each matrix
// brought to that representation from its per-64 mirror right before its GEMM; the norms, GDN
// conv / row scalars / scan, attention, SwiGLU and residual adds keep the decode path's
// arithmetic. The MTP prompt pass fills only the draft KV cache (src/q27_main.cpp:2647-2688).
constexpr int kPfAttnRows = 128;    // query rows per attention launch
// rows per attention row tile: up to 16, at most 64 query vectors per kv head (one block holds
// them); a launch's tiles take the work area of ceil(kPfAttnRows / tile) whole tiles
static int pf_attn_tile(const q27x_config& c) { return std::max(1, std::min(16, 64 / (c.n_q / c.n_kv))); }
static int pf_attn_work_rows(const q27x_config& c) {
    const int zr = pf_attn_tile(c);
    return (kPfAttnRows + zr - 1) / zr * zr;
}
static int env_int(const char* name, int def);
// Rows per pass over the layers for an n-token prompt: 1024 from 2048 tokens on, else 512 (with the two
// streams below, smaller chunks overlap more: at 4096 tokens 1024-row chunks measured 15.1K tok/s
// against 14.0K with 2048 and 11.3K with one stream; 512 and 768 were slower). Q27X_PF_CHUNK
// (8 .. 4096) overrides, read per call.
static int pf_chunk(int n) {
    const int v = env_int("Q27X_PF_CHUNK", n >= 2048 ? 1024 : 512);
    return v < 8 ? 8 : (v > 4096 ? 4096 : v);
}
// successive chunks on two streams, chunk c + 1's layer l behind chunk c's layer l (Q27X_PF_PIPE=0: one
// stream)
static int pf_streams() {   // chunks in flight: Q27X_PF_STREAMS (1 .. 3), default 2
    const int v = env_int("Q27X_PF_STREAMS", 2);
    return v < 1 ? 1 : (v > 3 ? 3 : v);
}
// K-group of the trunk's prefill GEMMs: the whole K (pf_gs 0, the reference default) or pf_gs
// columns when they divide K
static int pf_gs(const q27x_config& c, int K) { return (c.pf_gs > 0 && K % c.pf_gs == 0) ? c.pf_gs : K; }

static int pf_alloc(q27x_ctx* x, int cap, PfBuf** slot) {
    if (*slot && (*slot)->cap >= cap) return Q27X_OK;
    if (*slot) {
        Q27X_HIP(hipStreamSynchronize(x->stream));
        for (hipStream_t ps : x->pf_stream) if (ps) Q27X_HIP(hipStreamSynchronize(ps));
        for (void* p : (*slot)->allocs) (void)hipFree(p);
        delete *slot;
        *slot = nullptr;
    }
    const q27x_config& c = x->c;
    const int H = x->H, I = x->I;
    const int wz = x->nqkv + x->nz, wq = x->qr + 2 * x->kvr;
    const int kmax = std::max(std::max(H, I), std::max(x->nz, x->att));
    const int wmax = std::max(std::max(wz, wq), H);
    PfBuf* B = new PfBuf();
    B->cap = cap;
    auto A = [&](void** p, size_t bytes) -> int {
        const hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc (prefill buffers)");
        B->allocs.push_back(*p);
        return Q27X_OK;
    };
    const size_t C = (size_t)cap;
    const size_t ms = (size_t)x->max_splits;
    int rc = 0;
    if ((rc = A((void**)&B->x, C * H * 4)) || (rc = A((void**)&B->h, C * H * 2)) || (rc = A((void**)&B->y, C * H * 2)) ||
        (rc = A((void**)&B->yf, C * std::max(H, 2 * c.gdn_kh * x->D) * 4)) || (rc = A((void**)&B->xq, C * kmax)) || (rc = A((void**)&B->xs, C * 32 * 4)) ||
        (rc = A((void**)&B->xq2, C * H)) || (rc = A((void**)&B->xs2, C * 32 * 4)) ||
        (rc = A((void**)&B->pb, C * wmax * 2)) || (rc = A((void**)&B->qh, C * std::max(x->att, 1) * 2)) ||
        (rc = A((void**)&B->gu, C * std::max(2 * I, x->nz) * 4)) || (rc = A((void**)&B->mix, C * std::max(x->nz, x->att) * 2)) ||
        (rc = A((void**)&B->rowsc, 3 * C * c.gdn_vh * 4)) ||
        (rc = A((void**)&B->work, attn_work_floats(c.n_q, c.head_dim, (int)ms, pf_attn_work_rows(c)) * 4)) ||
        (rc = A((void**)&B->cv, C * x->nqkv * 2))) {
        for (void* p : B->allocs) (void)hipFree(p);
        delete B;
        return rc;
    }
    *slot = B;
    return Q27X_OK;
}

// y = GEMM(rows [r0, r0 + nrows) of W, the codes xq/xs of M rows) (+ the bf16 residual), y bf16
// or fp32 with row stride ldy
static int pf_gemm(q27x_ctx* x, const Mat& W, int r0, int nrows, const int8_t* xq, const float* xs, int M, void* y,
                   int ldy, int out_bf16, const void* res, int res_bf16 = 1) {
    const int K = W.K, gs = W.pgs;
    if (!W.pw || gs < 1) { set_error("prefill: no GEMM representation of a %d x %d matrix", W.rows, K); return Q27X_E_STATE; }
    // the stacked tensors' scales, for rows counted from r0
    AlphaSel as = W.asel;
    float a0 = W.alpha;
    if (r0 > 0 && !as.alpha_gu) {
        a0 = alpha_of(W.alpha, W.asel, r0);
        as.split_b = as.split_b > r0 ? as.split_b - r0 : 0;
        as.split_c = as.split_c > r0 ? as.split_c - r0 : 0;
        if (as.split_b == 0 && as.split_c > 0) { as.split_b = as.split_c; as.alpha_b = as.alpha_c; as.split_c = 0; }
    }
    return launch_gemm_i8g(W.pw + (size_t)r0 * K, W.ps + (size_t)r0 * (K / gs), nrows, K, gs, a0, xq, xs, M, y, ldy,
                           out_bf16, res, x->H, res_bf16, res ? 1.0f : 0.0f, x->pfs, &as);
}
// every matrix of the model in the GEMM representation (the reference keeps such per-(row, group)
// mirrors from load time, src/q27_epi.hip:14-35); made once per load, kept on the device
static int pf_weights(q27x_ctx* x) {
    if (x->pf_wready) return Q27X_OK;
    std::vector<Mat*> ms;
    for (LayerDev& Y : x->L) {
        for (Mat* m : { &Y.qkvz, &Y.out_proj, &Y.qkv, &Y.o, &Y.gu, &Y.down }) if (m->w) ms.push_back(m);
    }
    const size_t n_trunk = ms.size();
    for (Mat* m : { &x->fc0, &x->fc1, &x->mtp.qkv }) if (m->w) ms.push_back(m);
    for (size_t i = 0; i < ms.size(); ++i) {
        Mat* m = ms[i];
        // the MTP layer's matrices always in whole-K groups (src/q27_main.cpp:2625-2628, 2665-2668)
        const int K = m->K, gs = i < n_trunk ? pf_gs(x->c, K) : K;
        if (m->pw && m->pgs != gs) { set_error("prefill: GEMM representation group changed"); return Q27X_E_STATE; }
        m->pgs = gs;
        if (!m->pw) {
            hipError_t e = hipMalloc((void**)&m->pw, (size_t)m->rows * K);
            if (e != hipSuccess) return hip_fail(e, "hipMalloc (prefill weights)");
            x->pf_walloc.push_back(m->pw);
            e = hipMalloc((void**)&m->ps, (size_t)m->rows * (K / gs) * 4);
            if (e != hipSuccess) return hip_fail(e, "hipMalloc (prefill weight scales)");
            x->pf_walloc.push_back(m->ps);
        }
        const int rc = q27x_i8g64_to_grp(m->w, m->s, m->rows, K, gs, m->pw, m->ps, (q27x_stream_t)x->stream);
        if (rc) return rc;
    }
    x->pf_wready = 1;
    return Q27X_OK;
}
// norm of C rows (values to B.yf) and their per-(token, group) codes in groups of gs columns
static int pf_norm_quant(q27x_ctx* x, NormArgs n, int C, int8_t* xq, float* xs, int gs, float in_scale = 1.0f) {
    PfBuf& B = *x->pfc;
    n.yf = B.yf; n.yfstride = x->H;
    int rc = launch_norm(n, C, x->pfs);
    if (rc) return rc;
    return launch_quant_tok_grp(B.yf, x->H, C, x->H, gs, in_scale, xq, xs, x->pfs);
}

static int pf_layer(q27x_ctx* x, int l, int p0, int C) {
    const q27x_config& c = x->c;
    hipStream_t s = x->pfs;
    Dctl* d = x->dctl;
    PfBuf& B = *x->pfc;
    LayerDev& Y = x->L[l];
    const int H = x->H, I = x->I;
    int rc;
    NormArgs nin;
    if (l == 0) {
        nin = norm_of(x, nullptr, 1, Y.in_norm, 1.0f, 1, B.h, Y.is_attn ? nullptr : B.y);
        nin.emb = x->emb; nin.tok = x->prompt_dev + p0;
    } else {
        nin = norm_of(x, B.x, 0, Y.in_norm, 1.0f, 0, B.h, Y.is_attn ? nullptr : B.y);
    }
    const int gH = pf_gs(c, H);
    if ((rc = pf_norm_quant(x, nin, C, B.xq, B.xs, gH, Y.in_s_in))) return rc;
    if (Y.is_attn) {
        const int wq = Y.qkv.rows;
        if ((rc = pf_gemm(x, Y.qkv, 0, wq, B.xq, B.xs, C, B.pb, wq, 1, nullptr))) return rc;
        AttnArgs a{};
        a.qkv = B.pb; a.qkv_stride = wq; a.q_norm_w = Y.q_norm; a.k_norm_w = Y.k_norm;
        a.rope_cos = x->rope_cos; a.rope_sin = x->rope_sin; a.rot = c.rot_dims;
        a.kc = Y.kc; a.ks = Y.ks; a.vc = Y.vc; a.vs = Y.vs; a.kv_group = c.kv_group; a.qh = B.qh;
        a.nq = c.n_q; a.nkv = c.n_kv; a.hd = c.head_dim; a.gate = c.attn_gate; a.eps = c.rms_eps;
        a.pos0_imm = p0; a.sl2e = x->sl2e; a.stop = &d->stop;
        if ((rc = launch_attn_prep_rows(a, C, s))) return rc;
        const int zr = pf_attn_tile(c);
        for (int q0 = 0; q0 < C; q0 += kPfAttnRows) {
            const int cq = std::min(kPfAttnRows, C - q0);
            AttnArgs t = a;
            t.qh = B.qh + (size_t)q0 * x->att; t.qkv = B.pb + (size_t)q0 * wq; t.pos0_imm = p0 + q0;
            t.work = B.work; t.max_splits = (p0 + q0 + cq + kSplit - 1) / kSplit;
            t.zrows = zr; t.ztotal = cq; t.out = B.mix + (size_t)q0 * x->att;
            if ((rc = launch_attn(t, zr, s, false))) return rc;
        }
        if ((rc = launch_pf_quant_bf16(B.mix, x->att, C, x->att, pf_gs(c, x->att), Y.in_s_out, B.xq, B.xs, s))) return rc;
        if ((rc = pf_gemm(x, Y.o, 0, H, B.xq, B.xs, C, B.x, H, 0, B.h))) return rc;
    } else {
        const int wz = Y.qkvz.rows;
        if ((rc = pf_gemm(x, Y.qkvz, 0, wz, B.xq, B.xs, C, B.pb, wz, 1, nullptr))) return rc;
        if ((rc = launch_pf_ab(Y.in_a, Y.in_b, Y.A_log, Y.dt_bias, B.y, H, H, c.gdn_vh, C, B.rowsc, s))) return rc;
        if ((rc = launch_pf_conv(B.pb, wz, C, x->nqkv, Y.conv_w, Y.conv_st, 0, B.cv, x->nqkv, s))) return rc;
        GdnArgs g{};
        g.qkv = B.cv; g.qkv_stride = x->nqkv; g.z = B.pb + x->nqkv; g.z_stride = wz;
        g.rowsc = B.rowsc; g.norm_w = Y.gdn_norm; g.S = Y.S;
        g.kh = c.gdn_kh; g.vh = c.gdn_vh; g.d = x->D; g.eps = c.rms_eps;
        g.out = B.mix; g.out_stride = x->nz; g.stop = &d->stop;
        // scratch: yf (free after the in_qkv|in_z GEMM's quantizer) for q^|k^, the third rowsc
        // slab for k^.q^, the gate|up output (free until the MLP) for the mixed rows
        if ((rc = launch_gdn_scan(g, C, B.yf, B.rowsc + (size_t)2 * B.cap * c.gdn_vh, B.gu, s))) return rc;
        if ((rc = launch_pf_quant_bf16(B.mix, x->nz, C, x->nz, pf_gs(c, x->nz), Y.in_s_out, B.xq, B.xs, s))) return rc;
        if ((rc = pf_gemm(x, Y.out_proj, 0, H, B.xq, B.xs, C, B.x, H, 0, B.h))) return rc;
    }
    if ((rc = pf_norm_quant(x, norm_of(x, B.x, 0, Y.post_norm, 1.0f, 0, B.h, nullptr), C, B.xq, B.xs, gH,
                            Y.in_s_post)))
        return rc;
    if ((rc = pf_gemm(x, Y.gu, 0, 2 * I, B.xq, B.xs, C, B.gu, 2 * I, 0, nullptr))) return rc;
    if ((rc = launch_pf_swiglu_quant(B.gu, I, pf_gs(c, I), 1.0f / Y.in_s_down, C, B.xq, B.xs, s))) return rc;
    return pf_gemm(x, Y.down, 0, H, B.xq, B.xs, C, B.x, H, 0, B.h);
}

// the MTP prompt pass over draft positions p0 .. p0 + C - 1 (final residual rows hall[p], token p+1)
static int pf_mtp(q27x_ctx* x, int p0, int C) {
    const q27x_config& c = x->c;
    Dctl* d = x->dctl;
    PfBuf& B = *x->pfc;
    LayerDev& M = x->mtp;
    const int H = x->H;
    const float po = c.mtp_plus_one ? 1.0f : 0.0f;
    int rc;
    NormArgs ne = norm_of(x, nullptr, 1, x->pre_emb, po, 0, nullptr, nullptr);
    ne.emb = x->emb; ne.tok = x->prompt_dev + p0 + 1;
    // (every quantizer of the MTP prompt pass in whole-K groups, as its GEMM weights)
    if ((rc = pf_norm_quant(x, ne, C, B.xq, B.xs, H))) return rc;
    if ((rc = pf_norm_quant(x, norm_of(x, x->hall + (size_t)p0 * H, 1, x->pre_hid, po, 0, nullptr, nullptr), C,
                            B.xq2, B.xs2, H))) return rc;
    const Mat& fe = c.mtp_swap ? x->fc0 : x->fc1;    // the half that multiplies the embedding
    const Mat& fh = c.mtp_swap ? x->fc1 : x->fc0;
    if ((rc = pf_gemm(x, fe, 0, H, B.xq, B.xs, C, B.x, H, 0, nullptr))) return rc;
    // (fp32 residual: the first half's output, read and written in place)
    if ((rc = pf_gemm(x, fh, 0, H, B.xq2, B.xs2, C, B.x, H, 0, B.x, 0))) return rc;
    if ((rc = pf_norm_quant(x, norm_of(x, B.x, 0, M.in_norm, po, 0, nullptr, nullptr), C, B.xq, B.xs, H))) return rc;
    const int wq = M.qkv.rows;
    if ((rc = pf_gemm(x, M.qkv, x->qr, 2 * x->kvr, B.xq, B.xs, C, B.pb + x->qr, wq, 1, nullptr))) return rc;
    AttnArgs a{};
    a.qkv = B.pb; a.qkv_stride = wq; a.q_norm_w = M.q_norm; a.k_norm_w = M.k_norm;
    a.rope_cos = x->rope_cos; a.rope_sin = x->rope_sin; a.rot = c.rot_dims;
    a.kc = M.kc; a.ks = M.ks; a.vc = M.vc; a.vs = M.vs; a.kv_group = c.kv_group;
    a.nq = c.n_q; a.nkv = c.n_kv; a.hd = c.head_dim; a.gate = c.attn_gate; a.eps = c.rms_eps;
    a.pos0_imm = p0; a.prep_kv_only = 1; a.stop = &d->stop;
    return launch_attn_prep_rows(a, C, x->pfs);
}

int q27x_prefill_gemm(q27x_ctx* x, const int32_t* ids, int n, int32_t* first_token) {
    if (!x || !ids || n < 1) { set_error("q27x_prefill_gemm: bad arguments"); return Q27X_E_ARG; }
    if (!x->loaded) { set_error("q27x_prefill_gemm: no weights"); return Q27X_E_STATE; }
    if (n + x->c.spec_k + 2 > x->c.ctx || n > x->prompt_cap) {
        set_error("q27x_prefill_gemm: prompt of %d exceeds ctx %d", n, x->c.ctx);
        return Q27X_E_RANGE;
    }
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= x->V) { set_error("q27x_prefill_gemm: token %d out of range", ids[i]); return Q27X_E_RANGE; }
    int rc = q27x_reset(x);
    if (rc) return rc;
    const int chunk = pf_chunk(n);
    const int NS = (n > chunk) ? std::min(pf_streams(), (n + chunk - 1) / chunk) : 1;
    const bool pipe = NS > 1;
    if ((rc = pf_alloc(x, std::min(n, chunk), &x->pf))) return rc;
    for (int k = 1; k < NS; ++k)
        if ((rc = pf_alloc(x, chunk, &x->pfx[k - 1]))) return rc;
    if ((rc = pf_weights(x))) return rc;
    hipStream_t s = x->stream;
    Dctl* d = x->dctl;
    const q27x_config& c = x->c;
    const int H = x->H;
    const int NE = c.n_layers + 2;                 // per buffer set: one event per layer, the MTP pass, the end
    if (pipe) {
        for (int k = 1; k < NS; ++k)
            if (!x->pf_stream[k - 1]) {
                const hipError_t e = hipStreamCreateWithFlags(&x->pf_stream[k - 1], hipStreamNonBlocking);
                if (e != hipSuccess) return hip_fail(e, "hipStreamCreate (prefill)");
            }
        while ((int)x->pf_ev.size() < 3 * NE + 1) {
            hipEvent_t ev;
            const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
            if (e != hipSuccess) return hip_fail(e, "hipEventCreate (prefill)");
            x->pf_ev.push_back(ev);
        }
    }
    Q27X_HIP(hipMemcpyAsync(x->prompt_dev, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
    if (pipe) {                                     // the other streams start behind the upload and the weights
        Q27X_HIP(hipEventRecord(x->pf_ev[3 * NE], s));
        for (int k = 1; k < NS; ++k) Q27X_HIP(hipStreamWaitEvent(x->pf_stream[k - 1], x->pf_ev[3 * NE], 0));
    }
    // Chunk i runs on buffer set and stream i % NS. Its layer l waits for chunk i - 1's layer l (the
    // GDN state and conv records, the KV cache rows before its own), its MTP pass for chunk i - 1's
    // (the draft KV); its buffers were last used by chunk i - NS on the same stream.
    int ci = 0;
    for (int p0 = 0; p0 < n; p0 += chunk, ++ci) {
        const int C = std::min(chunk, n - p0);
        const int sl = ci % NS, sp = (ci + NS - 1) % NS;
        x->pfc = sl ? x->pfx[sl - 1] : x->pf;
        x->pfs = sl ? x->pf_stream[sl - 1] : s;
        hipEvent_t* ev = pipe ? &x->pf_ev[(size_t)sl * NE] : nullptr;
        hipEvent_t* evp = pipe ? &x->pf_ev[(size_t)sp * NE] : nullptr;
        for (int l = 0; l < c.n_layers; ++l) {
            if (pipe && ci > 0) Q27X_HIP(hipStreamWaitEvent(x->pfs, evp[l], 0));
            if ((rc = pf_layer(x, l, p0, C))) return rc;
            if (pipe) Q27X_HIP(hipEventRecord(ev[l], x->pfs));
        }
        // the rows' final residuals: bf16(bf16(r1) + r2) (the reference's double add) or bf16(r2)
        NormArgs hn{};
        hn.x = x->pfc->x; hn.x_bf16 = 0; hn.xstride = H; hn.hadd = c.head_double_residual ? x->pfc->h : nullptr;
        hn.hout = x->hall + (size_t)p0 * H; hn.w = x->final_norm; hn.plus = 1.0f; hn.eps = c.rms_eps; hn.n = H;
        hn.ystride = H; hn.in_scale = 1.0f; hn.stop = &d->stop;
        if ((rc = launch_norm(hn, C, x->pfs))) return rc;
        const int cm = (p0 + C < n) ? C : C - 1;     // MTP positions p with p + 1 < n
        if (pipe && ci > 0) Q27X_HIP(hipStreamWaitEvent(x->pfs, evp[c.n_layers], 0));
        if (cm > 0 && (rc = pf_mtp(x, p0, cm))) return rc;
        if (pipe) {
            Q27X_HIP(hipEventRecord(ev[c.n_layers], x->pfs));
            Q27X_HIP(hipEventRecord(ev[c.n_layers + 1], x->pfs));
        }
    }
    if (pipe) Q27X_HIP(hipStreamWaitEvent(s, x->pf_ev[(size_t)((ci - 1) % NS) * NE + c.n_layers + 1], 0));
    x->pfc = x->pf;
    x->pfs = s;
    // head of the last row: final norm, lm_head, argmax
    NormArgs hf = norm_of(x, x->hall + (size_t)(n - 1) * H, 1, x->final_norm, 1.0f, 1, nullptr, x->ynorm);
    if ((rc = launch_norm(hf, 1, s))) return rc;
    GemvArgs ga{};
    ga.W = x->lm_head; ga.rows = x->V; ga.K = H; ga.x = x->ynorm; ga.xst = H;
    ga.pval = x->pval; ga.pidx = x->pidx; ga.pstride = x->pstride; ga.stop = &d->stop;
    int nb = 0;
    if ((rc = launch_gemv(ga, 1, 1, &nb, s))) return rc;
    if ((rc = launch_argmax_final(x->pval, x->pidx, x->pstride, nb, 1, d->nx, d->nxval, &d->stop, s))) return rc;
    int32_t first = 0;
    Q27X_HIP(hipMemcpyAsync(&first, &d->nx[0], 4, hipMemcpyDeviceToHost, s));
    Q27X_HIP(hipMemcpyAsync(x->hprev, x->hall + (size_t)(n - 1) * H, (size_t)H * 2, hipMemcpyDeviceToDevice, s));
    Q27X_HIP(hipStreamSynchronize(s));
    if ((rc = set_ints(x, 4, DOFF(pos), n, DOFF(tok), first, DOFF(ncatch), 0, DOFF(gdn_npend), 0))) return rc;
    if ((rc = set_ints(x, 4, DOFF(committed), 1, DOFF(rounds), 0, DOFF(stop), 0, DOFF(max_new), 0x7fffffff))) return rc;
    Q27X_HIP(hipMemcpyAsync(x->out_ring, &first, 4, hipMemcpyHostToDevice, s));
    Q27X_HIP(hipStreamSynchronize(s));
    if ((rc = check_device_err(x))) return rc;
    x->prefilled = 1;
    x->n_prompt = n;
    if (first_token) *first_token = first;
    return Q27X_OK;
}

// The graph of a speculative round (spec = 1) or a plain step (spec = 0), built on first use.
static int ensure_graph(q27x_ctx* x, int spec) {
    if (!use_graphs()) return Q27X_OK;
    hipGraphExec_t* g = spec ? &x->g_spec : &x->g_plain;
    if (spec && x->g_spec && x->g_spec_k != x->c.spec_k) { (void)hipGraphExecDestroy(x->g_spec); x->g_spec = nullptr; }
    if (!*g) {
        int rc = build_graph(x, spec, g);
        if (rc) return rc;
        if (spec) x->g_spec_k = x->c.spec_k;
    }
    return Q27X_OK;
}
static int run_step(q27x_ctx* x, int spec) {
    if (use_graphs()) {
        int rc = ensure_graph(x, spec);
        if (rc) return rc;
        Q27X_HIP(hipGraphLaunch(spec ? x->g_spec : x->g_plain, x->stream));
        return Q27X_OK;
    }
    return spec ? enqueue_spec_round(x) : enqueue_plain_step(x);
}

// Start of every decode call: wait for the stream, read the control block into h, and re-arm it
// for a call that may commit up to max_new tokens in total. A call that reached its budget left
// stop = 1; the next call clears it, so decode continues from the current state. A device error
// stays set and is reported (a new prompt resets it).
// Arms the next launches: max_new, the stop flag, and the stop tokens (eos: q27x_generate; the
// single-step entries pass none). With stop tokens, the tokens already committed since the prompt
// (its first token, earlier calls) are searched first: a request that already holds one is over.
static int arm(q27x_ctx* x, int max_new, Dctl* h, bool eos = false) {
    Q27X_HIP(hipStreamSynchronize(x->stream));
    Q27X_HIP(hipMemcpy(h, x->dctl, sizeof *h, hipMemcpyDeviceToHost));
    if (h->err) return check_device_err(x);
    int e0 = -1, e1 = -1, emit = 0;
    if (eos) {
        e0 = x->c.eos_id;
        e1 = x->c.eos_id2;
        const int n = h->committed < x->ring_cap ? h->committed : x->ring_cap;
        if (n > 0 && (e0 >= 0 || e1 >= 0)) {
            std::vector<int32_t> toks((size_t)n);
            Q27X_HIP(hipMemcpy(toks.data(), x->out_ring, (size_t)n * 4, hipMemcpyDeviceToHost));
            for (int i = 0; i < n && !emit; ++i)
                if (toks[i] == e0 || toks[i] == e1) emit = i + 1;
        }
    }
    const int stop = (h->committed >= max_new || emit > 0) ? 1 : 0;
    int rc = set_ints(x, 2, DOFF(max_new), max_new, DOFF(stop), stop);
    if (!rc) rc = set_ints(x, 3, DOFF(eos0), e0, DOFF(eos1), e1, DOFF(emit_end), emit);
    if (rc) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    h->max_new = max_new;
    h->stop = stop;
    h->eos0 = e0;
    h->eos1 = e1;
    h->emit_end = emit;
    memset((void*)x->mbox, 0, sizeof(Mailbox));   // no kernel is in flight
    return Q27X_OK;
}

static void fill_stats(q27x_ctx* x, q27x_stats* st, const Dctl& h0, const Dctl& h, long long committed, double ms) {
    if (!st) return;
    memset(st, 0, sizeof *st);
    st->rounds = h.rounds - h0.rounds;
    st->committed = committed;
    st->accepted = h.accepted - h0.accepted;
    for (int j = 0; j < 9; ++j) st->acc_hist[j] = h.acc_hist[j] - h0.acc_hist[j];
    st->decode_ms = ms;
    const double tick_ms = x->wclk_khz > 0 ? 1.0 / x->wclk_khz : 0.0;
    st->draft_ms = (double)(h.sp_t[0] - h0.sp_t[0]) * tick_ms;
    st->verify_ms = (double)(h.sp_t[1] - h0.sp_t[1]) * tick_ms;
    st->head_ms = (double)(h.sp_t[2] - h0.sp_t[2]) * tick_ms;
    st->tail_ms = (double)(h.sp_t[3] - h0.sp_t[3]) * tick_ms;
}

int q27x_decode_step(q27x_ctx* x, int32_t* out_token) {
    if (!x || !x->prefilled) { set_error("q27x_decode_step: no prefill"); return Q27X_E_STATE; }
    Dctl h;
    int rc = arm(x, 0x7fffffff, &h);
    if (rc) return rc;
    if (h.pos >= x->c.ctx) { set_error("context capacity exhausted (ctx=%d)", x->c.ctx); return Q27X_E_RANGE; }
    if ((rc = run_step(x, 0))) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    if ((rc = check_device_err(x))) return rc;
    int32_t t = 0;
    Q27X_HIP(hipMemcpy(&t, &x->dctl->nx[0], 4, hipMemcpyDeviceToHost));
    if (out_token) *out_token = t;
    return Q27X_OK;
}

// One round. As in the reference's decode loop, a speculative round runs only while pos + K < ctx
// (src/q27_main.cpp:6391); nearer the end of the context the call takes a plain step (ncommit = 1).
int q27x_spec_round(q27x_ctx* x, int32_t* out_tokens, int* ncommit) {
    if (!x || !x->prefilled) { set_error("q27x_spec_round: no prefill"); return Q27X_E_STATE; }
    Dctl h;
    int rc = arm(x, 0x7fffffff, &h);
    if (rc) return rc;
    if (h.pos >= x->c.ctx) { set_error("context capacity exhausted (ctx=%d)", x->c.ctx); return Q27X_E_RANGE; }
    const int spec = h.pos + x->c.spec_k < x->c.ctx;
    if ((rc = run_step(x, spec))) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    if ((rc = check_device_err(x))) return rc;
    Q27X_HIP(hipMemcpy(&h, x->dctl, sizeof h, hipMemcpyDeviceToHost));
    const int nc = spec ? h.ncommit_last : 1;
    if (ncommit) *ncommit = nc;
    if (out_tokens) for (int j = 0; j < nc; ++j) out_tokens[j] = h.nx[j];
    return Q27X_OK;
}

int q27x_mtp_draft(q27x_ctx* x, const uint16_t* hrows, const int32_t* toks, int nr, int dpos0, int head_row,
                   uint16_t* res, int32_t* token, q27x_stream_t s) {
    if (!x || !hrows || !toks || nr < 1 || nr > kMaxRows || dpos0 < 0 || dpos0 + nr > x->c.ctx || head_row >= nr ||
        (token && head_row < 0)) {
        set_error("q27x_mtp_draft: bad arguments (nr=%d dpos0=%d head_row=%d)", nr, dpos0, head_row);
        return Q27X_E_ARG;
    }
    if (!x->loaded) { set_error("q27x_mtp_draft: no weights"); return Q27X_E_STATE; }
    const int H = x->H;
    hipEvent_t e;
    Q27X_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    int rc = Q27X_OK;
    auto run = [&]() -> int {
        Q27X_HIP(hipEventRecord(e, (hipStream_t)s));
        Q27X_HIP(hipStreamWaitEvent(x->stream, e, 0));
        Q27X_HIP(hipMemcpyAsync(x->mtp_hin, hrows, (size_t)nr * H * 2, hipMemcpyDeviceToDevice, x->stream));
        Q27X_HIP(hipMemcpyAsync(x->dctl->mtp_tok, toks, (size_t)nr * 4, hipMemcpyDeviceToDevice, x->stream));
        int r = set_ints(x, 4, DOFF(mtp_nact), nr, DOFF(mtp_dpos0), dpos0, DOFF(mtp_head), head_row < 0 ? 0 : head_row,
                         DOFF(stop), 0);
        if (r) return r;
        if ((r = mtp_pass(x, nr, head_row >= 0, 0))) return r;
        if (res) Q27X_HIP(hipMemcpyAsync(res, x->mtp_res, (size_t)nr * H * 2, hipMemcpyDeviceToDevice, x->stream));
        if (token) Q27X_HIP(hipMemcpyAsync(token, &x->dctl->mtp_out, 4, hipMemcpyDeviceToDevice, x->stream));
        Q27X_HIP(hipEventRecord(e, x->stream));
        Q27X_HIP(hipStreamWaitEvent((hipStream_t)s, e, 0));
        return Q27X_OK;
    };
    rc = run();
    (void)hipEventDestroy(e);
    return rc;
}

int q27x_set_forced_drafts(q27x_ctx* x, const int32_t* toks, int n) {
    if (!x || n < 0 || (n > 0 && !toks) || n > x->forced_cap) { set_error("q27x_set_forced_drafts: bad arguments"); return Q27X_E_ARG; }
    for (int i = 0; i < n; ++i)
        if (toks[i] < 0 || toks[i] >= x->V) { set_error("q27x_set_forced_drafts: token %d out of range", toks[i]); return Q27X_E_RANGE; }
    if (n) Q27X_HIP(hipMemcpy(x->forced, toks, (size_t)n * 4, hipMemcpyHostToDevice));
    const int base = x->n_prompt;
    int rc = set_ints(x, 3, DOFF(forced_on), n > 0 ? 1 : 0, DOFF(forced_n), n, DOFF(forced_base), base);
    if (rc) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    return Q27X_OK;
}

// The decode loop (src/q27_main.cpp:6382-6696). Steps are launched with two in flight; the host
// learns each one's outcome from the pinned mailbox one step late. Near the end of the context
// (when the position bound of the launched steps says the next round might not fit) it drains
// the stream, reads the exact position, and switches to plain steps once pos + K >= ctx, as the
// reference does (6391); the request ends when max_new tokens are committed or the context is full.
int q27x_generate(q27x_ctx* x, int max_new, int spec, int32_t* out, int* n_out, q27x_stats* st) {
    if (!x || !x->prefilled || max_new < 1 || !out) { set_error("q27x_generate: bad arguments"); return Q27X_E_ARG; }
    if (max_new > x->ring_cap) max_new = x->ring_cap;   // a request never commits more than the context holds
    Dctl h0;
    int rc = arm(x, max_new, &h0, true);
    if (rc) return rc;
    const int K = x->c.spec_k, ctx = x->c.ctx;
    // graphs built outside the timed loop (the plain one is needed at the context edge)
    if ((rc = ensure_graph(x, 0))) return rc;
    if (spec && (rc = ensure_graph(x, 1))) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<hipEvent_t> ev(2, nullptr);
    for (auto& e : ev) Q27X_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    long long launched = 0;
    long long pos_hi = h0.pos;              // bound of the position after every launched step
    int mode = spec ? 1 : 0;
    bool done = h0.stop != 0;
    while (!done && launched < (long long)ctx + 2) {
        if (launched >= 2) {
            if ((rc = (int)hipEventSynchronize(ev[launched & 1])) != 0) { rc = hip_fail((hipError_t)rc, "hipEventSynchronize"); break; }
            if (x->mbox->stop || x->mbox->committed >= max_new) break;
        }
        if (pos_hi + (mode ? K + 1 : 1) > ctx) {
            if ((rc = (int)hipStreamSynchronize(x->stream)) != 0) { rc = hip_fail((hipError_t)rc, "hipStreamSynchronize"); break; }
            Dctl h;
            if ((rc = (int)hipMemcpy(&h, x->dctl, sizeof h, hipMemcpyDeviceToHost)) != 0) { rc = hip_fail((hipError_t)rc, "hipMemcpy"); break; }
            if (h.stop || h.err || h.committed >= max_new) break;
            pos_hi = h.pos;
            if (mode && h.pos + K >= ctx) mode = 0;
            if (!mode && h.pos >= ctx) break;
        }
        if ((rc = run_step(x, mode))) break;
        if ((rc = (int)hipEventRecord(ev[launched & 1], x->stream)) != 0) { rc = hip_fail((hipError_t)rc, "hipEventRecord"); break; }
        ++launched;
        pos_hi += mode ? K + 1 : 1;
    }
    Q27X_HIP(hipStreamSynchronize(x->stream));
    const auto t1 = std::chrono::steady_clock::now();
    for (auto& e : ev) (void)hipEventDestroy(e);
    if (rc) return rc;
    if ((rc = check_device_err(x))) return rc;
    Dctl h;
    Q27X_HIP(hipMemcpy(&h, x->dctl, sizeof h, hipMemcpyDeviceToHost));
    int n = h.committed < max_new ? h.committed : max_new;
    if (h.emit_end > 0 && h.emit_end < n) n = h.emit_end;   // through the first stop token
    Q27X_HIP(hipMemcpy(out, x->out_ring, (size_t)n * 4, hipMemcpyDeviceToHost));
    if (n_out) *n_out = n;
    fill_stats(x, st, h0, h, h.committed - h0.committed, std::chrono::duration<double, std::milli>(t1 - t0).count());
    return Q27X_OK;
}

// Exactly n rounds (spec) or plain steps back to back from the current state, one graph launch
// each, no host synchronisation in between; stats over those rounds (wall clock around the launches
// and the final synchronisation). A round past the end of the context is an error (Q27X_E_RANGE).
int q27x_run_rounds(q27x_ctx* x, int n, int spec, q27x_stats* st) {
    if (!x || !x->prefilled || n < 1) { set_error("q27x_run_rounds: bad arguments"); return Q27X_E_ARG; }
    Dctl h0;
    int rc = arm(x, 0x7fffffff, &h0);
    if (rc) return rc;
    if ((rc = ensure_graph(x, spec))) return rc;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n && !rc; ++i) rc = run_step(x, spec);
    Q27X_HIP(hipStreamSynchronize(x->stream));
    const auto t1 = std::chrono::steady_clock::now();
    if (rc) return rc;
    if ((rc = check_device_err(x))) return rc;
    Dctl h;
    Q27X_HIP(hipMemcpy(&h, x->dctl, sizeof h, hipMemcpyDeviceToHost));
    fill_stats(x, st, h0, h, h.committed - h0.committed, std::chrono::duration<double, std::milli>(t1 - t0).count());
    return Q27X_OK;
}

int q27x_bench_verify(q27x_ctx* x, int nr, int iters, float* ms) {
    if (!x || !x->loaded || nr < 1 || nr > kMaxRows || iters < 1 || !ms) return Q27X_E_ARG;
    // a finished request leaves the stop flag set, which would make every kernel return at once
    int rc = set_ints(x, 1, DOFF(stop), 0);
    if (rc) return rc;
    hipEvent_t a, b;
    Q27X_HIP(hipEventCreate(&a));
    Q27X_HIP(hipEventCreate(&b));
    if ((rc = verify_pass(x, nr, 1, nullptr))) return rc;
    Q27X_HIP(hipEventRecord(a, x->stream));
    for (int i = 0; i < iters && !rc; ++i) rc = verify_pass(x, nr, 1, nullptr);
    Q27X_HIP(hipEventRecord(b, x->stream));
    Q27X_HIP(hipEventSynchronize(b));
    float t = 0.0f;
    Q27X_HIP(hipEventElapsedTime(&t, a, b));
    *ms = t / (float)iters;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return rc;
}

// Time one projection launch of the verify path (hipEvents on the engine's stream) and report its
// algorithmic bytes (weights + scales + activations + outputs). which: 0 in_qkv|in_z (GDN epilogue),
// 1 gate|up (SwiGLU epilogue), 2 down (+residual), 3 out_proj (+residual), 4 lm_head (bf16 +
// argmax partials).
// One kernel of the verify step timed over `iters` launches with device events on the engine
// stream. Consecutive launches cycle through the layers of the same kind, starting at `layer`,
// so no launch finds its weights in the 256 MB Infinity Cache from the previous one (the real
// step streams 27 GB per round).
int q27x_bench_kernel(q27x_ctx* x, int layer, int which, int nr, int iters, float* ms, double* bytes) {
    if (!x || !x->loaded || nr < 1 || nr > kMaxRows || iters < 1 || !ms || !bytes) return Q27X_E_ARG;
    const q27x_config& c = x->c;
    if (layer < 0 || layer >= c.n_layers) return Q27X_E_ARG;
    hipStream_t s = x->stream;
    Dctl* d = x->dctl;
    const int H = x->H, I = x->I;
    const bool need_gdn = (which == 0 || which == 3 || which == 5);
    std::vector<int> ls;
    for (int k = 0; k < c.n_layers; ++k) {
        const int l = (layer + k) % c.n_layers;
        if (!need_gdn || !x->L[l].is_attn) ls.push_back(l);
    }
    if (ls.empty()) return Q27X_E_ARG;
    int epi = EPI_STORE;
    double b = 0;
    auto make = [&](int l) {
        LayerDev& Y = x->L[l];
        ProjArgs p{};
        p.alpha = 1.0f; p.stop = &d->stop;
        if (which == 0) {   // as in the verify pass: input-norm prologue, conv epilogue, GDN row scalars
            p.W = Y.qkvz.w; p.WS = Y.qkvz.s; p.rows = Y.qkvz.rows; p.K = H;
            p.y = x->pb; p.ystride = Y.qkvz.rows; p.out_bf16 = 1;
            p.conv_w = Y.conv_w; p.conv_st = Y.conv_st; p.nconv = x->nqkv; p.npend_ptr = &d->gdn_npend;
            p.in_a = Y.in_a; p.in_b = Y.in_b; p.A_log = Y.A_log; p.dt_bias = Y.dt_bias; p.ab_vh = c.gdn_vh;
            p.ab_out = x->gab;
            set_pre(p, norm_of(x, x->xres, 0, Y.in_norm, 1.0f, 0, x->hid, nullptr));
            epi = EPI_CONV;
            b = (double)p.rows * H * (1 + 4.0 / 64) + (double)nr * H * 4 + (double)nr * p.rows * 2 +
                2.0 * c.gdn_vh * H * 2 + (double)x->nqkv * (8 + 2 * 32);
        } else if (which == 5) {   // in_qkv|in_z from pre-quantized rows (no prologue), for comparison
            p.W = Y.qkvz.w; p.WS = Y.qkvz.s; p.rows = Y.qkvz.rows; p.K = H; p.xq = x->xq; p.xst = H; p.xs = x->xs;
            p.y = x->pb; p.ystride = Y.qkvz.rows; p.out_bf16 = 1;
            b = (double)p.rows * H * (1 + 4.0 / 64) + (double)nr * H * (1 + 4.0 / 16) + (double)nr * p.rows * 2;
        } else if (which == 6) {   // gate|up from pre-quantized rows (no prologue), for comparison
            p.W = Y.gu.w; p.WS = Y.gu.s; p.rows = 2 * I; p.K = H; p.xq = x->xq; p.xst = H; p.xs = x->xs;
            p.act_q = x->xq + x->act_off; p.act_s = x->xs + x->act_off / 16; p.act_stride = I;
            p.gscale = 1.0f; p.sw_part = x->sw_part; p.sw_cnt = x->sw_cnt;
            epi = EPI_SWIGLU;
            b = (double)p.rows * H * (1 + 4.0 / 64) + (double)nr * H * (1 + 4.0 / 16) + (double)nr * I * (1 + 4.0 / 16);
        } else if (which == 1) {   // post-norm prologue, SwiGLU + quantize epilogue
            p.W = Y.gu.w; p.WS = Y.gu.s; p.rows = 2 * I; p.K = H;
            p.act_q = x->xq + x->act_off; p.act_s = x->xs + x->act_off / 16; p.act_stride = I;
            p.gscale = 1.0f; p.sw_part = x->sw_part; p.sw_cnt = x->sw_cnt;
            set_pre(p, norm_of(x, x->xres, 0, Y.post_norm, 1.0f, 0, x->hid, nullptr));
            epi = EPI_SWIGLU;
            b = (double)p.rows * H * (1 + 4.0 / 64) + (double)nr * H * 4 + (double)nr * I * (1 + 4.0 / 16);
        } else {
            const Mat& m = (which == 2) ? Y.down : Y.out_proj;
            p.W = m.w; p.WS = m.s; p.rows = H; p.K = m.K; p.xq = x->xq; p.xst = m.K; p.xs = x->xs;
            p.y = x->xres; p.ystride = H; p.res = x->hid; p.res_bf16 = 1; p.rstride = H; p.rs = 1.0f;
            b = (double)H * m.K * (1 + 4.0 / 64) + (double)nr * m.K * (1 + 4.0 / 16) + (double)nr * H * (2 + 4);
        }
        return p;
    };
    std::vector<ProjArgs> ps;
    GemvArgs ga{};
    if ((which >= 0 && which <= 3) || which == 5 || which == 6) {
        for (int l : ls) ps.push_back(make(l));
    } else if (which == 4) {
        ga.W = x->lm_head; ga.rows = x->V; ga.K = H; ga.x = x->ynorm; ga.xst = H;
        ga.pval = x->pval; ga.pidx = x->pidx; ga.pstride = x->pstride; ga.stop = &d->stop;
        b = (double)x->V * H * 2 + (double)nr * H * 2;
    } else return Q27X_E_ARG;
    int rc = set_ints(x, 1, DOFF(stop), 0);     // (a finished request leaves it set)
    if (rc) return rc;
    hipEvent_t e0, e1;
    Q27X_HIP(hipEventCreate(&e0));
    Q27X_HIP(hipEventCreate(&e1));
    int nb = 0;
    auto launch = [&](int i) {
        return which == 4 ? launch_gemv(ga, 1, nr, &nb, s) : launch_proj(ps[(size_t)i % ps.size()], epi, nr, s);
    };
    for (int i = 0; i < 3 && !rc; ++i) rc = launch(i);
    Q27X_HIP(hipEventRecord(e0, s));
    for (int i = 0; i < iters && !rc; ++i) rc = launch(i + 3);
    Q27X_HIP(hipEventRecord(e1, s));
    Q27X_HIP(hipEventSynchronize(e1));
    float t = 0.0f;
    Q27X_HIP(hipEventElapsedTime(&t, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms = t / (float)iters;
    *bytes = b;
    return rc;
}

// The mixer half of one verify layer (benchmark config 1: GDN -- in_qkv|in_z with its input-norm
// prologue, the GDN kernel, out_proj + residual; config 2: attention -- q|k|v with its prologue,
// the attention over positions 0 .. pos+nr-1, o_proj + residual), timed with device events over
// iters launches that cycle through the layers of that kind (layer 0 excluded: its prologue reads
// the embedding), so no launch finds its weights in the Infinity Cache. Runs at position pos; the
// control block is restored afterwards, but the layers' recurrent state, KV cache and the
// activation scratch are overwritten (prefill again before decoding).
int q27x_bench_mixer(q27x_ctx* x, int attn, int pos, int nr, int iters, float* ms, double* bytes) {
    if (!x || !x->loaded || nr < 1 || nr > kMaxRows || iters < 1 || !ms || !bytes || pos < 0 || pos + nr > x->c.ctx) {
        set_error("q27x_bench_mixer: bad arguments");
        return Q27X_E_ARG;
    }
    const q27x_config& c = x->c;
    std::vector<int> ls;
    for (int l = 1; l < c.n_layers; ++l)
        if (x->L[l].is_attn == (attn ? 1 : 0)) ls.push_back(l);
    if (ls.empty()) { set_error("q27x_bench_mixer: no layer of that kind"); return Q27X_E_ARG; }
    Dctl h0;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    Q27X_HIP(hipMemcpy(&h0, x->dctl, sizeof h0, hipMemcpyDeviceToHost));
    int rc = set_ints(x, 3, DOFF(pos), pos, DOFF(stop), 0, DOFF(gdn_npend), 0);
    if (rc) return rc;
    const double H = x->H, i8 = 1.0 + 4.0 / 64;
    double b;
    if (attn) {
        const double qkvr = x->qr + 2 * x->kvr;
        b = qkvr * H * i8 + nr * H * 4 + nr * qkvr * 2 +
            2.0 * (pos + nr) * x->kvr * (1.0 + 4.0 / c.kv_group) + H * x->att * i8 + nr * H * 6;
    } else {
        const double rows = x->nqkv + x->nz;
        b = rows * H * i8 + nr * H * 4 + nr * rows * 2 + 2.0 * c.gdn_vh * H * 2 + (double)x->nqkv * 4 * 2 +
            2.0 * c.gdn_vh * 128 * 128 * 4 + H * x->nz * i8 + nr * H * 6;
    }
    hipEvent_t e0, e1;
    Q27X_HIP(hipEventCreate(&e0));
    Q27X_HIP(hipEventCreate(&e1));
    for (int i = 0; i < 3 && !rc; ++i) rc = layer_pass(x, ls[(size_t)i % ls.size()], nr, 0);
    if (!rc) rc = (int)hipEventRecord(e0, x->stream);
    for (int i = 0; i < iters && !rc; ++i) rc = layer_pass(x, ls[(size_t)(i + 3) % ls.size()], nr, 0);
    if (!rc) rc = (int)hipEventRecord(e1, x->stream);
    float t = 0.0f;
    if (!rc) rc = (int)hipEventSynchronize(e1);
    if (!rc) rc = (int)hipEventElapsedTime(&t, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc) return rc < 0 ? rc : hip_fail((hipError_t)rc, "q27x_bench_mixer");
    Q27X_HIP(hipMemcpy(x->dctl, &h0, sizeof h0, hipMemcpyHostToDevice));
    *ms = t / (float)iters;
    *bytes = b;
    return Q27X_OK;
}

int q27x_debug_read(q27x_ctx* x, const char* name, int layer, void* dst, size_t bytes) {
    if (!x || !name || !dst) return Q27X_E_ARG;
    if (!strcmp(name, "pf_allocs")) {   // device allocations held for the prefill GEMM's weight copies
        const int32_t cnt = (int32_t)x->pf_walloc.size();
        if (bytes < 4) return Q27X_E_ARG;
        memcpy(dst, &cnt, 4);
        return Q27X_OK;
    }
    const void* src = nullptr;
    size_t n = 0;
    const LayerDev* Y = (layer >= 0 && layer < x->c.n_layers) ? &x->L[layer] : &x->mtp;
    const size_t kvn = (size_t)x->c.ctx * x->kvr;
    if (!strcmp(name, "S") && Y->S) { src = Y->S; n = (size_t)x->c.gdn_vh * 128 * 128 * 4; }
    else if (!strcmp(name, "conv_hist") && Y->conv_st) {
        // the committed conv history [nqkv][3] bf16, unpacked from the channel records
        std::vector<uint16_t> rec((size_t)x->nqkv * 16), h3((size_t)x->nqkv * 3);
        Q27X_HIP(hipStreamSynchronize(x->stream));
        Q27X_HIP(hipMemcpy(rec.data(), Y->conv_st, rec.size() * 2, hipMemcpyDeviceToHost));
        for (size_t ch = 0; ch < (size_t)x->nqkv; ++ch)
            for (int i = 0; i < 3; ++i) h3[ch * 3 + i] = rec[ch * 16 + i];
        const size_t nb = bytes < h3.size() * 2 ? bytes : h3.size() * 2;
        memcpy(dst, h3.data(), nb);
        return Q27X_OK;
    }
    else if (!strcmp(name, "kc") && Y->kc) { src = Y->kc; n = kvn; }
    else if (!strcmp(name, "vc") && Y->vc) { src = Y->vc; n = kvn; }
    else if (!strcmp(name, "ks") && Y->ks) { src = Y->ks; n = kvn / x->c.kv_group * 4; }
    else if (!strcmp(name, "vs") && Y->vs) { src = Y->vs; n = kvn / x->c.kv_group * 4; }
    else if (!strcmp(name, "mtp_res")) { src = x->mtp_res; n = (size_t)kMaxRows * x->H * 2; }
    else if (!strcmp(name, "hcatch")) { src = x->hcatch; n = (size_t)kMaxRows * x->H * 2; }
    else if (!strcmp(name, "dt")) { src = x->dctl->dt; n = 8 * 4; }
    else if (!strcmp(name, "dt_raw")) { src = x->dctl->dt_raw; n = 8 * 4; }
    else if (!strcmp(name, "nx")) { src = x->dctl->nx; n = 8 * 4; }
    else if (!strcmp(name, "catch_tok")) { src = x->dctl->catch_tok; n = 8 * 4; }
    else if (!strcmp(name, "ncatch")) { src = &x->dctl->ncatch; n = 4; }
    else if (!strcmp(name, "mtp_head")) { src = &x->dctl->mtp_head; n = 4; }
    else if (!strcmp(name, "pos")) { src = &x->dctl->pos; n = 4; }
    else if (!strcmp(name, "tok")) { src = &x->dctl->tok; n = 4; }
    else if (!strcmp(name, "hprev")) { src = x->hprev; n = (size_t)x->H * 2; }
    else if (!strcmp(name, "hfinal")) { src = x->hfinal; n = (size_t)kMaxRows * x->H * 2; }
    else if (!strcmp(name, "emb")) { src = x->emb; n = (size_t)x->V * x->H * 2; }
    else if (!strcmp(name, "lm_head")) { src = x->lm_head; n = (size_t)x->V * x->H * 2; }
    else if (!strcmp(name, "gu_w")) { src = Y->gu.w; n = (size_t)2 * x->I * x->H; }
    else if (!strcmp(name, "gu_s")) { src = Y->gu.s; n = (size_t)2 * x->I * (x->H / 64) * 4; }
    else if (!strcmp(name, "conv_w") && Y->conv_w) { src = Y->conv_w; n = (size_t)x->nqkv * 4 * 2; }
    else if (!strcmp(name, "dctl")) { src = x->dctl; n = sizeof(Dctl); }
    if (!src) { set_error("q27x_debug_read: unknown tensor %s", name); return Q27X_E_ARG; }
    if (bytes < n) n = bytes;
    Q27X_HIP(hipStreamSynchronize(x->stream));
    Q27X_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return Q27X_OK;
}

int q27x_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val, q27x_stream_t s) {
    if (!logits || !idx || n < 1 || ld < n || nr < 1 || nr > kMaxRows) { set_error("q27x_argmax_rows: bad arguments"); return Q27X_E_ARG; }
    float* pv = nullptr; uint32_t* pi = nullptr;
    int rc = argmax_scratch(&pv, &pi);
    if (rc) return rc;
    return launch_argmax_rows(logits, n, ld, nr, idx, val, pv, pi, (hipStream_t)s);
}

int q27x_accept(const int32_t* nx, const int32_t* dt, int k, int32_t* nacc_ncommit, int32_t* committed, q27x_stream_t s) {
    if (!nx || !dt || !nacc_ncommit || !committed || k < 0 || k > 7) { set_error("q27x_accept: bad arguments"); return Q27X_E_ARG; }
    hipLaunchKernelGGL(k_accept_rows, dim3(1), dim3(64), 0, (hipStream_t)s, nx, dt, k, nacc_ncommit, committed);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // extern "C"
