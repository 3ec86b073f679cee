/* q27o_model.c -- CPU oracle of the whole chained-MTP decode (R1-R4, R17-R21). TEST
 * INFRASTRUCTURE ONLY (see q27o.h). Mirrors the engine's per-row arithmetic exactly; every
 * function cites the reference routine whose semantics it restates. */
#include "q27o.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* tensor ids shared with the device generator: ((layer code) << 8) | kind;
 * layer code = L+1 for trunk layer L, 0 for globals, 1000 for the MTP layer */
enum {
    T_IN_NORM = 1, T_POST_NORM = 2,
    T_IN_QKV = 10, T_IN_Z = 11, T_IN_A = 12, T_IN_B = 13, T_A_LOG = 14, T_DT_BIAS = 15,
    T_GDN_NORM = 16, T_CONV_W = 17, T_OUT_PROJ = 18,
    T_Q = 20, T_K = 21, T_V = 22, T_Q_NORM = 23, T_K_NORM = 24, T_O = 25,
    T_GATE = 30, T_UP = 31, T_DOWN = 32, T_DOWN_S0 = 33,   /* MTP down slices: 33..36 */
    T_EMB = 40, T_FINAL_NORM = 41, T_LM_HEAD = 42,
    T_PRE_EMB = 50, T_PRE_HID = 51, T_FC0 = 52, T_FC1 = 53, T_MTP_NORM = 54
};
static uint64_t tid(int code, int kind) { return ((uint64_t)code << 8) | (uint64_t)kind; }

typedef struct { int8_t* w; float* s; int rows, K; } i8m;

typedef struct {
    int is_attn;
    uint16_t *in_norm, *post_norm;
    /* GDN */
    i8m qkvz;                /* in_qkv rows then in_z rows, one stacked matrix */
    uint16_t *in_a, *in_b, *A_log, *dt_bias, *gdn_norm, *conv_w;
    i8m out_proj;
    /* attention */
    i8m qkv;                 /* q (with gate) | k | v stacked */
    uint16_t *q_norm, *k_norm;
    i8m o;
    /* MLP */
    i8m gate, up, down;
    i8m down4[4];            /* MTP layer only: down as four column slices (src/q27_main.cpp:2605-2612) */
    /* state */
    int8_t *kc, *vc; float *ks, *vs;
    float* S; uint16_t* conv_hist; void* pend;
    /* checkpoint scales (1 for generated weights): alpha per source tensor of the stacked
     * projections (q, k, v or in_qkv, in_z), o / out_proj, gate, up, down; input_scale of the input
     * norm, the post norm, the SwiGLU output and the mixer output */
    float al_qkv[3], al_o, al_gate, al_up, al_down;
    float is_in, is_post, is_down, is_out;
} layer_t;

struct q27o_model {
    q27o_cfg c;
    uint64_t seed;
    layer_t* L;
    layer_t mtp;
    uint16_t *pre_emb, *pre_hid, *mtp_norm;
    i8m fc0, fc1;
    uint16_t *emb, *final_norm, *lm_head;
    float *rope_cos, *rope_sin;
    /* speculation state (src/q27_main.cpp:360-379 Dev NR fields) */
    int pos, tok, ncatch, gdn_npend, have_h;
    int catch_tok[8];
    uint16_t *hprev, *hcatch;     /* [H], [8][H] */
    uint16_t* hfinal;             /* [rows][H] last verify's final residual rows */
    uint16_t* hchain;             /* [H] */
    /* the last round's drafts (dt: what the verify saw; dt_raw: the MTP argmax before any forced
     * replacement), verify argmaxes and acceptance */
    int32_t dt[8], dt_raw[8], nx[8];
    int nacc_last;
    double wbytes;
    float* vlogits;               /* when set, the next verify's logits [rows][vocab] go here */
    /* when set, the next verify records per layer L (each [n_layers][rows][...]): the fp32
     * residual after the mixer r1 and after the MLP r2, and the post norm's int8 codes and per-16
     * scales (the MLP's input) */
    float *tr_r1, *tr_r2, *tr_ps; int8_t* tr_pq;
};

/* ------------------------------------------------------------------ generation */
static uint16_t* gen_bf16(uint64_t seed, uint64_t t, size_t n, float stdv, float mean) {
    uint16_t* p = (uint16_t*)malloc(n * 2);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        p[i] = q27o_f2bf(mean + q27o_normal(seed, t, (uint64_t)i) * stdv);
    return p;
}
static uint16_t* gen_uniform_bf16(uint64_t seed, uint64_t t, size_t n, float scale) {
    uint16_t* p = (uint16_t*)malloc(n * 2);
    for (size_t i = 0; i < n; ++i) p[i] = q27o_f2bf(q27o_uniform(seed, t, i) * scale);
    return p;
}
/* int8 projection: N(0, 0.02) draws through the R8 per-64 rule, rows stacked at row0 */
static void gen_i8_into(uint64_t seed, uint64_t t, int rows, int K, int8_t* w, float* s) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float v[64];
        for (int g = 0; g < K / 64; ++g) {
            for (int j = 0; j < 64; ++j)
                v[j] = q27o_normal(seed, t, (uint64_t)r * K + (uint64_t)g * 64 + j) * 0.02f;
            q27o_quant_f32(v, 64, 64, w + (size_t)r * K + (size_t)g * 64, s + (size_t)r * (K / 64) + g);
        }
    }
}
static i8m alloc_i8(int rows, int K) {
    i8m m; m.rows = rows; m.K = K;
    m.w = (int8_t*)malloc((size_t)rows * K);
    m.s = (float*)malloc((size_t)rows * (K / 64) * 4);
    return m;
}
static i8m gen_i8(uint64_t seed, uint64_t t, int rows, int K) {
    i8m m = alloc_i8(rows, K);
    gen_i8_into(seed, t, rows, K, m.w, m.s);
    return m;
}
static void free_i8(i8m* m) { free(m->w); free(m->s); m->w = NULL; m->s = NULL; }

static int is_attn_layer(const q27o_cfg* c, int L) { return (L % c->attn_period) == c->attn_period - 1; }
static int qrows_of(const q27o_cfg* c) { return c->n_q * (c->attn_gate ? 2 * c->head_dim : c->head_dim); }

static void gen_attn(q27o_model* m, layer_t* Y, int code) {
    const q27o_cfg* c = &m->c;
    const int H = c->hidden, qr = qrows_of(c), kvr = c->n_kv * c->head_dim;
    Y->qkv = alloc_i8(qr + 2 * kvr, H);
    gen_i8_into(m->seed, tid(code, T_Q), qr, H, Y->qkv.w, Y->qkv.s);
    gen_i8_into(m->seed, tid(code, T_K), kvr, H, Y->qkv.w + (size_t)qr * H, Y->qkv.s + (size_t)qr * (H / 64));
    gen_i8_into(m->seed, tid(code, T_V), kvr, H, Y->qkv.w + (size_t)(qr + kvr) * H, Y->qkv.s + (size_t)(qr + kvr) * (H / 64));
    Y->q_norm = gen_bf16(m->seed, tid(code, T_Q_NORM), c->head_dim, 0.02f, 0.0f);
    Y->k_norm = gen_bf16(m->seed, tid(code, T_K_NORM), c->head_dim, 0.02f, 0.0f);
    Y->o = gen_i8(m->seed, tid(code, T_O), H, c->n_q * c->head_dim);
    const size_t kvn = (size_t)c->ctx * kvr;
    Y->kc = (int8_t*)calloc(kvn, 1); Y->vc = (int8_t*)calloc(kvn, 1);
    Y->ks = (float*)calloc(kvn / c->kv_group, 4); Y->vs = (float*)calloc(kvn / c->kv_group, 4);
    m->wbytes += (double)(qr + 2 * kvr) * H * (1.0 + 4.0 / 64) + (double)H * c->n_q * c->head_dim * (1.0 + 4.0 / 64);
}
/* slices: 0 = one down matrix [H][I] (trunk layers); 4 = four [H][I/4] column slices, each its
 * own per-64-scaled tensor (the MTP layer, whose reference checkpoint stores mtp down as four
 * K = 4352 tensors, src/q27_main.cpp:2605-2612) */
static void gen_mlp(q27o_model* m, layer_t* Y, int code, int slices) {
    const q27o_cfg* c = &m->c;
    Y->in_norm = gen_bf16(m->seed, tid(code, T_IN_NORM), c->hidden, 0.02f, 0.0f);
    Y->post_norm = gen_bf16(m->seed, tid(code, T_POST_NORM), c->hidden, 0.02f, 0.0f);
    Y->gate = gen_i8(m->seed, tid(code, T_GATE), c->inter, c->hidden);
    Y->up = gen_i8(m->seed, tid(code, T_UP), c->inter, c->hidden);
    if (slices)
        for (int j = 0; j < 4; ++j) Y->down4[j] = gen_i8(m->seed, tid(code, T_DOWN_S0 + j), c->hidden, c->inter / 4);
    else
        Y->down = gen_i8(m->seed, tid(code, T_DOWN), c->hidden, c->inter);
    m->wbytes += 3.0 * c->inter * c->hidden * (1.0 + 4.0 / 64) + 4.0 * c->hidden;
}

q27o_model* q27o_model_create(const q27o_cfg* c, uint64_t seed) {
    q27o_model* m = (q27o_model*)calloc(1, sizeof(q27o_model));
    m->c = *c; m->seed = seed;
    const int H = c->hidden, D = c->gdn_d;
    const int nqkv = (2 * c->gdn_kh + c->gdn_vh) * D, nz = c->gdn_vh * D;
    m->L = (layer_t*)calloc((size_t)c->n_layers, sizeof(layer_t));
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* Y = &m->L[L];
        const int code = L + 1;
        Y->is_attn = is_attn_layer(c, L);
        gen_mlp(m, Y, code, 0);
        if (Y->is_attn) { gen_attn(m, Y, code); continue; }
        Y->qkvz = alloc_i8(nqkv + nz, H);
        gen_i8_into(seed, tid(code, T_IN_QKV), nqkv, H, Y->qkvz.w, Y->qkvz.s);
        gen_i8_into(seed, tid(code, T_IN_Z), nz, H, Y->qkvz.w + (size_t)nqkv * H, Y->qkvz.s + (size_t)nqkv * (H / 64));
        Y->in_a = gen_bf16(seed, tid(code, T_IN_A), (size_t)c->gdn_vh * H, 0.02f, 0.0f);
        Y->in_b = gen_bf16(seed, tid(code, T_IN_B), (size_t)c->gdn_vh * H, 0.02f, 0.0f);
        Y->A_log = gen_uniform_bf16(seed, tid(code, T_A_LOG), c->gdn_vh, 2.7f);
        Y->dt_bias = gen_bf16(seed, tid(code, T_DT_BIAS), c->gdn_vh, 0.1f, 0.0f);
        Y->gdn_norm = gen_bf16(seed, tid(code, T_GDN_NORM), D, 0.02f, 1.0f);
        Y->conv_w = gen_bf16(seed, tid(code, T_CONV_W), (size_t)nqkv * 4, 0.3f, 0.0f);
        Y->out_proj = gen_i8(seed, tid(code, T_OUT_PROJ), H, nz);
        Y->S = (float*)calloc((size_t)c->gdn_vh * D * D, 4);
        Y->conv_hist = (uint16_t*)calloc((size_t)nqkv * 3, 2);
        Y->pend = calloc(1, q27o_gdn_pend_bytes(c->gdn_kh, c->gdn_vh, D, 8));
        m->wbytes += (double)(nqkv + nz) * H * (1.0 + 4.0 / 64) + (double)H * nz * (1.0 + 4.0 / 64) +
                     2.0 * 2 * c->gdn_vh * H + 2.0 * 4 * nqkv + 2.0 * (2 * c->gdn_vh + D);
    }
    /* MTP layer: a full-attention decoder layer (src/q27_mtp_defs.h:22-33) */
    gen_mlp(m, &m->mtp, 1000, 1);
    m->mtp.is_attn = 1;
    gen_attn(m, &m->mtp, 1000);
    m->pre_emb = gen_bf16(seed, tid(1000, T_PRE_EMB), H, 0.02f, 0.0f);
    m->pre_hid = gen_bf16(seed, tid(1000, T_PRE_HID), H, 0.02f, 0.0f);
    m->mtp_norm = gen_bf16(seed, tid(1000, T_MTP_NORM), H, 0.02f, 0.0f);
    m->fc0 = gen_i8(seed, tid(1000, T_FC0), H, H);
    m->fc1 = gen_i8(seed, tid(1000, T_FC1), H, H);
    m->emb = gen_bf16(seed, tid(0, T_EMB), (size_t)c->vocab * H, 1.0f, 0.0f);
    m->final_norm = gen_bf16(seed, tid(0, T_FINAL_NORM), H, 0.02f, 0.0f);
    m->lm_head = gen_bf16(seed, tid(0, T_LM_HEAD), (size_t)c->vocab * H, 0.02f, 0.0f);
    m->wbytes += 2.0 * c->vocab * H;
    const int half = c->rot_dims / 2;
    m->rope_cos = (float*)malloc((size_t)c->ctx * half * 4);
    m->rope_sin = (float*)malloc((size_t)c->ctx * half * 4);
    q27o_rope_table(c->ctx, c->rot_dims, c->rope_theta, m->rope_cos, m->rope_sin);
    m->hprev = (uint16_t*)calloc(H, 2);
    m->hcatch = (uint16_t*)calloc((size_t)8 * H, 2);
    m->hfinal = (uint16_t*)calloc((size_t)8 * H, 2);
    m->hchain = (uint16_t*)calloc(H, 2);
    q27o_model_reset(m);
    for (int L = -1; L < c->n_layers; ++L) {
        layer_t* Y = (L < 0) ? &m->mtp : &m->L[L];
        Y->al_qkv[0] = Y->al_qkv[1] = Y->al_qkv[2] = 1.0f;
        Y->al_o = Y->al_gate = Y->al_up = Y->al_down = 1.0f;
        Y->is_in = Y->is_post = Y->is_down = Y->is_out = 1.0f;
    }
    return m;
}

static void free_layer(layer_t* Y) {
    free(Y->in_norm); free(Y->post_norm);
    free_i8(&Y->gate); free_i8(&Y->up); free_i8(&Y->down);
    for (int j = 0; j < 4; ++j) free_i8(&Y->down4[j]);
    if (Y->is_attn) {
        free_i8(&Y->qkv); free(Y->q_norm); free(Y->k_norm); free_i8(&Y->o);
        free(Y->kc); free(Y->vc); free(Y->ks); free(Y->vs);
    } else {
        free_i8(&Y->qkvz); free(Y->in_a); free(Y->in_b); free(Y->A_log); free(Y->dt_bias);
        free(Y->gdn_norm); free(Y->conv_w); free_i8(&Y->out_proj);
        free(Y->S); free(Y->conv_hist); free(Y->pend);
    }
}
void q27o_model_destroy(q27o_model* m) {
    if (!m) return;
    for (int L = 0; L < m->c.n_layers; ++L) free_layer(&m->L[L]);
    free(m->L);
    free_layer(&m->mtp);
    free(m->pre_emb); free(m->pre_hid); free(m->mtp_norm); free_i8(&m->fc0); free_i8(&m->fc1);
    free(m->emb); free(m->final_norm); free(m->lm_head); free(m->rope_cos); free(m->rope_sin);
    free(m->hprev); free(m->hcatch); free(m->hfinal); free(m->hchain);
    free(m);
}

void q27o_model_reset(q27o_model* m) {
    const q27o_cfg* c = &m->c;
    const int D = c->gdn_d, nqkv = (2 * c->gdn_kh + c->gdn_vh) * D;
    const size_t kvn = (size_t)c->ctx * c->n_kv * c->head_dim;
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* Y = &m->L[L];
        if (Y->is_attn) {
            memset(Y->kc, 0, kvn); memset(Y->vc, 0, kvn);
            memset(Y->ks, 0, kvn / c->kv_group * 4); memset(Y->vs, 0, kvn / c->kv_group * 4);
        } else {
            memset(Y->S, 0, (size_t)c->gdn_vh * D * D * 4);
            memset(Y->conv_hist, 0, (size_t)nqkv * 3 * 2);
            memset(Y->pend, 0, q27o_gdn_pend_bytes(c->gdn_kh, c->gdn_vh, D, 8));
        }
    }
    memset(m->mtp.kc, 0, kvn); memset(m->mtp.vc, 0, kvn);
    memset(m->mtp.ks, 0, kvn / c->kv_group * 4); memset(m->mtp.vs, 0, kvn / c->kv_group * 4);
    m->pos = 0; m->tok = 0; m->ncatch = 0; m->gdn_npend = 0; m->have_h = 0;
}

double q27o_model_weight_bytes(const q27o_model* m) { return m->wbytes; }

/* A stacked projection with one alpha per source tensor: rows [r[i], r[i+1]) take al[i]
 * (bf16 out at y + r[i], row stride ld; the decode path's projection). */
static void proj_stacked(const i8m* W, int nparts, const int* r, const float* al, const int8_t* xq,
                         const float* xs, uint16_t* y, int ld, int nr) {
    const int K = W->K;
    for (int i = 0; i < nparts; ++i)
        q27o_proj_rows_epi(W->w + (size_t)r[i] * K, W->s + (size_t)r[i] * (K / 64), al[i], r[i + 1] - r[i], K, xq, K,
                           xs, y + r[i], ld, 1, NULL, 0, 0, 0.0f, nr);
}

void q27o_model_set_scales(q27o_model* m, int layer, const float* v) {
    layer_t* Y = (layer >= 0 && layer < m->c.n_layers) ? &m->L[layer] : &m->mtp;
    Y->al_qkv[0] = v[0]; Y->al_qkv[1] = v[1]; Y->al_qkv[2] = v[2]; Y->al_o = v[3];
    Y->al_gate = v[4]; Y->al_up = v[5]; Y->al_down = v[6];
    Y->is_in = v[7]; Y->is_post = v[8]; Y->is_down = v[9]; Y->is_out = v[10];
}

/* ------------------------------------------------------------------ one verify pass */
/* run_layer_tp_nr (src/q27_main.cpp:2271-2489) on one card: residual share rs = 1. Rows are
 * tokens toks[0..nr-1] at positions m->pos .. m->pos+nr-1. Leaves the final residual rows in
 * m->hfinal (R17) and, if nx != NULL, the per-row argmax of the logits (R18). */
static void verify(q27o_model* m, int nr, const int32_t* toks, int32_t* nx) {
    const q27o_cfg* c = &m->c;
    const int H = c->hidden, I = c->inter, D = c->gdn_d;
    const int nqkv = (2 * c->gdn_kh + c->gdn_vh) * D, nz = c->gdn_vh * D;
    const int qr = qrows_of(c), kvr = c->n_kv * c->head_dim, att = c->n_q * c->head_dim;
    const int pos0 = m->pos;
    uint16_t* h = (uint16_t*)malloc((size_t)nr * H * 2);       /* bf16 residual copy */
    float* x = (float*)malloc((size_t)nr * H * 4);             /* fp32 residual (r1 / r2) */
    uint16_t* y = (uint16_t*)malloc((size_t)nr * H * 2);       /* bf16 normed */
    int8_t* xq = (int8_t*)malloc((size_t)nr * (I > H ? I : H) * 2);
    float* xs = (float*)malloc((size_t)nr * (I > H ? I : H) / 16 * 4 * 2);
    const int wmax = (nqkv + nz) > (qr + 2 * kvr) ? (nqkv + nz) : (qr + 2 * kvr);
    uint16_t* pb = (uint16_t*)malloc((size_t)nr * wmax * 2);
    uint16_t* mix = (uint16_t*)malloc((size_t)nr * (nz > att ? nz : att) * 2);
    float* g = (float*)malloc((size_t)nr * I * 4);
    float* u = (float*)malloc((size_t)nr * I * 4);
    float* ab = (float*)malloc((size_t)nr * c->gdn_vh * 4 * 2);
    float* tmp = (float*)malloc((size_t)nr * c->gdn_vh * 4);
    for (int r = 0; r < nr; ++r) memcpy(h + (size_t)r * H, m->emb + (size_t)toks[r] * H, (size_t)H * 2);
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* Y = &m->L[L];
        /* input norm: layer 0 from the bf16 embedding rows (q27_rmsnorm_quant_fp8), later layers
         * from the fp32 residual r2 (q27_rmsnorm_hostss_fp8_b) */
        if (L == 0) q27o_rmsnorm_quant_rows(h, 1, H, Y->in_norm, 1.0f, c->rms_eps, H, NULL, y, H, xq, xs, 1, Y->is_in, nr);
        else q27o_rmsnorm_quant_rows(x, 0, H, Y->in_norm, 1.0f, c->rms_eps, H, h, y, H, xq, xs, 0, Y->is_in, nr);
        if (Y->is_attn) {
            const int rr[4] = { 0, qr, qr + kvr, qr + 2 * kvr };
            proj_stacked(&Y->qkv, 3, rr, Y->al_qkv, xq, xs, pb, qr + 2 * kvr, nr);
            q27o_attn_prep_rows(pb, qr + 2 * kvr, Y->q_norm, Y->k_norm, m->rope_cos, m->rope_sin, c->rot_dims,
                                Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, mix, c->n_q, c->n_kv, c->head_dim,
                                c->attn_gate, c->rms_eps, pos0, nr);
            uint16_t* ao = (uint16_t*)malloc((size_t)nr * att * 2);
            q27o_attn_rows(mix, pb, qr + 2 * kvr, Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, c->n_q, c->n_kv,
                           c->head_dim, c->attn_gate, pos0, nr, ao, NULL, NULL);
            q27o_quant_rows(ao, att, xq, att, xs, att / 16, att, Y->is_out, nr);   /* o_proj's input_scale */
            free(ao);
            q27o_proj_rows_epi(Y->o.w, Y->o.s, Y->al_o, H, att, xq, att, xs, x, H, 0, h, 1, H, 1.0f, nr);
        } else {
            const int rr[3] = { 0, nqkv, nqkv + nz };
            proj_stacked(&Y->qkvz, 2, rr, Y->al_qkv, xq, xs, pb, nqkv + nz, nr);
            /* a / b: bf16 GEMV on the bf16 normed rows, bf16 outputs (src/q27_util.hip:158-162) */
            q27o_bf16_gemv_rows(Y->in_a, c->gdn_vh, H, y, H, tmp, c->gdn_vh, nr);
            for (int i = 0; i < nr * c->gdn_vh; ++i) ab[i] = q27o_bf2f(q27o_f2bf(tmp[i]));
            q27o_bf16_gemv_rows(Y->in_b, c->gdn_vh, H, y, H, tmp, c->gdn_vh, nr);
            for (int i = 0; i < nr * c->gdn_vh; ++i) ab[nr * c->gdn_vh + i] = q27o_bf2f(q27o_f2bf(tmp[i]));
            q27o_gdn_verify(pb, nqkv + nz, pb + nqkv, nqkv + nz, ab, ab + nr * c->gdn_vh, c->gdn_vh,
                            Y->A_log, Y->dt_bias, Y->gdn_norm, Y->conv_w, Y->S, Y->conv_hist, Y->pend,
                            m->gdn_npend, c->gdn_kh, c->gdn_vh, D, c->rms_eps, mix, nz, NULL, NULL, nr);
            q27o_quant_rows(mix, nz, xq, nz, xs, nz / 16, nz, Y->is_out, nr);       /* out_proj's input_scale */
            q27o_proj_rows_epi(Y->out_proj.w, Y->out_proj.s, Y->al_o, H, nz, xq, nz, xs, x, H, 0, h, 1, H, 1.0f, nr);
        }
        if (m->tr_r1) memcpy(m->tr_r1 + (size_t)L * nr * H, x, (size_t)nr * H * 4);
        /* post norm (q27_rmsnorm_hostss_perm_b, natural order here): h = bf16(r1) */
        q27o_rmsnorm_quant_rows(x, 0, H, Y->post_norm, 1.0f, c->rms_eps, H, h, NULL, H, xq, xs, 0, Y->is_post, nr);
        if (m->tr_pq) {
            memcpy(m->tr_pq + (size_t)L * nr * H, xq, (size_t)nr * H);
            memcpy(m->tr_ps + (size_t)L * nr * (H / 16), xs, (size_t)nr * (H / 16) * 4);
        }
        q27o_proj_rows(Y->gate.w, Y->gate.s, Y->al_gate, I, H, xq, H, xs, g, I, nr);
        q27o_proj_rows(Y->up.w, Y->up.s, Y->al_up, I, H, xq, H, xs, u, I, nr);
        q27o_swiglu_quant_rows(g, u, I, xq, xs, I, Y->is_down, nr);
        q27o_proj_rows_epi(Y->down.w, Y->down.s, Y->al_down, H, I, xq, I, xs, x, H, 0, h, 1, H, 1.0f, nr);
        if (m->tr_r2) memcpy(m->tr_r2 + (size_t)L * nr * H, x, (size_t)nr * H * 4);
    }
    /* head (src/q27_main.cpp:2457-2481): hid = bf16(bf16(r1) + r2) -- the residual the reference
     * adds twice -- or bf16(r2); final norm; lm_head; argmax */
    for (int r = 0; r < nr; ++r)
        for (int k = 0; k < H; ++k) {
            const float v = c->head_double_residual ? q27o_bf2f(h[(size_t)r * H + k]) + x[(size_t)r * H + k]
                                                    : x[(size_t)r * H + k];
            m->hfinal[(size_t)r * H + k] = q27o_f2bf(v);
        }
    if (nx) {
        q27o_rmsnorm_quant_rows(m->hfinal, 1, H, m->final_norm, 1.0f, c->rms_eps, H, NULL, y, H, NULL, NULL, 1, 1.0f, nr);
        float* logits = (float*)malloc((size_t)nr * c->vocab * 4);
        q27o_bf16_gemv_rows(m->lm_head, c->vocab, H, y, H, logits, c->vocab, nr);
        float val[8];
        q27o_argmax_rows(logits, c->vocab, c->vocab, nr, nx, val);
        if (m->vlogits) memcpy(m->vlogits, logits, (size_t)nr * c->vocab * 4);
        free(logits);
    }
    m->gdn_npend = nr;   /* default: every row committed (plain step / prefill); spec overrides */
    free(h); free(x); free(y); free(xq); free(xs); free(pb); free(mix); free(g); free(u); free(ab); free(tmp);
}

/* ------------------------------------------------------------------ MTP pass */
/* mtp_pass_nr (src/q27_main.cpp:2551-2618). Rows: hidden hrows[r] (bf16) and token toks[r] at
 * draft positions dpos0 + r. Leaves the layer's residual rows in res (bf16 [nr][H]); returns the
 * head row's argmax (head_row >= 0) or -1. */
static int mtp_pass(q27o_model* m, int nr, const uint16_t* const* hrows, const int32_t* toks,
                    int dpos0, int head_row, uint16_t* res, float* logits_out) {
    const q27o_cfg* c = &m->c;
    layer_t* Y = &m->mtp;
    const int H = c->hidden, I = c->inter;
    const int qr = qrows_of(c), kvr = c->n_kv * c->head_dim, att = c->n_q * c->head_dim;
    const float po = c->mtp_plus_one ? 1.0f : 0.0f;
    uint16_t* cat = (uint16_t*)calloc((size_t)nr * 2 * H, 2);
    uint16_t* t1 = (uint16_t*)malloc((size_t)nr * H * 2);
    int8_t* xa = (int8_t*)malloc((size_t)nr * (I > 2 * H ? I : 2 * H));
    float* sa = (float*)malloc((size_t)nr * (I > 2 * H ? I : 2 * H) / 16 * 4);
    float* f0 = (float*)malloc((size_t)nr * (I > H ? I : H) * 4);
    float* f1 = (float*)malloc((size_t)nr * I * 4);
    uint16_t* pb = (uint16_t*)malloc((size_t)nr * (qr + 2 * kvr) * 2);
    uint16_t* qh = (uint16_t*)malloc((size_t)nr * att * 2);
    uint16_t* ao = (uint16_t*)malloc((size_t)nr * att * 2);
    const int eoff = c->mtp_swap ? 0 : H, hoff = c->mtp_swap ? H : 0;   /* src/q27_mtp_defs.h:108-109 */
    for (int r = 0; r < nr; ++r) {
        q27o_rmsnorm_quant_rows(m->emb + (size_t)toks[r] * H, 1, H, m->pre_emb, po, c->rms_eps, H, NULL,
                                cat + (size_t)r * 2 * H + eoff, H, NULL, NULL, 1, 1.0f, 1);
        q27o_rmsnorm_quant_rows(hrows[r], 1, H, m->pre_hid, po, c->rms_eps, H, NULL,
                                cat + (size_t)r * 2 * H + hoff, H, NULL, NULL, 1, 1.0f, 1);
    }
    /* fc as two K = H halves (src/q27_main.cpp:2563-2572): res = bf16(bf16(fc0.a) + fc1.b) */
    q27o_quant_rows(cat, 2 * H, xa, 2 * H, sa, 2 * H / 16, 2 * H, 1.0f, nr);
    q27o_proj_rows_epi(m->fc0.w, m->fc0.s, 1.0f, H, H, xa, 2 * H, sa, res, H, 1, NULL, 0, 0, 0.0f, nr);
    {   /* fc1 consumes the second half: its rows start H bytes into each 2H row */
        int8_t* xb = (int8_t*)malloc((size_t)nr * H);
        float* sb = (float*)malloc((size_t)nr * H / 16 * 4);
        for (int r = 0; r < nr; ++r) {
            memcpy(xb + (size_t)r * H, xa + (size_t)r * 2 * H + H, (size_t)H);
            memcpy(sb + (size_t)r * (H / 16), sa + (size_t)r * (2 * H / 16) + H / 16, (size_t)H / 16 * 4);
        }
        q27o_proj_rows_epi(m->fc1.w, m->fc1.s, 1.0f, H, H, xb, H, sb, res, H, 1, res, 1, H, 1.0f, nr);
        free(xb); free(sb);
    }
    /* input norm from the bf16 residual, quantize the bf16 normed rows */
    q27o_rmsnorm_quant_rows(res, 1, H, Y->in_norm, po, c->rms_eps, H, NULL, t1, H, xa, sa, 1, 1.0f, nr);
    q27o_proj_rows_epi(Y->qkv.w, Y->qkv.s, 1.0f, qr + 2 * kvr, H, xa, H, sa, pb, qr + 2 * kvr, 1, NULL, 0, 0, 0.0f, nr);
    q27o_attn_prep_rows(pb, qr + 2 * kvr, Y->q_norm, Y->k_norm, m->rope_cos, m->rope_sin, c->rot_dims,
                        Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, qh, c->n_q, c->n_kv, c->head_dim,
                        c->attn_gate, c->rms_eps, dpos0, nr);
    q27o_attn_rows(qh, pb, qr + 2 * kvr, Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, c->n_q, c->n_kv,
                   c->head_dim, c->attn_gate, dpos0, nr, ao, xa, sa);
    /* o_proj to bf16, then the bf16 residual add (q27_proj_fp8_bf16_nrs + q27_add_inplace_bf16) */
    q27o_proj_rows_epi(Y->o.w, Y->o.s, 1.0f, H, att, xa, att, sa, t1, H, 1, NULL, 0, 0, 0.0f, nr);
    for (size_t i = 0; i < (size_t)nr * H; ++i) res[i] = q27o_f2bf(q27o_bf2f(res[i]) + q27o_bf2f(t1[i]));
    q27o_rmsnorm_quant_rows(res, 1, H, Y->post_norm, po, c->rms_eps, H, NULL, t1, H, xa, sa, 1, 1.0f, nr);
    q27o_proj_rows(Y->gate.w, Y->gate.s, 1.0f, I, H, xa, H, sa, f0, I, nr);
    q27o_proj_rows(Y->up.w, Y->up.s, 1.0f, I, H, xa, H, sa, f1, I, nr);
    q27o_swiglu_quant_rows(f0, f1, I, xa, sa, I, 1.0f, nr);
    /* down as four K = inter/4 column slices, each projected on its own and added into the bf16
     * residual, which is rounded to bf16 after every slice (src/q27_main.cpp:2605-2612:
     * q27_proj_nvfp4_down_nrs into fp32 pd, then q27_add_inplace(nrm, pd) per slice) */
    const int I4 = I / 4;
    for (int j = 0; j < 4; ++j)
        q27o_proj_rows_epi(Y->down4[j].w, Y->down4[j].s, 1.0f, H, I4, xa + (size_t)j * I4, I,
                           sa + (size_t)j * (I4 / 16), res, H, 1, res, 1, H, 1.0f, nr);
    int tok = -1;
    if (head_row >= 0) {
        q27o_rmsnorm_quant_rows(res + (size_t)head_row * H, 1, H, m->mtp_norm, 1.0f, c->rms_eps, H, NULL, t1, H,
                                NULL, NULL, 1, 1.0f, 1);
        float* logits = logits_out ? logits_out : (float*)malloc((size_t)c->vocab * 4);
        q27o_bf16_gemv_rows(m->lm_head, c->vocab, H, t1, H, logits, c->vocab, 1);
        int32_t ix; float vv;
        q27o_argmax_rows(logits, c->vocab, c->vocab, 1, &ix, &vv);
        tok = ix;
        if (!logits_out) free(logits);
    }
    free(cat); free(t1); free(xa); free(sa); free(f0); free(f1); free(pb); free(qh); free(ao);
    return tok;
}

/* ------------------------------------------------------------------ driver-level entries */
/* The prompt goes through the verify path in chunks of 8 rows (every row committed); the last
 * position's argmax is the first decode token; the MTP layer is then prompt-conditioned over
 * positions 0..n-2 with (final residual at p, embedding of token p+1) -- mtp_prompt_pass,
 * src/q27_main.cpp:2649-2692 -- and h_prev = final residual at n-1 (5131-5136). */
int q27o_model_prefill(q27o_model* m, const int32_t* ids, int n) {
    const int H = m->c.hidden;
    uint16_t* hall = (uint16_t*)malloc((size_t)n * H * 2);
    int32_t nx[8];
    int first = 0;
    q27o_model_reset(m);                       /* a prompt starts a new request */
    for (int c0 = 0; c0 < n; c0 += 8) {
        const int cn = (n - c0 < 8) ? n - c0 : 8;
        const int last = (c0 + cn == n);
        verify(m, cn, ids + c0, last ? nx : NULL);
        memcpy(hall + (size_t)c0 * H, m->hfinal, (size_t)cn * H * 2);
        m->pos += cn;
        if (last) first = nx[cn - 1];
    }
    uint16_t* res = (uint16_t*)malloc((size_t)8 * H * 2);
    for (int p0 = 0; p0 < n - 1; p0 += 8) {
        const int cn = (n - 1 - p0 < 8) ? n - 1 - p0 : 8;
        const uint16_t* hr[8];
        for (int r = 0; r < cn; ++r) hr[r] = hall + (size_t)(p0 + r) * H;
        mtp_pass(m, cn, hr, ids + p0 + 1, p0, -1, res, NULL);
    }
    free(res);
    memcpy(m->hprev, hall + (size_t)(n - 1) * H, (size_t)H * 2);
    free(hall);
    m->tok = first; m->ncatch = 0; m->have_h = 1;
    return first;
}

/* ------------------------------------------------------------------ prefill on the GEMM path */
/* Test knob: plants one composition mistake in the prefill restatement so the tests can show
 * that their tolerance rejects it (0 = none; 1 = down without its residual, 2 = the MTP fc
 * halves exchanged, 3 = the GDN scan not committing between sub-chunks, 4 = the a/b logits
 * exchanged). Never set outside tests. */
static int g_pf_plant = 0;
void q27o_debug_plant(int code) { g_pf_plant = code; }

/* Group size of the trunk's prefill GEMMs over K (the reference's Q27_Q8_GS, src/q27_load.cpp:1623,
 * src/q27_main.cpp:4020): the whole K (0, the default) or pf_gs columns when they divide K. */
static int pf_gs(const q27o_cfg* c, int K) { return (c->pf_gs > 0 && K % c->pf_gs == 0) ? c->pf_gs : K; }
/* y[M][rows] = GEMM(W, act) * 1 (+ rs * res), W's per-64 mirror requantized per (row, group)
 * (src/q27_epi.hip:14-35) and act quantized per (token, group) from fp32 values v [M][K]
 * (src/q27_epi.hip:64-75); the GEMM and its fp32 fold follow src/q27_rb.cpp:43-55 and
 * src/q27_epi.hip:189-243. rows0/nrows select a row range of W. */
static void pf_proj(const i8m* W, int row0, int nrows, const float* v, int M, float* y, int ldy,
                    const float* res, int ldr, float rs, float alpha, float in_scale, int gs) {
    const int K = W->K, ng = K / gs;
    int8_t* wg = (int8_t*)malloc((size_t)nrows * K);
    float* sg = (float*)malloc((size_t)nrows * ng * 4);
    q27o_i8g64_to_grp(W->w + (size_t)row0 * K, W->s + (size_t)row0 * (K / 64), nrows, K, gs, wg, sg);
    int8_t* xq = (int8_t*)malloc((size_t)M * K);
    float* xs = (float*)malloc((size_t)M * ng * 4);
    q27o_quant_tok_groups_g(v, K, M, K, gs, 1.0f / in_scale, xq, xs);
    q27o_gemm_i8g(wg, sg, nrows, K, gs, alpha, xq, xs, M, y, ldy, res, ldr, rs);
    free(wg); free(sg); free(xq); free(xs);
}
static void bf_to_f(const uint16_t* b, float* f, size_t n) { for (size_t i = 0; i < n; ++i) f[i] = q27o_bf2f(b[i]); }
static void f_to_bf(const float* f, uint16_t* b, size_t n) { for (size_t i = 0; i < n; ++i) b[i] = q27o_f2bf(f[i]); }

/* One chunk of C prompt rows at positions p0.. through every layer (ls_q8_layer's stage order,
 * src/q27_main.cpp:4076-4316): input norm -> q|k|v or in_qkv|in_z GEMM -> attention over the
 * cache / conv + GDN scan -> o / out_proj GEMM + residual -> post norm -> gate, up GEMMs ->
 * SwiGLU -> down GEMM + residual. The mixers, norms and residual adds are the decode path's
 * (a row's attention and recurrence are those of verify()); hall gets the rows' final residuals. */
static void pf_chunk(q27o_model* m, const int32_t* ids, int p0, int C, uint16_t* hall) {
    const q27o_cfg* c = &m->c;
    const int H = c->hidden, I = c->inter, D = c->gdn_d, VH = c->gdn_vh;
    const int nqkv = (2 * c->gdn_kh + VH) * D, nz = VH * D;
    const int qr = qrows_of(c), kvr = c->n_kv * c->head_dim, att = c->n_q * c->head_dim;
    const int wq = qr + 2 * kvr, wz = nqkv + nz, wmax = wq > wz ? wq : wz, mmax = nz > att ? nz : att;
    uint16_t* h = (uint16_t*)malloc((size_t)C * H * 2);        /* bf16 residual copy */
    float* hf = (float*)malloc((size_t)C * H * 4);             /* the same as fp32 */
    float* x = (float*)malloc((size_t)C * H * 4);              /* fp32 residual */
    uint16_t* y = (uint16_t*)malloc((size_t)C * H * 2);        /* bf16 normed (a/b) */
    float* v = (float*)malloc((size_t)C * (I > wmax ? I : wmax) * 4);   /* values to quantize / GEMM out */
    uint16_t* pb = (uint16_t*)malloc((size_t)C * wmax * 2);
    uint16_t* mix = (uint16_t*)malloc((size_t)C * mmax * 2);
    uint16_t* qh = (uint16_t*)malloc((size_t)8 * att * 2);
    float* g = (float*)malloc((size_t)C * I * 4);
    float* u = (float*)malloc((size_t)C * I * 4);
    float* ab = (float*)malloc((size_t)C * VH * 4 * 2);
    float* tmp = (float*)malloc((size_t)C * VH * 4);
    for (int r = 0; r < C; ++r) memcpy(h + (size_t)r * H, m->emb + (size_t)ids[p0 + r] * H, (size_t)H * 2);
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* Y = &m->L[L];
        if (L == 0) q27o_rmsnorm_f32_rows(h, 1, H, Y->in_norm, 1.0f, c->rms_eps, H, NULL, y, H, v, H, 1, C);
        else q27o_rmsnorm_f32_rows(x, 0, H, Y->in_norm, 1.0f, c->rms_eps, H, h, y, H, v, H, 0, C);
        bf_to_f(h, hf, (size_t)C * H);
        if (Y->is_attn) {
            float* o = (float*)malloc((size_t)C * wq * 4);
            const int rq[4] = { 0, qr, qr + kvr, wq };
            for (int i = 0; i < 3; ++i)
                pf_proj(&Y->qkv, rq[i], rq[i + 1] - rq[i], v, C, o + rq[i], wq, NULL, 0, 0.0f, Y->al_qkv[i], Y->is_in, pf_gs(c, Y->qkv.K));
            f_to_bf(o, pb, (size_t)C * wq);
            free(o);
            for (int r0 = 0; r0 < C; r0 += 8) {
                const int cn = (C - r0 < 8) ? C - r0 : 8;
                q27o_attn_prep_rows(pb + (size_t)r0 * wq, wq, Y->q_norm, Y->k_norm, m->rope_cos, m->rope_sin,
                                    c->rot_dims, Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, qh, c->n_q, c->n_kv,
                                    c->head_dim, c->attn_gate, c->rms_eps, p0 + r0, cn);
                q27o_attn_rows(qh, pb + (size_t)r0 * wq, wq, Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, c->n_q,
                               c->n_kv, c->head_dim, c->attn_gate, p0 + r0, cn, mix + (size_t)r0 * att, NULL, NULL);
            }
            bf_to_f(mix, v, (size_t)C * att);
            pf_proj(&Y->o, 0, H, v, C, x, H, hf, H, 1.0f, Y->al_o, Y->is_out, pf_gs(c, Y->o.K));
        } else {
            float* o = (float*)malloc((size_t)C * wz * 4);
            pf_proj(&Y->qkvz, 0, nqkv, v, C, o, wz, NULL, 0, 0.0f, Y->al_qkv[0], Y->is_in, pf_gs(c, Y->qkvz.K));
            pf_proj(&Y->qkvz, nqkv, nz, v, C, o + nqkv, wz, NULL, 0, 0.0f, Y->al_qkv[1], Y->is_in, pf_gs(c, Y->qkvz.K));
            f_to_bf(o, pb, (size_t)C * wz);
            free(o);
            /* a / b: the decode path's bf16 GEMV on the bf16 normed rows, bf16 outputs */
            q27o_bf16_gemv_rows(Y->in_a, VH, H, y, H, tmp, VH, C);
            for (int i = 0; i < C * VH; ++i) ab[i] = q27o_bf2f(q27o_f2bf(tmp[i]));
            q27o_bf16_gemv_rows(Y->in_b, VH, H, y, H, tmp, VH, C);
            for (int i = 0; i < C * VH; ++i) ab[C * VH + i] = q27o_bf2f(q27o_f2bf(tmp[i]));
            /* the scan: rows in order, each committed before the next (sub-chunks of 8 rows, each
             * call committing the previous one -- the same updates as one continuous scan) */
            int npend = m->gdn_npend;
            for (int r0 = 0; r0 < C; r0 += 8) {
                const int cn = (C - r0 < 8) ? C - r0 : 8;
                const float* la = ab + (size_t)(g_pf_plant == 4 ? C + r0 : r0) * VH;
                const float* lb = ab + (size_t)(g_pf_plant == 4 ? r0 : C + r0) * VH;
                q27o_gdn_verify(pb + (size_t)r0 * wz, wz, pb + (size_t)r0 * wz + nqkv, wz, la, lb, VH, Y->A_log, Y->dt_bias, Y->gdn_norm, Y->conv_w,
                                Y->S, Y->conv_hist, Y->pend, npend, c->gdn_kh, VH, D, c->rms_eps,
                                mix + (size_t)r0 * nz, nz, NULL, NULL, cn);
                npend = g_pf_plant == 3 ? 0 : cn;
            }
            q27o_gdn_verify(NULL, 0, NULL, 0, NULL, NULL, 0, Y->A_log, Y->dt_bias, Y->gdn_norm, Y->conv_w, Y->S,
                            Y->conv_hist, Y->pend, npend, c->gdn_kh, VH, D, c->rms_eps, NULL, 0, NULL, NULL, 0);
            bf_to_f(mix, v, (size_t)C * nz);
            pf_proj(&Y->out_proj, 0, H, v, C, x, H, hf, H, 1.0f, Y->al_o, Y->is_out, pf_gs(c, Y->out_proj.K));
        }
        q27o_rmsnorm_f32_rows(x, 0, H, Y->post_norm, 1.0f, c->rms_eps, H, h, NULL, H, v, H, 0, C);
        bf_to_f(h, hf, (size_t)C * H);
        pf_proj(&Y->gate, 0, I, v, C, g, I, NULL, 0, 0.0f, Y->al_gate, Y->is_post, pf_gs(c, Y->gate.K));
        pf_proj(&Y->up, 0, I, v, C, u, I, NULL, 0, 0.0f, Y->al_up, Y->is_post, pf_gs(c, Y->up.K));
        const float gsc = 1.0f / Y->is_down;
        for (size_t i = 0; i < (size_t)C * I; ++i) {   /* q27o_swiglu_quant_rows' value */
            const float a = g[i];
            const float sw = a / (1.0f + q27o_exp(-a));
            v[i] = sw * u[i] * gsc;
        }
        pf_proj(&Y->down, 0, H, v, C, x, H, hf, H, g_pf_plant == 1 ? 0.0f : 1.0f, Y->al_down, 1.0f, pf_gs(c, Y->down.K));
    }
    m->gdn_npend = 0;
    for (int r = 0; r < C; ++r)
        for (int k = 0; k < H; ++k) {
            const float t = c->head_double_residual ? q27o_bf2f(h[(size_t)r * H + k]) + x[(size_t)r * H + k]
                                                    : x[(size_t)r * H + k];
            hall[(size_t)r * H + k] = q27o_f2bf(t);
        }
    free(h); free(hf); free(x); free(y); free(v); free(pb); free(mix); free(qh); free(g); free(u); free(ab); free(tmp);
}

/* The MTP prompt pass over positions [p0, p0 + C) (mtp_prompt_pass, src/q27_main.cpp:2647-2688):
 * position p pairs the final residual at p with the embedding of token p+1; pre-norms (fp32
 * values, per-(token, group) quantized), fc as two GEMMs (the embedding half first, the hidden
 * half added in fp32), the layer's input norm, then only k|v: their rows' GEMM -> bf16 -> K/V
 * cache (k_norm, RoPE, int8) at draft positions p. */
static void pf_mtp(q27o_model* m, const int32_t* ids, int p0, int C, const uint16_t* hall) {
    const q27o_cfg* c = &m->c;
    layer_t* Y = &m->mtp;
    const int H = c->hidden;
    const int qr = qrows_of(c), kvr = c->n_kv * c->head_dim, att = c->n_q * c->head_dim, wq = qr + 2 * kvr;
    const float po = c->mtp_plus_one ? 1.0f : 0.0f;
    float* ve = (float*)malloc((size_t)C * H * 4);
    float* vh = (float*)malloc((size_t)C * H * 4);
    float* res = (float*)malloc((size_t)C * H * 4);
    float* kv = (float*)malloc((size_t)C * 2 * kvr * 4);
    uint16_t* pb = (uint16_t*)calloc((size_t)C * wq, 2);
    uint16_t* qh = (uint16_t*)malloc((size_t)8 * att * 2);
    uint16_t* e = (uint16_t*)malloc((size_t)C * H * 2);
    for (int r = 0; r < C; ++r) memcpy(e + (size_t)r * H, m->emb + (size_t)ids[p0 + r + 1] * H, (size_t)H * 2);
    q27o_rmsnorm_f32_rows(e, 1, H, m->pre_emb, po, c->rms_eps, H, NULL, NULL, H, ve, H, 0, C);
    q27o_rmsnorm_f32_rows(hall + (size_t)p0 * H, 1, H, m->pre_hid, po, c->rms_eps, H, NULL, NULL, H, vh, H, 0, C);
    const int sw = c->mtp_swap ^ (g_pf_plant == 2);
    const i8m* fe = sw ? &m->fc0 : &m->fc1;   /* the half that multiplies the embedding */
    const i8m* fh = sw ? &m->fc1 : &m->fc0;
    pf_proj(fe, 0, H, ve, C, res, H, NULL, 0, 0.0f, 1.0f, 1.0f, fe->K);
    pf_proj(fh, 0, H, vh, C, res, H, res, H, 1.0f, 1.0f, 1.0f, fh->K);
    q27o_rmsnorm_f32_rows(res, 0, H, Y->in_norm, po, c->rms_eps, H, NULL, NULL, H, ve, H, 0, C);
    pf_proj(&Y->qkv, qr, 2 * kvr, ve, C, kv, 2 * kvr, NULL, 0, 0.0f, 1.0f, 1.0f, Y->qkv.K);
    for (int r = 0; r < C; ++r)
        for (int k = 0; k < 2 * kvr; ++k) pb[(size_t)r * wq + qr + k] = q27o_f2bf(kv[(size_t)r * 2 * kvr + k]);
    for (int r0 = 0; r0 < C; r0 += 8) {
        const int cn = (C - r0 < 8) ? C - r0 : 8;
        q27o_attn_prep_rows(pb + (size_t)r0 * wq, wq, Y->q_norm, Y->k_norm, m->rope_cos, m->rope_sin, c->rot_dims,
                            Y->kc, Y->ks, Y->vc, Y->vs, c->kv_group, qh, c->n_q, c->n_kv, c->head_dim, c->attn_gate,
                            c->rms_eps, p0 + r0, cn);
    }
    free(ve); free(vh); free(res); free(kv); free(pb); free(qh); free(e);
}

int q27o_model_prefill_gemm(q27o_model* m, const int32_t* ids, int n, int chunk) {
    const q27o_cfg* c = &m->c;
    const int H = c->hidden;
    if (chunk < 1) chunk = n;
    q27o_model_reset(m);
    uint16_t* hall = (uint16_t*)malloc((size_t)n * H * 2);
    for (int p0 = 0; p0 < n; p0 += chunk) {
        const int C = (n - p0 < chunk) ? n - p0 : chunk;
        pf_chunk(m, ids, p0, C, hall + (size_t)p0 * H);
        const int cm = (p0 + C < n) ? C : C - 1;    /* MTP positions of this chunk (p + 1 < n) */
        if (cm > 0) pf_mtp(m, ids, p0, cm, hall);
    }
    /* head of the last row: final norm, lm_head, argmax */
    uint16_t* y = (uint16_t*)malloc((size_t)H * 2);
    float* logits = (float*)malloc((size_t)c->vocab * 4);
    q27o_rmsnorm_quant_rows(hall + (size_t)(n - 1) * H, 1, H, m->final_norm, 1.0f, c->rms_eps, H, NULL, y, H, NULL,
                            NULL, 1, 1.0f, 1);
    q27o_bf16_gemv_rows(m->lm_head, c->vocab, H, y, H, logits, c->vocab, 1);
    int32_t first = 0;
    float val = 0.0f;
    q27o_argmax_rows(logits, c->vocab, c->vocab, 1, &first, &val);
    memcpy(m->hprev, hall + (size_t)(n - 1) * H, (size_t)H * 2);
    free(y); free(logits); free(hall);
    m->pos = n; m->tok = first; m->ncatch = 0; m->have_h = 1; m->gdn_npend = 0;
    return first;
}

/* plain greedy step (the Q27_SPEC=0 path, src/q27_main.cpp:6396-6502) */
int q27o_model_decode_step(q27o_model* m) {
    int32_t t = m->tok, nx;
    verify(m, 1, &t, &nx);
    memcpy(m->hprev, m->hfinal, (size_t)m->c.hidden * 2);
    m->ncatch = 0;
    m->pos += 1;
    m->tok = nx;
    return nx;
}

/* One MTP pass on its own (the kernel-tier q27x_mtp_draft): nr rows (hidden rows hrows [nr][H]
 * bf16, tokens toks) at draft positions dpos0.. of the layer's KV cache; writes the layer's
 * residual rows res [nr][H] bf16 and, for head_row >= 0, that row's logits [vocab] fp32; returns
 * the head row's argmax (or -1). */
int q27o_model_mtp_pass(q27o_model* m, int nr, const uint16_t* hrows, const int32_t* toks, int dpos0,
                        int head_row, uint16_t* res, float* logits) {
    const uint16_t* hr[8];
    if (nr < 1 || nr > 8) return -2;
    for (int r = 0; r < nr; ++r) hr[r] = hrows + (size_t)r * m->c.hidden;
    return mtp_pass(m, nr, hr, toks, dpos0, head_row, res, logits);
}

int q27o_model_verify_rows(q27o_model* m, int nr, const int32_t* toks, int32_t* nx) {
    verify(m, nr, toks, nx);
    return 0;
}

/* Benchmark set-up: the next verify runs at position pos (rows pos.., attending to whatever the
 * caches hold below it), the next draft pass at pos - 1; every committed row of the GDN layers is
 * taken as applied. */
int q27o_model_set_pos(q27o_model* m, int pos) {
    if (pos < 1 || pos + 8 > m->c.ctx) return -1;
    m->pos = pos; m->gdn_npend = 0; m->ncatch = 0; m->have_h = 1;
    return 0;
}

/* One verify pass at the current position with its logits [nr][vocab] (for the float64 pin of the
 * trunk composition). advance != 0 commits the rows as a prompt chunk does: pos += nr. */
int q27o_model_verify_logits(q27o_model* m, int nr, const int32_t* toks, int32_t* nx, float* logits, int advance) {
    return q27o_model_verify_trace(m, nr, toks, nx, logits, advance, NULL, NULL, NULL, NULL);
}
int q27o_model_verify_trace(q27o_model* m, int nr, const int32_t* toks, int32_t* nx, float* logits, int advance,
                            float* r1, float* r2, int8_t* pq, float* ps) {
    if (nr < 1 || nr > 8 || m->pos + nr > m->c.ctx || (pq && !ps)) return -1;
    m->vlogits = logits;
    m->tr_r1 = r1; m->tr_r2 = r2; m->tr_pq = pq; m->tr_ps = ps;
    verify(m, nr, toks, nx);
    m->vlogits = NULL;
    m->tr_r1 = m->tr_r2 = m->tr_ps = NULL; m->tr_pq = NULL;
    if (advance) m->pos += nr;
    return 0;
}

/* spec_round (src/q27_main.cpp:2702-2958). forced != NULL: forced[j] replaces the MTP argmax of
 * draft j (forced-acceptance mode; the draft work is unchanged). */
int q27o_model_spec_round(q27o_model* m, int32_t* out, const int32_t* forced) {
    const int H = m->c.hidden, K = m->c.spec_k;
    int32_t dt[8], nx[8], toks[8];
    uint16_t* res = (uint16_t*)malloc((size_t)8 * H * 2);
    /* [1] draft 0 over the catch-up rows plus (h_prev, tok); drafts 1..K-1 chained on the MTP
     * layer's own residual */
    {
        const uint16_t* hr[8]; int32_t tk[8]; int nrm = 0;
        for (int cc = 0; cc < m->ncatch; ++cc) { hr[nrm] = m->hcatch + (size_t)cc * H; tk[nrm] = m->catch_tok[cc]; ++nrm; }
        hr[nrm] = m->hprev; tk[nrm] = m->tok; ++nrm;
        const int dpos0 = m->pos - 1 - m->ncatch;
        int d0 = mtp_pass(m, nrm, hr, tk, dpos0, nrm - 1, res, NULL);
        m->dt_raw[0] = d0;
        if (forced) d0 = forced[0];
        dt[0] = d0;
        memcpy(m->hchain, res + (size_t)(nrm - 1) * H, (size_t)H * 2);
        m->ncatch = 0;
    }
    for (int j = 1; j < K; ++j) {
        const uint16_t* hr[1] = { m->hchain };
        const int32_t tk[1] = { dt[j - 1] };
        int dj = mtp_pass(m, 1, hr, tk, m->pos - 1 + j, 0, res, NULL);
        m->dt_raw[j] = dj;
        if (forced) dj = forced[j];
        dt[j] = dj;
        memcpy(m->hchain, res, (size_t)H * 2);
    }
    /* [2] verify [tok @ pos, dt[0] @ pos+1, ..., dt[K-1] @ pos+K] */
    toks[0] = m->tok;
    for (int r = 1; r <= K; ++r) toks[r] = dt[r - 1];
    verify(m, K + 1, toks, nx);
    /* [3] greedy acceptance; [4] rollback = commit only rows 0..nacc; hand-off */
    const int nacc = q27o_accept(nx, dt, K, out);
    for (int j = 0; j < 8; ++j) {
        m->dt[j] = j < K ? dt[j] : 0;
        m->nx[j] = j <= K ? nx[j] : 0;
        if (j >= K) m->dt_raw[j] = 0;
    }
    m->nacc_last = nacc;
    m->gdn_npend = nacc + 1;
    for (int j = 0; j < nacc; ++j) {
        memcpy(m->hcatch + (size_t)j * H, m->hfinal + (size_t)j * H, (size_t)H * 2);
        m->catch_tok[j] = nx[j];
    }
    m->ncatch = nacc;
    memcpy(m->hprev, m->hfinal + (size_t)nacc * H, (size_t)H * 2);
    m->tok = nx[nacc];
    m->pos += nacc + 1;
    free(res);
    return nacc + 1;
}

void* q27o_model_tensor(q27o_model* m, const char* name, int layer, size_t* bytes) {
    const q27o_cfg* c = &m->c;
    const int H = c->hidden, D = c->gdn_d;
    const int nqkv = (2 * c->gdn_kh + c->gdn_vh) * D;
    layer_t* Y = (layer >= 0 && layer < c->n_layers) ? &m->L[layer] : &m->mtp;
    size_t b = 0; void* p = NULL;
    if (!strcmp(name, "S") && !Y->is_attn) { p = Y->S; b = (size_t)c->gdn_vh * D * D * 4; }
    else if (!strcmp(name, "conv_hist") && !Y->is_attn) { p = Y->conv_hist; b = (size_t)nqkv * 3 * 2; }
    else if (!strcmp(name, "kc") && Y->is_attn) { p = Y->kc; b = (size_t)c->ctx * c->n_kv * c->head_dim; }
    else if (!strcmp(name, "hprev")) { p = m->hprev; b = (size_t)H * 2; }
    else if (!strcmp(name, "hfinal")) { p = m->hfinal; b = (size_t)8 * H * 2; }
    else if (!strcmp(name, "emb")) { p = m->emb; b = (size_t)c->vocab * H * 2; }
    else if (!strcmp(name, "lm_head")) { p = m->lm_head; b = (size_t)c->vocab * H * 2; }
    else if (!strcmp(name, "gate_w")) { p = Y->gate.w; b = (size_t)c->inter * H; }
    else if (!strcmp(name, "gate_s")) { p = Y->gate.s; b = (size_t)c->inter * (H / 64) * 4; }
    else if (!strcmp(name, "conv_w") && !Y->is_attn) { p = Y->conv_w; b = (size_t)nqkv * 4 * 2; }
    else if (!strcmp(name, "ks") && Y->is_attn) { p = Y->ks; b = (size_t)c->ctx * c->n_kv * c->head_dim / c->kv_group * 4; }
    else if (!strcmp(name, "vc") && Y->is_attn) { p = Y->vc; b = (size_t)c->ctx * c->n_kv * c->head_dim; }
    else if (!strcmp(name, "vs") && Y->is_attn) { p = Y->vs; b = (size_t)c->ctx * c->n_kv * c->head_dim / c->kv_group * 4; }
    else if (!strcmp(name, "hcatch")) { p = m->hcatch; b = (size_t)8 * H * 2; }
    else if (!strcmp(name, "hchain")) { p = m->hchain; b = (size_t)H * 2; }
    else if (!strcmp(name, "dt")) { p = m->dt; b = 8 * 4; }
    else if (!strcmp(name, "dt_raw")) { p = m->dt_raw; b = 8 * 4; }
    else if (!strcmp(name, "nx")) { p = m->nx; b = 8 * 4; }
    else if (!strcmp(name, "catch_tok")) { p = m->catch_tok; b = 8 * 4; }
    else if (!strcmp(name, "pos")) { static int v; v = m->pos; p = &v; b = 4; }
    else if (!strcmp(name, "tok")) { static int v2; v2 = m->tok; p = &v2; b = 4; }
    else if (!strcmp(name, "ncatch")) { static int v3; v3 = m->ncatch; p = &v3; b = 4; }
    else if (!strcmp(name, "nacc")) { static int v4; v4 = m->nacc_last; p = &v4; b = 4; }
    /* weights of a layer (layer < 0: the MTP layer) and the MTP globals, for float64 forwards */
    else if (!strcmp(name, "in_norm")) { p = Y->in_norm; b = (size_t)H * 2; }
    else if (!strcmp(name, "post_norm")) { p = Y->post_norm; b = (size_t)H * 2; }
    else if (!strcmp(name, "up_w")) { p = Y->up.w; b = (size_t)c->inter * H; }
    else if (!strcmp(name, "up_s")) { p = Y->up.s; b = (size_t)c->inter * (H / 64) * 4; }
    else if (!strcmp(name, "down_w") && Y->down.w) { p = Y->down.w; b = (size_t)H * c->inter; }
    else if (!strcmp(name, "down_s") && Y->down.s) { p = Y->down.s; b = (size_t)H * (c->inter / 64) * 4; }
    else if (!strncmp(name, "down4_w", 7) && Y->down4[0].w) {
        const int j = name[7] - '0'; if (j >= 0 && j < 4) { p = Y->down4[j].w; b = (size_t)H * (c->inter / 4); } }
    else if (!strncmp(name, "down4_s", 7) && Y->down4[0].s) {
        const int j = name[7] - '0'; if (j >= 0 && j < 4) { p = Y->down4[j].s; b = (size_t)H * (c->inter / 256) * 4; } }
    else if (!strcmp(name, "qkv_w") && Y->is_attn) { p = Y->qkv.w; b = (size_t)Y->qkv.rows * H; }
    else if (!strcmp(name, "qkv_s") && Y->is_attn) { p = Y->qkv.s; b = (size_t)Y->qkv.rows * (H / 64) * 4; }
    else if (!strcmp(name, "q_norm") && Y->is_attn) { p = Y->q_norm; b = (size_t)c->head_dim * 2; }
    else if (!strcmp(name, "k_norm") && Y->is_attn) { p = Y->k_norm; b = (size_t)c->head_dim * 2; }
    else if (!strcmp(name, "o_w") && Y->is_attn) { p = Y->o.w; b = (size_t)H * Y->o.K; }
    else if (!strcmp(name, "o_s") && Y->is_attn) { p = Y->o.s; b = (size_t)H * (Y->o.K / 64) * 4; }
    else if (!strcmp(name, "fc0_w")) { p = m->fc0.w; b = (size_t)H * H; }
    else if (!strcmp(name, "fc0_s")) { p = m->fc0.s; b = (size_t)H * (H / 64) * 4; }
    else if (!strcmp(name, "fc1_w")) { p = m->fc1.w; b = (size_t)H * H; }
    else if (!strcmp(name, "fc1_s")) { p = m->fc1.s; b = (size_t)H * (H / 64) * 4; }
    else if (!strcmp(name, "pre_emb")) { p = m->pre_emb; b = (size_t)H * 2; }
    else if (!strcmp(name, "pre_hid")) { p = m->pre_hid; b = (size_t)H * 2; }
    else if (!strcmp(name, "mtp_norm")) { p = m->mtp_norm; b = (size_t)H * 2; }
    else if (!strcmp(name, "final_norm")) { p = m->final_norm; b = (size_t)H * 2; }
    else if (!strcmp(name, "gate_s")) { p = Y->gate.s; b = (size_t)c->inter * (H / 64) * 4; }
    else if (!strcmp(name, "qkvz_w") && !Y->is_attn && Y->qkvz.w) { p = Y->qkvz.w; b = (size_t)Y->qkvz.rows * H; }
    else if (!strcmp(name, "qkvz_s") && !Y->is_attn && Y->qkvz.s) { p = Y->qkvz.s; b = (size_t)Y->qkvz.rows * (H / 64) * 4; }
    else if (!strcmp(name, "out_w") && !Y->is_attn && Y->out_proj.w) { p = Y->out_proj.w; b = (size_t)H * Y->out_proj.K; }
    else if (!strcmp(name, "out_s") && !Y->is_attn && Y->out_proj.s) { p = Y->out_proj.s; b = (size_t)H * (Y->out_proj.K / 64) * 4; }
    else if (!strcmp(name, "in_a") && !Y->is_attn && Y->in_a) { p = Y->in_a; b = (size_t)c->gdn_vh * H * 2; }
    else if (!strcmp(name, "in_b") && !Y->is_attn && Y->in_b) { p = Y->in_b; b = (size_t)c->gdn_vh * H * 2; }
    else if (!strcmp(name, "A_log") && !Y->is_attn && Y->A_log) { p = Y->A_log; b = (size_t)c->gdn_vh * 2; }
    else if (!strcmp(name, "dt_bias") && !Y->is_attn && Y->dt_bias) { p = Y->dt_bias; b = (size_t)c->gdn_vh * 2; }
    else if (!strcmp(name, "gdn_norm") && !Y->is_attn && Y->gdn_norm) { p = Y->gdn_norm; b = (size_t)D * 2; }
    if (bytes) *bytes = b;
    return p;
}
