/* q27o.c -- CPU oracle, kernel-level functions. TEST INFRASTRUCTURE ONLY (see q27o.h).
 * Build: -O2 -ffp-contract=off -fno-fast-math (every fused multiply-add is an explicit fmaf). */
#include "q27o.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ scalars */
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t q27o_f2bf(float f) {   /* include/q27.h:136-139: (u + 0x7FFF + ((u >> 16) & 1)) >> 16 */
    const uint32_t u = f_bits(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float q27o_bf2f(uint16_t b) { return bits_f((uint32_t)b << 16); }

/* p * 2^n for p in [0.5, 2) and n in [-152, 130], one rounding at the final product. */
static inline float scale2(float p, int n) {
    if (n > 127) { p = p * 0x1p127f; n -= 127; }
    if (n < -126) { p = p * 0x1p-64f; n += 64; }
    return p * bits_f((uint32_t)(n + 127) << 23);
}

/* e^x: Cody-Waite reduction x = k ln2 + r (ln2 split hi/lo), Taylor polynomial of degree 7 on
 * |r| <= ln2/2 (truncation < 0.05 ulp), Horner with fmaf. */
float q27o_exp(float x) {
    if (x != x) return x;
    if (x > 88.7228393555f) return INFINITY;
    if (x < -103.972084045f) return 0.0f;
    const float kf = rintf(x * 1.44269502163f);
    float r = fmaf(kf, -0.693145751953125f, x);
    r = fmaf(kf, -1.42860682e-06f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333377e-3f);
    p = fmaf(p, r, 4.16666679e-2f);
    p = fmaf(p, r, 1.66666672e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return scale2(p, (int)kf);
}

/* 2^x: x = k + r exactly (|r| <= 1/2), e^(r ln2) by its degree-7 Taylor polynomial. */
float q27o_exp2(float x) {
    if (x != x) return x;
    if (x >= 128.0f) return INFINITY;
    if (x < -150.0f) return 0.0f;
    const float kf = rintf(x);
    const float r = x - kf;
    float p = 1.52527336e-5f;
    p = fmaf(p, r, 1.54035304e-4f);
    p = fmaf(p, r, 1.33335581e-3f);
    p = fmaf(p, r, 9.61812911e-3f);
    p = fmaf(p, r, 5.55041087e-2f);
    p = fmaf(p, r, 2.40226507e-1f);
    p = fmaf(p, r, 6.93147182e-1f);
    p = fmaf(p, r, 1.0f);
    return scale2(p, (int)kf);
}

/* log(u) for finite normal u > 0: u = m 2^e, m in (sqrt(1/2), sqrt(2)], s = (m-1)/(m+1),
 * log m = 2 atanh s by its odd series to s^9. */
static float log_pos(float u) {
    const uint32_t b = f_bits(u);
    int e = (int)((b >> 23) & 0xffu) - 127;
    float m = bits_f((b & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float p = 0.222222224f;
    p = fmaf(p, s2, 0.285714298f);
    p = fmaf(p, s2, 0.400000006f);
    p = fmaf(p, s2, 0.666666687f);
    p = p * s2;
    const float lm = fmaf(s, p, s + s);
    const float ef = (float)e;
    return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.42860682e-06f, lm));
}

/* log(1+y), y > -1: log(u) * y/(u-1) with u = fl(1+y) corrects the rounding of 1+y. */
float q27o_log1p(float y) {
    if (y != y) return y;
    if (y == INFINITY) return y;
    const float u = 1.0f + y;
    if (u == 1.0f) return y;
    return log_pos(u) * (y / (u - 1.0f));
}
float q27o_sigmoid(float x) { return 1.0f / (1.0f + q27o_exp(-x)); }
float q27o_silu(float x) { return x / (1.0f + q27o_exp(-x)); }
float q27o_softplus(float x) { return (x > 20.0f) ? x : q27o_log1p(q27o_exp(x)); }

void q27o_math_vec(const float* x, float* y, int n, int op) {
    for (int i = 0; i < n; ++i) {
        const float v = x[i];
        float r;
        switch (op) {
            case 0: r = q27o_exp(v); break;
            case 1: r = q27o_exp2(v); break;
            case 2: r = q27o_log1p(v); break;
            case 3: r = q27o_sigmoid(v); break;
            case 4: r = q27o_silu(v); break;
            default: r = q27o_softplus(v); break;
        }
        y[i] = r;
    }
}

/* ------------------------------------------------------------------ generator */
static inline uint64_t sm64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
uint64_t q27o_hash(uint64_t seed, uint64_t tensor, uint64_t idx) {
    return sm64(sm64(seed ^ (tensor * 0xD6E8FEB86659FD93ull)) + idx);
}
/* Irwin-Hall(4) on four 16-bit fields of one hash: integer sum (exact), one float subtraction
 * (exact), one multiply by sqrt(3)/65536 -> mean 0, variance 1, support +-3.46. */
float q27o_normal(uint64_t seed, uint64_t tensor, uint64_t idx) {
    const uint64_t h = q27o_hash(seed, tensor, idx);
    const uint32_t s = (uint32_t)(h & 0xffffu) + (uint32_t)((h >> 16) & 0xffffu) +
                       (uint32_t)((h >> 32) & 0xffffu) + (uint32_t)(h >> 48);
    return ((float)s - 131070.0f) * 2.64289800e-05f;
}
float q27o_uniform(uint64_t seed, uint64_t tensor, uint64_t idx) {
    const uint64_t h = q27o_hash(seed, tensor, idx);
    return (float)(uint32_t)(h >> 40) * 0x1p-24f;
}

/* ------------------------------------------------------------------ quantizers */
static inline int8_t q_code(float v, float inv) {
    int c = (int)rintf(v * inv);
    c = c < -127 ? -127 : (c > 127 ? 127 : c);
    return (int8_t)c;
}

/* R5: src/q27_fp8.hip:373-425 (q27_quant_fp8_body), natural order, g = 1/in_scale. */
void q27o_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs,
                     int sstride, int n, float in_scale, int nrows) {
    const float g = 1.0f / in_scale;
    for (int r = 0; r < nrows; ++r) {
        const uint16_t* xr = x + (size_t)r * xstride;
        for (int k0 = 0; k0 < n; k0 += 16) {
            float v[16], mx = 0.0f;
            for (int j = 0; j < 16; ++j) { v[j] = q27o_bf2f(xr[k0 + j]); mx = fmaxf(mx, fabsf(v[j])); }
            const float s = mx * g * (1.0f / 127.0f);
            const float inv = (s > 0.0f) ? (g / s) : 0.0f;
            xs[(size_t)r * sstride + (k0 >> 4)] = s;
            for (int j = 0; j < 16; ++j) xq[(size_t)r * qstride + k0 + j] = q_code(v[j], inv);
        }
    }
}

/* Group quantizer of fp32 values: sc = mx*(1/127), inv = sc>0 ? 1/sc : 0 -- the form shared by
 * the weight mirror (src/q27_nvfp4.hip:4270-4276), the KV writer (src/q27_attn.hip:156-168) and
 * the SwiGLU quantizer (src/q27_nvfp4.hip:4008-4010). */
void q27o_quant_f32(const float* v, int n, int group, int8_t* q, float* s) {
    for (int g0 = 0; g0 < n; g0 += group) {
        float mx = 0.0f;
        for (int j = 0; j < group; ++j) mx = fmaxf(mx, fabsf(v[g0 + j]));
        const float sc = mx * (1.0f / 127.0f);
        const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
        s[g0 / group] = sc;
        for (int j = 0; j < group; ++j) q[g0 + j] = q_code(v[g0 + j], inv);
    }
}

/* R8: src/q27_nvfp4.hip:4259-4289 (q27_k_fp8_to_i8g64) */
void q27o_quant_weights_i8g64(const float* w, int rows, int K, int8_t* wq, float* ws) {
    for (int r = 0; r < rows; ++r)
        q27o_quant_f32(w + (size_t)r * K, K, 64, wq + (size_t)r * K, ws + (size_t)r * (K / 64));
}

/* ------------------------------------------------------------------ prefill GEMM (per group) */
/* Weights, per-64 mirror -> per-(row, group of gs): src/q27_epi.hip:14-35 (q27_k_i8g64_to_grp).
 * sg = max of the group's per-64 scales; inv = sg>0 ? 1/sg : 0; code = clamp(rint((w*s64)*inv)). */
void q27o_i8g64_to_grp(const int8_t* w, const float* s64, int rows, int K, int gs, int8_t* wg, float* sg) {
    const int ns = K / 64, ng = K / gs;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < ng; ++g) {
            float mx = 0.0f;
            for (int i = 0; i < gs / 64; ++i) mx = fmaxf(mx, s64[(size_t)r * ns + g * (gs / 64) + i]);
            const float inv = (mx > 0.0f) ? 1.0f / mx : 0.0f;
            sg[(size_t)r * ng + g] = mx;
            for (int k = g * gs; k < (g + 1) * gs; ++k)
                wg[(size_t)r * K + k] = q_code((float)w[(size_t)r * K + k] * s64[(size_t)r * ns + (k >> 6)], inv);
        }
}

/* Activations per (token, group of gs): q27_quant_group, src/q27_epi.hip:64-75 (the same
 * sc = mx*(1/127), inv = 1/sc form as q27o_quant_f32). Row t of x at x + t*xstride. */
void q27o_quant_tok_groups(const float* x, int xstride, int M, int K, int gs, int8_t* xq, float* xs) {
    for (int t = 0; t < M; ++t)
        q27o_quant_f32(x + (size_t)t * xstride, K, gs, xq + (size_t)t * K, xs + (size_t)t * (K / gs));
}

/* The int32 slabs of src/q27_rb.cpp:43-55: part[g][t][n] = sum over group g of x[t][k]*w[n][k]. */
void q27o_gemm_i8g_partials(const int8_t* w, int N, int K, int gs, const int8_t* x, int M, int32_t* part) {
    const int ng = K / gs;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int t = 0; t < M; ++t)
            for (int g = 0; g < ng; ++g) {
                int32_t acc = 0;
                const int8_t* wr = w + (size_t)n * K + (size_t)g * gs;
                const int8_t* xr = x + (size_t)t * K + (size_t)g * gs;
                for (int k = 0; k < gs; ++k) acc += (int32_t)wr[k] * (int32_t)xr[k];
                part[((size_t)g * M + t) * N + n] = acc;
            }
}

/* The slab-sum epilogue, src/q27_epi.hip:189-203 (q27_slab4) and 235-243 (q27_k_epi_f32r):
 * o = 0; for g ascending: o = fmaf((float)acc_g, sw[n][g]*sx[t][g], o); y = o*alpha (+ rs*res). */
void q27o_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                   const float* sx, int M, float* y, int ldy, const float* res, int ldr, float rs) {
    const int ng = K / gs;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int t = 0; t < M; ++t) {
            float o = 0.0f;
            for (int g = 0; g < ng; ++g) {
                int32_t acc = 0;
                const int8_t* wr = w + (size_t)n * K + (size_t)g * gs;
                const int8_t* xr = x + (size_t)t * K + (size_t)g * gs;
                for (int k = 0; k < gs; ++k) acc += (int32_t)wr[k] * (int32_t)xr[k];
                o = fmaf((float)acc, sw[(size_t)n * ng + g] * sx[(size_t)t * ng + g], o);
            }
            o = o * alpha;
            if (res) o = o + rs * res[(size_t)t * ldr + n];
            y[(size_t)t * ldy + n] = o;
        }
}

/* R16: src/q27_nvfp4.hip:3984-4031 (natural order here): sw = g/(1+e^-g); v = sw*u*gscale. */
void q27o_swiglu_quant_rows(const float* gate, const float* up, int stride, int8_t* xq,
                            float* xs, int n, float in_scale, int nr) {
    const float gs = 1.0f / in_scale;
    float* v = (float*)malloc((size_t)n * sizeof(float));
    for (int r = 0; r < nr; ++r) {
        const float* G = gate + (size_t)r * stride;
        const float* U = up + (size_t)r * stride;
        for (int i = 0; i < n; ++i) {
            const float a = G[i];
            const float sw = a / (1.0f + q27o_exp(-a));
            v[i] = sw * U[i] * gs;
        }
        q27o_quant_f32(v, n, 16, xq + (size_t)r * n, xs + (size_t)r * (n / 16));
    }
    free(v);
}

/* ------------------------------------------------------------------ reductions */
/* shfl_down tree over 64 lane values (offsets 32..1): lane l < o takes a[l] + a[l+o]. */
static inline float tree64(float* a) {
    for (int o = 32; o > 0; o >>= 1)
        for (int l = 0; l < o; ++l) a[l] = a[l] + a[l + o];
    return a[0];
}

/* Row sum of squares, the 256-thread layout: element 1024i + 4t + e to thread t. */
float q27o_rowsumsq(const float* x, int n) {
    float acc[256];
    for (int t = 0; t < 256; ++t) {
        float a = 0.0f;
        for (int i = 0; i * 1024 < n; ++i)
            for (int e = 0; e < 4; ++e) {
                const int k = i * 1024 + 4 * t + e;
                if (k < n) a = fmaf(x[k], x[k], a);
            }
        acc[t] = a;
    }
    const float w0 = tree64(acc), w1 = tree64(acc + 64), w2 = tree64(acc + 128), w3 = tree64(acc + 192);
    return ((w0 + w1) + w2) + w3;
}

/* Head sum of products: chunks of 64 elements, one lane each, tree per chunk, chunks added in
 * order (src/q27_gdn.hip:291-300: two waves' ladders then r0[0] + r0[1]). */
float q27o_headsum(const float* a, const float* b, int n) {
    float tot = 0.0f;
    for (int c = 0; c < n; c += 64) {
        float t[64];
        for (int l = 0; l < 64; ++l) t[l] = a[c + l] * b[c + l];
        const float w = tree64(t);
        tot = (c == 0) ? w : tot + w;
    }
    return tot;
}

/* ------------------------------------------------------------------ R7 projection */
static inline int32_t dot16(const int8_t* w, const int8_t* x) {
    int32_t d = 0;
    for (int i = 0; i < 16; ++i) d += (int32_t)w[i] * (int32_t)x[i];
    return d;
}

/* src/q27_fp8.hip:3814-3871 (q27_k_proj_i8g_snr): lane l, step t covers slab 64t + l. */
void q27o_proj_rows(const int8_t* W, const float* WS, float alpha, int rows, int K,
                    const int8_t* xq, int xstride, const float* xs, float* y, int ystride,
                    int nr) {
    const int nslab = K / 16;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const int8_t* wr = W + (size_t)r * K;
        const float* wsr = WS + (size_t)r * (K / 64);
        for (int n = 0; n < nr; ++n) {
            const int8_t* xr = xq + (size_t)n * xstride;
            const float* xsr = xs + (size_t)n * (xstride / 16);
            float acc[64];
            for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
            for (int s = 0; s < nslab; ++s) {
                const int32_t d = dot16(wr + 16 * s, xr + 16 * s);
                acc[s & 63] = fmaf((float)d, wsr[s >> 2] * xsr[s], acc[s & 63]);
            }
            y[(size_t)n * ystride + r] = tree64(acc) * alpha;
        }
    }
}

void q27o_proj_partials(const int8_t* W, int rows, int K, const int8_t* xq, int xstride,
                        int32_t* part, int nr) {
    const int nslab = K / 16;
    for (int n = 0; n < nr; ++n)
        for (int r = 0; r < rows; ++r)
            for (int s = 0; s < nslab; ++s)
                part[((size_t)n * rows + r) * nslab + s] =
                    dot16(W + (size_t)r * K + 16 * s, xq + (size_t)n * xstride + 16 * s);
}

void q27o_proj_rows_epi(const int8_t* W, const float* WS, float alpha, int rows, int K,
                        const int8_t* xq, int xstride, const float* xs, void* y, int ystride,
                        int out_bf16, const void* res, int res_bf16, int rstride, float rs,
                        int nr) {
    float* t = (float*)malloc((size_t)nr * rows * sizeof(float));
    q27o_proj_rows(W, WS, alpha, rows, K, xq, xstride, xs, t, rows, nr);
    for (int n = 0; n < nr; ++n)
        for (int r = 0; r < rows; ++r) {
            float v = t[(size_t)n * rows + r];
            if (res) {
                const float rv = res_bf16 ? q27o_bf2f(((const uint16_t*)res)[(size_t)n * rstride + r])
                                          : ((const float*)res)[(size_t)n * rstride + r];
                v = v + rs * rv;
            }
            if (out_bf16) ((uint16_t*)y)[(size_t)n * ystride + r] = q27o_f2bf(v);
            else ((float*)y)[(size_t)n * ystride + r] = v;
        }
    free(t);
}

/* ------------------------------------------------------------------ bf16 GEMV */
/* src/q27_util.hip:114-157 (k_bf16_gemv2_tile) arithmetic, this build's lane-chunk order:
 * chunk c of 8 elements to lane c%64, fmaf per element. */
void q27o_bf16_gemv_rows(const uint16_t* W, int rows, int K, const uint16_t* x, int xstride,
                         float* y, int ystride, int nr) {
    const int nch = K / 8;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint16_t* wr = W + (size_t)r * K;
        for (int n = 0; n < nr; ++n) {
            const uint16_t* xr = x + (size_t)n * xstride;
            float acc[64];
            for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
            for (int c = 0; c < nch; ++c) {
                float a = acc[c & 63];
                for (int e = 0; e < 8; ++e) a = fmaf(q27o_bf2f(wr[8 * c + e]), q27o_bf2f(xr[8 * c + e]), a);
                acc[c & 63] = a;
            }
            y[(size_t)n * ystride + r] = tree64(acc);
        }
    }
}

/* ------------------------------------------------------------------ R22 RMSNorm + quantize */
/* src/q27_elem.hip:453-613 (bf16 input, quantize the bf16 normed vector) and 835-910 (fp32
 * input, quantize the fp32 normed vector); inv = 1/sqrt(ss/n + eps) with correctly rounded
 * sqrt and divide in place of v_rsq. */
void q27o_rmsnorm_quant_rows(const void* x, int x_bf16, int xstride, const uint16_t* w,
                             float plus, float eps, int n, uint16_t* hcopy, uint16_t* y,
                             int ystride, int8_t* xq, float* xs, int quant_bf16,
                             float in_scale, int nr) {
    float* xv = (float*)malloc((size_t)n * sizeof(float));
    float* nv = (float*)malloc((size_t)n * sizeof(float));
    const float rn = 1.0f / (float)n;
    const float g = 1.0f / in_scale;
    for (int r = 0; r < nr; ++r) {
        for (int k = 0; k < n; ++k)
            xv[k] = x_bf16 ? q27o_bf2f(((const uint16_t*)x)[(size_t)r * xstride + k])
                           : ((const float*)x)[(size_t)r * xstride + k];
        const float ss = q27o_rowsumsq(xv, n);
        const float inv = 1.0f / sqrtf(ss * rn + eps);
        for (int k = 0; k < n; ++k) {
            const float nm = xv[k] * inv * (plus + q27o_bf2f(w[k]));
            const uint16_t yb = q27o_f2bf(nm);
            if (hcopy) hcopy[(size_t)r * n + k] = q27o_f2bf(xv[k]);
            if (y) y[(size_t)r * ystride + k] = yb;
            nv[k] = quant_bf16 ? q27o_bf2f(yb) : nm;
        }
        if (xq) {
            for (int k0 = 0; k0 < n; k0 += 16) {
                float mx = 0.0f;
                for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(nv[k0 + j]));
                const float s = mx * g * (1.0f / 127.0f);
                const float inv2 = (s > 0.0f) ? (g / s) : 0.0f;
                xs[(size_t)r * (n / 16) + (k0 >> 4)] = s;
                for (int j = 0; j < 16; ++j) xq[(size_t)r * n + k0 + j] = q_code(nv[k0 + j], inv2);
            }
        }
    }
    free(xv);
    free(nv);
}

/* The same norm with the normed values as fp32 (bf16-rounded when round_bf16), for the prefill's
 * per-(token, group) quantizer (q27_red_rn_tok_b1 / q27_rmsnorm_hostss_tok_b,
 * src/q27_main.cpp:4123-4124): identical arithmetic to q27o_rmsnorm_quant_rows up to the value
 * it quantizes. hcopy = bf16(x), y = bf16(normed); any output may be NULL. */
void q27o_rmsnorm_f32_rows(const void* x, int x_bf16, int xstride, const uint16_t* w, float plus,
                           float eps, int n, uint16_t* hcopy, uint16_t* y, int ystride, float* yf,
                           int yfstride, int round_bf16, int nr) {
    float* xv = (float*)malloc((size_t)n * sizeof(float));
    const float rn = 1.0f / (float)n;
    for (int r = 0; r < nr; ++r) {
        for (int k = 0; k < n; ++k)
            xv[k] = x_bf16 ? q27o_bf2f(((const uint16_t*)x)[(size_t)r * xstride + k])
                           : ((const float*)x)[(size_t)r * xstride + k];
        const float ss = q27o_rowsumsq(xv, n);
        const float inv = 1.0f / sqrtf(ss * rn + eps);
        for (int k = 0; k < n; ++k) {
            const float nm = xv[k] * inv * (plus + q27o_bf2f(w[k]));
            const uint16_t yb = q27o_f2bf(nm);
            if (hcopy) hcopy[(size_t)r * n + k] = q27o_f2bf(xv[k]);
            if (y) y[(size_t)r * ystride + k] = yb;
            if (yf) yf[(size_t)r * yfstride + k] = round_bf16 ? q27o_bf2f(yb) : nm;
        }
    }
    free(xv);
}

/* Per-(token, group) quantizer with g = 1/in_scale (the prefill's norm / mixer quantizers):
 * sc = mx g / 127, inv = sc > 0 ? g / sc : 0. g = 1 gives q27o_quant_tok_groups' bits. */
void q27o_quant_tok_groups_g(const float* x, int xstride, int M, int K, int gs, float g, int8_t* xq, float* xs) {
    for (int t = 0; t < M; ++t)
        for (int g0 = 0; g0 < K; g0 += gs) {
            const float* v = x + (size_t)t * xstride + g0;
            float mx = 0.0f;
            for (int j = 0; j < gs; ++j) mx = fmaxf(mx, fabsf(v[j]));
            const float sc = mx * g * (1.0f / 127.0f);
            const float inv = (sc > 0.0f) ? (g / sc) : 0.0f;
            xs[(size_t)t * (K / gs) + g0 / gs] = sc;
            for (int j = 0; j < gs; ++j) xq[(size_t)t * K + g0 + j] = q_code(v[j], inv);
        }
}

/* ------------------------------------------------------------------ checkpoint formats */
/* E4M3 byte (include/q27.h:95-114): sign bit 7, exponent bits 6-3 (bias 7), mantissa bits 2-0;
 * exponent 0 is subnormal (m 2^-9); exponent 15 with mantissa 7 decodes as infinity (the
 * reference's choice for the code the OCP format calls NaN). */
float q27o_e4m3(uint8_t b) {
    const unsigned e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 0) v = (float)m * 0x1p-9f;
    else if (e == 15 && m == 7) v = INFINITY;
    else { const uint32_t u = ((e + 120u) << 23) | (m << 20); memcpy(&v, &u, 4); }
    return (b & 0x80u) ? -v : v;
}
/* E2M1 nibble (sign bit 3, exponent bits 2-1 with bias 1, mantissa bit 0) */
static float e2m1(unsigned nib) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    return mag[nib & 7u] * ((nib & 8u) ? -1.0f : 1.0f);
}
static void i8g64_of(const float* v, int n64, int8_t* w8, float* s64) {
    for (int g = 0; g < n64; ++g) {
        float mx = 0.0f;
        for (int j = 0; j < 64; ++j) mx = fmaxf(mx, fabsf(v[g * 64 + j]));
        const float sc = mx * (1.0f / 127.0f);
        const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
        s64[g] = sc;
        for (int j = 0; j < 64; ++j) w8[g * 64 + j] = q_code(v[g * 64 + j], inv);
    }
}
/* fp8 E4M3 [rows][ld] -> int8 per 64 (q27_k_fp8_to_i8g64, src/q27_nvfp4.hip:4259-4289) */
void q27o_fp8_to_i8g64(const uint8_t* f8, int rows, int K, int ld, int8_t* w8, float* s64) {
    float* v = (float*)malloc((size_t)K * 4);
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < K; ++k) v[k] = q27o_e4m3(f8[(size_t)r * ld + k]);
        i8g64_of(v, K / 64, w8 + (size_t)r * K, s64 + (size_t)r * (K / 64));
    }
    free(v);
}
/* NVFP4 [rows][K/2] (element 2j in the low nibble) with E4M3 per-16 scales [rows][K/16]
 * -> int8 per 64 (q27_k_nvfp4_to_i8g64, src/q27_nvfp4.hip:4166-4208): v = e2m1 x e4m3(scale) */
void q27o_nvfp4_to_i8g64(const uint8_t* w, const uint8_t* gs, int rows, int K, int8_t* w8, float* s64) {
    float* v = (float*)malloc((size_t)K * 4);
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < K; ++k) {
            const unsigned b = w[(size_t)r * (K / 2) + k / 2];
            v[k] = e2m1((k & 1) ? (b >> 4) : (b & 15u)) * q27o_e4m3(gs[(size_t)r * (K / 16) + k / 16] & 0x7Fu);
        }
        i8g64_of(v, K / 64, w8 + (size_t)r * K, s64 + (size_t)r * (K / 64));
    }
    free(v);
}
/* NVFP4 -> bf16 values bf16((e2m1 x e4m3(scale)) x weight_scale_2) (the engine's bf16 lm_head) */
void q27o_nvfp4_to_bf16(const uint8_t* w, const uint8_t* gs, float ws2, int rows, int K, uint16_t* out) {
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < K; ++k) {
            const unsigned b = w[(size_t)r * (K / 2) + k / 2];
            const float v = e2m1((k & 1) ? (b >> 4) : (b & 15u)) * q27o_e4m3(gs[(size_t)r * (K / 16) + k / 16] & 0x7Fu);
            out[(size_t)r * K + k] = q27o_f2bf(v * ws2);
        }
}
/* bf16 [rows][ld] columns 0..K-1 -> int8 per 64 (the MTP head, quantized from its values) */
void q27o_bf16_to_i8g64(const uint16_t* x, int rows, int K, int ld, int8_t* w8, float* s64) {
    float* v = (float*)malloc((size_t)K * 4);
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < K; ++k) v[k] = q27o_bf2f(x[(size_t)r * ld + k]);
        i8g64_of(v, K / 64, w8 + (size_t)r * K, s64 + (size_t)r * (K / 64));
    }
    free(v);
}

/* ------------------------------------------------------------------ R10-R12 GDN */
/* pend layout (per layer): khat [R][KH][D] f32 | delta [R][VH][D] f32 | decay [R][VH] f32 |
 * raw [R][NQKV] bf16, R = max rows. */
typedef struct { float* khat; float* delta; float* decay; uint16_t* raw; } pend_view;
static pend_view pend_map(void* pend, int kh, int vh, int d, int R) {
    pend_view p;
    char* b = (char*)pend;
    p.khat = (float*)b;  b += (size_t)R * kh * d * 4;
    p.delta = (float*)b; b += (size_t)R * vh * d * 4;
    p.decay = (float*)b; b += (size_t)R * vh * 4;
    p.raw = (uint16_t*)b;
    return p;
}
size_t q27o_gdn_pend_bytes(int kh, int vh, int d, int max_rows) {
    const size_t nqkv = (size_t)(2 * kh + vh) * d;
    return (size_t)max_rows * ((size_t)kh * d * 4 + (size_t)vh * d * 4 + (size_t)vh * 4 + nqkv * 2);
}
#define Q27O_GDN_R 8

/* k_gdn_conv_tp_tile (src/q27_gdn.hip:411-439): shift register of RAW bf16 inputs, tap order
 * 0..3 with the first tap a plain product, SiLU, bf16. gdn_step_body (src/q27_gdn.hip:206-372):
 * the recurrence below. Deferred commit replaces the snapshot banks of
 * src/q27_main.cpp:2933-2941. */
void q27o_gdn_verify(const uint16_t* qkv_raw, int qkv_stride, const uint16_t* z, int z_stride,
                     const float* a, const float* b, int ab_stride, const uint16_t* A_log,
                     const uint16_t* dt_bias, const uint16_t* norm_w, const uint16_t* conv_w,
                     float* S, uint16_t* conv_hist, void* pend, int npend, int kh, int vh,
                     int d, float eps, uint16_t* out, int out_stride, int8_t* xq, float* xs,
                     int nr) {
    const int nqkv = (2 * kh + vh) * d;
    const int ratio = vh / kh;
    const size_t hs = (size_t)d * d;
    pend_view P = pend_map(pend, kh, vh, d, Q27O_GDN_R);
    /* 1. commit the pending rows of the previous call */
    for (int c = 0; c < nqkv; ++c) {
        uint16_t h[3] = { conv_hist[3 * c], conv_hist[3 * c + 1], conv_hist[3 * c + 2] };
        for (int p = 0; p < npend; ++p) { h[0] = h[1]; h[1] = h[2]; h[2] = P.raw[(size_t)p * nqkv + c]; }
        conv_hist[3 * c] = h[0]; conv_hist[3 * c + 1] = h[1]; conv_hist[3 * c + 2] = h[2];
    }
#pragma omp parallel for schedule(static)
    for (int hh = 0; hh < vh; ++hh) {
        const int kk = hh / ratio;
        float* Sh = S + (size_t)hh * hs;
        for (int p = 0; p < npend; ++p) {
            const float* kp = P.khat + ((size_t)p * kh + kk) * d;
            const float* dp = P.delta + ((size_t)p * vh + hh) * d;
            const float dc = P.decay[(size_t)p * vh + hh];
            for (int j = 0; j < d; ++j)
                for (int e = 0; e < d; ++e) Sh[(size_t)j * d + e] = fmaf(kp[j], dp[e], dc * Sh[(size_t)j * d + e]);
        }
    }
    /* 2. the new rows, on working copies of the committed state */
    float* Sw = (float*)malloc((size_t)vh * hs * sizeof(float));
    memcpy(Sw, S, (size_t)vh * hs * sizeof(float));
    uint16_t* hw = (uint16_t*)malloc((size_t)nqkv * 3 * sizeof(uint16_t));
    memcpy(hw, conv_hist, (size_t)nqkv * 3 * sizeof(uint16_t));
    float* cv = (float*)malloc((size_t)nqkv * sizeof(float));
    for (int n = 0; n < nr; ++n) {
        const uint16_t* xr = qkv_raw + (size_t)n * qkv_stride;
        for (int c = 0; c < nqkv; ++c) {
            const uint16_t x = xr[c];
            const uint16_t* wc = conv_w + (size_t)4 * c;
            float acc = q27o_bf2f(hw[3 * c]) * q27o_bf2f(wc[0]);
            acc = fmaf(q27o_bf2f(hw[3 * c + 1]), q27o_bf2f(wc[1]), acc);
            acc = fmaf(q27o_bf2f(hw[3 * c + 2]), q27o_bf2f(wc[2]), acc);
            acc = fmaf(q27o_bf2f(x), q27o_bf2f(wc[3]), acc);
            hw[3 * c] = hw[3 * c + 1]; hw[3 * c + 1] = hw[3 * c + 2]; hw[3 * c + 2] = x;
            cv[c] = q27o_bf2f(q27o_f2bf(q27o_silu(acc)));
            P.raw[(size_t)n * nqkv + c] = x;
        }
        /* value heads are independent within a row (each writes only its own state, pending
         * slots and outputs; the key-head k^ slot by its first value head only): threads over them */
#pragma omp parallel for schedule(static)
        for (int hh = 0; hh < vh; ++hh) {
            float qn[128], kn[128], qh_[128], kh_[128], mixed[128], A[128], B[128];
            const int kk = hh / ratio;
            const float* qv = cv + (size_t)kk * d;
            const float* kv = cv + (size_t)kh * d + (size_t)kk * d;
            const float* vv = cv + (size_t)2 * kh * d + (size_t)hh * d;
            for (int j = 0; j < d; ++j) { qn[j] = qv[j]; kn[j] = kv[j]; }
            const float sumq2 = q27o_headsum(qn, qn, d);
            const float sumk2 = q27o_headsum(kn, kn, d);
            const float sumqk = q27o_headsum(qn, kn, d);
            const float invq = (1.0f / sqrtf(sumq2 + 1e-6f)) * 0.0883883476f;
            const float invk = 1.0f / sqrtf(sumk2 + 1e-6f);
            const float kq = sumqk * invq * invk;
            for (int j = 0; j < d; ++j) { qh_[j] = qn[j] * invq; kh_[j] = kn[j] * invk; }
            const float beta = q27o_sigmoid(b[(size_t)n * ab_stride + hh]);
            const float t = a[(size_t)n * ab_stride + hh] + q27o_bf2f(dt_bias[hh]);
            const float sp = q27o_softplus(t);
            const float Aexp = q27o_exp(q27o_bf2f(A_log[hh]));
            const float decay = q27o_exp(-(Aexp * sp));
            float* Sh = Sw + (size_t)hh * hs;
            for (int e = 0; e < d; ++e) {
                float pa[4], pb[4];
                for (int g = 0; g < 4; ++g) {
                    float aa = 0.0f, bb = 0.0f;
                    for (int j = g * (d / 4); j < (g + 1) * (d / 4); ++j) {
                        const float sv = Sh[(size_t)j * d + e];
                        aa = fmaf(sv, kh_[j], aa);
                        bb = fmaf(sv, qh_[j], bb);
                    }
                    pa[g] = aa; pb[g] = bb;
                }
                A[e] = ((pa[0] + pa[1]) + pa[2]) + pa[3];
                B[e] = ((pb[0] + pb[1]) + pb[2]) + pb[3];
            }
            float* dl = P.delta + ((size_t)n * vh + hh) * d;
            for (int e = 0; e < d; ++e) {
                const float delta = (vv[e] - decay * A[e]) * beta;
                mixed[e] = fmaf(delta, kq, decay * B[e]);
                dl[e] = delta;
            }
            for (int j = 0; j < d; ++j)
                for (int e = 0; e < d; ++e) Sh[(size_t)j * d + e] = fmaf(kh_[j], dl[e], decay * Sh[(size_t)j * d + e]);
            P.decay[(size_t)n * vh + hh] = decay;
            if (hh % ratio == 0)
                for (int j = 0; j < d; ++j) P.khat[((size_t)n * kh + kk) * d + j] = kh_[j];
            const float summ = q27o_headsum(mixed, mixed, d);
            const float inv = 1.0f / sqrtf(summ * (1.0f / (float)d) + eps);
            float yv[128];
            for (int e = 0; e < d; ++e) {
                const float zz = q27o_bf2f(z[(size_t)n * z_stride + (size_t)hh * d + e]);
                const float yy = mixed[e] * inv * q27o_bf2f(norm_w[e]) * q27o_silu(zz);
                const uint16_t yb = q27o_f2bf(yy);
                out[(size_t)n * out_stride + (size_t)hh * d + e] = yb;
                yv[e] = q27o_bf2f(yb);
            }
            if (xq) {
                for (int g0 = 0; g0 < d; g0 += 16) {
                    float mx = 0.0f;
                    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(yv[g0 + j]));
                    const float sc = mx * (1.0f / 127.0f);
                    const float qi = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
                    const size_t kq0 = (size_t)n * vh * d + (size_t)hh * d + g0;
                    xs[kq0 >> 4] = sc;
                    for (int j = 0; j < 16; ++j) xq[kq0 + j] = q_code(yv[g0 + j], qi);
                }
            }
        }
    }
    free(Sw); free(hw); free(cv);
}

/* ------------------------------------------------------------------ R14/R15 attention */
/* src/q27_attn.hip:239-247: inv_freq = 2^(-(2f/rot) log2 theta), angle = pos*inv_freq, both in
 * double, then rounded to float. */
void q27o_rope_table(int ctx, int rot, double theta, float* cosv, float* sinv) {
    const int half = rot / 2;
    const double l2t = log2(theta);
    for (int p = 0; p < ctx; ++p)
        for (int f = 0; f < half; ++f) {
            const double ifq = exp2(-((double)(2 * f) / (double)rot) * l2t);
            const double ang = (double)p * ifq;
            cosv[(size_t)p * half + f] = (float)cos(ang);
            sinv[(size_t)p * half + f] = (float)sin(ang);
        }
}

/* src/q27_attn.hip:177-253 (q27_attn_prep_k): head RMSNorm (1+w), rotate-half RoPE on the
 * first `rot` dims, q -> bf16, K/V -> int8 with per-kv_group scales. */
void q27o_attn_prep_rows(const uint16_t* qkv, int qkv_stride, const uint16_t* q_norm_w,
                         const uint16_t* k_norm_w, const float* rope_cos,
                         const float* rope_sin, int rot, int8_t* kc, float* ks, int8_t* vc,
                         float* vs, int kv_group, uint16_t* qh, int nq, int nkv, int hd,
                         int gate, float eps, int pos0, int nr) {
    const int qw = gate ? 2 * hd : hd;
    const int qrows = nq * qw, kvrows = nkv * hd;
    const int half = rot / 2;
    float x[256], y[256], yr[256];
    for (int r = 0; r < nr; ++r) {
        const int pos = pos0 + r;
        const uint16_t* row = qkv + (size_t)r * qkv_stride;
        for (int u = 0; u < nq + nkv; ++u) {
            const int isq = u < nq;
            const int head = isq ? u : u - nq;
            const uint16_t* src = isq ? row + (size_t)head * qw : row + qrows + (size_t)head * hd;
            const uint16_t* wgt = isq ? q_norm_w : k_norm_w;
            for (int i = 0; i < hd; ++i) x[i] = q27o_bf2f(src[i]);
            const float ss = q27o_headsum(x, x, hd);
            const float inv = 1.0f / sqrtf(ss * (1.0f / (float)hd) + eps);
            for (int i = 0; i < hd; ++i) y[i] = x[i] * inv * (1.0f + q27o_bf2f(wgt[i]));
            for (int i = 0; i < hd; ++i) {
                if (i < rot) {
                    const int f = i % half;
                    const float rv = (i < half) ? -y[i + half] : y[i - half];
                    const float cs = rope_cos[(size_t)pos * half + f], sn = rope_sin[(size_t)pos * half + f];
                    yr[i] = y[i] * cs + rv * sn;
                } else yr[i] = y[i];
            }
            if (isq) {
                for (int i = 0; i < hd; ++i) qh[(size_t)r * nq * hd + (size_t)head * hd + i] = q27o_f2bf(yr[i]);
            } else {
                const size_t off = (size_t)pos * kvrows + (size_t)head * hd;
                q27o_quant_f32(yr, hd, kv_group, kc + off, ks + off / kv_group);
                float vv[256];
                const uint16_t* vsrc = row + qrows + kvrows + (size_t)head * hd;
                for (int i = 0; i < hd; ++i) vv[i] = q27o_bf2f(vsrc[i]);
                q27o_quant_f32(vv, hd, kv_group, vc + off, vs + off / kv_group);
            }
        }
    }
}

/* score: four fmaf chains over the head dims in order, chain c over dims [c hd/4, (c+1) hd/4),
 * summed ((c0 + c1) + c2) + c3 (the GPU's matrix-core tiles run the four chains side by side) */
static float score_4chain(const float* q, const float* k, int hd) {
    float c[4];
    const int w = hd / 4;
    for (int j = 0; j < 4; ++j) {
        float a = 0.0f;
        for (int i = j * w; i < (j + 1) * w; ++i) a = fmaf(q[i], k[i], a);
        c[j] = a;
    }
    return ((c[0] + c[1]) + c[2]) + c[3];
}

#define Q27O_SPLIT 64
/* src/q27_attn.hip:258-463 semantics (GQA, causal over pos0+r, log2-domain softmax, split
 * combine, sigmoid output gate); this build's order: fixed 64-key splits, scores as four fmaf
 * chains over the head dims (score_4chain), per split m = max, p = 2^(x - m), l = shfl_down tree
 * over the split's 64 lanes, o = four fmaf chains over the split's 16-key blocks in ascending key
 * order, summed ((o0 + o1) + o2) + o3; splits combined in ascending order. */
void q27o_attn_rows(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride,
                    const int8_t* kc, const float* ks, const int8_t* vc, const float* vs,
                    int kv_group, int nq, int nkv, int hd, int gate, int pos0, int nr,
                    uint16_t* out, int8_t* xq, float* xs) {
    const int G = nq / nkv;
    const int kvrows = nkv * hd;
    const int qw = gate ? 2 * hd : hd;
    const float sl2e = (float)((1.0 / sqrt((double)hd)) * 1.4426950408889634);
    float* yv = (float*)malloc((size_t)nr * nq * hd * sizeof(float));
    /* every (row, query head) is independent and keeps its own fixed order: threads over them */
#pragma omp parallel for schedule(dynamic, 1)
    for (int rh = 0; rh < nr * nq; ++rh) {
        const int r = rh / nq, hq = rh % nq;
        const int L = pos0 + r + 1;
        const int ns = (L + Q27O_SPLIT - 1) / Q27O_SPLIT;
        const int kvh = hq / G;
        float q[256], kd[256], o[256], os[256];
        for (int i = 0; i < hd; ++i) q[i] = q27o_bf2f(qh[(size_t)r * nq * hd + (size_t)hq * hd + i]);
        float M = -INFINITY, den = 0.0f;
        float* ms = (float*)malloc((size_t)ns * sizeof(float));
        float* ls = (float*)malloc((size_t)ns * sizeof(float));
        float* ob = (float*)malloc((size_t)ns * hd * sizeof(float));
        for (int s = 0; s < ns; ++s) {
            const int k0 = s * Q27O_SPLIT;
            const int k1 = (k0 + Q27O_SPLIT < L) ? k0 + Q27O_SPLIT : L;
            float xsc[Q27O_SPLIT];
            float m = -INFINITY;
            for (int k = k0; k < k1; ++k) {
                const size_t off = (size_t)k * kvrows + (size_t)kvh * hd;
                for (int i = 0; i < hd; ++i) kd[i] = (float)kc[off + i] * ks[(off + i) / kv_group];
                const float x = score_4chain(q, kd, hd) * sl2e;
                xsc[k - k0] = x;
                m = fmaxf(m, x);
            }
            /* l: the 64 keys' p (0 past the valid ones) summed by the shfl_down tree */
            float pl[Q27O_SPLIT];
            for (int i = 0; i < Q27O_SPLIT; ++i) pl[i] = 0.0f;
            float oc[4][256];
            for (int j = 0; j < 4; ++j)
                for (int i = 0; i < hd; ++i) oc[j][i] = 0.0f;
            for (int k = k0; k < k1; ++k) {
                const float p = q27o_exp2(xsc[k - k0] - m);
                pl[k - k0] = p;
                const size_t off = (size_t)k * kvrows + (size_t)kvh * hd;
                float* oj = oc[(k - k0) / (Q27O_SPLIT / 4)];
                for (int i = 0; i < hd; ++i) oj[i] = fmaf(p, (float)vc[off + i] * vs[(off + i) / kv_group], oj[i]);
            }
            for (int i = 0; i < hd; ++i) os[i] = ((oc[0][i] + oc[1][i]) + oc[2][i]) + oc[3][i];
            const float l = tree64(pl);
            ms[s] = m; ls[s] = l;
            memcpy(ob + (size_t)s * hd, os, (size_t)hd * sizeof(float));
            M = fmaxf(M, m);
        }
        for (int i = 0; i < hd; ++i) o[i] = 0.0f;
        for (int s = 0; s < ns; ++s) {
            const float w = q27o_exp2(ms[s] - M);
            den = fmaf(ls[s], w, den);
            for (int i = 0; i < hd; ++i) o[i] = fmaf(ob[(size_t)s * hd + i], w, o[i]);
        }
        const float inv = 1.0f / den;
        for (int i = 0; i < hd; ++i) {
            float v = o[i] * inv;
            if (gate) {
                const float gt = q27o_bf2f(qkv_gate[(size_t)r * qkv_stride + (size_t)hq * qw + hd + i]);
                v = v * q27o_sigmoid(gt);
            }
            const uint16_t bv = q27o_f2bf(v);
            out[(size_t)r * nq * hd + (size_t)hq * hd + i] = bv;
            yv[(size_t)r * nq * hd + (size_t)hq * hd + i] = q27o_bf2f(bv);
        }
        free(ms); free(ls); free(ob);
    }
    if (xq)
        for (int r = 0; r < nr; ++r)
            q27o_quant_f32(yv + (size_t)r * nq * hd, nq * hd, 16, xq + (size_t)r * nq * hd, xs + (size_t)r * (nq * hd / 16));
    free(yv);
}

/* ------------------------------------------------------------------ R18 / R20 */
/* src/q27_elem.hip:216-322: finite filter, (value desc, index asc) total order. */
void q27o_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val) {
    for (int r = 0; r < nr; ++r) {
        const float* p = logits + (size_t)r * ld;
        float bv = -INFINITY;
        int bi = -1;
        for (int i = 0; i < n; ++i) {
            const float v = p[i];
            if (!isfinite(v)) continue;
            if (bi < 0 || v > bv) { bv = v; bi = i; }
        }
        idx[r] = bi < 0 ? 0 : bi;
        val[r] = bi < 0 ? -INFINITY : bv;
    }
}

/* src/q27_main.cpp:2811-2812, 2929-2932 */
int q27o_accept(const int32_t* nx, const int32_t* dt, int k, int32_t* committed) {
    int nacc = 0;
    while (nacc < k && nx[nacc] == dt[nacc]) ++nacc;
    for (int j = 0; j <= nacc; ++j) committed[j] = nx[j];
    return nacc;
}
