// q27x_norm.h -- the RMSNorm + per-16 quantize of activation rows, as one 256-thread block.
//
// Canonical order (q27_rmsnorm_quant_fp8 / q27_rmsnorm_hostss_fp8_b, src/q27_fp8.hip): thread t
// owns elements 1024 i + 4 t + e; its squares are accumulated with fmaf in (i, e) order, the four
// waves reduce with the shfl_down tree and meet as ((w0 + w1) + w2) + w3; inv = 1/sqrt(ss/n + eps);
// nrm = x * inv * (plus + w); a group of 16 is 4 adjacent threads (exact max, s = mx/127 * 1/in_scale).
// Used by the standalone norm kernel (one block per row) and by the last block of a residual
// projection (all rows of the step), so both write the same bits.
#pragma once
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

// Rows [r0, r0 + nrows) of `a` (source row index rs = row_sel ? *row_sel : r), RB rows per pass.
// NCH = n / 1024. wsum: __shared__ float[RB][4]. Every thread of the 256-thread block calls it.
template <int NCH, int RB>
__device__ __forceinline__ void norm_rows(const NormArgs& a, int r0, int nrows, float (*wsum)[4]) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    constexpr int n = NCH * 1024;
    float wf[NCH][4];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const uint2 wu = *(const uint2*)(a.w + i * 1024 + 4 * t);
        wf[i][0] = __uint_as_float(wu.x << 16); wf[i][1] = __uint_as_float(wu.x & 0xFFFF0000u);
        wf[i][2] = __uint_as_float(wu.y << 16); wf[i][3] = __uint_as_float(wu.y & 0xFFFF0000u);
    }
    const float g = 1.0f / a.in_scale;
    for (int rb = 0; rb < nrows; rb += RB) {
        float xv[RB][NCH][4];
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + rb + j;
            if (rb + j >= nrows) break;
            const int rs = a.row_sel ? *a.row_sel : r;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int k = i * 1024 + 4 * t;
                float* v = xv[j][i];
                if (a.emb) {
                    const uint2 u = *(const uint2*)(a.emb + (size_t)a.tok[rs] * n + k);
                    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
                    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
                } else if (a.x_bf16) {
                    const uint2 u = *(const uint2*)((const uint16_t*)a.x + (size_t)rs * a.xstride + k);
                    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
                    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
                } else {
                    const float4 f = *(const float4*)((const float*)a.x + (size_t)rs * a.xstride + k);
                    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + rb + j;
            if (rb + j >= nrows) break;
            const int rs = a.row_sel ? *a.row_sel : r;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int k = i * 1024 + 4 * t;
                float* v = xv[j][i];
                if (a.hout) {   // head: the final residual row, bf16(bf16(r1) + r2) or bf16(r2)
                    uint16_t hb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float s = a.hadd ? bf2f(a.hadd[(size_t)rs * n + k + e]) + v[e] : v[e];
                        hb[e] = f2bf(s);
                        v[e] = bf2f(hb[e]);
                    }
                    *(uint2*)(a.hout + (size_t)r * n + k) = make_uint2((uint32_t)hb[0] | ((uint32_t)hb[1] << 16),
                                                                      (uint32_t)hb[2] | ((uint32_t)hb[3] << 16));
                }
                if (a.hcopy)
                    *(uint2*)(a.hcopy + (size_t)r * n + k) =
                        make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                                   (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(v[e], v[e], acc);
            }
            acc = tree64(acc);
            if (lane == 0) wsum[j][wv] = acc;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + rb + j;
            if (rb + j >= nrows) break;
            const float ss = ((wsum[j][0] + wsum[j][1]) + wsum[j][2]) + wsum[j][3];
            const float inv = rsqrt_cr(ss * (1.0f / (float)n) + a.eps);
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int k = i * 1024 + 4 * t;
                float nm[4];
                uint16_t yb[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    nm[e] = xv[j][i][e] * inv * (a.plus + wf[i][e]);
                    yb[e] = f2bf(nm[e]);
                }
                if (a.y)
                    *(uint2*)(a.y + (size_t)r * a.ystride + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                           (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
                if (a.yf)
                    *(float4*)(a.yf + (size_t)r * a.yfstride + k) =
                        a.quant_bf16 ? make_float4(bf2f(yb[0]), bf2f(yb[1]), bf2f(yb[2]), bf2f(yb[3]))
                                     : make_float4(nm[0], nm[1], nm[2], nm[3]);
                if (a.xq) {
                    float q[4], mx = 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) { q[e] = a.quant_bf16 ? bf2f(yb[e]) : nm[e]; mx = fmaxf(mx, fabsf(q[e])); }
                    mx = max_xor(mx, 4);
                    const float s = mx * g * (1.0f / 127.0f);
                    const float qi = (s > 0.0f) ? (g / s) : 0.0f;
                    uint32_t pk = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) pk |= ((uint32_t)(uint8_t)qcode(q[e], qi)) << (8 * e);
                    *(uint32_t*)(a.xq + (size_t)r * n + k) = pk;
                    if ((t & 3) == 0) a.xs[(size_t)r * (n >> 4) + (k >> 4)] = s;
                }
            }
        }
        __syncthreads();   // wsum reused by the next pass
    }
}

}  // namespace q27x

namespace q27x {

// Prologue form of the same RMSNorm + quantize for a 1024-thread block: every block of a consumer
// projection normalizes the NR input rows itself (n = NCH * 1024 = the projection's K) and writes
// the codes and scales straight into its LDS activation stage, in the slab layout of k_proj:
// element k = 1024 i + 4 t + e lands in slab 64 i + t/4 at byte 4 (t % 4). The four 256-thread
// groups take rows tg, tg + 4, ... (tg = thread / 256), each in the canonical order above, so all
// blocks hold the bits a standalone norm writes. Block 0 also stores the side outputs (hcopy, y,
// xq/xs) for later kernels. Loads are split from the arithmetic so the caller can issue its
// weight prefetch in between (vector-memory counters retire in order: the input rows must be
// requested before the weights to be waited on alone).
template <int NCH, int NR>
struct PreNorm {
    static constexpr int GR = 4;                          // 256-thread groups
    static constexpr int RPG = (NR + GR - 1) / GR;        // rows per group
    uint2 wb[NCH];                                        // 4 bf16 norm weights per chunk
    float xv[RPG][NCH][4];

    __device__ __forceinline__ void load(const NormArgs& a) {
        const int t = threadIdx.x & 255, tg = threadIdx.x >> 8;
        constexpr int n = NCH * 1024;
#pragma unroll
        for (int i = 0; i < NCH; ++i) wb[i] = *(const uint2*)(a.w + i * 1024 + 4 * t);
#pragma unroll
        for (int j = 0; j < RPG; ++j) {
            const int r = tg + GR * j;
            if (r >= NR) break;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int k = i * 1024 + 4 * t;
                float* v = xv[j][i];
                if (a.emb || a.x_bf16) {
                    const uint16_t* src = a.emb ? a.emb + (size_t)a.tok[r] * n : (const uint16_t*)a.x + (size_t)r * a.xstride;
                    const uint2 u = *(const uint2*)(src + k);
                    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
                    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
                } else {
                    const float4 f = *(const float4*)((const float*)a.x + (size_t)r * a.xstride + k);
                    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
                }
            }
        }
    }
    // sxw: the LDS code stage as 32-bit words ([NR][SL] slabs of 4 words); ssc: [NR][SL] scales;
    // wsum: __shared__ float[RPG][GR][4]. Block 0 (writer) also stores the side outputs; the other
    // blocks run a copy without them, and the bf16 rounding of the normalized values is compiled
    // in only where it is used (side output y, quant_bf16, or ylds), about halving their
    // instructions. ylds (optional): LDS rows [NR][n] that receive the bf16 normalized values.
    __device__ __forceinline__ void finish(const NormArgs& a, uint32_t* sxw, float* ssc, int SL,
                                           float (*wsum)[GR][4], bool writer, uint16_t* ylds = nullptr) {
        if (writer || ylds) {
            if (a.quant_bf16) fin<true, true>(a, sxw, ssc, SL, wsum, writer, ylds);
            else fin<true, false>(a, sxw, ssc, SL, wsum, writer, ylds);
        } else {
            if (a.quant_bf16) fin<false, true>(a, sxw, ssc, SL, wsum, false, nullptr);
            else fin<false, false>(a, sxw, ssc, SL, wsum, false, nullptr);
        }
    }
    // YB: the bf16 values are formed (the writer's side outputs, or ylds)
    template <bool YB, bool QB>
    __device__ __forceinline__ void fin(const NormArgs& a, uint32_t* sxw, float* ssc, int SL,
                                        float (*wsum)[GR][4], bool writer, uint16_t* ylds) {
        constexpr bool WR = YB;
        const int t = threadIdx.x & 255, tg = threadIdx.x >> 8, lane = t & 63, wv = t >> 6;
        constexpr int n = NCH * 1024;
#pragma unroll
        for (int j = 0; j < RPG; ++j) {
            const int r = tg + GR * j;
            if (r >= NR) break;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const float* v = xv[j][i];
                if (WR && writer && a.hcopy)
                    *(uint2*)(a.hcopy + (size_t)r * n + i * 1024 + 4 * t) =
                        make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                                   (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(v[e], v[e], acc);
            }
            acc = tree64(acc);
            if (lane == 0) wsum[j][tg][wv] = acc;
        }
        __syncthreads();
        const float g = 1.0f / a.in_scale;
#pragma unroll
        for (int j = 0; j < RPG; ++j) {
            const int r = tg + GR * j;
            if (r >= NR) break;
            const float ss = ((wsum[j][tg][0] + wsum[j][tg][1]) + wsum[j][tg][2]) + wsum[j][tg][3];
            const float inv = rsqrt_cr(ss * (1.0f / (float)n) + a.eps);
            // (the two-rows form below, applied at one row per group, made in_qkv|in_z at 3 rows
            // 18.65 -> 19.0 us; at 8 rows it took gate|up 42.0 -> 41.6 us, in_qkv|in_z 25.4 ->
            // 25.1 us and the K=7 round 9.67 -> 9.59 ms)
            if constexpr (RPG == 1) {
                // one chunk at a time: values, group maximum, the quotient g / s, codes
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    const int k = i * 1024 + 4 * t;
                    const float wf[4] = {__uint_as_float(wb[i].x << 16), __uint_as_float(wb[i].x & 0xFFFF0000u),
                                         __uint_as_float(wb[i].y << 16), __uint_as_float(wb[i].y & 0xFFFF0000u)};
                    float q[4], mx = 0.0f;
                    uint16_t yb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float nm = xv[j][i][e] * inv * (a.plus + wf[e]);
                        if constexpr (WR || QB) yb[e] = f2bf(nm);
                        q[e] = QB ? bf2f(yb[e]) : nm;
                        mx = fmaxf(mx, fabsf(q[e]));
                    }
                    if (WR && writer && a.y)
                        *(uint2*)(a.y + (size_t)r * a.ystride + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                               (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
                    if (WR && ylds)
                        *(uint2*)(ylds + (size_t)r * n + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                        (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
                    mx = max_quad(mx);
                    const float s = mx * g * (1.0f / 127.0f);
                    const float qi = (s > 0.0f) ? (g / s) : 0.0f;
                    uint32_t pk = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) pk |= ((uint32_t)(uint8_t)qcode(q[e], qi)) << (8 * e);
                    const int slab = 64 * i + (t >> 2);
                    sxw[((size_t)r * SL + slab) * 4 + (t & 3)] = pk;
                    if ((t & 3) == 0) ssc[r * SL + slab] = s;
                    if (WR && writer && a.xq) {
                        *(uint32_t*)(a.xq + (size_t)r * n + k) = pk;
                        if ((t & 3) == 0) a.xs[(size_t)r * (n >> 4) + (k >> 4)] = s;
                    }
                }
            } else {
                // two rows per group: the row's normalized values and each group's scale first (a
                // group of 16 is a quad of lanes)
                float qv[NCH][4], sv[NCH];
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    const int k = i * 1024 + 4 * t;
                    const float wf[4] = {__uint_as_float(wb[i].x << 16), __uint_as_float(wb[i].x & 0xFFFF0000u),
                                         __uint_as_float(wb[i].y << 16), __uint_as_float(wb[i].y & 0xFFFF0000u)};
                    float mx = 0.0f;
                    uint16_t yb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float nm = xv[j][i][e] * inv * (a.plus + wf[e]);
                        if constexpr (WR || QB) yb[e] = f2bf(nm);
                        qv[i][e] = QB ? bf2f(yb[e]) : nm;
                        mx = fmaxf(mx, fabsf(qv[i][e]));
                    }
                    if (WR && writer && a.y)
                        *(uint2*)(a.y + (size_t)r * a.ystride + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                               (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
                    if (WR && ylds)
                        *(uint2*)(ylds + (size_t)r * n + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                        (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
                    sv[i] = max_quad(mx) * g * (1.0f / 127.0f);
                }
                // the groups' quotients g / s: lane m of a quad divides for the chunks m, m + 4, ...
                // (every lane of the quad holds the same s), then each chunk's quotient is broadcast
                // from its lane; the same correctly rounded division as in every lane, a quarter of
                // the instructions
                constexpr int ND = (NCH + 3) / 4;
                const int m = t & 3;
                float qd[ND];
#pragma unroll
                for (int d = 0; d < ND; ++d) {
                    float den = sv[4 * d];
#pragma unroll
                    for (int u = 1; u < 4; ++u)
                        if (4 * d + u < NCH) den = (m == u) ? sv[(4 * d + u < NCH) ? 4 * d + u : 0] : den;
                    qd[d] = (den > 0.0f) ? (g / den) : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    const int k = i * 1024 + 4 * t;
                    const float s = sv[i];
                    const float qi = quad_bcast(qd[i >> 2], i);
                    int c[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) c[e] = qcode(qv[i][e], qi);
                    // the four codes' low bytes, in order
                    const uint32_t pk = __builtin_amdgcn_perm((uint32_t)c[1], (uint32_t)c[0], 0x0c0c0400u) |
                                        __builtin_amdgcn_perm((uint32_t)c[3], (uint32_t)c[2], 0x04000c0cu);
                    const int slab = 64 * i + (t >> 2);
                    sxw[((size_t)r * SL + slab) * 4 + (t & 3)] = pk;
                    if ((t & 3) == 0) ssc[r * SL + slab] = s;
                    if (WR && writer && a.xq) {
                        *(uint32_t*)(a.xq + (size_t)r * n + k) = pk;
                        if ((t & 3) == 0) a.xs[(size_t)r * (n >> 4) + (k >> 4)] = s;
                    }
                }
            }
        }
    }
};

}  // namespace q27x
