// k_attn.hip -- full attention of NR verify rows over the int8 KV cache (R14, R15).
//
// prep (src/q27_attn.hip:177-253): one wave per (head, row): RMSNorm over the head (1+w), lane l
//   holds dims l and l+64; rotate-half RoPE on the first `rot` dims from the host's cos/sin
//   tables; q -> bf16; K (normed, roped) and V (raw) -> int8 with one fp32 scale per kv_group.
// attention (src/q27_attn.hip:258-463 semantics): GQA, row r attends keys 0..pos0+r. Keys are cut
//   into FIXED 64-key splits, so a row's result depends only on its own keys and never on how
//   many rows share the launch (the verify row and the plain step agree bit for bit). A block
//   owns (split, kv head) for all rows and all GQA heads: K/V tile dequantised into LDS once,
//   scores by 16-lane dot products, two-pass softmax in base 2, p.V in key order; the combine
//   merges splits in order, applies sigmoid(gate) and quantises for o_proj.
#include <mutex>

#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

constexpr int kHD = 128;
constexpr int kMaxQ = kMaxRows * 8;   // rows x GQA heads per kv head held by one block

// RMSNorm (1 + w) and rotate-half RoPE of one head row at position pos by one wave: lane l holds
// dims l and l + 64 of the head's 128 bf16 values at src.
__device__ __forceinline__ void norm_rope(const AttnArgs& a, const uint16_t* src, const uint16_t* wgt, int pos,
                                          int l, float& y0, float& y1) {
    const float x0 = bf2f(src[l]), x1 = bf2f(src[l + 64]);
    const float wg0 = bf2f(wgt[l]), wg1 = bf2f(wgt[l + 64]);
    // the RoPE table entries are read by every lane (in bounds for any lane) with the inputs
    const int half = a.rot >> 1;
    const int f = (a.rot <= 64) ? (l & (half - 1)) : l;
    const float c = a.rope_cos[(size_t)pos * half + f], s = a.rope_sin[(size_t)pos * half + f];
    const float w0 = tree64(x0 * x0), w1 = tree64(x1 * x1);
    const float ss = bcast0(w0) + bcast0(w1);
    const float inv = rsqrt_cr(ss * (1.0f / (float)kHD) + a.eps);
    y0 = x0 * inv * (1.0f + wg0);
    y1 = x1 * inv * (1.0f + wg1);
    if (a.rot <= 64) {
        const float pv = __shfl_xor(y0, half, 64);
        if (l < a.rot) {
            const float rv = (l < half) ? -pv : pv;
            y0 = y0 * c + rv * s;
        }
    } else {   // rot == 128: dims l and l+64 are partners
        const float n0 = y0 * c + (-y1) * s;
        const float n1 = y1 * c + y0 * s;
        y0 = n0; y1 = n1;
    }
}

// K (normed, roped: y0, y1) and V (raw: v0, v1) of one kv head row -> int8 codes with one fp32
// scale per kv_group at cache element offset off; deq gets code * scale, the values the attention
// reads back.
__device__ __forceinline__ void store_kv(const AttnArgs& a, float y0, float y1, float v0, float v1, size_t off,
                                         int l, float (&deq)[4]) {
    const int G = a.kv_group;
    const float vals[4] = { y0, y1, v0, v1 };
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float v = vals[q];
        const float mx = max_xor(fabsf(v), G);
        const float sc = mx * (1.0f / 127.0f);
        const float qi = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
        const int dd = l + ((q & 1) ? 64 : 0);
        int8_t* c8 = (q < 2) ? a.kc : a.vc;
        float* cs8 = (q < 2) ? a.ks : a.vs;
        const int8_t code = qcode(v, qi);
        c8[off + dd] = code;
        if ((dd % G) == 0) cs8[(off + dd) / G] = sc;
        deq[q] = (float)code * sc;
    }
}

// The same prep for a head of HD = 64 NC dims (128 or 256): lane l holds dims l + 64 i, i < NC.
// The head's sum of squares adds the 64-dim chunks' trees in order (((w0 + w1) + w2) + w3); RoPE on
// the first rot <= 64 dims (all in chunk 0, partner lane l ^ rot/2), or on all 128 dims of a
// 128-wide head (partners l and l + 64).
template <int HD>
__device__ __forceinline__ void norm_rope_n(const AttnArgs& a, const uint16_t* src, const uint16_t* wgt, int pos, int l,
                                            float (&y)[HD / 64]) {
    constexpr int NC = HD / 64;
    float x[NC], wg[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) { x[i] = bf2f(src[l + 64 * i]); wg[i] = bf2f(wgt[l + 64 * i]); }
    const int half = a.rot >> 1;
    const int f = (a.rot <= 64) ? (l & (half - 1)) : l;
    const float c = a.rope_cos[(size_t)pos * half + f], s = a.rope_sin[(size_t)pos * half + f];
    float ss = bcast0(tree64(x[0] * x[0]));
#pragma unroll
    for (int i = 1; i < NC; ++i) ss = ss + bcast0(tree64(x[i] * x[i]));
    const float inv = rsqrt_cr(ss * (1.0f / (float)HD) + a.eps);
#pragma unroll
    for (int i = 0; i < NC; ++i) y[i] = x[i] * inv * (1.0f + wg[i]);
    if (a.rot <= 64) {
        const float pv = __shfl_xor(y[0], half, 64);
        if (l < a.rot) {
            const float rv = (l < half) ? -pv : pv;
            y[0] = y[0] * c + rv * s;
        }
    } else if constexpr (HD == 128) {   // rot == 128
        const float n0 = y[0] * c + (-y[1]) * s;
        const float n1 = y[1] * c + y[0] * s;
        y[0] = n0; y[1] = n1;
    }
}
// K (normed, roped) and V (raw) of one kv head row of HD dims -> int8 with one fp32 scale per
// kv_group (<= 64: a group lies inside one 64-dim chunk) at cache element offset off.
template <int HD>
__device__ __forceinline__ void store_kv_n(const AttnArgs& a, const float (&yk)[HD / 64], const float (&yv)[HD / 64],
                                           size_t off, int l) {
    const int G = a.kv_group;
#pragma unroll
    for (int q = 0; q < 2 * (HD / 64); ++q) {
        const int i = q % (HD / 64);
        const float v = (q < HD / 64) ? yk[i] : yv[i];
        const float mx = max_xor(fabsf(v), G);
        const float sc = mx * (1.0f / 127.0f);
        const float qi = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
        const int dd = l + 64 * i;
        int8_t* c8 = (q < HD / 64) ? a.kc : a.vc;
        float* cs8 = (q < HD / 64) ? a.ks : a.vs;
        c8[off + dd] = qcode(v, qi);
        if ((dd % G) == 0) cs8[(off + dd) / G] = sc;
    }
}

template <int HD>
__global__ __launch_bounds__(64) void k_attn_prep(AttnArgs a) {
    constexpr int NC = HD / 64;
    if (stopped(a.stop)) return;
    const int r = blockIdx.y;
    if (a.nact_ptr && r >= ld_uniform(a.nact_ptr)) return;
    const int pos = (a.pos0_ptr ? ld_uniform(a.pos0_ptr) : a.pos0_imm) + r;
    const int l = threadIdx.x;
    const int u = blockIdx.x + (a.prep_kv_only ? a.nq : 0);
    const bool isq = u < a.nq;
    const int head = isq ? u : u - a.nq;
    const int qw = a.gate ? 2 * HD : HD;
    const int qrows = a.nq * qw, kvrows = a.nkv * HD;
    const uint16_t* row = a.qkv + (size_t)r * a.qkv_stride;
    const uint16_t* src = isq ? row + (size_t)head * qw : row + qrows + (size_t)head * HD;
    float y[NC];
    norm_rope_n<HD>(a, src, isq ? a.q_norm_w : a.k_norm_w, pos, l, y);
    if (isq) {
        uint16_t* dst = a.qh + (size_t)r * a.nq * HD + (size_t)head * HD;
#pragma unroll
        for (int i = 0; i < NC; ++i) dst[l + 64 * i] = f2bf(y[i]);
        return;
    }
    const uint16_t* vsrc = row + qrows + kvrows + (size_t)head * HD;
    float v[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) v[i] = bf2f(vsrc[l + 64 * i]);
    store_kv_n<HD>(a, y, v, (size_t)pos * kvrows + (size_t)head * HD, l);
}

size_t attn_work_floats(int nq, int hd, int max_splits, int nr) {
    return (size_t)nr * nq * max_splits * (size_t)(hd + 2);
}

// work layout: o [nr][nq][ms][hd] | m [nr][nq][ms] | l [nr][nq][ms]
// Block = (split of 64 keys, kv head), all rows and all GQA heads of the kv head (nqr query
// vectors), 8 waves. The block requests its int8 K and V tiles, their scales and the queries up
// front, dequantizes K and V once into LDS as fp32 (k8 * ks, v8 * vs: the host restatement's
// values), K rows padded to 132 floats so 16 lanes reading 16 different keys hit distinct banks.
//   scores: lane = key, wave w = queries w + 8 i (i < NQW); x = sl2e * (fmaf over the 128 dims in
//           order of q[d] * k[d]);
//   softmax of the split: m = wave max over the valid keys, p = 2^(x - m), l = shfl_down tree of
//           the 64 lanes' p (0 for invalid keys);
//   P.V: thread = (4 dims, queries t/32 + 16 u, u < QPT), o = fmaf(p_k, v_k, o) over the valid keys
//        in order.
// Dynamic LDS: queries [nqr][128] fp32 | p [nqr][65] fp32.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kKStride = kHD + 4;     // LDS row strides chosen so the MFMA operand reads of 64
constexpr int kQStride = kHD + 4;     // lanes (16 rows x 4 columns) hit every bank twice
constexpr int kVStride = kHD + 16;
constexpr int kSpStride = kSplit + 4;
constexpr int kAttnThreads = 512;
constexpr int kSplitBlocks = 256;
// PREP: the block also does the prep of its rows: the queries of its kv head are normed and roped
// here (once per block) instead of read back, and the split that holds
// the step's new positions computes their K and V, writes them to the cache and puts the
// dequantized values straight into its tile.
// Row tiles (a.zrows > 0, prefill): block z of grid.z works on rows z zrows .. of the query rows,
// at their positions, with its own work region, exactly as a launch of those rows alone would.
template <int HD = kHD>
__device__ __forceinline__ void tile_rows(AttnArgs& a, int nr, int& pos0, int& nact) {
    const int z = blockIdx.z;
    const int r0 = z * a.zrows;
    pos0 += r0;
    nact = (a.ztotal - r0 < a.zrows) ? a.ztotal - r0 : a.zrows;
    a.qh += (size_t)r0 * a.nq * HD;
    a.qkv += (size_t)r0 * a.qkv_stride;
    a.work += (size_t)z * nr * a.nq * a.max_splits * (size_t)(HD + 2);   // attn_work_floats of the tile
    a.out += (size_t)r0 * a.nq * HD;
    if (a.xq) { a.xq += (size_t)r0 * a.nq * HD; a.xs += (size_t)r0 * a.nq * HD / 16; }
}
template <int NQW, int QPT, bool PREP>
__global__ __launch_bounds__(kAttnThreads) void k_attn_split(AttnArgs a, int nr) {
    warm_args(a);
    if (stopped(a.stop)) return;
    const int kvh = blockIdx.y;
    const int G = a.nq / a.nkv;
    const int gsq = __builtin_ctz(G);               // G is a power of two: query i = (row i >> gsq, head i & (G - 1))
    int nact = a.nact_ptr ? ld_uniform(a.nact_ptr) : nr;
    int pos0 = a.pos0_ptr ? ld_uniform(a.pos0_ptr) : a.pos0_imm;
    if (!PREP && a.zrows) tile_rows(a, nr, pos0, nact);
    const int Lmax = pos0 + nact;
    const int nqr = nact * G;                       // query vectors of this kv head
    const int kvrows = a.nkv * kHD;
    const int ms = a.max_splits;
    const int gsh = __builtin_ctz(a.kv_group);      // kv_group is a power of two
    __shared__ float kd[kSplit * kKStride];
    __shared__ float vd[kSplit * kVStride];
    extern __shared__ float dyn[];
    float* qf = dyn;                                // [nqr_max][kQStride]
    float* sp = dyn + (size_t)nr * G * kQStride;    // [nqr_max][kSpStride]: scores, then p
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    float* wo = a.work;
    float* wm = a.work + (size_t)nr * a.nq * ms * kHD;
    float* wl = wm + (size_t)nr * a.nq * ms;
    bool staged_q = false;
    // the int8 K/V words of split s (thread: 16-byte words t and t + 512; K words 0..511, V
    // 512..1023) and their scales; the step's new positions (PREP) are computed, not read
    // (every thread loads its two words unconditionally, keys past the cached ones from key 0 of
    // the split, and the dequantization below zeroes them; the load addresses stay live until
    // then, so the matrix-core work in between never reuses their registers, which would make it
    // wait for the prefetch)
    uint4 kv4[2];
    float scl[2];
    const int8_t* lp[2];
    const float* lsp[2];
    auto load_tile = [&](int s) __attribute__((always_inline)) {
        const int k0 = s * kSplit;
        const int nk = (Lmax - k0 < kSplit) ? (Lmax - k0) : kSplit;
        const int kn0 = PREP ? ((pos0 - k0 > 0) ? (pos0 - k0 < nk ? pos0 - k0 : nk) : 0) : nk;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = t + kAttnThreads * u, isv = i >> 9, j = i & 511, k = j >> 3, c = j & 7;
            const size_t off = (size_t)(k0 + (k < kn0 ? k : 0)) * kvrows + (size_t)kvh * kHD + 16 * c;
            lp[u] = (isv ? a.vc : a.kc) + off;
            lsp[u] = (isv ? a.vs : a.ks) + (off >> gsh);
            kv4[u] = *(const uint4*)lp[u];
            scl[u] = *lsp[u];
        }
    };
    if (blockIdx.x * kSplit < Lmax) load_tile(blockIdx.x);
    for (int s = blockIdx.x; s * kSplit < Lmax; s += gridDim.x) {
        const int k0 = s * kSplit;
        const int nk = (Lmax - k0 < kSplit) ? (Lmax - k0) : kSplit;
        // keys [kn0, nk) are this step's new positions (PREP: computed below, not read)
        const int kn0 = PREP ? ((pos0 - k0 > 0) ? (pos0 - k0 < nk ? pos0 - k0 : nk) : 0) : nk;
        uint4 q4[2] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
        if (!PREP && !staged_q) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i = t + kAttnThreads * u;   // query vector i/16, 8 dims (i%16)*8
                const int qi = i >> 4, c = i & 15;
                if (qi < nqr) {
                    const int r = qi >> gsq, g = qi & (G - 1);
                    q4[u] = *(const uint4*)(a.qh + (size_t)r * a.nq * kHD + (size_t)(kvh * G + g) * kHD + 8 * c);
                }
            }
        }
        // (before the barrier: these write only the query stage and the new keys' tile rows,
        // which the dequantization below leaves alone, and their loads overlap the tile's)
        if (PREP && !staged_q) {
            // queries: one wave per query vector (row r, GQA head g): norm, RoPE, bf16
            const int qw = a.gate ? 2 * kHD : kHD;
            // (unrolled over the wave's NQW vectors with clamped indices, so every load is issued
            // before the first wait)
            float qy[NQW][2];
#pragma unroll
            for (int i = 0; i < NQW; ++i) {
                const int qi = wv + (kAttnThreads / 64) * i, qc = qi < nqr ? qi : nqr - 1;
                const int r = qc >> gsq, g = qc & (G - 1);
                const uint16_t* src = a.qkv + (size_t)r * a.qkv_stride + (size_t)(kvh * G + g) * qw;
                norm_rope(a, src, a.q_norm_w, pos0 + r, lane, qy[i][0], qy[i][1]);
            }
#pragma unroll
            for (int i = 0; i < NQW; ++i) {
                const int qi = wv + (kAttnThreads / 64) * i;
                if (qi < nqr) {
                    qf[qi * kQStride + lane] = bfr(qy[i][0]);
                    qf[qi * kQStride + 64 + lane] = bfr(qy[i][1]);
                }
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0): as at the end of new_keys below
        }
        // new positions of this split (in whichever of the block's splits holds them): one wave
        // per key. In the block's first split this runs before the barrier below (nothing to
        // overwrite yet, and its loads overlap the tile's); in a later split only after it, when
        // the previous split's tiles are consumed.
        auto new_keys = [&]() __attribute__((always_inline)) {
            const int qw = a.gate ? 2 * kHD : kHD;
            const int qrows = a.nq * qw;
            for (int k = kn0 + wv; k < nk; k += kAttnThreads / 64) {
                const int pos = k0 + k, r = pos - pos0;
                const uint16_t* row = a.qkv + (size_t)r * a.qkv_stride;
                const uint16_t* ksrc = row + qrows + (size_t)kvh * kHD;
                const uint16_t* vsrc = row + qrows + kvrows + (size_t)kvh * kHD;
                float y0, y1, deq[4];
                norm_rope(a, ksrc, a.k_norm_w, pos, lane, y0, y1);
                store_kv(a, y0, y1, bf2f(vsrc[lane]), bf2f(vsrc[lane + 64]), (size_t)pos * kvrows + (size_t)kvh * kHD,
                         lane, deq);
                kd[k * kKStride + lane] = deq[0];
                kd[k * kKStride + 64 + lane] = deq[1];
                vd[k * kVStride + lane] = deq[2];
                vd[k * kVStride + 64 + lane] = deq[3];
            }
            // the cache stores retire here: left in flight, their data registers would be
            // protected at the next register reuse (the score tiles) by a wait for every vector
            // memory operation, the tile prefetch included, in every split
            __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0)
        };
        if (PREP && !staged_q && kn0 < nk) new_keys();
        __syncthreads();                           // the previous split's tiles are consumed
        if (PREP && staged_q && kn0 < nk) new_keys();
        asm volatile("" :: "v"(lp[0]), "v"(lp[1]), "v"(lsp[0]), "v"(lsp[1]));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = t + kAttnThreads * u, isv = i >> 9, j = i & 511, k = j >> 3, c = j & 7;
            if (k >= kn0 && k < nk) continue;      // a new position (PREP)
            if (k >= kn0) { kv4[u] = make_uint4(0u, 0u, 0u, 0u); scl[u] = 0.0f; }   // past the split's keys
            const uint32_t w4[4] = {kv4[u].x, kv4[u].y, kv4[u].z, kv4[u].w};
            float* dst = isv ? &vd[k * kVStride + 16 * c] : &kd[k * kKStride + 16 * c];
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                float4 f;
                f.x = (float)(int8_t)(w4[e4] & 0xFFu) * scl[u];
                f.y = (float)(int8_t)((w4[e4] >> 8) & 0xFFu) * scl[u];
                f.z = (float)(int8_t)((w4[e4] >> 16) & 0xFFu) * scl[u];
                f.w = (float)(int8_t)(w4[e4] >> 24) * scl[u];
                *(float4*)(dst + 4 * e4) = f;
            }
        }
        // the block's next split: its tile loads stay in flight through this split's work
        if ((s + (int)gridDim.x) * kSplit < Lmax) load_tile(s + gridDim.x);
        if (!PREP && !staged_q) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i = t + kAttnThreads * u;
                const int qi = i >> 4, c = i & 15;
                if (qi < nqr) {
                    float4* d = (float4*)&qf[qi * kQStride + 8 * c];
                    d[0] = make_float4(__uint_as_float(q4[u].x << 16), __uint_as_float(q4[u].x & 0xFFFF0000u),
                                       __uint_as_float(q4[u].y << 16), __uint_as_float(q4[u].y & 0xFFFF0000u));
                    d[1] = make_float4(__uint_as_float(q4[u].z << 16), __uint_as_float(q4[u].z & 0xFFFF0000u),
                                       __uint_as_float(q4[u].w << 16), __uint_as_float(q4[u].w & 0xFFFF0000u));
                }
            }
        }
        staged_q = true;
        __syncthreads();
        // ---- scores on the matrix cores: query tile qt (16 queries) x key tile kt (16 keys) per
        // wave, v_mfma_f32_16x16x4f32 over the head dims in order. Each instruction adds its four
        // products one after another with fused multiply-adds (k = 0..3), so a chain of 8
        // instructions is exactly an fmaf loop over 32 dims; four such chains (dims 32c..32c+31)
        // run side by side and are summed ((c0 + c1) + c2) + c3, the oracle's score order.
        // Operand lanes: lane 16 g + j gives A[j][g] = q(16 qt + j)[4 s + g] and
        // B[g][j] = k(16 kt + j)[4 s + g]; result r of lane 16 g + j is score(query 4 g + r, key j).
        constexpr int QT = (8 * NQW + 15) / 16;   // query tiles of the kernel's capacity
        const int g4 = lane >> 4, j16 = lane & 15;
        for (int ti = wv; ti < 4 * QT; ti += kAttnThreads / 64) {
            const int qt = ti >> 2, kt = ti & 3;
            const int qa = (16 * qt + j16 < nqr) ? 16 * qt + j16 : 0;     // rows past nqr: discarded
            const float* qrow = qf + (size_t)qa * kQStride + g4;
            const float* krow = kd + (size_t)(16 * kt + j16) * kKStride + g4;
            v4f c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
            for (int st4 = 0; st4 < kHD / 16; ++st4) {
                c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qrow[4 * st4], krow[4 * st4], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qrow[32 + 4 * st4], krow[32 + 4 * st4], c1, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(qrow[64 + 4 * st4], krow[64 + 4 * st4], c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(qrow[96 + 4 * st4], krow[96 + 4 * st4], c3, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = 16 * qt + 4 * g4 + r;
                if (qi < nqr) sp[qi * kSpStride + 16 * kt + j16] = ((c0[r] + c1[r]) + c2[r]) + c3[r];
            }
        }
        __syncthreads();
        // ---- split softmax, p replacing the score: this wave's queries wv + 8 i, four at a time,
        // query i of a pass in lane row i (lanes 16 i .. 16 i + 15), lane 16 i + c holding keys c,
        // c + 16, c + 32, c + 48. The 64-lane shfl_down tree for l pairs key c with c + 32, then
        // c with c + 16: those two levels are this lane's ((p_c + p_c+32) + (p_c+16 + p_c+48)),
        // and the levels 8, 4, 2, 1 run in every row at once (DPP row shifts), l landing in lane
        // 16 i; the max is exact in any order. (Query rows past the wave's NQW run on a clamped
        // query and are discarded.)
        {
            const int qrow = lane >> 4, c = lane & 15;
#pragma unroll
            for (int pass = 0; pass < (NQW + 3) / 4; ++pass) {
                const int iq = 4 * pass + qrow;
                const int qi = wv + 8 * iq, qc = (qi < nqr && iq < NQW) ? qi : nqr - 1;
                const int r = qc >> gsq;
                const int L = pos0 + r + 1;
                const int nv = (L - k0 < nk) ? (L - k0) : nk;   // valid keys of this row in the split
                float x[4], p[4];
                float m = -__builtin_huge_valf();
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = sp[qc * kSpStride + c + 16 * e] * a.sl2e;
                    if (c + 16 * e < nv) m = fmaxf(m, x[e]);
                }
                m = max_xor(m, 16);
#pragma unroll
                for (int e = 0; e < 4; ++e) p[e] = (c + 16 * e < nv) ? qexp2(x[e] - m) : 0.0f;
                float l = (p[0] + p[2]) + (p[1] + p[3]);
                l = down_add<8>(l);
                l = down_add<4>(l);
                l = down_add<2>(l);
                l = down_add<1>(l);
                if (qi < nqr && iq < NQW) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) sp[qi * kSpStride + c + 16 * e] = p[e];
                    const int g = qi & (G - 1);
                    if (c == 0 && L - k0 > 0) {
                        const size_t mi = ((size_t)r * a.nq + (size_t)(kvh * G + g)) * ms + s;
                        wm[mi] = m;
                        wl[mi] = l;
                    }
                }
            }
        }
        __syncthreads();
        // ---- o = sum_k p_k v_k on the matrix cores: query tile qt x dim tile dt per wave; four
        // chains of 4 instructions over the 16-key blocks of the split in key order, summed
        // ((o0 + o1) + o2) + o3 (p = 0 for the keys a row does not see, whose V rows are finite:
        // fma(0, v, o) leaves o unchanged).
        // A[j][g] = p(16 qt + j)[4 s + g], B[g][j] = v[4 s + g][16 dt + j]; result r of lane
        // 16 g + j is o(query 16 qt + 4 g + r)[16 dt + j].
        for (int ti = wv; ti < 8 * QT; ti += kAttnThreads / 64) {
            const int qt = ti >> 3, dt = ti & 7;
            const int qa = (16 * qt + j16 < nqr) ? 16 * qt + j16 : 0;
            const float* prow = sp + (size_t)qa * kSpStride + g4;
            const float* vcol = vd + (size_t)g4 * kVStride + 16 * dt + j16;
            v4f o0 = {0.0f, 0.0f, 0.0f, 0.0f}, o1 = o0, o2 = o0, o3 = o0;
#pragma unroll
            for (int st4 = 0; st4 < kSplit / 16; ++st4) {
                o0 = __builtin_amdgcn_mfma_f32_16x16x4f32(prow[4 * st4], vcol[4 * st4 * kVStride], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_16x16x4f32(prow[16 + 4 * st4], vcol[(16 + 4 * st4) * kVStride], o1, 0, 0, 0);
                o2 = __builtin_amdgcn_mfma_f32_16x16x4f32(prow[32 + 4 * st4], vcol[(32 + 4 * st4) * kVStride], o2, 0, 0, 0);
                o3 = __builtin_amdgcn_mfma_f32_16x16x4f32(prow[48 + 4 * st4], vcol[(48 + 4 * st4) * kVStride], o3, 0, 0, 0);
            }
            v4f acc;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = ((o0[r] + o1[r]) + o2[r]) + o3[r];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = 16 * qt + 4 * g4 + r;
                if (qi >= nqr) continue;
                const int rr = qi >> gsq, g = qi & (G - 1);
                const int L = pos0 + rr + 1;
                if (L - k0 <= 0) continue;        // no key of this split is visible to the row
                wo[(((size_t)rr * a.nq + (size_t)(kvh * G + g)) * ms + s) * kHD + 16 * dt + j16] = acc[r];
            }
        }
    }
}

// Merge the splits of one (row, query head): M = max m_s; w_s = 2^(m_s - M); den and o accumulated
// over the splits in order (fmaf); x sigmoid(gate) -> bf16 -> per-16 quantize. Thread t owns dim
// t. The split outputs of a window of splits (contiguous in the work area) go to LDS at once by
// 16-byte LDS DMA, 1 KiB per wave instruction (up to ~150 KiB per block in flight; staged 32
// splits at a time, each chunk waited a full memory round trip), requested right behind the first
// batch of the m_s and l_s loads, whose values then give the first window's weights without a
// second round trip. The waits after that cover every transfer (their count is a run-time loop,
// so the compiler's waits count all of them), then a barrier: one round trip for the whole
// window. Longer contexts take further windows.
// splits per LDS window at most: 296 for 128-wide heads (18,944 positions), 150 for 256-wide
__host__ __device__ constexpr int comb_cap(int hd) { return hd == 128 ? 296 : 150; }
// the window of a launch: its split count, capped (short contexts keep several blocks per CU)
__host__ __device__ inline int comb_win(int max_splits, int hd = kHD) {
    return max_splits < comb_cap(hd) ? max_splits : comb_cap(hd);
}
// the window's split outputs, a 1 KiB pad (the tail of the last 16-byte transfer block), the
// window's weights and sums
__host__ __device__ inline size_t comb_lds(int max_splits, int hd = kHD) {
    return ((size_t)comb_win(max_splits, hd) * (hd + 2) + 256) * 4;
}
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(AttnArgs a, int nr) {
    if (stopped(a.stop)) return;
    const int hq = blockIdx.x, r = blockIdx.y;
    if (a.nact_ptr && r >= ld_uniform(a.nact_ptr)) return;
    int pos0 = a.pos0_ptr ? ld_uniform(a.pos0_ptr) : a.pos0_imm;
    if (a.zrows) {
        int nact = 0;
        tile_rows<HD>(a, nr, pos0, nact);
        if (r >= nact) return;
    }
    const int L = pos0 + r + 1;
    const int ns = (L + kSplit - 1) / kSplit;
    const int ms = a.max_splits;
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const float* wo = a.work;
    const float* wm = a.work + (size_t)nr * a.nq * ms * HD;
    const float* wl = wm + (size_t)nr * a.nq * ms;
    const size_t base = ((size_t)r * a.nq + hq) * ms;
    constexpr int NWV = HD / 64;
    __shared__ float smax[NWV];
    extern __shared__ __attribute__((aligned(16))) float cwin[];   // [W][HD] outputs | 256 pad | [W] w | [W] l
    const int W = comb_win(ms, HD);
    float* so = cwin;
    float* cw = cwin + (size_t)W * HD + 256;
    float* cl = cw + W;
    // splits w0 .. w0 + wn - 1 (wn HD contiguous floats of the work area) into LDS in 1 KiB blocks,
    // block b by wave b % NWV, 16 bytes per lane; lanes past the window's end re-read its first
    // bytes into the pad behind it
    const uint32_t so_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)so;
    auto dma = [&](int w0, int wn) __attribute__((always_inline)) {
        const float* src = wo + (base + w0) * HD;
        const int nf = wn * HD;
        for (int b = wv; 256 * b < nf; b += NWV) {
            const int f = 256 * b + 4 * lane;
            lds_dma16(src + (f < nf ? f : 0), __builtin_amdgcn_readfirstlane(so_lds + 1024u * b));
        }
    };
    // M over all splits: m and l of 4 splits per thread per batch, all issued before the first use;
    // the first batch's values stay in registers for the first window's weights (4 HD splits cover
    // any window). The first window's transfers are issued behind the first batch by every thread
    // (a transfer moves the lanes that execute it).
    float M = -__builtin_huge_valf();
    float m0v[4], l0v[4];
    const int wn0 = ns < W ? ns : W;
    for (int s0 = t; s0 - t < ns; s0 += 4 * HD) {
        float mv[4], lv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t i = base + ((s0 + u * HD < ns) ? s0 + u * HD : ns - 1);
            mv[u] = wm[i];
            lv[u] = wl[i];
        }
        if (s0 == t) {
            dma(0, wn0);
#pragma unroll
            for (int u = 0; u < 4; ++u) { m0v[u] = mv[u]; l0v[u] = lv[u]; }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (s0 + u * HD < ns) M = fmaxf(M, mv[u]);
    }
    M = max_xor(M, 64);
    if (lane == 0) smax[t >> 6] = M;
    __syncthreads();
    M = smax[0];
#pragma unroll
    for (int w = 1; w < HD / 64; ++w) M = fmaxf(M, smax[w]);
    float den = 0.0f, o = 0.0f;
    for (int w0 = 0; w0 < ns; w0 += W) {
        const int wn = (ns - w0 < W) ? ns - w0 : W;
        if (w0 > 0) {
            __syncthreads();                        // the previous window is consumed
            dma(w0, wn);
            for (int j = t; j < wn; j += HD) { cw[j] = qexp2(wm[base + w0 + j] - M); cl[j] = wl[base + w0 + j]; }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = t + u * HD;
                if (j < wn) { cw[j] = qexp2(m0v[u] - M); cl[j] = l0v[u]; }
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0): this wave's transfers have landed
        __syncthreads();                            // every thread's weights are in LDS
        for (int j = 0; j < wn; ++j) {
            const float w = cw[j];
            den = __builtin_fmaf(cl[j], w, den);
            o = __builtin_fmaf(so[j * HD + t], w, o);
        }
    }
    const float inv = 1.0f / den;
    float v = o * inv;
    const int qw = a.gate ? 2 * HD : HD;
    if (a.gate) v = v * qsigmoid(bf2f(a.qkv[(size_t)r * a.qkv_stride + (size_t)hq * qw + HD + t]));
    const uint16_t vb = f2bf(v);
    const size_t k = (size_t)r * a.nq * HD + (size_t)hq * HD + t;
    a.out[k] = vb;
    if (a.xq) {   // the per-16 quantizer with g = 1/in_scale (s = mx g / 127, 1/s -> g / s)
        const float g = (a.in_scale > 0.0f) ? 1.0f / a.in_scale : 1.0f;
        const float yv = bf2f(vb);
        const float m16 = max_xor(fabsf(yv), 16);
        const float sc = m16 * g * (1.0f / 127.0f);
        const float qi = (sc > 0.0f) ? (g / sc) : 0.0f;
        a.xq[k] = qcode(yv, qi);
        if ((t & 15) == 0) a.xs[k >> 4] = sc;
    }
}

// ---------------------------------------------------------------- general geometry
// Heads of HD = 256 dims (the reference trunk's 24q / 4kv x 256, include/q27.h:25-35) or GQA groups
// that are not a power of two. Queries come from qh (the prep runs as its own launch before), K and
// V from the cache. The splits, and the order of every sum, are those of the kernels above and of
// the oracle: score = ((c0 + c1) + c2) + c3 with c_j the fmaf chain over dims [j HD/4, (j+1) HD/4),
// on K values code x scale; the split softmax m = max, p = 2^(x - m), l = the 64-lane shfl_down
// tree; o = ((o0 + o1) + o2) + o3 with o_j the fmaf chain over the row's visible keys of the split's
// j-th 16-key block, in key order. Block = (split, kv head), all rows and GQA heads of the kv head:
// the int8 K/V tile and its scales in LDS (an fp32 tile of 256-wide rows would not leave room for
// the queries), plain VALU chains, one thread per (query, key) score and per (query, dim) output.
constexpr int kGThreads = 512;
constexpr int kSpG = kSplit + 1;                 // score row stride (floats)
template <int HD>
__host__ __device__ constexpr int tile_stride_g() { return HD + 16; }   // int8 K/V tile row stride
template <int HD>
__global__ __launch_bounds__(kGThreads) void k_attn_split_g(AttnArgs a, int nr) {
    if (stopped(a.stop)) return;
    constexpr int KS = tile_stride_g<HD>();
    constexpr int NSC = HD / 16;                 // scales per key row at most (kv_group >= 16)
    const int kvh = blockIdx.y;
    const int G = a.nq / a.nkv;
    int nact = a.nact_ptr ? ld_uniform(a.nact_ptr) : nr;
    int pos0 = a.pos0_ptr ? ld_uniform(a.pos0_ptr) : a.pos0_imm;
    if (a.zrows) tile_rows<HD>(a, nr, pos0, nact);
    const int Lmax = pos0 + nact;
    const int nqr = nact * G;
    const int kvrows = a.nkv * HD;
    const int ms = a.max_splits;
    const int KG = a.kv_group, nsc = HD / KG;
    __shared__ __attribute__((aligned(16))) int8_t k8[kSplit * KS];
    __shared__ __attribute__((aligned(16))) int8_t v8[kSplit * KS];
    __shared__ float ksc[kSplit * NSC];
    __shared__ float vsc[kSplit * NSC];
    extern __shared__ float dyn[];
    float* qf = dyn;                                // [nr G][HD] queries as fp32
    float* sp = dyn + (size_t)nr * G * HD;          // [nr G][kSpG] scores, then p
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    float* wo = a.work;
    float* wm = a.work + (size_t)nr * a.nq * ms * HD;
    float* wl = wm + (size_t)nr * a.nq * ms;
    for (int i = t; i < nqr * HD; i += kGThreads) {
        const int qi = i / HD, d = i - qi * HD;
        const int r = qi / G, g = qi - r * G;
        qf[i] = bf2f(a.qh[(size_t)r * a.nq * HD + (size_t)(kvh * G + g) * HD + d]);
    }
    for (int s = blockIdx.x; s * kSplit < Lmax; s += gridDim.x) {
        const int k0 = s * kSplit;
        const int nk = (Lmax - k0 < kSplit) ? (Lmax - k0) : kSplit;
        __syncthreads();                            // the previous split's tiles are consumed
        for (int i = t; i < nk * (HD / 16); i += kGThreads) {
            const int k = i / (HD / 16), c = i - k * (HD / 16);
            const size_t off = (size_t)(k0 + k) * kvrows + (size_t)kvh * HD + 16 * c;
            *(uint4*)&k8[k * KS + 16 * c] = *(const uint4*)(a.kc + off);
            *(uint4*)&v8[k * KS + 16 * c] = *(const uint4*)(a.vc + off);
        }
        for (int i = t; i < nk * nsc; i += kGThreads) {
            const int k = i / nsc, c = i - k * nsc;
            const size_t off = ((size_t)(k0 + k) * kvrows + (size_t)kvh * HD) / KG + c;
            ksc[k * NSC + c] = a.ks[off];
            vsc[k * NSC + c] = a.vs[off];
        }
        __syncthreads();
        // scores, one (query, key) pair per thread at a time
        for (int i = t; i < nqr * kSplit; i += kGThreads) {
            const int qi = i >> 6, key = i & (kSplit - 1);
            if (key >= nk) continue;
            const float* q = qf + (size_t)qi * HD;
            const int8_t* kr = k8 + key * KS;
            const float* kscr = ksc + key * NSC;
            float c4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float acc = 0.0f;
                for (int d = j * (HD / 4); d < (j + 1) * (HD / 4); ++d)
                    acc = __builtin_fmaf(q[d], (float)kr[d] * kscr[d / KG], acc);
                c4[j] = acc;
            }
            sp[(size_t)qi * kSpG + key] = (((c4[0] + c4[1]) + c4[2]) + c4[3]) * a.sl2e;
        }
        __syncthreads();
        // split softmax, one wave per query, lane = key
        for (int qi = wv; qi < nqr; qi += kGThreads / 64) {
            const int r = qi / G, g = qi - r * G;
            const int L = pos0 + r + 1;
            const int nv = (L - k0 < nk) ? (L - k0) : nk;       // visible keys of this row in the split
            const float x = (lane < nv) ? sp[(size_t)qi * kSpG + lane] : -__builtin_huge_valf();
            const float m = max_xor(x, 64);
            const float p = (lane < nv) ? qexp2(x - m) : 0.0f;
            const float l = tree64(p);
            sp[(size_t)qi * kSpG + lane] = p;
            if (lane == 0 && nv > 0) {
                const size_t mi = ((size_t)r * a.nq + (size_t)(kvh * G + g)) * ms + s;
                wm[mi] = m;
                wl[mi] = l;
            }
        }
        __syncthreads();
        // o = sum_k p_k v_k, one (query, dim) pair per thread at a time
        for (int i = t; i < nqr * HD; i += kGThreads) {
            const int qi = i / HD, d = i - qi * HD;
            const int r = qi / G, g = qi - r * G;
            const int L = pos0 + r + 1;
            const int nv = (L - k0 < nk) ? (L - k0) : nk;
            if (nv <= 0) continue;
            const float* pr = sp + (size_t)qi * kSpG;
            float o4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float acc = 0.0f;
                const int e = (16 * (j + 1) < nv) ? 16 * (j + 1) : nv;
                for (int key = 16 * j; key < e; ++key)
                    acc = __builtin_fmaf(pr[key], (float)v8[key * KS + d] * vsc[key * NSC + d / KG], acc);
                o4[j] = acc;
            }
            wo[(((size_t)r * a.nq + (size_t)(kvh * G + g)) * ms + s) * HD + d] = ((o4[0] + o4[1]) + o4[2]) + o4[3];
        }
    }
}

// The 128-wide kernels above need a power-of-two GQA group; the general kernel takes the rest.
static bool attn_general(const AttnArgs& a) {
    const int G = a.nq / a.nkv;
    return a.hd != kHD || (G & (G - 1));
}

static int attn_check(const AttnArgs& a, int nr) {
    const bool rot_ok = a.rot >= 2 && (a.rot & (a.rot - 1)) == 0 && (a.rot <= 64 || (a.rot == kHD && a.hd == kHD));
    // (row tiles of a prefill may hold more rows than a verify step, as many as kMaxQ query vectors)
    if ((a.hd != 128 && a.hd != 256) || a.nkv < 1 || a.nq % a.nkv || nr < 1 || nr > (a.zrows ? kMaxQ : kMaxRows) ||
        nr * (a.nq / a.nkv) > kMaxQ || (a.kv_group != 16 && a.kv_group != 32 && a.kv_group != 64) || !rot_ok) {
        set_error("attn: unsupported shape (nq=%d nkv=%d hd=%d nr=%d kv_group=%d rot=%d: hd 128 or 256, at most %d "
                  "query vectors per kv head, rot a power of two <= 64 or the whole 128-wide head)", a.nq, a.nkv, a.hd,
                  nr, a.kv_group, a.rot, kMaxQ);
        return Q27X_E_SHAPE;
    }
    return Q27X_OK;
}

int launch_attn_prep(const AttnArgs& a, int nr, hipStream_t s) {
    if (int rc = attn_check(a, nr)) return rc;
    if (a.hd == 256) hipLaunchKernelGGL(k_attn_prep<256>, dim3(a.nq + a.nkv, nr), dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_attn_prep<128>, dim3(a.nq + a.nkv, nr), dim3(64), 0, s, a);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// prep of any number of rows (prefill): one wave per (head, row); K/V only when a.prep_kv_only
int launch_attn_prep_rows(const AttnArgs& a, int nrows, hipStream_t s) {
    if (int rc = attn_check(a, 1)) return rc;
    if (nrows < 1 || a.nact_ptr) {
        set_error("attn prep: rows=%d unsupported", nrows);
        return Q27X_E_SHAPE;
    }
    const dim3 grid(a.prep_kv_only ? a.nkv : a.nq + a.nkv, nrows);
    if (a.hd == 256) hipLaunchKernelGGL(k_attn_prep<256>, grid, dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_attn_prep<128>, grid, dim3(64), 0, s, a);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

template <int HD>
static int launch_split_g(const AttnArgs& a, int nr, hipStream_t s) {
    const size_t lds = (size_t)nr * (a.nq / a.nkv) * (HD + kSpG) * 4;
    static std::once_flag attr;
    static hipError_t attr_e = hipSuccess;
    std::call_once(attr, [] {
        attr_e = hipFuncSetAttribute((const void*)k_attn_split_g<HD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)((size_t)kMaxQ * (HD + kSpG) * 4));
    });
    Q27X_HIP(attr_e);
    const int bx = a.max_splits < kSplitBlocks / a.nkv ? a.max_splits : (kSplitBlocks / a.nkv > 0 ? kSplitBlocks / a.nkv : 1);
    const dim3 grid(bx, a.nkv, a.zrows ? (unsigned)((a.ztotal + a.zrows - 1) / a.zrows) : 1u);
    hipLaunchKernelGGL(k_attn_split_g<HD>, grid, dim3(kGThreads), lds, s, a, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

template <bool PREP>
static int launch_split(const AttnArgs& a, int nr, hipStream_t s) {
    const int nqr = nr * (a.nq / a.nkv);
    const size_t lds = (size_t)nqr * (kQStride + kSpStride) * 4;
    static bool lds_set = false;                  // queries + p of up to 64 query vectors: 50 KiB
    if (!lds_set) {
        const int mx = 64 * (kQStride + kSpStride) * 4;
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<1, 1, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<2, 1, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<3, 2, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<4, 2, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<6, 3, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_attn_split<8, 4, PREP>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        lds_set = true;
    }
    // at most kSplitBlocks blocks (about one per CU); a block takes splits blockIdx.x + i gridDim.x
    const int bx = a.max_splits < kSplitBlocks / a.nkv ? a.max_splits : (kSplitBlocks / a.nkv > 0 ? kSplitBlocks / a.nkv : 1);
    const dim3 grid(bx, a.nkv, a.zrows ? (unsigned)((a.ztotal + a.zrows - 1) / a.zrows) : 1u);
    if (nqr <= 8) hipLaunchKernelGGL((k_attn_split<1, 1, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    else if (nqr <= 16) hipLaunchKernelGGL((k_attn_split<2, 1, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    else if (nqr <= 24) hipLaunchKernelGGL((k_attn_split<3, 2, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    else if (nqr <= 32) hipLaunchKernelGGL((k_attn_split<4, 2, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    else if (nqr <= 48) hipLaunchKernelGGL((k_attn_split<6, 3, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    else hipLaunchKernelGGL((k_attn_split<8, 4, PREP>), grid, dim3(kAttnThreads), lds, s, a, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// prep_fused: the split kernel does the prep as well (no k_attn_prep launch before it)
int launch_attn(const AttnArgs& a, int nr, hipStream_t s, bool prep_fused) {
    if (int rc = attn_check(a, nr)) return rc;
    if (!a.work || a.max_splits < 1) { set_error("attn: no work buffer"); return Q27X_E_ARG; }
    static std::once_flag comb_attr;
    static hipError_t comb_e = hipSuccess;
    std::call_once(comb_attr, [] {
        comb_e = hipFuncSetAttribute((const void*)k_attn_combine<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)comb_lds(comb_cap(128), 128));
        if (comb_e == hipSuccess)
            comb_e = hipFuncSetAttribute((const void*)k_attn_combine<256>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)comb_lds(comb_cap(256), 256));
    });
    Q27X_HIP(comb_e);
    if (a.zrows && (prep_fused || a.zrows != nr || a.ztotal < 1 || a.nact_ptr)) {
        set_error("attn: row tiles need separate prep, zrows == nr and no active-row count");
        return Q27X_E_ARG;
    }
    const dim3 cgrid(a.nq, nr, a.zrows ? (unsigned)((a.ztotal + a.zrows - 1) / a.zrows) : 1u);
    if (attn_general(a)) {
        // the prep (queries to qh, the new K/V to the cache) as a launch of its own, then the splits
        if (prep_fused) {
            if (!a.qh) { set_error("attn: the general geometry needs a query buffer"); return Q27X_E_ARG; }
            if (int rc = launch_attn_prep(a, nr, s)) return rc;
        }
        const int rc = a.hd == 256 ? launch_split_g<256>(a, nr, s) : launch_split_g<128>(a, nr, s);
        if (rc) return rc;
        if (a.hd == 256) hipLaunchKernelGGL(k_attn_combine<256>, cgrid, dim3(256), comb_lds(a.max_splits, 256), s, a, nr);
        else hipLaunchKernelGGL(k_attn_combine<128>, cgrid, dim3(128), comb_lds(a.max_splits, 128), s, a, nr);
        Q27X_HIP(hipGetLastError());
        return Q27X_OK;
    }
    const int rc = prep_fused ? launch_split<true>(a, nr, s) : launch_split<false>(a, nr, s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_attn_combine<128>, cgrid, dim3(kHD), comb_lds(a.max_splits), s, a, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // namespace q27x

using namespace q27x;
extern "C" size_t q27x_attn_work_bytes(int nq, int hd, int ctx, int nr) {
    return attn_work_floats(nq, hd, (ctx + kSplit - 1) / kSplit, nr) * 4;
}

extern "C" int q27x_attn_prep_rows(const uint16_t* qkv, int qkv_stride, const uint16_t* q_norm_w,
                                   const uint16_t* k_norm_w, const float* rope_cos, const float* rope_sin, int rot,
                                   int8_t* kc, float* ks, int8_t* vc, float* vs, int kv_group, uint16_t* qh, int nq,
                                   int nkv, int hd, int gate, float eps, int pos0, int nr, q27x_stream_t s) {
    if (!qkv || !q_norm_w || !k_norm_w || !rope_cos || !rope_sin || !kc || !ks || !vc || !vs || !qh || pos0 < 0) {
        set_error("q27x_attn_prep_rows: null argument");
        return Q27X_E_ARG;
    }
    AttnArgs a{};
    a.qkv = qkv; a.qkv_stride = qkv_stride; a.q_norm_w = q_norm_w; a.k_norm_w = k_norm_w;
    a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.rot = rot;
    a.kc = kc; a.ks = ks; a.vc = vc; a.vs = vs; a.kv_group = kv_group; a.qh = qh;
    a.nq = nq; a.nkv = nkv; a.hd = hd; a.gate = gate; a.eps = eps; a.pos0_imm = pos0;
    return launch_attn_prep(a, nr, (hipStream_t)s);
}

extern "C" int q27x_attn_rows(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride, const int8_t* kc,
                              const float* ks, const int8_t* vc, const float* vs, int kv_group, int nq, int nkv,
                              int hd, int gate, int pos0, int nr, void* work, uint16_t* out, int8_t* xq, float* xs,
                              q27x_stream_t s) {
    if (!qh || (gate && !qkv_gate) || !kc || !ks || !vc || !vs || !work || !out || pos0 < 0) {
        set_error("q27x_attn_rows: null argument");
        return Q27X_E_ARG;
    }
    AttnArgs a{};
    a.qh = const_cast<uint16_t*>(qh); a.qkv = qkv_gate; a.qkv_stride = qkv_stride;
    a.kc = const_cast<int8_t*>(kc); a.ks = const_cast<float*>(ks);
    a.vc = const_cast<int8_t*>(vc); a.vs = const_cast<float*>(vs);
    a.kv_group = kv_group; a.nq = nq; a.nkv = nkv; a.hd = hd; a.gate = gate; a.rot = 2;
    a.pos0_imm = pos0; a.work = (float*)work; a.max_splits = (pos0 + nr + kSplit - 1) / kSplit;
    a.sl2e = (float)((1.0 / sqrt((double)hd)) * 1.4426950408889634);
    a.out = out; a.xq = xq; a.xs = xs;
    return launch_attn(a, nr, (hipStream_t)s);
}

// ---------------------------------------------------------------- allocation-free variant
// Scratch of q27x_attn_rows_noalloc: the split partials of one call, o [nr][nq][splits][128] |
// m | l, at most kNoAllocRows (row, query head, split) triples -- 32 query heads x 8 rows x 256
// splits of 64 keys (16384 positions): 32.5 MiB of device memory, held on every GPU the library
// runs on until the process ends. Every partial the combine reads is written earlier in the same
// call, so nothing in it has to start at zero.
namespace q27x {
constexpr size_t kNoAllocRows = 65536;
constexpr size_t kNoAllocFloats = kNoAllocRows * (kHD + 2);
static __device__ __align__(256) float scratch[kNoAllocFloats];

// Device address of `scratch` on the current device. The array's name in host code is only a
// host-side stand-in, so the address is looked up once per device (with that device current) and
// kept; kernels and copies get this pointer, never the name.
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_dev[kMaxDevices];
static int scratch_ptr(float** out) {
    int dev = 0;
    Q27X_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) { set_error("attn: device %d out of range", dev); return Q27X_E_ARG; }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) { set_error("attn: no device address for the scratch array"); return Q27X_E_HIP; }
        g_scratch_dev[dev] = (float*)p;
    }
    *out = g_scratch_dev[dev];
    return Q27X_OK;
}
}  // namespace q27x

extern "C" int q27x_attn_rows_noalloc(const uint16_t* qh, const uint16_t* qkv_gate, int qkv_stride, const int8_t* kc,
                                      const float* ks, const int8_t* vc, const float* vs, int kv_group, int nq, int nkv,
                                      int hd, int gate, int pos0, int nr, uint16_t* out, int8_t* xq, float* xs,
                                      q27x_stream_t s) {
    if (!qh || (gate && !qkv_gate) || !kc || !ks || !vc || !vs || !out || pos0 < 0 || nq < 1 || nr < 1 || hd != kHD) {
        set_error("q27x_attn_rows_noalloc: bad arguments");
        return Q27X_E_ARG;
    }
    const size_t splits = ((size_t)pos0 + nr + kSplit - 1) / kSplit;
    if ((size_t)nr * nq * splits > kNoAllocRows) {
        set_error("q27x_attn_rows_noalloc: nr x nq x splits = %zu exceeds the scratch limit of %zu "
                  "(e.g. 8 rows x 32 heads at 16384 positions)", (size_t)nr * nq * splits, kNoAllocRows);
        return Q27X_E_RANGE;
    }
    float* w = nullptr;
    const int rc = scratch_ptr(&w);
    if (rc) return rc;
    return q27x_attn_rows(qh, qkv_gate, qkv_stride, kc, ks, vc, vs, kv_group, nq, nkv, hd, gate, pos0, nr, w, out, xq,
                          xs, s);
}
