// k_proj.hip -- W8A8 projection of NR <= 8 rows and the bf16 GEMV (lm_head, GDN a/b).
//
// Memory-bound: one pass over the weights serves every verify row. A wave owns RPW weight rows
// at a time; lane l streams 16 B of each row per 1024-element step (the 64 lanes of a step read
// one contiguous 1 KiB run per row, non-temporal), so slab s = 64*step + lane of the row meets
// the same slab of every activation row staged once per block in LDS. Per slab:
//   int d = sdot4 x 4 (exact int32), acc = fmaf((float)d, ws64 * xs16, acc)
// then the 64 lane sums meet in the shfl_down tree -- the reference's order
// (src/q27_fp8.hip:3814-3871), kept so results match its host restatement bit for bit.
// Pipelining: each weight register is refilled with the next row group's slab once its dot
// products have issued (the compiler issues the group's refills together, which measured faster
// than spreading them over the steps), so a full group of loads stays in flight through the
// reduction and the epilogue; epilogue inputs are requested before those refills (vector-memory
// counters retire in order, so a later load would make its wait drain the prefetch).
#include <stdlib.h>

#include <type_traits>

#include "q27x_dev.h"
#include "q27x_int.h"
#include "q27x_norm.h"

namespace q27x {


template <int V> struct Pow2 {
    static constexpr int value = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : V <= 32 ? 32 : 64;
};

// shfl_down levels O, O/2, ..., 1 (down_add: DPP for offsets <= 8)
template <int O>
__device__ __forceinline__ float down_tree(float y) {
    if constexpr (O == 0) return y;
    else return down_tree<O / 2>(down_add<O>(y));
}

// Transposed shfl tree: P values per lane, each reduced over the 64 lanes with exactly the pairs
// of the shfl_down tree (offsets 32..1; a + b and b + a are the same float); value v ends in lane
// v * (64 / P). The halving levels exchange half of the values per step, so P values cost
// P - 1 + log2(64 / P) shuffles instead of 6 P.
template <int P>
__device__ __forceinline__ float tree_t(float (&x)[P], int lane) {
    // levels 32 and 16: one lane-half (row) swap of the pair (v, v + h) puts value v's partners
    // side by side in the lower half (rows 0, 2) and value v + h's in the upper half (rows 1, 3),
    // the same pairs the exchange below forms
    int h = P / 2, o = 32;
#pragma unroll
    for (; h >= 1 && o >= 16; h >>= 1, o >>= 1) {
#pragma unroll
        for (int v = 0; v < h; ++v) {
            const auto r = (o == 32) ? __builtin_amdgcn_permlane32_swap(__float_as_uint(x[v]), __float_as_uint(x[v + h]), false, false)
                                     : __builtin_amdgcn_permlane16_swap(__float_as_uint(x[v]), __float_as_uint(x[v + h]), false, false);
            x[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    }
#pragma unroll
    for (; h >= 1; h >>= 1, o >>= 1) {
        // bitwise selects: a select between two array elements would become a select of
        // addresses and push the array out of registers
        const uint32_t up = (lane & o) ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int v = 0; v < h; ++v) {
            const uint32_t lo = __float_as_uint(x[v]), hi = __float_as_uint(x[v + h]);
            const float send = __uint_as_float((lo & up) | (hi & ~up));
            const float keep = __uint_as_float((hi & up) | (lo & ~up));
            // (an LDS-crossbar shuffle: the lane swaps used by tree64 changed how the compiler
            // places the next group's refills here and made the store kernels slower)
            x[v] = keep + __shfl_xor(send, o, 64);
        }
    }
    return down_tree<32 / P>(x[0]);
}

// Work assignment. A row group is RPW consecutive weight rows. Each block owns a list of groups;
// its waves take them one at a time from a counter in LDS (a wave that is served sooner takes
// more), so the block's waves finish together.
//   EPI_STORE: with 4-wave blocks (K = 17408 and the unaligned shapes, several blocks per CU),
//     block b owns the groups b NW + w + i nw (w < NW, nw = gridDim.x * NW); with 16-wave
//     blocks (one per CU) it owns the groups b + i gridDim.x, so every block gets the same count
//     to within one. Either way the waves of the grid stream adjacent rows at the same time.
//   EPI_SWIGLU (RPW = 1): the 32-row units (16 gate rows | 16 up rows = one 16-output quantization
//     group) are dealt so that every block streams the same number of rows. With
//     nunits = F * nb + E, block b takes the whole units b, b + nb, ..., b + (F-1) nb; the E
//     leftover units are cut into quarters (4 gate rows + the matching 4 up rows = 4 outputs)
//     dealt round-robin over the blocks (a block's quarters come first in its list). The dot
//     products of a block's rows meet in LDS, and an LDS counter per unit / quarter counts its
//     rows: the wave that stores the last row of a whole unit applies SwiGLU + quantize to it
//     (codes and scales staged in LDS, written out by the block at the end); for a quarter it
//     sends the 4 SwiGLU values to the scratch area with agent-scope stores and counts on the
//     unit's arrival counter; the wave that brings the count to 4 takes the exact
//     max over the unit's 16 values, quantizes them and resets the counter. No block waits for
//     another.
// FULL: K == 1024 * NSTEP (no slab bounds checks). PRE: the activation stage is the RMSNorm +
// quantize of the raw input rows (a.pre), computed by every block (K = NSTEP * 1024, NW = 16).
constexpr int kSwRows = 288;     // SwiGLU rows one block may hold: 32 F + 8 (quarters per block)
// The activation stage of NR rows at K = 1024 NSTEP: 16-byte code words and a 4-byte scale per
// slab in LDS. When all of it does not fit (K = 17408 at 8 rows), the scales of the rows from XL on
// stay in registers. (512 bytes are left for the kernel's other LDS variables.)
template <int NR, int NSTEP>
struct StageFit {
    static constexpr int kLds = 160 * 1024 - 512;
    static constexpr int kCodes = NR * NSTEP * 64 * 16;
    static constexpr int XL = (kCodes + NR * NSTEP * 64 * 4 <= kLds) ? NR : (kLds - kCodes) / (NSTEP * 64 * 4);
    static constexpr int kBytes = kCodes + XL * NSTEP * 64 * 4;
};
template <int NR, int NSTEP, int RPW, int EPI, bool FULL, bool PRE, int NW>
__global__ __launch_bounds__(NW * 64) void k_proj(ProjArgs a) {
    constexpr bool CV = (EPI == EPI_CONV);
    constexpr bool ST = (EPI == EPI_STORE || CV);
    static_assert(!CV || RPW == 1, "the conv epilogue takes one row per group");
    constexpr int SL = NSTEP * 64;
    constexpr int NT = NW * 64;
    constexpr int NSTG = (NR * SL + NT - 1) / NT;      // staging loads per thread
    constexpr int V = RPW * NR, P = Pow2<V>::value, LPV = 64 / P;
    static_assert(EPI != EPI_SWIGLU || RPW == 1, "SwiGLU deals single rows");
    static_assert(!PRE || NW == 16, "the norm prologue runs on 16-wave blocks");
    // XR: the K = 17408 stage of 8 rows (8 x 1088 slabs x 20 B) does not fit in 160 KB with all
    // its scales: rows 0..4 keep their scales in LDS, rows 5..7 in registers (each lane holds the
    // scales of its own slabs; with every row's scales in registers the kernel ran out of them).
    // XB: from 5 rows on each step's LDS reads are requested together ahead of its arithmetic;
    // left to itself the compiler waits for each read before the next (K = 17408 at 6 rows with
    // every scale in LDS: 32.6 us unbatched, 20.0 us batched; at 8 rows out_proj 12.9 -> 11.5 us,
    // o_proj 9.7 -> 9.2, in_qkv|in_z 29.3 -> 28.2, gate|up unchanged).
    constexpr int XL = StageFit<NR, NSTEP>::XL;        // rows whose scales are staged in LDS
    constexpr bool XR = XL < NR;
    constexpr bool XB = (NR > 4);
    static_assert(!XR || (!PRE && FULL && EPI == EPI_STORE), "register scales: plain full-K stage only");
    __shared__ uint4 sx[NR * SL];
    __shared__ float ssc[XL * SL];
    float XS[XR ? NR - XL : 1][XR ? NSTEP : 1];
    __shared__ float sacc[(EPI == EPI_SWIGLU) ? kSwRows * NR : 1];
    __shared__ float wsum[PRE ? PreNorm<NSTEP, NR>::RPG : 1][4][4];
    // EPI_CONV: the bf16 normalized input rows of the blocks that compute GDN row scalars
    __shared__ __attribute__((aligned(16))) uint16_t sybf[CV ? NR * NSTEP * 1024 : 1];
    // The round's stop flag is read once the prologue's loads are in flight (before any store),
    // so its read does not add a memory round trip in front of them.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, nslab = K >> 4, ng64 = K >> 6;
    const int nb = gridDim.x, bi = blockIdx.x;
    // The block's row groups form a list j = 0 .. nrb-1; wave w starts with group w, then takes
    // the next unclaimed group from a block counter in LDS, so waves that get their bytes sooner
    // do more groups and the block's waves finish together.
    const int ngroups = (a.rows + RPW - 1) / RPW;
    const int nw = nb * NW;
    const int nunits = a.rows >> 5, F = nunits / nb, E = nunits - F * nb;
    const int nq = 4 * E, myq = (nq > bi) ? (nq - 1 - bi) / nb + 1 : 0;   // leftover quarters
    int nrb;
    if constexpr (EPI == EPI_SWIGLU) {
        nrb = 32 * F + 8 * myq;                        // this block's rows
    } else if constexpr (NW == 16) {                   // groups bi + i*nb of the grid
        nrb = (ngroups - bi + nb - 1) / nb;
    } else {                                           // groups bi*NW + w + i*nw of the grid
        const int fr = ngroups / nw, rem = ngroups - fr * nw - bi * NW;
        nrb = fr * NW + (rem < 0 ? 0 : (rem > NW ? NW : rem));
    }
    __shared__ unsigned s_next;                        // groups handed out after the first NW
    if (threadIdx.x == 0) s_next = 0u;
    // SwiGLU: rows still owed per quarter / whole unit of the block (quarters first in the list)
    __shared__ unsigned s_gcnt[(EPI == EPI_SWIGLU) ? kSwRows / 8 : 1];
    __shared__ int8_t s_code[(EPI == EPI_SWIGLU) ? (kSwRows / 32) * NR * 16 : 1];
    __shared__ float s_scale[(EPI == EPI_SWIGLU) ? (kSwRows / 32) * NR : 1];
    if constexpr (EPI == EPI_SWIGLU)
        for (int i = threadIdx.x; i < kSwRows / 8; i += NT) s_gcnt[i] = 0u;
    auto row_of = [&](int j, int r) __attribute__((always_inline)) {
        if constexpr (EPI == EPI_SWIGLU) {
            if (j >= 8 * myq) return (bi + nb * ((j - 8 * myq) >> 5)) * 32 + ((j - 8 * myq) & 31);
            const int m = j >> 3, r8 = j & 7;
            const int p = bi + nb * m, u = F * nb + (p >> 2), q = p & 3;
            return u * 32 + (r8 < 4 ? 4 * q + r8 : 12 + 4 * q + r8);
        } else {
            if constexpr (NW == 16) return (bi + j * nb) * RPW + r;
            else return (bi * NW + (j % NW) + (j / NW) * nw) * RPW + r;
        }
    };
    auto valid = [&](int j) __attribute__((always_inline)) { return j < nrb; };
    uint4 W[RPW][NSTEP];
    float S[RPW][NSTEP];
    // Loads are issued on every path: a group past the wave's last (ok == false) reads the first
    // 16 bytes of the weights instead, so no branch merges a path that loaded with one that did
    // not, and each wait the compiler places counts exactly the loads still owed to later groups
    // (a merge of the two would make it wait for all of them).
    // rg: the group's first row (wave-uniform), computed once per group
    auto ld = [&](int rg, int r, int t, bool ok) __attribute__((always_inline)) {
        int row = rg + r;
        row = row < a.rows ? row : a.rows - 1;
        const int s = t * 64 + lane;
        if (FULL || s < nslab) {
            // (the row base is selected per wave, the lane's slab added after: a group past the
            // wave's last reads the first row's slabs)
            const int8_t* wrow = ok ? a.W + (size_t)row * K : a.W;
            const float* srow = ok ? a.WS + (size_t)row * ng64 : a.WS;
            W[r][t] = ld_nt16(wrow + 16 * s);
            S[r][t] = srow[s >> 2];
        } else {
            W[r][t] = make_uint4(0u, 0u, 0u, 0u);
            S[r][t] = 0.0f;
        }
    };
    auto prefetch = [&]() __attribute__((always_inline)) {
        const int rg = __builtin_amdgcn_readfirstlane(row_of(wave, 0));
#pragma unroll
        for (int t = 0; t < NSTEP; ++t)
#pragma unroll
            for (int r = 0; r < RPW; ++r) ld(rg, r, t, valid(wave));
    };
    if constexpr (PRE) {
        // input rows first, then the weights, so waiting for the rows leaves the weights in flight.
        // With two rows per 256-thread group (NR > 4) the held rows and the prefetch do not fit
        // in 128 registers together; the weights are then requested after the norm. So are the
        // conv-epilogue kernel's (in_qkv|in_z): with its prefetch in flight during the norm it took
        // 19.9-20.0 us at 3 rows, with the prefetch after the norm 19.0 (the same change in the
        // SwiGLU and plain-store kernels measured within the noise).
        PreNorm<NSTEP, NR> pn;
        constexpr bool EARLY = PreNorm<NSTEP, NR>::RPG == 1 && !CV;
        pn.load(a.pre);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (EARLY) prefetch();
        __builtin_amdgcn_sched_barrier(0);
        if (stopped(a.stop)) return;
        uint16_t* ylds = nullptr;
        if constexpr (CV) ylds = (bi < 2 * a.ab_vh) ? sybf : nullptr;
        pn.finish(a.pre, (uint32_t*)sx, ssc, SL, wsum, blockIdx.x == 0, ylds);
        if constexpr (!EARLY) prefetch();
    } else if constexpr (FULL) {
        // activation stage by LDS DMA (global_load_lds: each lane's 16-byte code word and 4-byte
        // scale land at the wave's LDS base + lane offset, no registers), requested together with
        // the weight prefetch; the barrier below waits for both
#pragma unroll
        for (int j = 0; j < NSTG; ++j) {
            const int i0 = j * NT + 64 * wave;              // first stage element of this wave
            const int i = i0 + lane;
            if (i0 < NR * SL && i < NR * SL) {
                const int n = i / SL, s = i - n * SL;
                __builtin_amdgcn_global_load_lds((const void*)(a.xq + (size_t)n * a.xst + 16 * s),
                                                 (__attribute__((address_space(3))) void*)&sx[i0], 16, 0, 0);
                if (i0 / SL < XL)                       // (the wave's row: SL is a multiple of 64)
                    __builtin_amdgcn_global_load_lds((const void*)(a.xs + (size_t)n * (a.xst >> 4) + s),
                                                     (__attribute__((address_space(3))) void*)&ssc[i0], 4, 0, 0);
            }
        }
        if constexpr (XR) {
            // (after the DMA requests and before the prefetch: the barrier's wait below counts the
            // prefetch as the only loads still owed)
#pragma unroll
            for (int n = XL; n < NR; ++n)
#pragma unroll
                for (int t = 0; t < NSTEP; ++t) XS[n - XL][t] = a.xs[(size_t)n * (a.xst >> 4) + t * 64 + lane];
        }
        prefetch();
        if (stopped(a.stop)) return;
        // this wave's LDS DMA writes are complete before the barrier: they are older than the
        // prefetch's 2 NSTEP RPW loads, which stay in flight (vector-memory counts retire in
        // order). A plain barrier plus an acquire fence, because the release half of
        // __syncthreads would wait for the prefetch as well.
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NSTEP * RPW) & ~(15 << 8));   // and the LDS counter
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    } else {
        // activation stage: every load issued before any LDS write (one round trip). When the
        // stage is small its registers coexist with the weight prefetch, which is then requested
        // before the stage is written, so the two round trips overlap.
        constexpr bool EARLY = NSTG <= 5;
        uint4 tv[NSTG];
        float ts[NSTG];
#pragma unroll
        for (int j = 0; j < NSTG; ++j) {
            const int i = threadIdx.x + j * NT;
            const int n = i / SL, s = i - n * SL;
            tv[j] = make_uint4(0u, 0u, 0u, 0u);
            ts[j] = 0.0f;
            if (i < NR * SL && (FULL || s < nslab)) {
                tv[j] = *(const uint4*)(a.xq + (size_t)n * a.xst + 16 * s);
                ts[j] = a.xs[(size_t)n * (a.xst >> 4) + s];
            }
        }
        if constexpr (EARLY) {
            __builtin_amdgcn_sched_barrier(0);
            prefetch();
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < NSTG; ++j) {
            const int i = threadIdx.x + j * NT;
            if (i < NR * SL) { sx[i] = tv[j]; ssc[i] = ts[j]; }
        }
        if constexpr (!EARLY) prefetch();
        if (stopped(a.stop)) return;
    }
    if constexpr (PRE || !FULL) __syncthreads();
    int npend_cv = 0;
    if constexpr (CV) npend_cv = ld_uniform(a.npend_ptr);
    // GDN row scalars (EPI_CONV): wave 0 of blocks b < 2 ab_vh, before its rows. The bf16 GEMV of
    // one in_a / in_b row: chunk c of 8 elements on lane c % 64 in ascending c, fmaf per element,
    // shfl tree, bf16 rounding (k_bf16_gemv2_tile, src/q27_util.hip:114-167); then, lane n for row
    // n, the scalar of src/q27_gdn.hip:206-372.
    if constexpr (CV) {
        if (wave == 0 && bi < 2 * a.ab_vh) {
            const int which = bi & 1, head = bi >> 1;
            const uint16_t* wrow = (which ? a.in_b : a.in_a) + (size_t)head * K;
            constexpr int NC = NSTEP * 2;              // 8-element chunks per lane
            float acc[NR];
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[n] = 0.0f;
#pragma unroll
            for (int c0 = 0; c0 < NC; c0 += 5) {
                uint4 wv4[5];
#pragma unroll
                for (int i = 0; i < 5; ++i)
                    if (c0 + i < NC) wv4[i] = *(const uint4*)(wrow + 8 * (lane + 64 * (c0 + i)));
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    if (c0 + i >= NC) break;
                    const uint4 w = wv4[i];
                    const int cc = lane + 64 * (c0 + i);
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        const uint4 y = *(const uint4*)(sybf + (size_t)n * K + 8 * cc);
                        float v = acc[n];
                        v = __builtin_fmaf(__uint_as_float(w.x << 16), __uint_as_float(y.x << 16), v);
                        v = __builtin_fmaf(__uint_as_float(w.x & 0xFFFF0000u), __uint_as_float(y.x & 0xFFFF0000u), v);
                        v = __builtin_fmaf(__uint_as_float(w.y << 16), __uint_as_float(y.y << 16), v);
                        v = __builtin_fmaf(__uint_as_float(w.y & 0xFFFF0000u), __uint_as_float(y.y & 0xFFFF0000u), v);
                        v = __builtin_fmaf(__uint_as_float(w.z << 16), __uint_as_float(y.z << 16), v);
                        v = __builtin_fmaf(__uint_as_float(w.z & 0xFFFF0000u), __uint_as_float(y.z & 0xFFFF0000u), v);
                        v = __builtin_fmaf(__uint_as_float(w.w << 16), __uint_as_float(y.w << 16), v);
                        v = __builtin_fmaf(__uint_as_float(w.w & 0xFFFF0000u), __uint_as_float(y.w & 0xFFFF0000u), v);
                        acc[n] = v;
                    }
                }
            }
            float mine = 0.0f;
#pragma unroll
            for (int n = 0; n < NR; ++n) {
                const float v = bcast0(tree64(acc[n]));
                if (lane == n) mine = v;
            }
            if (lane < NR) {
                const float v = bfr(mine);
                float r;
                if (which) r = qsigmoid(v);
                else r = qexp(-(qexp(bf2f(a.A_log[head])) * qsoftplus(v + bf2f(a.dt_bias[head]))));
                a.ab_out[(size_t)(which * kMaxRows + lane) * a.ab_vh + head] = r;
            }
        }
    }
    const int vi = lane / LPV;                         // the value this lane holds after the tree
    const bool holder = (lane % LPV) == 0 && vi < V;
    const int hn = (vi < V) ? vi / RPW : NR - 1, hr = (vi < V) ? vi - (vi / RPW) * RPW : 0;
    const uint32_t* resw = (const uint32_t*)a.res;
    // v = silu(g) * u * gscale for output j (rows j and 16 + j of its unit)
    auto swiglu = [&](float gv, float uv) __attribute__((always_inline)) {
        const float swv = gv / (1.0f + qexp(-gv));
        return swv * uv * a.gscale;
    };
    // 16 values in lanes c = lane & 15 -> one per-16 group: exact max, scale, codes
    auto quant16 = [&](float v, int8_t& code, float& sc) __attribute__((always_inline)) {
        const float mx = max_xor(fabsf(v), 16);
        sc = mx * (1.0f / 127.0f);
        const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
        code = qcode(v, inv);
    };
    // The wave that stores the last row of a whole unit quantizes the unit into LDS; the wave that
    // stores the last row of a leftover quarter hands its 4 SwiGLU values to the unit's other
    // blocks (agent-scope stores, then the unit's arrival counter; the fourth arrival quantizes
    // the unit). Quarters come first in the block's list, so their exchange overlaps the streaming.
    auto finish = [&](int j) __attribute__((always_inline)) {
        const int c16 = lane & 15;
        if (j >= 8 * myq) {
            const int k = (j - 8 * myq) >> 5, lr = 8 * myq + 32 * k;
#pragma unroll
            for (int nn = 0; nn < NR; ++nn) {
                int8_t code;
                float sc;
                quant16(swiglu(sacc[(lr + c16) * NR + nn], sacc[(lr + 16 + c16) * NR + nn]), code, sc);
                if (lane < 16) s_code[(k * NR + nn) * 16 + c16] = code;
                if (lane == 0) s_scale[k * NR + nn] = sc;
            }
        } else {
            const int m = j >> 3, p = bi + nb * m, e = p >> 2, q = p & 3, unit = F * nb + e, c = lane & 3;
            float* part = a.sw_part + (size_t)e * 16 * NR;   // [16 outputs][NR]
#pragma unroll
            for (int nn = 0; nn < NR; ++nn) {
                const float v = swiglu(sacc[(8 * m + c) * NR + nn], sacc[(8 * m + 4 + c) * NR + nn]);
                if (lane < 4) st_agent(part + (4 * q + c) * NR + nn, v);
            }
            __builtin_amdgcn_s_waitcnt(0);             // the stores are acknowledged before counting
            unsigned prev = 0u;
            if (lane == 0) prev = add_agent(a.sw_cnt + e, 1u);
            prev = (unsigned)__builtin_amdgcn_readfirstlane((int)prev);
            if (prev == 3u) {                          // the unit's fourth quarter: finish it
#pragma unroll
                for (int nn = 0; nn < NR; ++nn) {
                    int8_t code;
                    float sc;
                    quant16(__hip_atomic_load(part + c16 * NR + nn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), code, sc);
                    if (lane < 16) a.act_q[(size_t)nn * a.act_stride + unit * 16 + c16] = code;
                    if (lane == 0) a.act_s[(size_t)nn * (a.act_stride >> 4) + unit] = sc;
                }
                if (lane == 0) st_agent(a.sw_cnt + e, 0u);
            }
            // nothing of this path left in flight, so the loop's waits stay those of the plain path
            __builtin_amdgcn_s_waitcnt(0);
        }
    };
    // Conv epilogue of channel r0 (k_gdn_conv_tp_tile, src/q27_gdn.hip:411-439): the NR raw values
    // x_n = bf16(v_n) (v_n in lane n * LPV) follow the committed history (the record's history
    // and the first npend pending raw inputs) in one sequence h0 h1 h2 x_0 .. x_{NR-1}; lane n
    // convolves row n's window (the three values before x_n, then x_n: acc = s0 w0 + s1 w1 + s2 w2
    // + x_n w3, an fmaf chain), out = bf16(SiLU(acc)), and stores it; lane 0 rewrites the record
    // (committed history, this call's raw inputs as the new pending ones).
    auto conv_epilogue = [&](float tv, uint32_t cvd, int r0, int ln) __attribute__((always_inline)) {
        uint32_t dw[10];
#pragma unroll
        for (int i = 0; i < 10; ++i) dw[i] = (uint32_t)__builtin_amdgcn_readlane((int)cvd, i);
        uint32_t h0 = dw[0] & 0xFFFFu, h1 = dw[0] >> 16, h2 = dw[1] & 0xFFFFu;
#pragma unroll
        for (int p = 0; p < kMaxRows; ++p)
            if (p < npend_cv) { h0 = h1; h1 = h2; h2 = (dw[2 + (p >> 1)] >> (16 * (p & 1))) & 0xFFFFu; }
        uint32_t seq[NR + 3];
        seq[0] = h0; seq[1] = h1; seq[2] = h2;
#pragma unroll
        for (int n = 0; n < NR; ++n) seq[3 + n] = f2bf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(tv), n * LPV)));
        uint32_t s0 = seq[0], s1 = seq[1], s2 = seq[2], s3 = seq[3];
#pragma unroll
        for (int m = 1; m < NR; ++m)
            if (ln == m) { s0 = seq[m]; s1 = seq[m + 1]; s2 = seq[m + 2]; s3 = seq[m + 3]; }
        const float w0 = __uint_as_float(dw[8] << 16), w1 = __uint_as_float(dw[8] & 0xFFFF0000u);
        const float w2 = __uint_as_float(dw[9] << 16), w3 = __uint_as_float(dw[9] & 0xFFFF0000u);
        float cacc = __uint_as_float(s0 << 16) * w0;
        cacc = __builtin_fmaf(__uint_as_float(s1 << 16), w1, cacc);
        cacc = __builtin_fmaf(__uint_as_float(s2 << 16), w2, cacc);
        cacc = __builtin_fmaf(__uint_as_float(s3 << 16), w3, cacc);
        if (ln < NR) ((uint16_t*)a.y)[(size_t)ln * a.ystride + r0] = f2bf(qsilu(cacc));
        if (ln == 0) {
            uint32_t rec[8] = { h0 | (h1 << 16), h2, 0u, 0u, 0u, 0u, 0u, 0u };
#pragma unroll
            for (int n = 0; n < NR; ++n) rec[2 + (n >> 1)] |= seq[3 + n] << (16 * (n & 1));
            uint4* d = (uint4*)(a.conv_st + (size_t)r0 * 16);
            d[0] = make_uint4(rec[0], rec[1], rec[2], rec[3]);
            d[1] = make_uint4(rec[4], rec[5], rec[6], rec[7]);
        }
    };
    // the row group's epilogue: store (+ residual, conv) or SwiGLU accumulation
    auto emit = [&](int j, float tv, uint32_t rw, size_t ridx, uint32_t cvd) __attribute__((always_inline)) {
        bool conv_row = false;
        if constexpr (CV) {
            const int r0 = row_of(j, 0);                 // wave-uniform: one row per group
            if (r0 < a.nconv) {
                conv_row = true;
                conv_epilogue(tv, cvd, r0, lane);
            }
        }
        if constexpr (ST) {
            const int row = row_of(j, hr);
            if (!conv_row && holder && row < a.rows) {
                float v = tv;
                if (resw) {
                    const float rv = a.res_bf16 ? bf2f((uint16_t)((ridx & 1) ? (rw >> 16) : (rw & 0xFFFFu)))
                                                : __uint_as_float(rw);
                    if (a.res_round) v = bfr(v);
                    v = v + a.rs * rv;
                }
                const size_t yi = (size_t)hn * a.ystride + row;
                if (a.out_bf16) ((uint16_t*)a.y)[yi] = f2bf(v);
                else ((float*)a.y)[yi] = v;
            }
        } else {
            if (holder) sacc[j * NR + hn] = tv;
            // (LDS operations of a wave complete in order: the row's values are in LDS before
            // its count, and a wave that reads the count as complete reads them after it)
            const bool isq = j < 8 * myq;
            unsigned prev = 0u;
            if (lane == 0)
                prev = __hip_atomic_fetch_add(&s_gcnt[isq ? (j >> 3) : myq + ((j - 8 * myq) >> 5)], 1u,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            prev = (unsigned)__builtin_amdgcn_readfirstlane((int)prev);
            if (prev == (isq ? 7u : 31u)) {
                asm volatile("" ::: "memory");
                finish(j);
            }
        }
    };
    // the per-output scale of the group's row (one weight row per group), selected from the
    // group's first row, which the loop carries from one group to the next
    int rg_cur = __builtin_amdgcn_readfirstlane(row_of(wave, 0));
    for (int j = wave; j < nrb;) {
        float al = a.alpha;
        if constexpr (RPW == 1) al = alpha_of(a.alpha, a.asel, rg_cur);
        unsigned jn = 0u;
        if (lane == 0) jn = __hip_atomic_fetch_add(&s_next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int jnext = NW + __builtin_amdgcn_readfirstlane((int)jn);
        const bool more = valid(jnext);
        const int rg_next = __builtin_amdgcn_readfirstlane(row_of(jnext, 0));
        // residual: one raw dword per lane (bf16 pairs or fp32), decoded at the use; loaded
        // (from a harmless address) also when there is none, for the reason given at ld
        size_t ridx = 0;
        uint32_t rw = 0u;
        if constexpr (ST) {
            int row = row_of(j, hr);
            row = row < a.rows ? row : a.rows - 1;
            ridx = (size_t)hn * a.rstride + row;
            rw = *(resw ? resw + (a.res_bf16 ? (ridx >> 1) : ridx) : (const uint32_t*)a.W);
        }
        // conv channel: its record (8 dwords) and its 4 tap weights (2 dwords), one dword in each
        // of lanes 0..9, requested with the residual word
        uint32_t cvd = 0u;
        if constexpr (CV) {
            const int r0 = row_of(j, 0);
            const int rc = r0 < a.nconv ? r0 : 0;
            const uint32_t* rec = (const uint32_t*)a.conv_st + (size_t)rc * 8;
            const uint32_t* cw = (const uint32_t*)a.conv_w + (size_t)rc * 2;
            cvd = *((lane < 8) ? rec + lane : (lane < 10) ? cw + (lane - 8) : rec);
        }
        __builtin_amdgcn_sched_barrier(0);
        float acc[P];
#pragma unroll
        for (int v = 0; v < P; ++v) acc[v] = 0.0f;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            const int s = t * 64 + lane;
            // XB: the step's code and scale reads, requested together ahead of its arithmetic
            uint4 xb[XB ? NR : 1];
            float sb[XB ? XL : 1];
            if constexpr (XB) {
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    xb[n] = sx[n * SL + s];
                    if (n < XL) sb[n < XL ? n : 0] = ssc[n * SL + s];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int n = 0; n < NR; ++n) {
                const uint4 xa = XB ? xb[XB ? n : 0] : sx[n * SL + s];
                float sa;
                if (n >= XL) sa = XS[n >= XL ? n - XL : 0][t];
                else sa = XB ? sb[XB && n < XL ? n : 0] : ssc[n * SL + s];
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const int d = dot16(W[r][t], xa);
                    acc[n * RPW + r] = __builtin_fmaf((float)d, S[r][t] * sa, acc[n * RPW + r]);
                }
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) ld(rg_next, r, t, more);
        }
        const float tv = tree_t<P>(acc, lane) * al;
        emit(j, tv, rw, ridx, cvd);
        j = jnext;
        rg_cur = rg_next;
    }
    if constexpr (EPI == EPI_SWIGLU) {
        // the whole units' codes and scales, quantized in the loop, written out together
        __syncthreads();
        for (int i = threadIdx.x; i < F * NR * 16; i += NT) {
            const int k = i / (NR * 16), nn = (i / 16) % NR, c = i & 15;
            a.act_q[(size_t)nn * a.act_stride + (bi + nb * k) * 16 + c] = s_code[i];
            if (c == 0) a.act_s[(size_t)nn * (a.act_stride >> 4) + bi + nb * k] = s_scale[k * NR + nn];
        }
    }
}

static int g_ncu = 0;
static int num_cus() {
    if (!g_ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 256;
        g_ncu = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    }
    return g_ncu;
}

// Launch shape. The norm-prologue, SwiGLU and aligned K <= 6144 kernels run one 16-wave block per
// CU (the prologue is then computed once per CU; a block's waves share one row list). K = 17408
// (a 17 KiB-per-row prefetch in ~190 VGPRs) and the unaligned shapes run 4-wave blocks, wpc
// waves per CU (8 for K = 17408, 16 otherwise): for K = 17408 one 8-wave block per CU measured
// slower. Overridable for launch-shape sweeps (Q27X_WPC5, Q27X_WPC17).
static int env_knob(const char* name, int def, int lo, int hi) {
    const char* v = getenv(name);
    if (!v || !*v) return def;
    const int x = atoi(v);
    return (x < lo) ? lo : (x > hi ? hi : x);
}
static int knob_wpc5() { static const int v = env_knob("Q27X_WPC5", 16, 4, 32); return v; }
static int knob_wpc17() { static const int v = env_knob("Q27X_WPC17", 8, 4, 16); return v; }

template <int NR, int NSTEP, int EPI, bool FULL, bool PRE, int RPW>
static int run_proj_rpw(const ProjArgs& a, hipStream_t s) {
    // K = 17408: 4-wave blocks (two per CU up to 3 rows, one from 4 rows on, where the stage fills
    // the LDS), and one 8-wave block per CU (two waves per SIMD) at 7 and 8 rows. Measured per row
    // count (down, 5120 x 17408, 4 -> 8 waves): 23.9 -> 22.9 us at 7 rows and 27.0 -> 25.0 us at
    // 8, but slower at 4-6 rows (19.1 -> 19.6, 19.7 -> 20.5, 20.0 -> 21.6 us).
    constexpr int NW = (PRE || EPI == EPI_SWIGLU || (FULL && NSTEP < 17)) ? 16 : (NSTEP >= 17 && NR >= 7) ? 8 : 4;
    int grid;
    if (EPI == EPI_SWIGLU) {
        const int nunits = a.rows >> 5;
        grid = nunits < num_cus() ? nunits : num_cus();
        const int F = nunits / grid, E = nunits - F * grid;
        if (32 * F + 8 * ((4 * E + grid - 1) / grid) > kSwRows || E > kSwMaxSplit || (E && (!a.sw_part || !a.sw_cnt))) {
            set_error("proj: SwiGLU shape rows=%d over %d blocks needs %s", a.rows, grid,
                      (E && (!a.sw_part || !a.sw_cnt)) ? "the split-unit scratch" : "more LDS than it has");
            return Q27X_E_SHAPE;
        }
    } else if (NW == 16) {
        const int ngroups = (a.rows + RPW - 1) / RPW;
        const int nb = (ngroups + NW - 1) / NW;
        grid = nb < num_cus() ? nb : num_cus();
    } else {
        const int ngroups = (a.rows + RPW - 1) / RPW;
        int wpc = (NSTEP >= 17) ? knob_wpc17() : knob_wpc5();
        // no more waves per CU than the blocks whose LDS stages fit (160 KB per CU)
        constexpr int kStage = StageFit<NR, NSTEP>::kBytes;
        constexpr int kBpc = (160 * 1024) / kStage > 0 ? (160 * 1024) / kStage : 1;
        if (wpc > kBpc * NW) wpc = kBpc * NW;
        const int wmax = num_cus() * wpc;
        const int nwv = ngroups < wmax ? ngroups : wmax;
        grid = (nwv + NW - 1) / NW;
    }
    if (EPI == EPI_CONV && a.ab_vh && grid < 2 * a.ab_vh) {
        set_error("proj: %d blocks cannot hold the %d GDN row-scalar rows", grid, 2 * a.ab_vh);
        return Q27X_E_SHAPE;
    }
    hipLaunchKernelGGL((k_proj<NR, NSTEP, RPW, EPI, FULL, PRE, NW>), dim3(grid), dim3(NW * 64), 0, s, a);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
// One weight row per wave step: two rows per step (more bytes in flight per wave) measured slower
// on MI355X for every shape here, with and without the prologue.
template <int NR, int NSTEP, int EPI, bool FULL, bool PRE>
static int run_proj(const ProjArgs& a, hipStream_t s) {
    return run_proj_rpw<NR, NSTEP, EPI, FULL, PRE, 1>(a, s);
}

// Shape router. NSTEP = ceil(K/1024); the LDS stage is NR*NSTEP*1280 B, except K = 17408 at NR > 4
// (174 KB at NR = 8), whose scales are held in registers (NR*NSTEP*1024 B). The norm prologue (PRE)
// exists for the hidden sizes K = 1024 and 5120, the inputs of the layers' first projections.
template <int NR, int EPI, bool FULL>
static int route_k(const ProjArgs& a, hipStream_t s) {
    const int ns = (a.K + 1023) / 1024;
    if (a.has_pre) {
        if constexpr (FULL) {
            if (ns == 1) return run_proj<NR, 1, EPI, true, true>(a, s);
            if (ns == 5) return run_proj<NR, 5, EPI, true, true>(a, s);
        }
        return -2;
    }
    if constexpr (EPI == EPI_SWIGLU) {
        if (ns == 1) return run_proj<NR, 1, EPI, FULL, false>(a, s);
        if (ns == 5) return run_proj<NR, 5, EPI, FULL, false>(a, s);
        return -2;
    } else if constexpr (EPI == EPI_CONV) {
        return -2;                                     // prologue kernels only
    } else {
        switch (ns) {
            case 1: return run_proj<NR, 1, EPI, FULL, false>(a, s);
            case 2: return run_proj<NR, 2, EPI, FULL, false>(a, s);
            case 4: return run_proj<NR, 4, EPI, FULL, false>(a, s);
            case 5: return run_proj<NR, 5, EPI, FULL, false>(a, s);
            case 6: return run_proj<NR, 6, EPI, FULL, false>(a, s);
            case 17:
                if constexpr (FULL && EPI == EPI_STORE) return run_proj<NR, 17, EPI, FULL, false>(a, s);
                return -2;
            default: return -2;
        }
    }
}

template <int EPI, bool FULL>
static int route_nr(const ProjArgs& a, int nr, hipStream_t s) {
    switch (nr) {
        case 1: return route_k<1, EPI, FULL>(a, s);
        case 2: return route_k<2, EPI, FULL>(a, s);
        case 3: return route_k<3, EPI, FULL>(a, s);
        case 4: return route_k<4, EPI, FULL>(a, s);
        case 5: return route_k<5, EPI, FULL>(a, s);
        case 6: return route_k<6, EPI, FULL>(a, s);
        case 7: return route_k<7, EPI, FULL>(a, s);
        case 8: return route_k<8, EPI, FULL>(a, s);
        default: return -2;
    }
}

static int route(const ProjArgs& a, int epi, int nr, hipStream_t s) {
    const bool full = (a.K & 1023) == 0;
    if (epi == EPI_SWIGLU) return full ? route_nr<EPI_SWIGLU, true>(a, nr, s) : -2;   // K = 1024 k only
    if (epi == EPI_CONV) return (full && a.has_pre) ? route_nr<EPI_CONV, true>(a, nr, s) : -2;   // the GDN input
    return full ? route_nr<EPI_STORE, true>(a, nr, s) : route_nr<EPI_STORE, false>(a, nr, s);
}

bool proj_k_supported(int K) {
    if (K < 64 || (K & 63)) return false;
    const int ns = (K + 1023) / 1024;
    return ns == 1 || ns == 2 || ns == 4 || ns == 5 || ns == 6 || (ns == 17 && (K & 1023) == 0);
}

int launch_proj(const ProjArgs& a, int epi, int nr, hipStream_t s) {
    if (!a.W || !a.WS || a.rows < 1 || a.K < 64 || (a.K & 63) || nr < 1 || nr > kMaxRows) {
        set_error("proj: bad arguments (rows=%d K=%d nr=%d)", a.rows, a.K, nr);
        return Q27X_E_ARG;
    }
    if (a.has_pre) {
        const NormArgs& n = a.pre;
        if (n.n != a.K || !(a.K == 1024 || a.K == 5120) || !n.w || (!n.x && !(n.emb && n.tok)) || n.hout ||
            n.hadd || n.row_sel || (!n.x_bf16 && !n.emb && (n.xstride & 3)) || (n.xstride & 3) ||
            (n.xq && !n.xs) || (n.y && (n.ystride & 3))) {
            set_error("proj: unsupported norm prologue (n=%d K=%d)", n.n, a.K);
            return Q27X_E_SHAPE;
        }
    } else {
        if (!a.xq || !a.xs) { set_error("proj: no activations"); return Q27X_E_ARG; }
        if ((a.xst & 15) || a.xst < a.K) { set_error("proj: activation stride %d must be >= K and a multiple of 16", a.xst); return Q27X_E_ARG; }
    }
    if (a.res && ((size_t)a.res & 3)) { set_error("proj: residual must be 4-byte aligned"); return Q27X_E_ARG; }
    if (epi == EPI_SWIGLU && (a.rows & 31)) { set_error("proj: SwiGLU rows %d not a multiple of 32", a.rows); return Q27X_E_SHAPE; }
    if (epi == EPI_CONV && (!a.conv_w || !a.conv_st || !a.npend_ptr || a.nconv < 0 || a.nconv > a.rows || !a.out_bf16 ||
                            a.res || ((size_t)a.conv_w & 7) || ((size_t)a.conv_st & 15))) {
        set_error("proj: conv epilogue needs conv_w, conv_st, npend, bf16 out and no residual");
        return Q27X_E_ARG;
    }
    if (epi == EPI_CONV && a.ab_vh && (!a.in_a || !a.in_b || !a.A_log || !a.dt_bias || !a.ab_out || a.ab_vh > 128 ||
                                       ((size_t)a.in_a & 15) || ((size_t)a.in_b & 15))) {
        set_error("proj: GDN row scalars need in_a, in_b, A_log, dt_bias and ab_out (ab_vh <= 128)");
        return Q27X_E_ARG;
    }
    const int rc = route(a, epi, nr, s);
    if (rc == -2) { set_error("proj: no kernel for K=%d nr=%d epi=%d", a.K, nr, epi); return Q27X_E_SHAPE; }
    return rc;
}

// ---------------------------------------------------------------- the MTP layer's down, one launch
// The reference projects the MTP layer's down in four column slices of K/4 and adds each slice's
// fp32 result into the bf16 residual with its own bf16 rounding, slice after slice
// (src/q27_main.cpp:2605-2612). Four slice launches of the projection above do exactly that; this
// kernel gives the same bits in one launch for up to 4 rows. A wave takes the units (row r,
// slice j) of its rows in order: the unit's dot products in the lane-slab order (slab s on lane
// s % 64 at step s / 64, acc = fmaf((float)d, ws64 * xs16, acc)), the slice's own shfl_down tree,
// and after the fourth slice the four additions in slice order, each rounded to bf16. Units
// alternate between two weight register sets: a unit's set is refilled with the unit two ahead
// once its products have issued, so the next unit's bytes are in flight while one computes. The
// rows' codes and scales for the whole K are staged in LDS once per block.
constexpr int kD4Waves = 8;
template <int NR, int NS>
__global__ __launch_bounds__(kD4Waves * 64) void k_down4(Down4Args a) {
    constexpr int SLS = NS * 64;                       // staged slabs per slice and row
    constexpr int NT = kD4Waves * 64;
    constexpr int P = Pow2<NR>::value, LPV = 64 / P;
    __shared__ uint4 sx[NR * 4 * SLS];
    __shared__ float ssc[NR * 4 * SLS];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K4 = a.K4, nsl = K4 >> 4, ng = K4 >> 6;
    const int nw = gridDim.x * kD4Waves;
    uint4 W[2][NS];
    float S[2][NS];
    // unit (row, slice j) into set b: loads issued on every path (a unit past the wave's last reads
    // the last row, not used). A lane past the slice's slabs reads the row's first slab and scale:
    // its staged activation slab and scale are zero, so its product is dot 0 times scale 0 and
    // fmaf(0, 0, acc) leaves acc's bits as they are (acc starts at +0 and +0 + -0 is +0). No select
    // on the loaded values, which would wait for the loads where the select stands.
    auto ld = [&](int b, int row, int j) __attribute__((always_inline)) {
        row = row < a.rows ? row : a.rows - 1;
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int sl = t * 64 + lane;
            const int sc = sl < nsl ? sl : 0;
            W[b][t] = ld_nt16(a.W[j] + (size_t)row * K4 + 16 * sc);
            S[b][t] = a.WS[j][(size_t)row * ng + (sc >> 2)];
        }
    };
    // one unit from set b: its products, the set refilled with unit (rq, jq), the slice's tree
    auto unit = [&](int b, int j, int rq, int jq) __attribute__((always_inline)) -> float {
        // an opaque copy of the lane's slab index: the unit's LDS reads stay in the unit (they
        // do not depend on the row, and hoisted out of the row loop they would hold every slice's
        // activations in registers)
        int sl0 = lane;
        asm volatile("" : "+v"(sl0));
        float acc[P];
#pragma unroll
        for (int v = 0; v < P; ++v) acc[v] = 0.0f;
#pragma unroll
        for (int t = 0; t < NS; ++t) {
#pragma unroll
            for (int n = 0; n < NR; ++n) {
                const int si = (n * 4 + j) * SLS + t * 64 + sl0;
                const int d = dot16(W[b][t], sx[si]);
                acc[n] = __builtin_fmaf((float)d, S[b][t] * ssc[si], acc[n]);
            }
        }
        ld(b, rq, jq);
        return tree_t<P>(acc, lane) * a.alpha[j];
    };
    // stage: slice j's slab s of row n at (n * 4 + j) * SLS + s; slabs past the slice are zero
    for (int i = threadIdx.x; i < NR * 4 * SLS; i += NT) {
        const int nj = i / SLS, sb = i - nj * SLS, n = nj >> 2, j = nj & 3;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        float sc = 0.0f;
        if (sb < nsl) {
            v = *(const uint4*)(a.xq + (size_t)n * a.xst + (size_t)j * K4 + 16 * sb);
            sc = a.xs[(size_t)n * (a.xst >> 4) + (size_t)j * nsl + sb];
        }
        sx[i] = v;
        ssc[i] = sc;
    }
    int r = blockIdx.x * kD4Waves + wave;              // this wave's rows: r, r + nw, ...
    // set 0's loads all issue before set 1's, as in the loop (the wait counts at the loop's top
    // hold for both ways in)
    ld(0, r, 0);
    __builtin_amdgcn_sched_barrier(0);
    ld(1, r, 1);
    if (stopped(a.stop)) return;
    __syncthreads();
    // lane n LPV holds row n's four slice results after the trees
    const bool holder = (lane % LPV) == 0 && lane / LPV < NR;
    for (; r < a.rows; r += nw) {
        // the residual is read before the units' loads are issued (loads retire in order, and a
        // read issued after them would wait for all of them), by every lane (lanes that hold no
        // value read row 0's), so that no select or branch waits for it here
        uint16_t* yp = a.y + (size_t)(holder ? lane / LPV : 0) * a.ystride + r;
        uint16_t y = *yp;
        const float d0 = unit(0, 0, r, 2);
        const float d1 = unit(1, 1, r, 3);
        const float d2 = unit(0, 2, r + nw, 0);
        const float d3 = unit(1, 3, r + nw, 1);
        // add them into the residual in slice order
        if (holder) {
            y = f2bf(d0 + 1.0f * bf2f(y));
            y = f2bf(d1 + 1.0f * bf2f(y));
            y = f2bf(d2 + 1.0f * bf2f(y));
            y = f2bf(d3 + 1.0f * bf2f(y));
            *yp = y;
        }
    }
}
// instances: K/4 up to 2048 (the small test geometries) and 4097 .. 5120 (the model's 4352)
bool down4_supported(int K4, int nr) {
    const int ns = (K4 + 1023) / 1024;
    return nr >= 1 && nr <= 4 && K4 >= 64 && (K4 & 63) == 0 && (ns == 1 || ns == 2 || ns == 5);
}
int launch_down4(const Down4Args& a, int nr, hipStream_t s) {
    if (!down4_supported(a.K4, nr) || a.rows < 1 || !a.xq || !a.xs || !a.y ||
        (a.xst & 15) || a.xst < 4 * a.K4 || !a.W[0] || !a.W[1] || !a.W[2] || !a.W[3] || !a.WS[0] || !a.WS[1] ||
        !a.WS[2] || !a.WS[3]) {
        set_error("down4: no kernel for rows=%d K/4=%d nr=%d", a.rows, a.K4, nr);
        return Q27X_E_SHAPE;
    }
    const int grid = num_cus(), ns = (a.K4 + 1023) / 1024;
    auto go = [&](auto nsc) {
        constexpr int NS = decltype(nsc)::value;
        switch (nr) {
            case 1: hipLaunchKernelGGL((k_down4<1, NS>), dim3(grid), dim3(kD4Waves * 64), 0, s, a); break;
            case 2: hipLaunchKernelGGL((k_down4<2, NS>), dim3(grid), dim3(kD4Waves * 64), 0, s, a); break;
            case 3: hipLaunchKernelGGL((k_down4<3, NS>), dim3(grid), dim3(kD4Waves * 64), 0, s, a); break;
            default: hipLaunchKernelGGL((k_down4<4, NS>), dim3(grid), dim3(kD4Waves * 64), 0, s, a); break;
        }
    };
    if (ns == 1) go(std::integral_constant<int, 1>{});
    else if (ns == 2) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 5>{});
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// ---------------------------------------------------------------- int32 slab partials
__global__ __launch_bounds__(256) void k_proj_partials(const int8_t* __restrict__ W, int rows, int K,
                                                       const int8_t* __restrict__ xq, int xst,
                                                       int32_t* __restrict__ part, int nr) {
    const int nslab = K >> 4;
    const long long total = (long long)nr * rows * nslab;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int s = (int)(i % nslab);
        const long long rn = i / nslab;
        const int r = (int)(rn % rows), n = (int)(rn / rows);
        const uint4 w = *(const uint4*)(W + (size_t)r * K + 16 * s);
        const uint4 x = *(const uint4*)(xq + (size_t)n * xst + 16 * s);
        part[i] = dot16(w, x);
    }
}

// ---------------------------------------------------------------- bf16 GEMV
// Chunk c of 8 bf16 (16 B) belongs to lane c%64 at step c/64; fmaf per element in order; shfl
// tree. Activations staged as fp32 in LDS. MODE 1 keeps a running (value, index) argmax per row
// (non-finite filtered, ties to the lowest index: src/q27_elem.hip:226-236) and writes one
// partial per block.
__device__ __forceinline__ void am_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
    const bool take = (v > bv) || (v == bv && i < bi);
    bv = take ? v : bv;
    bi = take ? i : bi;
}
__device__ __forceinline__ bool finitef(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

template <int NR, int NSTEP, int RPW, int MODE>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a, int upw) {
    constexpr int CH = NSTEP * 64;
    __shared__ float sxf[NR * CH * 8];
    if (stopped(a.stop)) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, nch = K >> 3;
    const int ngroups = (a.rows + RPW - 1) / RPW;
    const int gw = blockIdx.x * 4 + wave;
    const int g0 = gw * upw, g1 = (g0 + upw < ngroups) ? g0 + upw : ngroups;
    uint4 wv[RPW][NSTEP];
    auto load = [&](int g, uint4 (&W_)[RPW][NSTEP]) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            int row = g * RPW + r;
            row = row < a.rows ? row : a.rows - 1;
            const uint16_t* wp = a.W + (size_t)row * K;
#pragma unroll
            for (int t = 0; t < NSTEP; ++t) {
                const int c = t * 64 + lane;
                W_[r][t] = (c < nch) ? ld_nt16(wp + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };
    if (g0 < g1) load(g0, wv);
    for (int i = threadIdx.x; i < NR * CH * 8; i += 256) {
        const int n = i / (CH * 8), k = i - n * (CH * 8);
        sxf[i] = (k < K) ? bf2f(a.x[(size_t)n * a.xst + k]) : 0.0f;
    }
    __syncthreads();
    float bv = -__builtin_huge_valf();                  // MODE 1: lane n < NR keeps row n's best
    uint32_t bi = 0xFFFFFFFFu;
    for (int g = g0; g < g1; ++g) {
        uint4 wn[RPW][NSTEP];
        if (g + 1 < g1) load(g + 1, wn);
        float acc[RPW][NR];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = 0.0f;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            const int c = t * 64 + lane;
            if (c < nch) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const uint4 w = wv[r][t];
                    float wf[8];
                    wf[0] = __uint_as_float(w.x << 16); wf[1] = __uint_as_float(w.x & 0xFFFF0000u);
                    wf[2] = __uint_as_float(w.y << 16); wf[3] = __uint_as_float(w.y & 0xFFFF0000u);
                    wf[4] = __uint_as_float(w.z << 16); wf[5] = __uint_as_float(w.z & 0xFFFF0000u);
                    wf[6] = __uint_as_float(w.w << 16); wf[7] = __uint_as_float(w.w & 0xFFFF0000u);
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        const float4 x0 = *(const float4*)&sxf[n * CH * 8 + 8 * c];
                        const float4 x1 = *(const float4*)&sxf[n * CH * 8 + 8 * c + 4];
                        float v = acc[r][n];
                        v = __builtin_fmaf(wf[0], x0.x, v); v = __builtin_fmaf(wf[1], x0.y, v);
                        v = __builtin_fmaf(wf[2], x0.z, v); v = __builtin_fmaf(wf[3], x0.w, v);
                        v = __builtin_fmaf(wf[4], x1.x, v); v = __builtin_fmaf(wf[5], x1.y, v);
                        v = __builtin_fmaf(wf[6], x1.z, v); v = __builtin_fmaf(wf[7], x1.w, v);
                        acc[r][n] = v;
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = bcast0(tree64(acc[r][n]));
        const int row0 = g * RPW;
        if (MODE == 0) {
            if (lane < RPW * NR) {
                const int r = lane % RPW, n = lane / RPW, row = row0 + r;
                float v = 0.0f;
#pragma unroll
                for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
                    for (int nn = 0; nn < NR; ++nn) if (rr == r && nn == n) v = acc[rr][nn];
                if (row < a.rows) {
                    if (a.out_bf16) ((uint16_t*)a.y)[(size_t)n * a.ystride + row] = f2bf(v);
                    else ((float*)a.y)[(size_t)n * a.ystride + row] = v;
                }
            }
        } else if (lane < NR) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int row = row0 + r;
                float v = 0.0f;
#pragma unroll
                for (int nn = 0; nn < NR; ++nn) if (nn == lane) v = acc[r][nn];
                if (row < a.rows && finitef(v)) am_merge(bv, bi, v, (uint32_t)row);
            }
        }
        if (g + 1 < g1) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int t = 0; t < NSTEP; ++t) wv[r][t] = wn[r][t];
        }
    }
    if (MODE == 1 && lane < NR) {
        a.pval[(size_t)lane * a.pstride + gw] = bv;
        a.pidx[(size_t)lane * a.pstride + gw] = bi;
    }
}

// Aligned form (K = NSTEP * 512, 16-byte aligned activation rows): one 16-wave block per CU.
// Block b owns the row groups b + i * gridDim.x; wave w starts with group w and then takes the
// next unclaimed group from an LDS counter, so the block's waves finish together. Each step's
// weights are refilled with the next group's right after they are used (one group in flight per
// wave, no register copies). The activation rows are staged as fp32 with 16-byte loads issued
// before the first group's weights. Same per-row arithmetic as k_gemv, so the same bits. MODE 1
// merges the waves' running argmax in LDS and writes one partial per block.
// More than 4 rows: rows 0..3 are staged as fp32 and rows 4.. as bf16 (widened at the read, which
// is exact), so 8 rows of K = 5120 fit in 120 KB and the LDS reads stay below the VALU time.
template <int NR, int NSTEP, int RPW, int MODE>
__global__ __launch_bounds__(1024) void k_gemv_full(GemvArgs a) {
    constexpr int NW = 16, NT = NW * 64, CH = NSTEP * 64, NCK = NR * CH, SI = (NCK + NT - 1) / NT;
    constexpr int NF = NR < 4 ? NR : 4;                // fp32-staged rows
    __shared__ float sxf[NF * CH * 8];
    __shared__ __attribute__((aligned(16))) uint16_t sxb[(NR > NF ? NR - NF : 1) * CH * 8];
    __shared__ unsigned s_next;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K;
    const int ngroups = (a.rows + RPW - 1) / RPW;
    const int nb = gridDim.x, bi = blockIdx.x;
    const int nrb = (ngroups - bi + nb - 1) / nb;      // this block's groups (the launch has nb <= ngroups)
    if (threadIdx.x == 0) s_next = 0u;
    uint4 W[RPW][NSTEP];
    // a group past the block's last reads the first 16 bytes of the weights instead (branch-free,
    // so each wait the compiler places counts only the loads owed to later steps)
    auto ld = [&](int rg, int r, int t, bool ok) __attribute__((always_inline)) {
        int row = rg + r;
        row = row < a.rows ? row : a.rows - 1;
        W[r][t] = ld_nt16(ok ? a.W + (size_t)row * K + 8 * (t * 64 + lane) : a.W);
    };
    // activation rows first, then the first group's weights: waiting for the rows leaves the
    // weights in flight
    uint4 xv[SI];
#pragma unroll
    for (int u = 0; u < SI; ++u) {
        const int i = threadIdx.x + u * NT;
        const int n = i / CH, c = i - n * CH;
        xv[u] = *(const uint4*)((i < NCK) ? a.x + (size_t)n * a.xst + 8 * c : a.x);
    }
    {
        const int rg = __builtin_amdgcn_readfirstlane((bi + wave * nb) * RPW);
#pragma unroll
        for (int t = 0; t < NSTEP; ++t)
#pragma unroll
            for (int r = 0; r < RPW; ++r) ld(rg, r, t, wave < nrb);
    }
    if (stopped(a.stop)) return;
#pragma unroll
    for (int u = 0; u < SI; ++u) {
        const int i = threadIdx.x + u * NT;
        if (i < NCK) {
            const int n = i / CH, c = i - n * CH;
            const uint4 v = xv[u];
            if (n < NF) {
                float* d = &sxf[n * CH * 8 + 8 * c];
                *(float4*)d = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                                          __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
                *(float4*)(d + 4) = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u),
                                                __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xFFFF0000u));
            } else {
                *(uint4*)&sxb[(n - NF) * CH * 8 + 8 * c] = v;
            }
        }
    }
    __syncthreads();
    float bv = -__builtin_huge_valf();                 // MODE 1: lane n < NR keeps row n's best
    uint32_t bx = 0xFFFFFFFFu;
    for (int j = wave; j < nrb;) {
        unsigned jn = 0u;
        if (lane == 0) jn = __hip_atomic_fetch_add(&s_next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int jnext = NW + __builtin_amdgcn_readfirstlane((int)jn);
        const bool more = jnext < nrb;
        const int rg_next = __builtin_amdgcn_readfirstlane((bi + jnext * nb) * RPW);
        float acc[RPW][NR];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = 0.0f;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            const int c = t * 64 + lane;
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const uint4 w = W[r][t];
                float wf[8];
                wf[0] = __uint_as_float(w.x << 16); wf[1] = __uint_as_float(w.x & 0xFFFF0000u);
                wf[2] = __uint_as_float(w.y << 16); wf[3] = __uint_as_float(w.y & 0xFFFF0000u);
                wf[4] = __uint_as_float(w.z << 16); wf[5] = __uint_as_float(w.z & 0xFFFF0000u);
                wf[6] = __uint_as_float(w.w << 16); wf[7] = __uint_as_float(w.w & 0xFFFF0000u);
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    float4 x0, x1;
                    if (n < NF) {
                        x0 = *(const float4*)&sxf[n * CH * 8 + 8 * c];
                        x1 = *(const float4*)&sxf[n * CH * 8 + 8 * c + 4];
                    } else {
                        const uint4 b = *(const uint4*)&sxb[(n - NF) * CH * 8 + 8 * c];
                        x0 = make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xFFFF0000u),
                                         __uint_as_float(b.y << 16), __uint_as_float(b.y & 0xFFFF0000u));
                        x1 = make_float4(__uint_as_float(b.z << 16), __uint_as_float(b.z & 0xFFFF0000u),
                                         __uint_as_float(b.w << 16), __uint_as_float(b.w & 0xFFFF0000u));
                    }
                    float v = acc[r][n];
                    v = __builtin_fmaf(wf[0], x0.x, v); v = __builtin_fmaf(wf[1], x0.y, v);
                    v = __builtin_fmaf(wf[2], x0.z, v); v = __builtin_fmaf(wf[3], x0.w, v);
                    v = __builtin_fmaf(wf[4], x1.x, v); v = __builtin_fmaf(wf[5], x1.y, v);
                    v = __builtin_fmaf(wf[6], x1.z, v); v = __builtin_fmaf(wf[7], x1.w, v);
                    acc[r][n] = v;
                }
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) ld(rg_next, r, t, more);
            __builtin_amdgcn_sched_barrier(0);          // keeps each step's activation reads in the step
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = bcast0(tree64(acc[r][n]));
        const int row0 = (bi + j * nb) * RPW;
        if (MODE == 0) {
            if (lane < RPW * NR) {
                const int r = lane % RPW, n = lane / RPW, row = row0 + r;
                float v = 0.0f;
#pragma unroll
                for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
                    for (int nn = 0; nn < NR; ++nn) if (rr == r && nn == n) v = acc[rr][nn];
                if (row < a.rows) {
                    if (a.out_bf16) ((uint16_t*)a.y)[(size_t)n * a.ystride + row] = f2bf(v);
                    else ((float*)a.y)[(size_t)n * a.ystride + row] = v;
                }
            }
        } else if (lane < NR) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int row = row0 + r;
                float v = 0.0f;
#pragma unroll
                for (int nn = 0; nn < NR; ++nn) if (nn == lane) v = acc[r][nn];
                if (row < a.rows && finitef(v)) am_merge(bv, bx, v, (uint32_t)row);
            }
        }
        j = jnext;
    }
    if constexpr (MODE == 1) {                         // one partial per block and row
        __shared__ float sbv[NW][NR];
        __shared__ uint32_t sbx[NW][NR];
        if (lane < NR) { sbv[wave][lane] = bv; sbx[wave][lane] = bx; }
        __syncthreads();
        if (threadIdx.x < NR) {
            const int n = threadIdx.x;
            for (int w = 0; w < NW; ++w)
                if (sbx[w][n] != 0xFFFFFFFFu) am_merge(bv, bx, sbv[w][n], sbx[w][n]);
            a.pval[(size_t)n * a.pstride + bi] = bv;
            a.pidx[(size_t)n * a.pstride + bi] = bx;
        }
    }
}

template <int NR, int MODE>
static int gemv_k(const GemvArgs& a, hipStream_t s, int* nb) {
    const int ns = (a.K + 511) / 512;
    constexpr int RPW = 2;
    const int ngroups = (a.rows + RPW - 1) / RPW;
    const bool aligned = a.K == ns * 512 && !((uintptr_t)a.x & 15) && !(a.xst & 7);
    if (aligned && (ns == 1 || ns == 2 || ns == 4 || ns == 10)) {
        int grid = a.rows < num_cus() ? a.rows : num_cus();
        if (MODE == 1 && grid > a.pstride) grid = a.pstride;
        if (grid < 1) return -2;
        if (nb) *nb = grid;
#define Q27X_GF(NS) hipLaunchKernelGGL((k_gemv_full<NR, NS, 1, MODE>), dim3(grid), dim3(1024), 0, s, a)
        switch (ns) {
            case 1: Q27X_GF(1); break;
            case 2: Q27X_GF(2); break;
            case 4: Q27X_GF(4); break;
            default: Q27X_GF(10); break;
        }
#undef Q27X_GF
        Q27X_HIP(hipGetLastError());
        return Q27X_OK;
    }
    if constexpr (NR > 4) {
        return -2;                                     // (the caller splits the rows)
    } else {
    int wmax = num_cus() * 8;
    if (MODE == 1 && wmax > a.pstride) wmax = a.pstride & ~3;
    const int upw = (ngroups + wmax - 1) / wmax;
    const int waves = (ngroups + upw - 1) / upw;
    const int grid = (waves + 3) / 4;
    if (nb) *nb = grid * 4;
    if (MODE == 1 && grid * 4 > a.pstride) return -2;
#define Q27X_G(NS) hipLaunchKernelGGL((k_gemv<NR, NS, RPW, MODE>), dim3(grid), dim3(256), 0, s, a, upw)
    switch (ns) {
        case 1: Q27X_G(1); break;
        case 2: Q27X_G(2); break;
        case 4: Q27X_G(4); break;
        case 10: Q27X_G(10); break;
        default: return -2;
    }
#undef Q27X_G
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
    }
}

int launch_gemv(const GemvArgs& a, int argmax_mode, int nr, int* nblocks_out, hipStream_t s) {
    if (!a.W || !a.x || a.rows < 1 || a.K < 8 || (a.K & 7) || nr < 1 || nr > kMaxRows) {
        set_error("gemv: bad arguments (rows=%d K=%d nr=%d)", a.rows, a.K, nr);
        return Q27X_E_ARG;
    }
    if (nr > 4) {
        // one pass over the weights for all rows (aligned shapes); otherwise two launches of <= 4
        // rows (the unaligned kernel's fp32 stage holds 4 rows)
        int rc = -2;
#define Q27X_GN(N) (argmax_mode ? gemv_k<N, 1>(a, s, nblocks_out) : gemv_k<N, 0>(a, s, nblocks_out))
        switch (nr) {
            case 5: rc = Q27X_GN(5); break;
            case 6: rc = Q27X_GN(6); break;
            case 7: rc = Q27X_GN(7); break;
            default: rc = Q27X_GN(8); break;
        }
#undef Q27X_GN
        if (rc != -2) return rc;
        GemvArgs b = a;
        int nb0 = 0, nb1 = 0;
        rc = launch_gemv(b, argmax_mode, 4, &nb0, s);
        if (rc) return rc;
        b.x = a.x + (size_t)4 * a.xst;
        if (argmax_mode) { b.pval = a.pval + (size_t)4 * a.pstride; b.pidx = a.pidx + (size_t)4 * a.pstride; }
        else b.y = (char*)a.y + (size_t)4 * a.ystride * (a.out_bf16 ? 2 : 4);
        rc = launch_gemv(b, argmax_mode, nr - 4, &nb1, s);
        if (nblocks_out) *nblocks_out = nb0;
        return rc;
    }
    int rc = -2;
#define Q27X_GN(N) (argmax_mode ? gemv_k<N, 1>(a, s, nblocks_out) : gemv_k<N, 0>(a, s, nblocks_out))
    switch (nr) {
        case 1: rc = Q27X_GN(1); break;
        case 2: rc = Q27X_GN(2); break;
        case 3: rc = Q27X_GN(3); break;
        case 4: rc = Q27X_GN(4); break;
        default: rc = -2; break;
    }
#undef Q27X_GN
    if (rc == -2) { set_error("gemv: no kernel for K=%d nr=%d", a.K, nr); return Q27X_E_SHAPE; }
    return rc;
}

// ---------------------------------------------------------------- argmax
__global__ __launch_bounds__(256) void k_argmax_final(const float* __restrict__ pval, const uint32_t* __restrict__ pidx,
                                                      int pstride, int nblocks, int32_t* __restrict__ idx,
                                                      float* __restrict__ val, const int* stop) {
    if (stopped(stop)) return;
    const int n = blockIdx.x;
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    float bv = -__builtin_huge_valf();
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = threadIdx.x; i < nblocks; i += 256) {
        const uint32_t ii = pidx[(size_t)n * pstride + i];
        if (ii != 0xFFFFFFFFu) am_merge(bv, bi, pval[(size_t)n * pstride + i], ii);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        if (oi != 0xFFFFFFFFu) am_merge(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < 4; ++w) if (si[w] != 0xFFFFFFFFu) am_merge(bv, bi, sv[w], si[w]);
        const bool none = (bi == 0xFFFFFFFFu);
        idx[n] = none ? 0 : (int32_t)bi;
        if (val) val[n] = none ? -__builtin_huge_valf() : bv;
    }
}
int launch_argmax_final(const float* pval, const uint32_t* pidx, int pstride, int nblocks, int nr,
                        int32_t* idx, float* val, const int* stop, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_final, dim3(nr), dim3(256), 0, s, pval, pidx, pstride, nblocks, idx, val, stop);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ logits, int n, int ld,
                                                     float* __restrict__ pval, uint32_t* __restrict__ pidx, int pstride) {
    const int r = blockIdx.y;
    const float* p = logits + (size_t)r * ld;
    float bv = -__builtin_huge_valf();
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float v = p[i];
        if (finitef(v)) am_merge(bv, bi, v, (uint32_t)i);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        if (oi != 0xFFFFFFFFu) am_merge(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < 4; ++w) if (si[w] != 0xFFFFFFFFu) am_merge(bv, bi, sv[w], si[w]);
        pval[(size_t)r * pstride + blockIdx.x] = bv;
        pidx[(size_t)r * pstride + blockIdx.x] = bi;
    }
}
// module-static partials of the kernel-tier argmax (as the reference's g_q27_am_val/idx arena,
// src/q27_elem.hip:221-222): 8 rows x 64 blocks
__device__ float g_am_val[kMaxRows * 64];
__device__ uint32_t g_am_idx[kMaxRows * 64];
int argmax_scratch(float** pv, uint32_t** pi) {
    Q27X_HIP(hipGetSymbolAddress((void**)pv, HIP_SYMBOL(g_am_val)));
    Q27X_HIP(hipGetSymbolAddress((void**)pi, HIP_SYMBOL(g_am_idx)));
    return Q27X_OK;
}
int launch_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val, float* pval,
                       uint32_t* pidx, hipStream_t s) {
    const int nb = 64;
    hipLaunchKernelGGL(k_argmax_part, dim3(nb, nr), dim3(256), 0, s, logits, n, ld, pval, pidx, nb);
    Q27X_HIP(hipGetLastError());
    return launch_argmax_final(pval, pidx, nb, nb, nr, idx, val, nullptr, s);
}

}  // namespace q27x

// ---------------------------------------------------------------- C ABI (kernel tier)
using namespace q27x;
extern "C" int q27x_proj_rows(const q27x_i8g_t* w, const int8_t* xq, int xstride, const float* xs, void* y,
                              int ystride, int out_bf16, const void* res, int res_bf16, int rstride, float rs,
                              int nr, q27x_stream_t s) {
    if (!w || !y) { set_error("q27x_proj_rows: null argument"); return Q27X_E_ARG; }
    ProjArgs a{};
    a.W = w->w; a.WS = w->s; a.rows = w->rows; a.K = w->K; a.alpha = w->alpha;
    a.xq = xq; a.xst = xstride; a.xs = xs;
    a.y = y; a.ystride = ystride; a.out_bf16 = out_bf16 ? 1 : 0;
    a.res = res; a.res_bf16 = res_bf16 ? 1 : 0; a.rstride = rstride; a.rs = rs;
    return launch_proj(a, EPI_STORE, nr, (hipStream_t)s);
}

extern "C" int q27x_proj_partials(const q27x_i8g_t* w, const int8_t* xq, int xstride, int32_t* part, int nr,
                                  q27x_stream_t s) {
    if (!w || !w->w || !xq || !part || nr < 1 || nr > kMaxRows || (w->K & 15)) {
        set_error("q27x_proj_partials: bad arguments");
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_proj_partials, dim3(1024), dim3(256), 0, (hipStream_t)s, w->w, w->rows, w->K, xq, xstride,
                       part, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_bf16_gemv_rows(const uint16_t* w, int rows, int K, const uint16_t* x, int xstride, void* y,
                                   int ystride, int out_bf16, int nr, q27x_stream_t s) {
    GemvArgs a{};
    a.W = w; a.rows = rows; a.K = K; a.x = x; a.xst = xstride; a.y = y; a.ystride = ystride;
    a.out_bf16 = out_bf16 ? 1 : 0;
    if (!y) { set_error("q27x_bf16_gemv_rows: null output"); return Q27X_E_ARG; }
    return launch_gemv(a, 0, nr, nullptr, (hipStream_t)s);
}
