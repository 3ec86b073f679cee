// k_gemm.hip -- prefill ingest on int8 MFMA: the per-(row, group) W8A8 GEMM of the reference's
// layer-split prefill and its two quantizers, as hand-written gfx950 kernels.
//
// Reference: one rocBLAS int8 gemm_ex per K group writes an int32 slab (src/q27_rb.cpp:43-55), and
// an epilogue sums the slabs with the product of the two scales (src/q27_epi.hip:189-203, fp32 +
// residual form 235-243). The groups are GS = 1024 columns (or the whole K); weights are the
// per-64 mirror requantized per (row, group) (src/q27_epi.hip:14-35), activations are quantized
// per (token, group) (q27_quant_group, src/q27_epi.hip:64-75).
//
// Semantics kept bit for bit:
//   weights:     sg = max of the group's per-64 scales; inv = sg > 0 ? 1/sg : 0;
//                code = clamp(rint(((float)w * s64) * inv), -127, 127)
//   activations: sc = max|v| * (1/127); qi = sc > 0 ? 1/sc : 0; code = clamp(rint(v * qi), -127, 127)
//   GEMM:        acc_g = exact int32 dot over group g; o = 0;
//                for g ascending: o = fmaf((float)acc_g, sw[n][g] * sx[t][g], o);
//                y[t][n] = o * alpha (+ rs * res[t][n])
// The int32 group sums do not depend on the order of their terms, so the MFMA tiling cannot
// change them; the fp32 part runs per output in the reference's group order.
//
// GEMM tiling: a 256-thread block computes a 128-token x 128-row tile; wave w owns the 64 x 64
// quarter (w / 2, w % 2) as 2 x 2 v_mfma_i32_32x32x32_i8 tiles, and two blocks share a CU. K
// advances 64 bytes per stage through a ring of 4 LDS stages (3 when the scales of 17+ groups
// take the room) filled by LDS DMA ahead of the multiply, so 96-128 KiB per CU stay in flight
// to cover the memory latency (one stage ahead measured 16% of the int8 peak: every stage waited
// for its own loads). At the end of each group the int32 tiles are folded into fp32
// accumulators with the group's scales (staged in LDS for the whole K at the start) and
// restarted from zero. Larger forms: 256-token tiles (k_gemm_i8g_rs, 8 waves), and with one group
// over the whole K 256 x 256 tiles (k_gemm_i8g_w4, 8 waves of 128 x 64) where the launch needs
// fewer tile rounds with them.
#include <stdlib.h>
#include <type_traits>

#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kGN = 128, kGK = 64;                // block tile: BM tokens x 128 weight rows, 64 K bytes per stage
constexpr int kGMaxG = 20;                         // groups per row held in LDS (K / GS)
template <int BM, int NS> struct GemmCfg {
    static constexpr int S = NS;                   // stages in the LDS ring
    static constexpr int NW = BM / 32;             // waves: BM / 64 token rows x 2 weight columns of 64
    static constexpr int Stage = (BM + kGN) * kGK; // bytes per stage: A rows, then B rows
    static constexpr int NI = Stage / (1024 * NW); // 1 KiB transfers per wave per stage
    static_assert(Stage % (1024 * NW) == 0, "whole transfers per wave");
};

struct GemmArgs {
    const int8_t* w;    // [N][K] per-(row, group) codes
    const float* sw;    // [N][ng]
    const int8_t* x;    // [M][K] per-(token, group) codes
    const float* sx;    // [M][ng]
    float* y;           // [M][ldy] (bf16 when out_bf16)
    const float* res;   // [M][ldr] or null (bf16 when res_bf16)
    float alpha, rs;
    int M, N, K, gs, ng, ldy, ldr;
    int out_bf16, res_bf16;
    AlphaSel asel;
};

template <int BM, int NS>
__global__ __launch_bounds__(BM * 2) void k_gemm_i8g(GemmArgs a) {
    constexpr int kGS = GemmCfg<BM, NS>::S, kGStage = GemmCfg<BM, NS>::Stage, NI = GemmCfg<BM, NS>::NI;
    constexpr int kGM = BM, BN = kGN, NT = BM * 2;
    constexpr int JT = 2;                          // 32-row weight tiles per wave
    __shared__ __align__(16) int8_t sR[kGS * kGStage];
    // the block's scales, [row][ng] floats: 128 token rows, then BN weight rows (dynamic LDS,
    // sized by the launch to the group count, so short K leaves room for a deeper ring)
    extern __shared__ float sScl[];
    float* sSx = sScl;
    float* sSw = sScl + kGM * a.ng;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;       // wave tile: tokens 64 wm .., weight rows (BN / 2) wn ..
    // Tile order. Blocks are dealt to the 8 XCDs round-robin (block b runs on XCD b % 8), and each
    // XCD has its own L2; block b therefore takes tile (b % 8) * T/8 + b / 8 of a grouped order
    // (groups of 4 token tiles, weight tile major within a group), so each XCD streams one
    // contiguous run of that order: with 32 token tiles, its own 4 token tiles (kept in its L2)
    // against every weight tile, and the 32 blocks it runs at once share 4 token tiles and 8
    // weight tiles. When T is not a multiple of 8 the order is the plain one.
    const int nt = a.N / BN, mt = (a.M + kGM - 1) / kGM, T = nt * mt;
    const int b = blockIdx.x;
    const int tile = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int grp = tile / (4 * nt), fm = grp * 4, gsz = (mt - fm < 4) ? mt - fm : 4;
    const int within = tile - grp * 4 * nt;
    const int m0 = (fm + within % gsz) * kGM, n0 = (within / gsz) * BN;
    const int K = a.K, ng = a.ng, spg = a.gs / kGK, nsteps = K / kGK;

    // Stage layout: rows of 64 bytes, A rows 0..BM-1 then B rows 0..BN-1; chunk c (16 bytes) of row
    // R sits in slot c ^ ((R >> 2) & 3) of its row, so the 16 consecutive rows one operand read
    // serves at a time (same c) fill the 16 distinct 16-byte positions of a 256-byte bank window
    // (SQ_LDS_BANK_CONFLICT reads 0; with (R >> 1) & 3 it was 17% of busy cycles). DMA: instruction i (< NI) of wave
    // w fills stage bytes 1 KiB (NI w + i) .. +1 KiB = stage rows 16 (NI w + i) .. +16; lane l writes
    // row 16 (NI w + i) + l / 4, slot l % 4, so it loads that row's chunk (l % 4) ^ ((row >> 2) & 3).
    const int8_t* gp[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int rs = 16 * (NI * wave + i) + (lane >> 2);         // stage row
        const int r = rs < kGM ? rs : rs - kGM;
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        if (rs < kGM) {
            const int t = (m0 + r < a.M) ? m0 + r : a.M - 1;       // rows past M repeat row M - 1
            gp[i] = a.x + (size_t)t * K + 16 * c;
        } else {
            gp[i] = a.w + (size_t)(n0 + r) * K + 16 * c;
        }
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)sR;
    auto issue = [&](int step, int slot) __attribute__((always_inline)) {
        const uint32_t base = lds0 + slot * kGStage + 1024 * NI * wave;
#pragma unroll
        for (int i = 0; i < NI; ++i) lds_dma16(gp[i] + step * kGK, __builtin_amdgcn_readfirstlane(base + 1024 * i));
    };

    // the first stages, then the block's scales for every group (rows past M read row M - 1;
    // their outputs are not stored)
#pragma unroll
    for (int p = 0; p < kGS - 1; ++p) issue(p < nsteps ? p : 0, p);
    for (int i = tid; i < kGM * ng; i += NT) {
        const int r = i / ng, g = i - r * ng;
        const int t = (m0 + r < a.M) ? m0 + r : a.M - 1;
        sSx[r * ng + g] = a.sx[(size_t)t * ng + g];
    }
    for (int i = tid; i < BN * ng; i += NT) {
        const int r = i / ng, g = i - r * ng;
        sSw[r * ng + g] = a.sw[(size_t)(n0 + r) * ng + g];
    }
    __syncthreads();

    v16i acc[2][JT];
    float facc[2][JT][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) { acc[i][j][r] = 0; facc[i][j][r] = 0.0f; }

    // operand rows of this lane: A row (token) wm*64 + 32 i + lane % 32, B row (weight row)
    // wn*BN/2 + 32 j + lane % 32; both take chunk 2 kk + lane / 32 of the stage's 32-byte K slice
    // kk, so A and B pair the same K positions
    const int arow = wm * 64 + (lane & 31), brow = wn * (BN / 2) + (lane & 31);
    const int swa = (arow >> 2) & 3, swb = (brow >> 2) & 3, kh = lane >> 5;
    for (int s = 0; s < nsteps; ++s) {
        // this wave's transfers for stage s are done once at most the NI (kGS - 2) issued after
        // them are outstanding (vector-memory counts retire in order); after the barrier every
        // wave's are, and every wave has finished reading stage s - 1, whose slot is refilled now
        // with stage s + kGS - 1 (past the end: stage 0 again, never read, so every iteration
        // issues the same transfers and the count stays exact)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(NI * (kGS - 2)));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        __builtin_amdgcn_sched_barrier(0);
        const int sn = s + kGS - 1;
        issue(sn < nsteps ? sn : 0, sn % kGS);
        const int8_t* st = sR + (s % kGS) * kGStage;
#pragma unroll
        for (int kk = 0; kk < kGK / 32; ++kk) {
            const int c = 2 * kk + kh;
            v4i av[2], bv[JT];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = *(const v4i*)(st + (arow + 32 * i) * kGK + ((c ^ swa) << 4));
#pragma unroll
            for (int j = 0; j < JT; ++j) bv[j] = *(const v4i*)(st + (kGM + brow + 32 * j) * kGK + ((c ^ swb) << 4));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if ((s + 1) % spg == 0) {
            // fold the group: accumulator element r of a 32 x 32 tile is row
            // 8 (r / 4) + 4 (lane / 32) + r % 4, column lane % 32
            const int g = (s + 1) / spg - 1;
#pragma unroll
            for (int j = 0; j < JT; ++j) {
                const float swv = sSw[(brow + 32 * j) * ng + g];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int tr = wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        const float sc = swv * sSx[tr * ng + g];
                        facc[i][j][r] = __builtin_fmaf((float)acc[i][j][r], sc, facc[i][j][r]);
                        acc[i][j][r] = 0;
                    }
            }
        }
    }
    // no transfer may still be writing LDS when the block ends
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const int n = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t < a.M) {
                    float o = facc[i][j][r] * alpha_of(a.alpha, a.asel, n);
                    if (a.res) o = o + a.rs * (a.res_bf16 ? bf2f(((const uint16_t*)a.res)[(size_t)t * a.ldr + n])
                                                          : a.res[(size_t)t * a.ldr + n]);
                    if (a.out_bf16) ((uint16_t*)a.y)[(size_t)t * a.ldy + n] = f2bf(o);
                    else a.y[(size_t)t * a.ldy + n] = o;
                }
            }
        }
}

// The same GEMM for 256-token tiles with register-staged loads and 128-byte stages: each thread
// moves six 16-byte chunks per stage with plain vector loads, issued three stages ahead into two
// register sets, and writes them to a double-buffered LDS stage one iteration before the
// multiply; 16 MFMAs per wave between barriers, each 32-byte slice's operands read from LDS
// while the previous slice multiplies. The loop is unrolled by two so the register sets
// are named at compile time; nsteps (K / 128) must be even. Rows are 128 bytes, chunk c of row R
// in slot c ^ ((R >> 1) & 7) (the 16 rows one operand read serves fill a 256-byte bank window).
// Same fold and tile order as k_gemm_i8g.
template <int RES, bool OBF>   // epilogue form, as k_gemm_i8g_w4's
__global__ __launch_bounds__(512) void k_gemm_i8g_rs(GemmArgs a) {
    constexpr int BM = 256, BN = kGN, NT = 512, KB = 128, kStage = (BM + BN) * KB;
    __shared__ __align__(16) int8_t sR[2 * kStage];
    extern __shared__ float sScl[];
    float* sSx = sScl;
    float* sSw = sScl + BM * a.ng;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nt = a.N / BN, mt = (a.M + BM - 1) / BM, T = nt * mt;
    const int b = blockIdx.x;
    const int tile = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int grp = tile / (4 * nt), fm = grp * 4, gsz = (mt - fm < 4) ? mt - fm : 4;
    const int within = tile - grp * 4 * nt;
    const int m0 = (fm + within % gsz) * BM, n0 = (within / gsz) * BN;
    const int K = a.K, ng = a.ng, spg = a.gs / KB, nsteps = K / KB;

    // thread tid moves chunk q = tid + 512 k (k < 6) of each stage: stage row q / 8 (A rows
    // first), natural chunk q % 8 of that row, stored at slot (q % 8) ^ ((row >> 1) & 7)
    const int8_t* gp[6];
    int lo[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const int q = tid + NT * k, rs = q >> 3, c = q & 7;
        const int r = rs < BM ? rs : rs - BM;
        if (rs < BM) {
            const int t = (m0 + r < a.M) ? m0 + r : a.M - 1;
            gp[k] = a.x + (size_t)t * K + 16 * c;
        } else {
            gp[k] = a.w + (size_t)(n0 + r) * K + 16 * c;
        }
        lo[k] = rs * KB + ((c ^ ((r >> 1) & 7)) << 4);
    }
    uint4 ra0, ra1, ra2, ra3, ra4, ra5, rb0, rb1, rb2, rb3, rb4, rb5;
#define Q27X_LD(R0, R1, R2, R3, R4, R5, step)                                                       \
    { const int k0_ = (step) * KB;                                                                  \
      R0 = *(const uint4*)(gp[0] + k0_); R1 = *(const uint4*)(gp[1] + k0_);                         \
      R2 = *(const uint4*)(gp[2] + k0_); R3 = *(const uint4*)(gp[3] + k0_);                         \
      R4 = *(const uint4*)(gp[4] + k0_); R5 = *(const uint4*)(gp[5] + k0_); }
#define Q27X_ST(R0, R1, R2, R3, R4, R5, slot)                                                       \
    { int8_t* d_ = sR + (slot) * kStage;                                                            \
      *(uint4*)(d_ + lo[0]) = R0; *(uint4*)(d_ + lo[1]) = R1; *(uint4*)(d_ + lo[2]) = R2;           \
      *(uint4*)(d_ + lo[3]) = R3; *(uint4*)(d_ + lo[4]) = R4; *(uint4*)(d_ + lo[5]) = R5; }

    for (int i = tid; i < BM * ng; i += NT) {
        const int r = i / ng, g = i - r * ng;
        const int t = (m0 + r < a.M) ? m0 + r : a.M - 1;
        sSx[r * ng + g] = a.sx[(size_t)t * ng + g];
    }
    for (int i = tid; i < BN * ng; i += NT) {
        const int r = i / ng, g = i - r * ng;
        sSw[r * ng + g] = a.sw[(size_t)(n0 + r) * ng + g];
    }
    // stages 0 and 1 in flight, stage 0 to LDS, stage 2 in flight behind stage 1
    Q27X_LD(ra0, ra1, ra2, ra3, ra4, ra5, 0)
    Q27X_LD(rb0, rb1, rb2, rb3, rb4, rb5, 1)
    Q27X_ST(ra0, ra1, ra2, ra3, ra4, ra5, 0)
    Q27X_LD(ra0, ra1, ra2, ra3, ra4, ra5, 2 < nsteps ? 2 : 0)
    __syncthreads();

    v16i acc[2][2];
    float facc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) { acc[i][j][r] = 0; facc[i][j][r] = 0.0f; }
    const int arow = wm * 64 + (lane & 31), brow = wn * 64 + (lane & 31);
    const int swa = (arow >> 1) & 7, swb = (brow >> 1) & 7, kh = lane >> 5;

    // iteration s: multiply stage s (LDS slot s % 2); store stage s + 1 (register set (s + 1) % 2)
    // into the other slot; reload that set with stage s + 3 (past the end: stage 0, stored into a
    // slot nobody reads again); barrier
#define Q27X_ITER(S_, N0, N1, N2, N3, N4, N5)                                                       \
    {                                                                                               \
        const int s_ = (S_);                                                                        \
        const int8_t* st = sR + (s_ & 1) * kStage;                                                  \
        v4i av[2][2], bv[2][2];                                                                     \
_Pragma("unroll")                                                                                   \
        for (int i = 0; i < 2; ++i) av[0][i] = *(const v4i*)(st + (arow + 32 * i) * KB + ((kh ^ swa) << 4)); \
_Pragma("unroll")                                                                                   \
        for (int j = 0; j < 2; ++j) bv[0][j] = *(const v4i*)(st + (BM + brow + 32 * j) * KB + ((kh ^ swb) << 4)); \
_Pragma("unroll")                                                                                   \
        for (int kk = 0; kk < KB / 32; ++kk) {                                                      \
            const int cu = kk & 1, nx = cu ^ 1;                                                     \
            if (kk + 1 < KB / 32) {                                                                 \
                const int c = 2 * (kk + 1) + kh;                                                    \
_Pragma("unroll")                                                                                   \
                for (int i = 0; i < 2; ++i) av[nx][i] = *(const v4i*)(st + (arow + 32 * i) * KB + ((c ^ swa) << 4)); \
_Pragma("unroll")                                                                                   \
                for (int j = 0; j < 2; ++j) bv[nx][j] = *(const v4i*)(st + (BM + brow + 32 * j) * KB + ((c ^ swb) << 4)); \
            }                                                                                       \
_Pragma("unroll")                                                                                   \
            for (int i = 0; i < 2; ++i)                                                             \
_Pragma("unroll")                                                                                   \
                for (int j = 0; j < 2; ++j)                                                         \
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[cu][i], bv[cu][j], acc[i][j], 0, 0, 0); \
        }                                                                                           \
        if ((s_ + 1) % spg == 0) {                                                                  \
            const int g = (s_ + 1) / spg - 1;                                                       \
_Pragma("unroll")                                                                                   \
            for (int j = 0; j < 2; ++j) {                                                           \
                const float swv = sSw[(brow + 32 * j) * ng + g];                                    \
_Pragma("unroll")                                                                                   \
                for (int i = 0; i < 2; ++i)                                                         \
_Pragma("unroll")                                                                                   \
                    for (int r = 0; r < 16; ++r) {                                                  \
                        const int tr = wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); \
                        const float sc = swv * sSx[tr * ng + g];                                    \
                        facc[i][j][r] = __builtin_fmaf((float)acc[i][j][r], sc, facc[i][j][r]);     \
                        acc[i][j][r] = 0;                                                           \
                    }                                                                               \
            }                                                                                       \
        }                                                                                           \
        Q27X_ST(N0, N1, N2, N3, N4, N5, (s_ + 1) & 1)                                               \
        Q27X_LD(N0, N1, N2, N3, N4, N5, s_ + 3 < nsteps ? s_ + 3 : 0)                               \
        __syncthreads();                                                                            \
    }
    for (int s = 0; s < nsteps; s += 2) {
        Q27X_ITER(s, rb0, rb1, rb2, rb3, rb4, rb5)        // stage s + 1 sits in the b set
        Q27X_ITER(s + 1, ra0, ra1, ra2, ra3, ra4, ra5)    // stage s + 2 in the a set
    }
#undef Q27X_ITER
#undef Q27X_LD
#undef Q27X_ST

    // outputs (32-bit element offsets: the launcher keeps M x ldy and M x ldr below 2^30)
    const uint32_t nb = (uint32_t)(n0 + wn * 64 + (lane & 31));
    float al[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) al[j] = alpha_of(a.alpha, a.asel, (int)nb + 32 * j);
    auto out = [&](auto full) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (decltype(full)::value || t < a.M) {
                    const uint32_t yo = (uint32_t)t * (uint32_t)a.ldy + nb;
                    const uint32_t ro = (uint32_t)t * (uint32_t)a.ldr + nb;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        float o = facc[i][j][r] * al[j];
                        if constexpr (RES == 1) o = o + a.rs * a.res[ro + 32 * j];
                        if constexpr (RES == 2) o = o + a.rs * bf2f(((const uint16_t*)a.res)[ro + 32 * j]);
                        if constexpr (OBF) ((uint16_t*)a.y)[yo + 32 * j] = f2bf(o);
                        else a.y[yo + 32 * j] = o;
                    }
                }
            }
    };
    if (m0 + BM <= a.M) out(std::true_type{});
    else out(std::false_type{});
}

// One group over the whole K (the reference's default arm) on 256-token x 256-row tiles: 8 waves,
// two per SIMD, each owning 128 tokens x 64 rows as 4 x 2 v_mfma_i32_32x32x32_i8 tiles (128
// accumulator registers; no fp32 group accumulators are needed, the scales apply once at the end),
// so each MFMA reads three quarters of a KiB of LDS operands instead of the 64 x 64 quarter's full
// KiB, and while one wave of a SIMD waits (a barrier, its operand reads) the other multiplies
// (with 4 waves of 128 x 128, one per SIMD, the same tile ran 17-20% slower). K
// advances 128 bytes per stage (each stage row is one whole 128-byte line of a row, which halves
// the load requests of 64-byte stages) through two 64 KiB LDS stages filled by LDS DMA. The
// operand reads are pipelined one 32-byte slice ahead of the MFMAs, across the stage barrier too:
// the barrier that certifies stage s + 1 sits before the last slice of stage s, whose operands
// are already in registers, and the next stage's first slice is read while that slice multiplies.
// Rows are 128 bytes, chunk c of row R in slot c ^ ((R >> 1) & 7) (the 16 rows of one operand read
// fill a 256-byte bank window). Same tile order as k_gemm_i8g; the int32 sums are exact, so the
// outputs are the other kernels' bits.
constexpr int kW4B = 256, kW4K = 128, kW4S = 2;
constexpr int kW4Stage = 2 * kW4B * kW4K;              // 64 KiB: A rows, then B rows
constexpr int kW4NI = kW4Stage / (1024 * 8);           // 1 KiB transfers per wave per stage (8)
// RES: no residual (0), fp32 (1) or bf16 (2) residual rows; OBF: bf16 output. Instances per
// epilogue form: with per-element branches on them the unrolled epilogue of 256 values per lane
// cost ~20 us per tile.
template <int RES, bool OBF>
__global__ __launch_bounds__(512) void k_gemm_i8g_w4(GemmArgs a) {
    __shared__ __align__(16) int8_t sR[kW4S * kW4Stage];
    __shared__ float sSx[kW4B], sSw[kW4B];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int nt = a.N / kW4B, mt = (a.M + kW4B - 1) / kW4B, T = nt * mt;
    const int b = blockIdx.x;
    const int tile = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int grp = tile / (4 * nt), fm = grp * 4, gsz = (mt - fm < 4) ? mt - fm : 4;
    const int within = tile - grp * 4 * nt;
    const int m0 = (fm + within % gsz) * kW4B, n0 = (within / gsz) * kW4B;
    const int K = a.K, nsteps = K / kW4K;
    // DMA: transfer i (< 8) of wave w fills stage rows 8 (8 w + i) .. +8; lane l writes row
    // 8 (8 w + i) + l / 8, slot l % 8, so it loads that row's chunk (l % 8) ^ ((row >> 1) & 7)
    // (waves 0-3 fill the A rows, waves 4-7 the B rows: one base per wave, byte offsets below
    // 2^31 for the row counts and K this kernel takes)
    const int8_t* gb = wave < 4 ? a.x : a.w;
    uint32_t go[kW4NI];
#pragma unroll
    for (int i = 0; i < kW4NI; ++i) {
        const int rs = 8 * (kW4NI * wave + i) + (lane >> 3);
        const int r = rs < kW4B ? rs : rs - kW4B;
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int row = rs < kW4B ? ((m0 + r < a.M) ? m0 + r : a.M - 1) : n0 + r;   // rows past M repeat row M - 1
        go[i] = (uint32_t)row * (uint32_t)K + 16 * c;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)sR;
    auto issue = [&](int step, int slot) __attribute__((always_inline)) {
        const uint32_t base = lds0 + slot * kW4Stage + 1024 * kW4NI * wave;
#pragma unroll
        for (int i = 0; i < kW4NI; ++i)
            lds_dma16(gb + go[i] + (uint32_t)(step * kW4K), __builtin_amdgcn_readfirstlane(base + 1024 * i));
    };
    issue(0, 0);
    if (tid < kW4B) {
        const int t = (m0 + tid < a.M) ? m0 + tid : a.M - 1;
        sSx[tid] = a.sx[t];
        sSw[tid] = a.sw[n0 + tid];
    }
    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    // operand rows of this lane: A (token) wm*128 + 32 i + lane % 32, B (weight row) wn*64 + 32 j +
    // lane % 32; both take chunk 2 kk + lane / 32 of the stage's 32-byte K slice kk
    const int arow = wm * 128 + (lane & 31), brow = kW4B + wn * 64 + (lane & 31);
    const int swa = (arow >> 1) & 7, swb = ((brow - kW4B) >> 1) & 7, kh = lane >> 5;
    auto rd = [&](v4i (&av)[4], v4i (&bv)[2], int slot, int kk) __attribute__((always_inline)) {
        const int8_t* st = sR + slot * kW4Stage;
        const int c = 2 * kk + kh;
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = *(const v4i*)(st + (arow + 32 * i) * kW4K + ((c ^ swa) << 4));
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[j] = *(const v4i*)(st + (brow + 32 * j) * kW4K + ((c ^ swb) << 4));
    };
    auto mm = [&](const v4i (&av)[4], const v4i (&bv)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
    };
    // this wave's transfers of the next stage done and its operand reads of the current one
    // returned; after the barrier every wave's are (nothing is scheduled across it)
    auto sync = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        __builtin_amdgcn_sched_barrier(0);
    };
    constexpr int SL = kW4K / 32;                      // 32-byte slices per stage
    v4i oa[2][4], ob[2][2];
    sync();                                            // stage 0 everywhere (and the scales)
    issue(1 < nsteps ? 1 : 0, 1);
    rd(oa[0], ob[0], 0, 0);
    for (int s = 0; s < nsteps; ++s) {
#pragma unroll
        for (int kk = 0; kk < SL; ++kk) {
            const int cu = kk & 1, nx = cu ^ 1;
            if (kk + 1 < SL) {
                rd(oa[nx], ob[nx], s & 1, kk + 1);
            } else {
                // stage s + 1 landed everywhere and stage s is read by all: its slot takes stage
                // s + 2 (past the end: stage 0 again into a slot nobody reads, so every iteration
                // issues the same transfers); the next stage's first slice is read meanwhile
                // (past the last stage that is a stale slot, not used)
                sync();
                issue(s + 2 < nsteps ? s + 2 : 0, s & 1);
                rd(oa[nx], ob[nx], (s + 1) & 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
            mm(oa[cu], ob[cu]);
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        }
    }
    // no transfer may still be writing LDS when the block ends
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // the tile's outputs; rows past M only in the last token tile. Element offsets are 32-bit
    // (the launcher keeps M x ldy and M x ldr below 2^30), so the stores take the output's base in
    // scalar registers.
    const uint32_t nb = (uint32_t)(n0 + wn * 64 + (lane & 31));
    float swv[2], al[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        swv[j] = sSw[wn * 64 + 32 * j + (lane & 31)];
        al[j] = alpha_of(a.alpha, a.asel, (int)nb + 32 * j);
    }
    auto out = [&](auto full) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tl = wm * 128 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), t = m0 + tl;
                if (decltype(full)::value || t < a.M) {
                    const float sxv = sSx[tl];
                    const uint32_t yo = (uint32_t)t * (uint32_t)a.ldy + nb;
                    const uint32_t ro = (uint32_t)t * (uint32_t)a.ldr + nb;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        float o = __builtin_fmaf((float)acc[i][j][r], swv[j] * sxv, 0.0f) * al[j];
                        if constexpr (RES == 1) o = o + a.rs * a.res[ro + 32 * j];
                        if constexpr (RES == 2) o = o + a.rs * bf2f(((const uint16_t*)a.res)[ro + 32 * j]);
                        if constexpr (OBF) ((uint16_t*)a.y)[yo + 32 * j] = f2bf(o);
                        else a.y[yo + 32 * j] = o;
                    }
                }
            }
    };
    if (m0 + kW4B <= a.M) out(std::true_type{});
    else out(std::false_type{});
}

// Weights: per-64 mirror -> per-(row, group) codes and scales; one 256-thread block per row.
// In place when wg == w (each element is read and written by the same thread).
__global__ __launch_bounds__(256) void k_i8g64_to_grp(const int8_t* w, const float* s64, int K, int gs,
                                                      int8_t* wg, float* sg) {
    const int r = blockIdx.x, t = threadIdx.x, ns = K >> 6, ng = K / gs;
    __shared__ float red[4];
    const int8_t* row = w + (size_t)r * K;
    int8_t* out = wg + (size_t)r * K;
    const float* sr = s64 + (size_t)r * ns;
    for (int g = 0; g < ng; ++g) {
        float mx = 0.0f;
        for (int i = t; i < (gs >> 6); i += 256) mx = fmaxf(mx, sr[g * (gs >> 6) + i]);
        mx = max_xor(mx, 64);
        if ((t & 63) == 0) red[t >> 6] = mx;
        __syncthreads();
        const float s = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        const float inv = (s > 0.0f) ? 1.0f / s : 0.0f;
        if (t == 0) sg[(size_t)r * ng + g] = s;
        for (int k = g * gs + t; k < (g + 1) * gs; k += 256) {
            out[k] = qcode((float)row[k] * sr[k >> 6], inv);
        }
    }
}

// Activations: fp32 rows -> per-(token, group) codes and scales; one 256-thread block per
// (group, token), four values per thread per 1024 columns.
__global__ __launch_bounds__(256) void k_quant_tok_grp(const float* x, int xstride, int K, int gs, int8_t* xq,
                                                       float* xs, float gq) {
    const int g = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, ng = K / gs;
    __shared__ float red[4];
    const float* row = x + (size_t)tok * xstride + (size_t)g * gs;
    float mx = 0.0f;
    for (int k = 4 * t; k < gs; k += 1024) {
        const float4 v = *(const float4*)(row + k);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mx = max_xor(mx, 64);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m * gq * (1.0f / 127.0f), qi = (sc > 0.0f) ? gq / sc : 0.0f;   // gq = 1/in_scale
    if (t == 0) xs[(size_t)tok * ng + g] = sc;
    int8_t* out = xq + (size_t)tok * K + (size_t)g * gs;
    for (int k = 4 * t; k < gs; k += 1024) {
        const float4 v = *(const float4*)(row + k);
        const uint32_t pk = (uint32_t)(uint8_t)qcode(v.x, qi) | ((uint32_t)(uint8_t)qcode(v.y, qi) << 8) |
                            ((uint32_t)(uint8_t)qcode(v.z, qi) << 16) | ((uint32_t)(uint8_t)qcode(v.w, qi) << 24);
        *(uint32_t*)(out + k) = pk;
    }
}

}  // namespace q27x

// ---------------------------------------------------------------- C ABI (prefill GEMM tier)
using namespace q27x;

extern "C" int q27x_i8g64_to_grp(const int8_t* w, const float* s64, int rows, int K, int gs, int8_t* wg,
                                 float* sg, q27x_stream_t s) {
    if (!w || !s64 || !wg || !sg || rows < 1 || K < 64 || gs < 64 || (gs & 63) || (K % gs)) {
        set_error("q27x_i8g64_to_grp: bad arguments (rows %d, K %d, gs %d)", rows, K, gs);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_i8g64_to_grp, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)s, w, s64, K, gs, wg, sg);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_quant_tok_groups(const float* x, int xstride, int M, int K, int gs, int8_t* xq, float* xs,
                                     q27x_stream_t s) {
    if (!x || !xq || !xs || M < 1 || K < 4 || gs < 4 || (gs & 3) || (K % gs) || xstride < K || (xstride & 3) ||
        ((uintptr_t)x & 15)) {
        set_error("q27x_quant_tok_groups: bad arguments (M %d, K %d, gs %d, xstride %d)", M, K, gs, xstride);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_quant_tok_grp, dim3((unsigned)(K / gs), (unsigned)M), dim3(256), 0, (hipStream_t)s, x,
                       xstride, K, gs, xq, xs, 1.0f);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                             const float* sx, int M, float* y, int ldy, const float* res, int ldr, float rs,
                             q27x_stream_t s) {
    if (!w || !sw || !x || !sx || !y || M < 1 || N < 1 || K < 1 || gs < 1 || ldy < N || (res && ldr < N)) {
        set_error("q27x_gemm_i8g: bad arguments");
        return Q27X_E_ARG;
    }
    if ((N % 128) || (K % kGK) || (gs % kGK) || (K % gs) || K / gs > kGMaxG || ((uintptr_t)w & 15) ||
        ((uintptr_t)x & 15)) {
        set_error("q27x_gemm_i8g: no kernel for N %d, K %d, gs %d (N %% 128, K %% %d, gs %% %d must be 0, "
                  "K/gs <= %d, 16-byte aligned codes)", N, K, gs, kGK, kGK, kGMaxG);
        return Q27X_E_SHAPE;
    }
    return launch_gemm_i8g(w, sw, N, K, gs, alpha, x, sx, M, y, ldy, 0, res, ldr, 0, rs, (hipStream_t)s);
}

namespace q27x {
static int g_gemm_cus = 0;
static int gemm_cus() {
    if (!g_gemm_cus) {
        int dev = 0;
        hipDeviceProp_t p;
        g_gemm_cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess &&
                      p.multiProcessorCount > 0) ? p.multiProcessorCount : 256;
    }
    return g_gemm_cus;
}
int launch_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                    const float* sx, int M, void* y, int ldy, int out_bf16, const void* res, int ldr, int res_bf16,
                    float rs, hipStream_t s, const AlphaSel* asel) {
    if ((N % 128) || (K % kGK) || (gs % kGK) || (K % gs) || K / gs > kGMaxG || ((uintptr_t)w & 15) ||
        ((uintptr_t)x & 15) || M < 1 || ldy < N || (res && ldr < N)) {
        set_error("gemm: no kernel for M %d, N %d, K %d, gs %d", M, N, K, gs);
        return Q27X_E_SHAPE;
    }
    GemmArgs a{};
    a.w = w; a.sw = sw; a.x = x; a.sx = sx; a.y = (float*)y; a.res = (const float*)res; a.alpha = alpha; a.rs = rs;
    a.M = M; a.N = N; a.K = K; a.gs = gs; a.ng = K / gs; a.ldy = ldy; a.ldr = ldr;
    a.out_bf16 = out_bf16; a.res_bf16 = res_bf16;
    if (asel) a.asel = *asel;
    // Weight tiles of 128 rows (256-row tiles need 433 registers per lane, one block per CU, and
    // measured 1-8% slower). Token tiles of 256 (8 waves, one block per CU, a 5-stage ring) from
    // 512 tokens on: a third fewer bytes per MAC through the CU's load path; else 128 (4 waves,
    // two blocks per CU, a 4-stage ring, or 3 when 17+ groups' scales take the room).
    // One group over the whole K: 256 x 256 tiles when their launch takes fewer tile rounds on the
    // CUs, counting a round of 256 x 256 tiles as 1.4 rounds of the rs kernel's 256 x 128 tiles
    // (measured per round at 4096 x 16384 x 5120: 90 and 63 us); with too few tiles for the CUs
    // the narrower tiles keep more of them busy. Q27X_GEMM_W4 = 1 / 0 takes / avoids them wherever
    // the shape allows (tests of the kernel at small shapes, measurements).
    if (M >= 512 && a.ng == 1 && N % kW4B == 0 && K % kW4K == 0 && K >= 2 * kW4K &&
        (long)(M > N ? M : N) * K < (1L << 31) && (long)M * ldy < (1L << 30) && (!res || (long)M * ldr < (1L << 30))) {
        const long mt = (M + 255) / 256, g = gemm_cus();
        const long rw = ((long)(N / kW4B) * mt + g - 1) / g, ro = ((long)(N / kGN) * mt + g - 1) / g;
        const char* f = getenv("Q27X_GEMM_W4");
        const bool force = f && f[0] == '1' && !f[1], avoid = f && f[0] == '0' && !f[1];
        if (force || (!avoid && rw * 14 < ro * 10)) {
            const dim3 grid((unsigned)((N / kW4B) * mt));
            const int rm = !res ? 0 : res_bf16 ? 2 : 1;
            if (out_bf16) {
                if (rm == 0) hipLaunchKernelGGL((k_gemm_i8g_w4<0, true>), grid, dim3(512), 0, s, a);
                else if (rm == 1) hipLaunchKernelGGL((k_gemm_i8g_w4<1, true>), grid, dim3(512), 0, s, a);
                else hipLaunchKernelGGL((k_gemm_i8g_w4<2, true>), grid, dim3(512), 0, s, a);
            } else {
                if (rm == 0) hipLaunchKernelGGL((k_gemm_i8g_w4<0, false>), grid, dim3(512), 0, s, a);
                else if (rm == 1) hipLaunchKernelGGL((k_gemm_i8g_w4<1, false>), grid, dim3(512), 0, s, a);
                else hipLaunchKernelGGL((k_gemm_i8g_w4<2, false>), grid, dim3(512), 0, s, a);
            }
            Q27X_HIP(hipGetLastError());
            return Q27X_OK;
        }
    }
    if (M >= 512 && K % 256 == 0 && gs % 128 == 0 && (long)M * ldy < (1L << 30) &&
        (!res || (long)M * ldr < (1L << 30))) {
        const unsigned mt = (unsigned)((M + 255) / 256);
        const size_t scl = (size_t)(256 + kGN) * a.ng * sizeof(float);
        const dim3 grid((unsigned)(N / kGN) * mt);
        const int rm = !res ? 0 : res_bf16 ? 2 : 1;
        if (out_bf16) {
            if (rm == 0) hipLaunchKernelGGL((k_gemm_i8g_rs<0, true>), grid, dim3(512), scl, s, a);
            else if (rm == 1) hipLaunchKernelGGL((k_gemm_i8g_rs<1, true>), grid, dim3(512), scl, s, a);
            else hipLaunchKernelGGL((k_gemm_i8g_rs<2, true>), grid, dim3(512), scl, s, a);
        } else {
            if (rm == 0) hipLaunchKernelGGL((k_gemm_i8g_rs<0, false>), grid, dim3(512), scl, s, a);
            else if (rm == 1) hipLaunchKernelGGL((k_gemm_i8g_rs<1, false>), grid, dim3(512), scl, s, a);
            else hipLaunchKernelGGL((k_gemm_i8g_rs<2, false>), grid, dim3(512), scl, s, a);
        }
    } else if (M >= 512) {
        const unsigned mt = (unsigned)((M + 255) / 256);
        const size_t scl = (size_t)(256 + kGN) * a.ng * sizeof(float);
        hipLaunchKernelGGL((k_gemm_i8g<256, 5>), dim3((unsigned)(N / kGN) * mt), dim3(512), scl, (hipStream_t)s, a);
    } else {
        const unsigned mt = (unsigned)((M + 127) / 128);
        const size_t scl = (size_t)(128 + kGN) * a.ng * sizeof(float);
        if (64 * 1024 + scl <= 80 * 1024)
            hipLaunchKernelGGL((k_gemm_i8g<128, 4>), dim3((unsigned)(N / kGN) * mt), dim3(256), scl, (hipStream_t)s, a);
        else
            hipLaunchKernelGGL((k_gemm_i8g<128, 3>), dim3((unsigned)(N / kGN) * mt), dim3(256), scl, (hipStream_t)s, a);
    }
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
// the per-(token, group) quantizer with g = 1/in_scale (s = mx g / 127, qi = g / s)
int launch_quant_tok_grp(const float* x, int xstride, int M, int K, int gs, float in_scale, int8_t* xq, float* xs,
                         hipStream_t s) {
    if (!x || !xq || !xs || M < 1 || K < 4 || gs < 4 || (gs & 3) || (K % gs) || xstride < K || (xstride & 3) ||
        ((uintptr_t)x & 15) || !(in_scale > 0.0f)) {
        set_error("quant tok groups: bad arguments (M %d, K %d, gs %d)", M, K, gs);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_quant_tok_grp, dim3((unsigned)(K / gs), (unsigned)M), dim3(256), 0, s, x, xstride, K, gs, xq,
                       xs, 1.0f / in_scale);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // namespace q27x
