// flare_ar_mfma.hip -- bf16-input MFMA kernels for phases 1 and 3 of the chunked
// causal FLARE forward on gfx950 (16x16x32 bf16/fp16 MFMA, fp32 accumulate).
//
// Notation for one (b,h), latent m, token t, in the log2 domain
// (S = scale * log2(e) * k_t . q_m):
//   R[m]      reference max of latent m.  It moves only when a score exceeds it
//             by more than kLazy, so every E below is at most 2^kLazy and the
//             numerator is rescaled rarely (lazy rescaling).
//   E[t,m]    = 2^(S[t,m] - R[m])
//   d[m]      = sum_t E[t,m]             U[m,:] = sum_t E[t,m] v_t
// The chunk summary (max, den, num) of the reference (training.py:914-1018) is
// (R_true, d 2^(R - R_true), U 2^(R - R_true)) in natural-log units.
//
// Phase 1, chunk_prepare_mfma: one workgroup per (chunk, b, h) holding every
// latent (M/32 waves, 32 latents each), so K and V are read once.  S = K Q^T
// is computed tokens-as-rows: its C layout gives each lane 8 tokens of one
// latent, which is the A-operand layout of E^T in U += E^T V.
//
// Phase 3, chunk_output_mfma: one workgroup replays one chunk.  Per 32-token
// subtile, with d0 = den at the subtile start and d_t = d0 + sum_{tau<=t} E:
//   z0[m]    = U[m] / d0                 |z0| <= max|v|
//   W1[t,m]  = alpha[t,m] d0 / d_t       in [0, alpha],   alpha = softmax_m(S[t,:])
//   W2[t,m]  = alpha[t,m] / d_t
//   G[t,tau] = sum_m W2[t,m] E[tau,m]    in [0, 1]
//   y_t      = sum_m W1[t,m] z0[m] + sum_{tau<=t} G[t,tau] v_tau
//   U       += E^T V_j
// This is the tokenwise recurrence of the reference (training.py:1282-1393,
// reference.py:446-496) regrouped into 16x16x32 contractions.  Scores, maxima,
// den and the softmax weights are split over waves by latent; U and y are split
// by value column; W1, E^T and the partials of G cross waves through LDS.
//
// Operand precision (all products accumulate in fp32):
//   S = Q K^T            bf16 x bf16 (the inputs)
//   U += E^T V           fp16 x fp16 (E <= 2^kLazy; bf16 V converts exactly)
//   y += W1 z0           fp16 x fp16 (both bounded, see above)
//   G  = W2 E^T          hi/lo bf16 splits of both, three MFMAs
//   y += G V             hi/lo fp16 split of G x fp16 V, two MFMAs
// The splits are needed: sum_tau G v cancels to the small early outputs, where
// a single bf16 rounding of E or G costs ~1e-1 relative error.  A value column
// with |v| > 65504 (outside fp16) switches that wave's subtile to bf16 V with
// hi/lo-split partners (exact, slower); a non-finite fp16 readout is redone
// in bf16.
#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {
namespace mfma {

// ---------------------------------------------------------------------------
// Phase 1.  grid = (NC, B*H), M/32 waves.  Wave w owns latents 32w .. 32w+31
// (two 16-latent tiles) and every value column.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(512) void chunk_prepare_mfma(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    int M, float scale2, int chunk, float* __restrict__ cmax, float* __restrict__ cden,
    float* __restrict__ cnum) {
    constexpr int KS = D / 32;     // k-steps for the scores
    constexpr int DT = D / 16;     // value-column tiles
    constexpr int VP = T + 8;      // padded row of the transposed V tile
    constexpr int QP = D + 8;      // padded row of Q in LDS
    __shared__ __attribute__((aligned(16))) f16 vtl[D * VP];
    __shared__ __attribute__((aligned(16))) bf16 qsh[kMaxPrepM * QP];  // Q[h], M rows
    __shared__ int vbig;

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int nthr = blockDim.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int m0 = 32 * w;                       // this wave's 32 latents

    for (int vi = tid; vi < M * D / 8; vi += nthr) {
        const int m = vi / (D / 8), d8 = vi % (D / 8);
        *reinterpret_cast<bf16x8*>(qsh + m * QP + 8 * d8) = load8<bf16x8>(Q + ((size_t)h * M + m) * D + 8 * d8);
    }
    f32x4 U[2][DT];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int di = 0; di < DT; ++di) U[mt][di] = f32x4{0.f, 0.f, 0.f, 0.f};
    // per latent m0 + 16 mt + c (replicated over the four rows g)
    float R[2] = {kNegInf, kNegInf}, Rt[2] = {kNegInf, kNegInf}, den[2] = {0.f, 0.f};

    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    if (tid == 0) vbig = 0;
    // K rows of the first subtile (A operands of S = K Q^T); each iteration
    // prefetches the next subtile's rows while it works on the current one.
    bf16x8 ka[2][KS];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
        const int t = t_begin + 16 * ti + c;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            ka[ti][ks] = t < t_end ? load8<bf16x8>(K + row0 + (size_t)t * stride + 32 * ks + 8 * g) : zero8();
    }
    for (int t0 = t_begin; t0 < t_end; t0 += T) {
        __syncthreads();
        if (stage_vt_f16<VP>(vtl, V, row0, stride, t0, t_end, 0, D, tid, nthr)) vbig = 1;
        // S = K Q^T, tokens as rows: s[mt][ti][r] = S[t = 16 ti + 4 g + r][m = 16 mt + c]
        float s[2][2][4];
        {
            f32x4 acc[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)   // B operand: Q rows of this wave's latents
                        acc[mt][ti] = mma(ka[ti][ks], load8<bf16x8>(qsh + (m0 + 16 * mt + c) * QP + 32 * ks + 8 * g),
                                          acc[mt][ti]);
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const int t = t0 + T + 16 * ti + c;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    ka[ti][ks] = t < t_end ? load8<bf16x8>(K + row0 + (size_t)t * stride + 32 * ks + 8 * g) : zero8();
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        s[mt][ti][r] = (t0 + 16 * ti + 4 * g + r < t_end) ? acc[mt][ti][r] * scale2 : kNegInf;
        }
        // per-latent maxima (lazy reference), E, den
        float e[2][2][4];
        bool need = false;
        float gam[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            float mx = kNegInf;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[mt][ti][r]);
            mx = rows_max4(mx);
            Rt[mt] = fmaxf(Rt[mt], mx);
            const bool mv = mx > R[mt] + kLazy;
            need |= mv;
            const float Rn = mv ? mx : R[mt];
            gam[mt] = mv ? exp2f_fast(R[mt] - Rn) : 1.0f;     // 0 when R = -inf
            R[mt] = Rn;
            float es = 0.0f;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    e[mt][ti][r] = exp2f_fast(s[mt][ti][r] - Rn);
                    es += e[mt][ti][r];
                }
            den[mt] = den[mt] * gam[mt] + rows_sum4(es);
        }
        if (__any(need)) {
            // rows of U are latents 16 mt + 4 g + r: fetch their factors
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float gr = __shfl(gam[mt], 4 * g + r, 64);
#pragma unroll
                    for (int di = 0; di < DT; ++di) U[mt][di][r] *= gr;
                }
        }
        __syncthreads();
        if (!vbig) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                f16x8 ea;   // E^T[m = c][tau = pi(g, .)]
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    ea[r] = (f16)e[mt][0][r];
                    ea[4 + r] = (f16)e[mt][1][r];
                }
#pragma unroll
                for (int di = 0; di < DT; ++di) {
                    const f16* vr = vtl + (16 * di + c) * VP;
                    const f16x8 vb = cat8<f16x8>(load4<f16x4>(vr + 4 * g), load4<f16x4>(vr + 16 + 4 * g));
                    U[mt][di] = mma(ea, vb, U[mt][di]);
                }
            }
        } else {
            // a value outside the fp16 range: bf16 V and an exact hi/lo split of E
            __syncthreads();
            bf16* vtb = reinterpret_cast<bf16*>(vtl);
            stage_vt_bf16<VP>(vtb, V, row0, stride, t0, t_end, 0, D, tid, nthr);
            __syncthreads();
            if (tid == 0) vbig = 0;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                bf16x8 eh, el;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    SPLIT2(bf16, e[mt][0][r], eh[r], el[r]);
                    SPLIT2(bf16, e[mt][1][r], eh[4 + r], el[4 + r]);
                }
#pragma unroll
                for (int di = 0; di < DT; ++di) {
                    const bf16* vr = vtb + (16 * di + c) * VP;
                    const bf16x8 vb = cat8<bf16x8>(load4<bf16x4>(vr + 4 * g), load4<bf16x4>(vr + 16 + 4 * g));
                    U[mt][di] = mma(eh, vb, U[mt][di]);
                    U[mt][di] = mma(el, vb, U[mt][di]);
                }
            }
        }
    }
    // Summary relative to the true chunk max (the reference's chunk_max).
    const size_t sbase = ((size_t)bh * NC + c_idx) * M;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const float f = exp2f_fast(R[mt] - Rt[mt]);    // <= 1
        if (g == 0) {
            cmax[sbase + m0 + 16 * mt + c] = Rt[mt] * kLn2;
            cden[sbase + m0 + 16 * mt + c] = den[mt] * f;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float fr = __shfl(f, 4 * g + r, 64);
#pragma unroll
            for (int di = 0; di < DT; ++di) cnum[(sbase + m0 + 16 * mt + 4 * g + r) * D + 16 * di + c] = U[mt][di][r] * fr;
        }
    }
}

// ---------------------------------------------------------------------------
// Phase 3.  grid = (NC, B*H), 64*NW threads, shared encoder/decoder weights.
// ---------------------------------------------------------------------------
template <int M, int D, int NW>
struct OutLayout {
    static constexpr int NT = 64 * NW;
    static constexpr int MW = M / NW;        // latents per wave (scores)
    static constexpr int MT = MW / 16;       // latent tiles per wave
    static constexpr int MTA = M / 16;       // latent tiles of the whole bank
    static constexpr int MB = M / 32;        // 32-latent k-blocks of the readout
    static constexpr int DW = D / NW;        // value columns per wave
    static constexpr int DTW = DW / 16;      // value tiles per wave
    static constexpr int KS = D / 32;        // k-steps of the scores
    static constexpr int WP = M + 8;         // padded row of W1[t][m]
    static constexpr int EP = T + 8;         // padded row of E^T[m][tau] and V^T[d][tau]
    static constexpr int GP = T + 4;         // padded row of G^T [t][tau]
    static constexpr int QP = D + 8;         // padded row of Q in LDS
    static constexpr int GROWS = T / NW;     // rows of G each wave reduces
    static_assert(MT % 2 == 0, "each wave needs an even number of latent tiles");
    static_assert(DW % 16 == 0, "value columns per wave must be a multiple of 16");
};

template <int M, int D, int NW>
__global__ __launch_bounds__(64 * NW, 1) void chunk_output_mfma(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, const float* __restrict__ pmax, const float* __restrict__ pden,
    const float* __restrict__ pnum, void* __restrict__ Y, int out_dtype) {
    using L = OutLayout<M, D, NW>;
    __shared__ __attribute__((aligned(16))) f16 wl[T * L::WP];         // W1[t][m]
    __shared__ __attribute__((aligned(16))) f16 etl[M * L::EP];        // E^T[m][tau]
    __shared__ __attribute__((aligned(16))) f16 vtl[D * L::EP];        // V^T[d][tau] (bf16 when moved)
    __shared__ __attribute__((aligned(16))) float gpl[NW * T * L::GP]; // partial G^T[t][tau] per wave
    __shared__ __attribute__((aligned(16))) float gfl[T * L::GP];      // reduced G^T[t][tau]
    __shared__ __attribute__((aligned(16))) float lsep[NW * T * 2];    // (max, sum) per wave/token
    __shared__ __attribute__((aligned(16))) float gaml[M];             // rescale factor per latent
    __shared__ __attribute__((aligned(16))) float invd[M];             // 1 / d0 (0 if d0 = 0)
    __shared__ int moved[NW];                                           // wave moved a reference max
    __shared__ __attribute__((aligned(16))) bf16 qs[M * L::QP];        // Q[h] (latent bank)

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int mw0 = w * L::MW;     // first latent of this wave's score slice
    const int dw0 = w * L::DW;     // first value column of this wave's state slice

    for (int vi = tid; vi < M * D / 8; vi += L::NT) {
        const int m = vi / (D / 8), d8 = vi % (D / 8);
        *reinterpret_cast<bf16x8*>(qs + m * L::QP + 8 * d8) = load8<bf16x8>(Q + ((size_t)h * M + m) * D + 8 * d8);
    }
    // Chunk prefix: max (log2 domain) and den of the score slice, and the
    // numerator U[all M][this wave's value columns].
    const size_t pbase = ((size_t)bh * NC + c_idx) * M;
    float R[L::MT][4], dn[L::MT][4];
#pragma unroll
    for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mw0 + 16 * mi + 4 * g + r;
            R[mi][r] = pmax[pbase + m] * kLog2e;
            dn[mi][r] = pden[pbase + m];
        }
    f32x4 U[L::MTA][L::DTW];
#pragma unroll
    for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
        for (int di = 0; di < L::DTW; ++di)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                U[mi][di][r] = pnum[(pbase + 16 * mi + 4 * g + r) * D + dw0 + 16 * di + c];
    __syncthreads();

    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    // K rows of the first subtile (B operands of S^T = Q K^T); each iteration
    // prefetches the next subtile's rows right after its scores are formed.
    bf16x8 kb[2][L::KS];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
        const int t = t_begin + 16 * ti + c;
#pragma unroll
        for (int ks = 0; ks < L::KS; ++ks)
            kb[ti][ks] = t < t_end ? load8<bf16x8>(K + row0 + (size_t)t * stride + 32 * ks + 8 * g) : zero8();
    }
    for (int t0 = t_begin; t0 < t_end; t0 += T) {
        // ---- V^T of this wave's value columns (wave-private rows of vtl), fp16
        const bool vbig = __any(stage_vt_f16<L::EP>(vtl, V, row0, stride, t0, t_end, dw0, L::DW, lane, 64));
        // ---- S^T = Q K^T for this wave's latents, log2 domain, invalid tokens -inf
        float s[L::MT][2][4];
        {
            f32x4 acc[L::MT][2];
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < L::KS; ++ks) {
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi) {
                    const bf16x8 qa = load8<bf16x8>(qs + (mw0 + 16 * mi + c) * L::QP + 32 * ks + 8 * g);
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) acc[mi][ti] = mma(qa, kb[ti][ks], acc[mi][ti]);
                }
            }
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const int t = t0 + T + 16 * ti + c;
#pragma unroll
                for (int ks = 0; ks < L::KS; ++ks)
                    kb[ti][ks] = t < t_end ? load8<bf16x8>(K + row0 + (size_t)t * stride + 32 * ks + 8 * g) : zero8();
            }
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const bool valid = t0 + 16 * ti + c < t_end;
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[mi][ti][r] = valid ? acc[mi][ti][r] * scale2 : kNegInf;
                }
        }
        // ---- per-latent reference max, E, cumulative den (rows of S^T, DPP over tokens)
        bf16x4 ehi[L::MT][2], elo[L::MT][2];   // E = hi + lo (bf16), for G
        float dt[L::MT][2][4], d0[L::MT][4];
        bool need = false;
#pragma unroll
        for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float mx = row_max16(fmaxf(s[mi][0][r], s[mi][1][r]));
                const bool mv = mx > R[mi][r] + kLazy;
                need |= mv;
                const float Rn = mv ? mx : R[mi][r];
                const float gam = mv ? exp2f_fast(R[mi][r] - Rn) : 1.0f;   // 0 when R = -inf
                R[mi][r] = Rn;
                const float e0 = exp2f_fast(s[mi][0][r] - Rn);
                const float e1 = exp2f_fast(s[mi][1][r] - Rn);
                SPLIT2(bf16, e0, ehi[mi][0][r], elo[mi][0][r]);
                SPLIT2(bf16, e1, ehi[mi][1][r], elo[mi][1][r]);
                const float base = dn[mi][r] * gam;
                d0[mi][r] = base;
                const float c0 = row_scan16(e0);
                const float tot0 = row_sum16(e0);
                const float c1 = row_scan16(e1);
                const float tot1 = row_sum16(e1);
                dt[mi][0][r] = base + c0;
                dt[mi][1][r] = base + tot0 + c1;
                dn[mi][r] = base + tot0 + tot1;
                const int m = mw0 + 16 * mi + 4 * g + r;
                if (c == 0) {
                    gaml[m] = gam;
                    invd[m] = base > 0.0f ? __builtin_amdgcn_rcpf(base) : 0.0f;
                }
                f16* er = etl + m * L::EP;     // E^T[m][tau] in fp16 for the update
                er[c] = (f16)e0;
                er[16 + c] = (f16)e1;
            }
        const bool wave_moved = __any(need);     // a wave-wide vote: every lane takes part
        if (lane == 0) moved[w] = wave_moved ? 1 : 0;
        // ---- decoder log-sum-exp over the latent bank, per token (cols of S^T)
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            float lm = kNegInf;
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) lm = fmaxf(lm, s[mi][ti][r]);
            lm = rows_max4(lm);
            float ls = 0.0f;
            if (lm != kNegInf) {
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) ls += exp2f_fast(s[mi][ti][r] - lm);
            }
            ls = rows_sum4(ls);
            if (g == 0) {
                lsep[(w * T + 16 * ti + c) * 2 + 0] = lm;
                lsep[(w * T + 16 * ti + c) * 2 + 1] = ls;
            }
        }
        __syncthreads();   // B1: lse partials, rescale factors, 1/d0, E^T visible

        float lse[2];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const int t = 16 * ti + c;
            float mm = kNegInf;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) mm = fmaxf(mm, lsep[(w2 * T + t) * 2]);
            float ss = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) {
                const float m2 = lsep[(w2 * T + t) * 2];
                if (m2 != kNegInf) ss += lsep[(w2 * T + t) * 2 + 1] * exp2f_fast(m2 - mm);
            }
            lse[ti] = mm + __log2f(ss);
        }
        // W1 (fp16 -> LDS) and W2 = hi + lo (bf16), one 32-latent block at a time,
        // each block folded straight into the partial G^T[tau][t] = sum_m E W2.
        f32x4 gacc[2][2];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) gacc[ti][0] = gacc[ti][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < L::MT / 2; ++kk) {
            bf16x4 whi[2][2], wlo[2][2];    // [latent tile of the block][t tile]
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int mi = 2 * kk + j;
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const bool valid = t0 + 16 * ti + c < t_end;
                    f16x4 w1;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float d_t = dt[mi][ti][r];
                        const float a = (valid && d_t > 0.0f) ? exp2f_fast(s[mi][ti][r] - lse[ti]) : 0.0f;
                        const float w2v = a * (d_t > 0.0f ? __builtin_amdgcn_rcpf(d_t) : 0.0f);
                        w1[r] = (f16)(w2v * d0[mi][r]);
                        SPLIT2(bf16, w2v, whi[j][ti][r], wlo[j][ti][r]);
                    }
                    *reinterpret_cast<f16x4*>(wl + (16 * ti + c) * L::WP + mw0 + 16 * mi + 4 * g) = w1;
                }
            }
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)          // t tile (cols of G^T)
#pragma unroll
                for (int ui = 0; ui < 2; ++ui) {    // tau tile (rows of G^T)
                    const bf16x8 wh = cat8<bf16x8>(whi[0][ti], whi[1][ti]);                  // W2^T[m][t]
                    const bf16x8 wo = cat8<bf16x8>(wlo[0][ti], wlo[1][ti]);
                    const bf16x8 eh = cat8<bf16x8>(ehi[2 * kk][ui], ehi[2 * kk + 1][ui]);    // E[tau][m]
                    const bf16x8 eo = cat8<bf16x8>(elo[2 * kk][ui], elo[2 * kk + 1][ui]);
                    gacc[ti][ui] = mma(eh, wh, gacc[ti][ui]);
                    gacc[ti][ui] = mma(eo, wh, gacc[ti][ui]);
                    gacc[ti][ui] = mma(eh, wo, gacc[ti][ui]);
                }
        }
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int ui = 0; ui < 2; ++ui)
                *reinterpret_cast<f32x4*>(gpl + (w * T + 16 * ti + c) * L::GP + 16 * ui + 4 * g) = gacc[ti][ui];
        // ---- move the numerator to the new reference maxima (rare after the first subtile)
        bool any_moved = false;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) any_moved |= moved[w2] != 0;
        if (any_moved) {
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi) {
                const f32x4 gm = *reinterpret_cast<const f32x4*>(gaml + 16 * mi + 4 * g);
#pragma unroll
                for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                    for (int r = 0; r < 4; ++r) U[mi][di][r] *= gm[r];
            }
        }
        __syncthreads();   // B2: W1 and the G^T partials visible

        // ---- reduce the G^T partials: wave w sums rows t in [w*GROWS, (w+1)*GROWS)
        for (int e2 = lane; e2 < L::GROWS * T; e2 += 64) {
            const int t = w * L::GROWS + e2 / T, tau = e2 % T;
            float acc = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) acc += gpl[(w2 * T + t) * L::GP + tau];
            gfl[t * L::GP + tau] = acc;
        }
        // ---- Y^T = z0^T W1^T with z0 = U / d0 (fp16 operands, both bounded)
        f32x4 yacc[L::DTW][2];
#pragma unroll
        for (int di = 0; di < L::DTW; ++di)
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < L::MB; ++kk) {
            f16x8 wb[2];
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const f16* wr = wl + (16 * ti + c) * L::WP + 32 * kk;
                wb[ti] = cat8<f16x8>(load4<f16x4>(wr + 4 * g), load4<f16x4>(wr + 16 + 4 * g));
            }
            const f32x4 ilo = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 4 * g);
            const f32x4 ihi = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 16 + 4 * g);
#pragma unroll
            for (int di = 0; di < L::DTW; ++di) {
                f16x8 za;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    za[r] = (f16)(U[2 * kk][di][r] * ilo[r]);
                    za[4 + r] = (f16)(U[2 * kk + 1][di][r] * ihi[r]);
                }
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = mma(za, wb[ti], yacc[di][ti]);
            }
        }
        {   // |z0| <= max|v|: only a value column with |v| > 65504 overflows fp16 -- redo in bf16
            bool bad = false;
#pragma unroll
            for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(yacc[di][ti][r]);
            if (__any(bad)) {
#pragma unroll
                for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int kk = 0; kk < L::MB; ++kk) {
                    bf16x8 wb[2];
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const f16* wr = wl + (16 * ti + c) * L::WP + 32 * kk;
#pragma unroll
                        for (int e2 = 0; e2 < 4; ++e2) {
                            wb[ti][e2] = (bf16)(float)wr[4 * g + e2];
                            wb[ti][4 + e2] = (bf16)(float)wr[16 + 4 * g + e2];
                        }
                    }
                    const f32x4 ilo = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 4 * g);
                    const f32x4 ihi = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 16 + 4 * g);
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di) {
                        bf16x8 za;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            za[r] = (bf16)(U[2 * kk][di][r] * ilo[r]);
                            za[4 + r] = (bf16)(U[2 * kk + 1][di][r] * ihi[r]);
                        }
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = mma(za, wb[ti], yacc[di][ti]);
                    }
                }
            }
        }
        __syncthreads();   // B2b: the reduced G^T is visible
        if (!vbig) {
            // ---- + V^T (G^T o causal), G = hi + lo (fp16) x V (fp16)
            f16x8 va[L::DTW];
#pragma unroll
            for (int di = 0; di < L::DTW; ++di) va[di] = load8<f16x8>(vtl + (dw0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const int t = 16 * ti + c;
                const float* gr = gfl + t * L::GP + 8 * g;
                const f32x4 ga = *reinterpret_cast<const f32x4*>(gr);
                const f32x4 gb = *reinterpret_cast<const f32x4*>(gr + 4);
                f16x8 gh, go;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    SPLIT2(f16, (8 * g + r <= t) ? ga[r] : 0.0f, gh[r], go[r]);
                    SPLIT2(f16, (8 * g + 4 + r <= t) ? gb[r] : 0.0f, gh[4 + r], go[4 + r]);
                }
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) {
                    yacc[di][ti] = mma(va[di], gh, yacc[di][ti]);
                    yacc[di][ti] = mma(va[di], go, yacc[di][ti]);
                }
            }
            // ---- U += E^T V (all latents, this wave's value columns), fp16 x fp16
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi) {
                const f16x8 ea = load8<f16x8>(etl + (16 * mi + c) * L::EP + 8 * g);
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) U[mi][di] = mma(ea, va[di], U[mi][di]);
            }
        } else {
            // a value outside the fp16 range in this wave's columns: bf16 V, exact splits
            bf16* vtb = reinterpret_cast<bf16*>(vtl);
            stage_vt_bf16<L::EP>(vtb, V, row0, stride, t0, t_end, dw0, L::DW, lane, 64);
            bf16x8 va[L::DTW];
#pragma unroll
            for (int di = 0; di < L::DTW; ++di) va[di] = load8<bf16x8>(vtb + (dw0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const int t = 16 * ti + c;
                bf16x8 gh, go;
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) {
                    const float x = gfl[t * L::GP + 8 * g + e2];
                    SPLIT2(bf16, (8 * g + e2 <= t) ? x : 0.0f, gh[e2], go[e2]);
                }
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) {
                    yacc[di][ti] = mma(va[di], gh, yacc[di][ti]);
                    yacc[di][ti] = mma(va[di], go, yacc[di][ti]);
                }
            }
            for (int mi = 0; mi < L::MTA; ++mi) {
                const f16x8 ea = load8<f16x8>(etl + (16 * mi + c) * L::EP + 8 * g);
                bf16x8 eh, el;
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) SPLIT2(bf16, (float)ea[e2], eh[e2], el[e2]);
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) {
                    U[mi][di] = mma(eh, va[di], U[mi][di]);
                    U[mi][di] = mma(el, va[di], U[mi][di]);
                }
            }
        }
        // ---- store Y[b, t, h, d] for this wave's value columns
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const int t = t0 + 16 * ti + c;
            if (t < t_end) {
#pragma unroll
                for (int di = 0; di < L::DTW; ++di)
                    store4(Y, row0 + (size_t)t * stride + dw0 + 16 * di + 4 * g, yacc[di][ti], out_dtype);
            }
        }
        __syncthreads();   // B3: LDS is rewritten by the next subtile
    }
}

}  // namespace mfma

using namespace mfma;

bool mfma_prepare_supported(int dtype, int64_t M, int64_t Dk, int64_t Dv) {
    return dtype == FLARE_BF16 && Dk == Dv && (Dk == 64 || Dk == 128) && M % 32 == 0 && M >= 32 && M <= kMaxPrepM;
}

bool mfma_output_supported(int dtype, int out_dtype, bool shared, int64_t M, int64_t Dk, int64_t Dv) {
    return dtype == FLARE_BF16 && shared && Dk == Dv && (Dk == 64 || Dk == 128) && (M == 128 || M == 256) &&
           (out_dtype == FLARE_BF16 || out_dtype == FLARE_F32);
}

int launch_prepare_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                        int64_t M, int64_t D, float scale, int64_t chunk, float* cmax, float* cden,
                        float* cnum, hipStream_t stream) {
    FLARE_REQUIRE(chunk % T == 0, "chunk_prepare_mfma: chunk must be a multiple of %d", T);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    dim3 block((unsigned)(64 * (M / 32)));
    const float s2 = scale * kLog2e;
    if (D == 64)
        hipLaunchKernelGGL(chunk_prepare_mfma<64>, grid, block, 0, stream, (const bf16*)Q, (const bf16*)K,
                           (const bf16*)V, (int)N, (int)H, (int)M, s2, (int)chunk, cmax, cden, cnum);
    else
        hipLaunchKernelGGL(chunk_prepare_mfma<128>, grid, block, 0, stream, (const bf16*)Q, (const bf16*)K,
                           (const bf16*)V, (int)N, (int)H, (int)M, s2, (int)chunk, cmax, cden, cnum);
    return check_launch("chunk_prepare_mfma");
}

int launch_output_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                       int64_t M, int64_t D, float scale, int64_t chunk, const float* pmax,
                       const float* pden, const float* pnum, void* Y, int out_dtype, hipStream_t stream) {
    FLARE_REQUIRE(chunk % T == 0, "chunk_output_mfma: chunk must be a multiple of %d", T);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_OUT_MFMA(MM, DD, NWW)                                                                    \
    hipLaunchKernelGGL((chunk_output_mfma<MM, DD, NWW>), grid, dim3(64 * NWW), 0, stream,             \
                       (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                       pmax, pden, pnum, Y, out_dtype)
    if (M == 128 && D == 64) FLARE_OUT_MFMA(128, 64, 4);
    else if (M == 128 && D == 128) FLARE_OUT_MFMA(128, 128, 4);
    else if (M == 256 && D == 64) FLARE_OUT_MFMA(256, 64, 4);
    else FLARE_OUT_MFMA(256, 128, 8);
#undef FLARE_OUT_MFMA
    return check_launch("chunk_output_mfma");
}

}  // namespace flare
