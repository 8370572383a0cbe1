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
// Phase 1.  grid = (NC, B*H), NWP = M/32 waves.  Wave w owns latents
// 32w .. 32w+31 (two 16-latent tiles; their Q rows stay in registers) and
// every value column.  V and K of the next subtile are fetched while the
// current one is processed; V^T is double-buffered in LDS so one barrier per
// subtile suffices.  The per-latent maximum and den are kept per lane and
// reduced over the four lanes of a latent only when a reference max moves
// and at the end.
// ---------------------------------------------------------------------------
template <int D, int NWP>
__global__ __launch_bounds__(64 * NWP) void chunk_prepare_mfma(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, float* __restrict__ cmax, float* __restrict__ cden, float* __restrict__ cnum) {
    constexpr int M = 32 * NWP;
    constexpr int NT = 64 * NWP;
    constexpr int KS = D / 32;     // k-steps for the scores
    constexpr int DT = D / 16;     // value-column tiles
    constexpr int VP = T + 8;      // padded row of the transposed V tile
    __shared__ __attribute__((aligned(16))) f16 vtl[2][D * VP];
    __shared__ __attribute__((aligned(16))) bf16 ksl[2][T * D];   // K rows of a subtile (swizzled)
    __shared__ int vbig[2];        // subtile index whose V^T buffer holds a value outside fp16

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int m0 = 32 * w;                       // this wave's 32 latents

    // this wave's Q rows as MFMA B operands (n = m, k = d), held in registers
    bf16x8 qb[2][KS];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kq = 0; kq < KS; ++kq)
            qb[mt][kq] = load8<bf16x8>(Q + ((size_t)h * M + m0 + 16 * mt + c) * D + 32 * kq + 8 * g);
    f32x4 U[2][DT];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int di = 0; di < DT; ++di) U[mt][di] = f32x4{0.f, 0.f, 0.f, 0.f};
    // per latent m0 + 16 mt + c: R replicated over the four rows g; rt, dl per lane
    float R[2] = {kNegInf, kNegInf}, rt[2] = {kNegInf, kNegInf}, dl[2] = {0.f, 0.f};

    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    if (tid < 2) vbig[tid] = -1;
    // K rows go through registers (loaded a subtile ahead, stored before the barrier);
    // V comes through registers, also one subtile ahead.
    VTile<D, NT> vt;
    KRows<D, NT> kr;
    kr.load(K, row0, stride, t_begin, N, tid);
    kr.store(ksl[0], tid);
    vt.load(V, row0, stride, t_begin, t_end, 0, tid);
    __syncthreads();
    int j = 0;
    for (int t0 = t_begin; t0 < t_end; t0 += T, ++j) {
        f16* vtj = vtl[j & 1];
        const bf16* kj = ksl[j & 1];
        if (vt.template store_f16<VP>(vtj, 0, tid)) vbig[j & 1] = j;
        const bool more = t0 + T < t_end;
        // the next subtile's K rows through registers (stored to LDS before this
        // subtile's barrier) and its V rows (staged at the next subtile's start);
        // K is issued first, so that waiting for it leaves the V loads in flight
        if (more) kr.load(K, row0, stride, t0 + T, N, tid);
        vt.load(V, row0, stride, t0 + T, t_end, 0, tid);
        // S = K Q^T, tokens as rows: s[mt][ti][r] = S[t = 16 ti + 4 g + r][m = 16 mt + c]
        float s[2][2][4];
        {
            f32x4 acc[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kq = 0; kq < KS; ++kq) {
                bf16x8 ka[2];
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) ka[ti] = load8<bf16x8>(kj + (16 * ti + c) * D + 8 * swz<D>(16 * ti + c, 4 * kq + g));
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) acc[mt][ti] = mma(ka[ti], qb[mt][kq], acc[mt][ti]);
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[mt][ti][r] = acc[mt][ti][r] * scale2;
            if (t0 + T > t_end) {      // the ragged last subtile
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (t0 + 16 * ti + 4 * g + r >= t_end) s[mt][ti][r] = kNegInf;
            }
        }
        // lazy reference max: checked per lane, moved (exact max over the latent) rarely
        float mx[2];
        bool need = false;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            mx[mt] = fmaxf(fmaxf(fmaxf(s[mt][0][0], s[mt][0][1]), fmaxf(s[mt][0][2], s[mt][0][3])),
                           fmaxf(fmaxf(s[mt][1][0], s[mt][1][1]), fmaxf(s[mt][1][2], s[mt][1][3])));
            rt[mt] = fmaxf(rt[mt], mx[mt]);
            need |= mx[mt] > R[mt] + kLazy;
        }
        if (__any(need)) {
            float gam[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float m4 = rows_max4(mx[mt]);
                const bool mv = m4 > R[mt] + kLazy;
                const float Rn = mv ? m4 : R[mt];
                gam[mt] = mv ? exp2f_fast(R[mt] - Rn) : 1.0f;     // 0 when R = -inf
                R[mt] = Rn;
                dl[mt] *= gam[mt];
            }
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
        float e[2][2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            float es = 0.0f;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    e[mt][ti][r] = exp2f_fast(s[mt][ti][r] - R[mt]);
                    es += e[mt][ti][r];
                }
            dl[mt] += es;
        }
        if (more) kr.store(ksl[(j + 1) & 1], tid);
        __syncthreads();   // V^T of this subtile (and its range flag), next K rows visible
        if (vbig[j & 1] != j) {
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
                    const f16* vr = vtj + (16 * di + c) * VP;
                    const f16x8 vb = cat8<f16x8>(load4<f16x4>(vr + 4 * g), load4<f16x4>(vr + 16 + 4 * g));
                    U[mt][di] = mma(ea, vb, U[mt][di]);
                }
            }
        } else {
            // a value outside the fp16 range: bf16 V and an exact hi/lo split of E
            __syncthreads();
            bf16* vtb = reinterpret_cast<bf16*>(vtj);
            stage_vt_bf16<VP>(vtb, V, row0, stride, t0, t_end, 0, D, tid, NT);
            __syncthreads();
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
        const float Rt = rows_max4(rt[mt]);
        const float den = rows_sum4(dl[mt]);
        const float f = exp2f_fast(R[mt] - Rt);    // <= 1
        if (g == 0) {
            cmax[sbase + m0 + 16 * mt + c] = Rt * kLn2;
            cden[sbase + m0 + 16 * mt + c] = den * f;
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
    static constexpr int EP = T + 8;         // padded row of E^T[m][tau], V^T[d][tau], G^T[t][tau] (16-bit)
    static constexpr int GP = 16 + 4;        // padded row of a 16x16 tile of the fp32 partials of G^T
    static constexpr int KC = D / 8;         // 16-byte chunks of a K / Q row in LDS (XOR-swizzled slots)
    static_assert(MT % 2 == 0, "each wave needs an even number of latent tiles");
    static_assert(DW % 16 == 0, "value columns per wave must be a multiple of 16");
};

template <int M, int D, int NW>
__global__ __launch_bounds__(64 * NW, 1) void chunk_output_mfma(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, const float* __restrict__ pmax, const float* __restrict__ pden,
    const float* __restrict__ pnum, void* __restrict__ Y, int out_dtype, int* __restrict__ redo) {
    using L = OutLayout<M, D, NW>;
    __shared__ __attribute__((aligned(16))) f16 wl[T * L::WP];         // W1[t][m]
    __shared__ __attribute__((aligned(16))) f16 etl[M * L::EP];        // E^T[m][tau] (fp16)
    __shared__ __attribute__((aligned(16))) f16 vtl[D * L::EP];        // V^T[d][tau], rows wave-private
    __shared__ __attribute__((aligned(16))) float gpl[NW * 3 * 16 * L::GP]; // partial G^T, 3 causal tiles per wave
    __shared__ __attribute__((aligned(16))) f16 gfh[T * L::EP];        // G^T = hi + lo (fp16), causal
    __shared__ __attribute__((aligned(16))) f16 gfo[T * L::EP];
    __shared__ __attribute__((aligned(16))) float2 lsep[NW * T];       // (max, sum) per wave/token
    __shared__ __attribute__((aligned(16))) float gaml[M];             // rescale factor per latent
    __shared__ __attribute__((aligned(16))) float d0l[M];              // den at the subtile start (after moves)
    __shared__ int moved[NW];                                           // wave moved a reference max
    __shared__ int redol;                                               // a reference jumped past kJumpMax
    __shared__ __attribute__((aligned(16))) bf16 qs[M * D];            // Q[h] (latent bank), swizzled rows
    __shared__ __attribute__((aligned(16))) bf16 ksl[T * D];           // K rows of the subtile, swizzled rows

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int mw0 = w * L::MW;     // first latent of this wave's score slice
    const int dw0 = w * L::DW;     // first value column of this wave's state slice

    // Rows of Q and K in LDS hold 16-byte chunk j at slot j ^ (row mod KC), so
    // that the 16 lanes reading one chunk of 16 consecutive rows hit distinct banks.
    auto slot = [](int row, int j) { return j ^ (row & (L::KC - 1)); };
    for (int vi = tid; vi < M * L::KC; vi += L::NT) {
        const int m = vi / L::KC, j = vi % L::KC;
        *reinterpret_cast<bf16x8*>(qs + m * D + 8 * slot(m, j)) = load8<bf16x8>(Q + ((size_t)h * M + m) * D + 8 * j);
    }
    // Chunk prefix: max (log2 domain) and den of the score slice, and the
    // numerator U[all M][this wave's value columns].
    const size_t pbase = ((size_t)bh * NC + c_idx) * M;
    // The reference R of a latent starts at the prefix's log-sum-exp, so that
    // den starts at 1 and the numerator at the prefix's normalised z.
    float R[L::MT][4], dn[L::MT][4];
#pragma unroll
    for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mw0 + 16 * mi + 4 * g + r;
            const float pd = pden[pbase + m];
            R[mi][r] = pd > 0.0f ? pmax[pbase + m] * kLog2e + __log2f(pd) : kNegInf;
            dn[mi][r] = pd > 0.0f ? 1.0f : 0.0f;
        }
    f32x4 U[L::MTA][L::DTW];
#pragma unroll
    for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pd = pden[pbase + 16 * mi + 4 * g + r];
            const float ip = pd > 0.0f ? 1.0f / pd : 0.0f;
#pragma unroll
            for (int di = 0; di < L::DTW; ++di)
                U[mi][di][r] = pnum[(pbase + 16 * mi + 4 * g + r) * D + dw0 + 16 * di + c] * ip;
        }

    if (tid == 0) redol = 0;     // visible after the first subtile's barriers
    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    VTile<L::DW, 64> vt;
    vt.load(V, row0, stride, t_begin, t_end, dw0, lane);
    // K rows of a subtile go straight from HBM to LDS (global_load_lds): each
    // lane moves one 16-byte chunk into slot `lane` of its wave's 1 KiB; rows
    // past the end of the sequence load row N-1 and are masked.  Issued for the
    // next subtile once every wave has formed its scores, waited for before the
    // barrier that precedes their use.
    auto load_k = [&](int t0n) {
        for (int e = tid; e < T * L::KC; e += L::NT) {
            const int row = e / L::KC, sl = e % L::KC;
            const int t = min(t0n + row, N - 1);
            const bf16* src = K + row0 + (size_t)t * stride + 8 * slot(row, sl);
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(ksl + (e - lane) * 8),
                                             16, 0, 0);
        }
    };
    load_k(t_begin);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int t0 = t_begin; t0 < t_end; t0 += T) {
        // ---- V^T of this wave's value columns (wave-private rows of vtl), fp16; fetch the next subtile
        const bool vbig = __any(vt.template store_f16<L::EP>(vtl, dw0, lane));
        vt.load(V, row0, stride, t0 + T, t_end, dw0, lane);
        // ---- S^T = Q K^T for this wave's latents, log2 domain, invalid tokens -inf
        float s[L::MT][2][4];
        {
            f32x4 acc[L::MT][2];
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kq = 0; kq < L::KS; ++kq) {
                bf16x8 kb[2];
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const int row = 16 * ti + c;
                    kb[ti] = load8<bf16x8>(ksl + row * D + 8 * slot(row, 4 * kq + g));
                }
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi) {
                    const int m = mw0 + 16 * mi + c;
                    const bf16x8 qa = load8<bf16x8>(qs + m * D + 8 * slot(m, 4 * kq + g));
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) acc[mi][ti] = mma(qa, kb[ti], acc[mi][ti]);
                }
            }
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[mi][ti][r] = acc[mi][ti][r] * scale2;
            if (t0 + T > t_end) {      // the ragged last subtile
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (t0 + 16 * ti + c >= t_end) s[mi][ti][r] = kNegInf;
            }
        }
        // ---- lazy reference: R moves when a score exceeds it by more than kLazy
        //      (to the exact row max) or when den has grown past 2^kDen (by
        //      log2 den), so E <= 2^kLazy and den, U / max|v| stay below 2^kDen
        //      at every subtile start.  Checked per lane; moved rarely.
        float gam[L::MT][4];
        bool need = false;
#pragma unroll
        for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                gam[mi][r] = 1.0f;
                need |= (fmaxf(s[mi][0][r], s[mi][1][r]) > R[mi][r] + kLazy) | (dn[mi][r] > kDenMax);
            }
        const bool wave_moved = __any(need);     // a wave-wide vote: every lane takes part
        if (wave_moved) {
            bool jump = false;
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float mx = row_max16(fmaxf(s[mi][0][r], s[mi][1][r]));
                    float Rn = mx > R[mi][r] + kLazy ? mx : R[mi][r];
                    // running max at the subtile's first valid token (R, or the smallest valid
                    // score when there is no reference yet); a move past kJumpMax above it
                    // sends the chunk to the tokenwise fp32 replay
                    const float s0 = s[mi][0][r], s1 = s[mi][1][r];
                    const float mn = -row_max16(fmaxf(s0 == kNegInf ? kNegInf : -s0, s1 == kNegInf ? kNegInf : -s1));
                    jump |= Rn - (R[mi][r] == kNegInf ? mn : R[mi][r]) > kJumpMax;
                    float g1 = exp2f_fast(R[mi][r] - Rn);                  // 0 when R = -inf
                    const float dd = dn[mi][r] * g1;
                    if (dd > kDenMax) {
                        const float lg = __log2f(dd);
                        Rn += lg;
                        g1 = exp2f_fast(R[mi][r] - Rn);
                    }
                    gam[mi][r] = Rn == R[mi][r] ? 1.0f : g1;
                    R[mi][r] = Rn;
                }
            if (jump) redol = 1;
        }
        // ---- decoder max over this wave's latents, per token (cols of S^T)
        float lm[2], off[2];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            float mx = kNegInf;
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
                mx = fmaxf(mx, fmaxf(fmaxf(s[mi][ti][0], s[mi][ti][1]), fmaxf(s[mi][ti][2], s[mi][ti][3])));
            lm[ti] = rows_max4(mx);
            off[ti] = lm[ti] == kNegInf ? 0.0f : lm[ti];
        }
        // ---- E = 2^(S - R) (hi + lo bf16 for G, fp16 E^T for the numerator), the
        //      cumulative den d_t (DPP scans over the token lanes), p = 2^(S - lm),
        //      and q = p / d_t
        bf16x4 ehi[L::MT][2], elo[L::MT][2];
        float q[L::MT][2][4], d0[L::MT][4];
        float ls[2] = {0.0f, 0.0f};
#pragma unroll
        for (int mi = 0; mi < L::MT; ++mi) {
            float e[2][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e0 = exp2f_fast(s[mi][0][r] - R[mi][r]);
                const float e1 = exp2f_fast(s[mi][1][r] - R[mi][r]);
                e[0][r] = e0;
                e[1][r] = e1;
                const int m = mw0 + 16 * mi + 4 * g + r;
                etl[m * L::EP + c] = (f16)e0;
                etl[m * L::EP + 16 + c] = (f16)e1;
                const float c0 = row_scan16(e0);
                const float c1 = row_scan16(e1);
                const float base = dn[mi][r] * gam[mi][r];
                const float b1 = base + row_bcast15(c0);
                d0[mi][r] = base;
                const float dt0 = base + c0, dt1 = b1 + c1;
                dn[mi][r] = b1 + row_bcast15(c1);
                const float p0 = exp2f_fast(s[mi][0][r] - off[0]);
                const float p1 = exp2f_fast(s[mi][1][r] - off[1]);
                ls[0] += p0;
                ls[1] += p1;
                q[mi][0][r] = dt0 > 0.0f ? p0 * __builtin_amdgcn_rcpf(dt0) : 0.0f;
                q[mi][1][r] = dt1 > 0.0f ? p1 * __builtin_amdgcn_rcpf(dt1) : 0.0f;
            }
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) split_bf16x4(e[ti][0], e[ti][1], e[ti][2], e[ti][3], ehi[mi][ti], elo[mi][ti]);
        }
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const float l = rows_sum4(ls[ti]);
            if (g == 0) lsep[w * T + 16 * ti + c] = float2{lm[ti], l};
        }
        // per-latent rescale factor and den at the subtile start (read by every
        // wave when any wave moved a reference): lanes c = 0..3 store rows r = c
#pragma unroll
        for (int mi = 0; mi < L::MT; ++mi) {
            float gsel = gam[mi][0], dsel = d0[mi][0];
#pragma unroll
            for (int r = 1; r < 4; ++r) {
                gsel = c == r ? gam[mi][r] : gsel;
                dsel = c == r ? d0[mi][r] : dsel;
            }
            if (c < 4) {
                gaml[mw0 + 16 * mi + 4 * g + c] = gsel;
                d0l[mw0 + 16 * mi + 4 * g + c] = dsel;
            }
        }
        if (lane == 0) moved[w] = wave_moved ? 1 : 0;
        __syncthreads();   // B1: lse partials, rescale factors, 1/d0, E^T visible; K rows consumed
        if (t0 + T < t_end) load_k(t0 + T);
        bool any_moved = false;     // some wave moved a reference in this subtile
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) any_moved |= moved[w2] != 0;

        // ---- f = 2^(lm_w - lse): alpha = p f, W2 = alpha / d_t = q f
        float f[2];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const int t = 16 * ti + c;
            float mm = kNegInf;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) mm = fmaxf(mm, lsep[w2 * T + t].x);
            float ss = 0.0f;     // NaN only when mm = -inf (no valid token), not used then
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) {
                const float2 e2 = lsep[w2 * T + t];
                ss += e2.y * exp2f_fast(e2.x - mm);
            }
            f[ti] = (mm == kNegInf) ? 0.0f : exp2f_fast(off[ti] - mm) * __builtin_amdgcn_rcpf(ss);
        }
        // W1 = W2 d0 (fp16 -> LDS) and W2 = hi + lo (bf16), one 32-latent block at a
        // time, each block folded straight into this wave's part of G^T[tau][t] = sum_m E W2.
        f32x4 gacc[3];    // (t tile, tau tile) = (0,0), (1,0), (1,1); (0,1) is above the diagonal
#pragma unroll
        for (int q3 = 0; q3 < 3; ++q3) gacc[q3] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < L::MT / 2; ++kk) {
            bf16x4 whi[2][2], wlo[2][2];    // [latent tile of the block][t tile]
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
                const int mi = 2 * kk + jb;
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    float w2v[4];
                    f16x4 w1;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        w2v[r] = q[mi][ti][r] * f[ti];
                        w1[r] = (f16)(any_moved ? w2v[r] * d0[mi][r] : w2v[r]);
                    }
                    split_bf16x4(w2v[0], w2v[1], w2v[2], w2v[3], whi[jb][ti], wlo[jb][ti]);
                    *reinterpret_cast<f16x4*>(wl + (16 * ti + c) * L::WP + mw0 + 16 * mi + 4 * g) = w1;
                }
            }
#pragma unroll
            for (int q3 = 0; q3 < 3; ++q3) {
                const int ti = q3 == 0 ? 0 : 1, ui = q3 == 2 ? 1 : 0;
                const bf16x8 wh = cat8<bf16x8>(whi[0][ti], whi[1][ti]);                  // W2^T[m][t]
                const bf16x8 wo = cat8<bf16x8>(wlo[0][ti], wlo[1][ti]);
                const bf16x8 e_h = cat8<bf16x8>(ehi[2 * kk][ui], ehi[2 * kk + 1][ui]);   // E[tau][m]
                const bf16x8 e_o = cat8<bf16x8>(elo[2 * kk][ui], elo[2 * kk + 1][ui]);
                gacc[q3] = mma(e_h, wh, gacc[q3]);
                gacc[q3] = mma(e_o, wh, gacc[q3]);
                gacc[q3] = mma(e_h, wo, gacc[q3]);
            }
        }
        // this wave's partial G^T: rows t = 16 ti + c, cols tau = 16 ui + 4 g .. + 3
#pragma unroll
        for (int q3 = 0; q3 < 3; ++q3) {
            const int ti = q3 == 0 ? 0 : 1, ui = q3 == 2 ? 1 : 0;
            *reinterpret_cast<f32x4*>(gpl + ((w * 3 + q3) * 16 + c) * L::GP + 4 * g) = gacc[q3];
        }
        // ---- a subtile where some reference moved (rare after the first): move the
        //      numerator and normalise it to z0 = U / d0 for the readout
        if (any_moved) {
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi) {
                const f32x4 ga = *reinterpret_cast<const f32x4*>(gaml + 16 * mi + 4 * g);
                const f32x4 da = *reinterpret_cast<const f32x4*>(d0l + 16 * mi + 4 * g);
                f32x4 gm;
#pragma unroll
                for (int r = 0; r < 4; ++r) gm[r] = da[r] > 0.0f ? ga[r] / da[r] : 0.0f;
#pragma unroll
                for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                    for (int r = 0; r < 4; ++r) U[mi][di][r] *= gm[r];
            }
        }
        __syncthreads();   // B2: W1 and the G^T partials visible

        // ---- reduce the partials into the causal G^T = hi + lo (fp16), two entries per step
        for (int e2 = tid; e2 < T * T / 2; e2 += L::NT) {
            const int t = e2 / (T / 2), tau = 2 * (e2 % (T / 2));
            float a0 = 0.0f, a1 = 0.0f;
            if (tau <= t) {
                const int q3 = (t >= 16) + (tau >= 16);
#pragma unroll
                for (int w2 = 0; w2 < NW; ++w2) {
                    const float2 pr = *reinterpret_cast<const float2*>(gpl + ((w2 * 3 + q3) * 16 + (t & 15)) * L::GP + (tau & 15));
                    a0 += pr.x;
                    a1 += pr.y;
                }
                if (tau + 1 > t) a1 = 0.0f;
            }
            f16x2 hh, ll;
            split_f16_pair(a0, a1, hh, ll);
            *reinterpret_cast<f16x2*>(gfh + t * L::EP + tau) = hh;
            *reinterpret_cast<f16x2*>(gfo + t * L::EP + tau) = ll;
        }
        // ---- Y^T = U^T W2^T at the subtile start.  No reference moved: d >= 1 so
        //      W2 <= 1 and |U| <= kDenMax max|v| (fp16 operands).  Some moved: the
        //      normalised pair z0 = U / d0, W1 = W2 d0 <= alpha instead.
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
#pragma unroll
            for (int di = 0; di < L::DTW; ++di) {
                f16x8 za;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    za[r] = (f16)U[2 * kk][di][r];
                    za[4 + r] = (f16)U[2 * kk + 1][di][r];
                }
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = mma(za, wb[ti], yacc[di][ti]);
            }
        }
        {   // an fp16 overflow (|v| beyond 65504 / kDenMax): redo in bf16 with z0, W1
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
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di) {
                        bf16x8 za;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            za[r] = (bf16)U[2 * kk][di][r];
                            za[4 + r] = (bf16)U[2 * kk + 1][di][r];
                        }
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) yacc[di][ti] = mma(za, wb[ti], yacc[di][ti]);
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);     // this wave's K rows of the next subtile have landed
        __syncthreads();   // B2b: the reduced G^T (and the next K rows) are visible
        if (any_moved) {    // back from z0 to the numerator
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi) {
                const f32x4 da = *reinterpret_cast<const f32x4*>(d0l + 16 * mi + 4 * g);
#pragma unroll
                for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                    for (int r = 0; r < 4; ++r) U[mi][di][r] *= da[r];
            }
        }
        if (!vbig) {
            // ---- + V^T G^T, G = hi + lo (fp16) x V (fp16)
            f16x8 va[L::DTW];
#pragma unroll
            for (int di = 0; di < L::DTW; ++di) va[di] = load8<f16x8>(vtl + (dw0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                const f16x8 gh = load8<f16x8>(gfh + (16 * ti + c) * L::EP + 8 * g);
                const f16x8 go = load8<f16x8>(gfo + (16 * ti + c) * L::EP + 8 * g);
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
                const f16x8 gh16 = load8<f16x8>(gfh + (16 * ti + c) * L::EP + 8 * g);
                const f16x8 go16 = load8<f16x8>(gfo + (16 * ti + c) * L::EP + 8 * g);
                bf16x8 gh, go;
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) SPLIT2(bf16, (float)gh16[e2] + (float)go16[e2], gh[e2], go[e2]);
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
    if (redo != nullptr && tid == 0) redo[(size_t)bh * NC + c_idx] = redol;
}

}  // namespace mfma

using namespace mfma;

bool mfma_prepare_supported(int dtype, int64_t M, int64_t Dk, int64_t Dv) {
    const bool shape = Dk == Dv && (Dk == 64 || Dk == 128);
    if (dtype == FLARE_BF16) return shape && M % 32 == 0 && M >= 32 && M <= kMaxPrepM;
    // fp16 inputs: the producer / consumer kernel only
    return dtype == FLARE_F16 && shape && output_pc_enabled() && (M == 128 || M == 256);
}

bool mfma_output_supported(int dtype, int out_dtype, bool shared, int64_t M, int64_t Dk, int64_t Dv) {
    const bool shape = shared && Dk == Dv && (Dk == 64 || Dk == 128) && (M == 128 || M == 256);
    if (dtype == FLARE_BF16) return shape && (out_dtype == FLARE_BF16 || out_dtype == FLARE_F32);
    return dtype == FLARE_F16 && shape && output_pc_enabled() && (out_dtype == FLARE_F16 || out_dtype == FLARE_F32);
}

int launch_prepare_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                        int64_t M, int64_t D, float scale, int64_t chunk, float* cmax, float* cden,
                        float* cnum, bool f16in, hipStream_t stream) {
    if (output_pc_enabled() && (M == 128 || M == 256))
        return launch_prepare_pc(Q, K, V, B, N, H, M, D, scale, chunk, cmax, cden, cnum, nullptr, f16in, stream);
    FLARE_REQUIRE(!f16in, "chunk_prepare_mfma: fp16 inputs need the producer/consumer kernel");
    FLARE_REQUIRE(chunk % T == 0, "chunk_prepare_mfma: chunk must be a multiple of %d", T);
    FLARE_REQUIRE(M % 32 == 0 && M >= 32 && M <= kMaxPrepM && (D == 64 || D == 128),
                  "chunk_prepare_mfma: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
    const int nwp = (int)(M / 32);
#define FLARE_PREP(DD, NN)                                                                              \
    hipLaunchKernelGGL((chunk_prepare_mfma<DD, NN>), grid, dim3(64 * NN), 0, stream, (const bf16*)Q,     \
                       (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, cmax, cden, cnum)
#define FLARE_PREP_D(DD)                      \
    switch (nwp) {                            \
        case 1: FLARE_PREP(DD, 1); break;     \
        case 2: FLARE_PREP(DD, 2); break;     \
        case 3: FLARE_PREP(DD, 3); break;     \
        case 4: FLARE_PREP(DD, 4); break;     \
        case 5: FLARE_PREP(DD, 5); break;     \
        case 6: FLARE_PREP(DD, 6); break;     \
        case 7: FLARE_PREP(DD, 7); break;     \
        default: FLARE_PREP(DD, 8); break;    \
    }
    if (D == 64) { FLARE_PREP_D(64) } else { FLARE_PREP_D(128) }
#undef FLARE_PREP_D
#undef FLARE_PREP
    return check_launch("chunk_prepare_mfma");
}

int launch_output_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                       int64_t M, int64_t D, float scale, int64_t chunk, const float* pmax,
                       const float* pden, const float* pnum, void* Y, int out_dtype, const int32_t* tmask,
                       bool f16in, int* redo, hipStream_t stream, bool record) {
    if (output_pc_enabled())
        return launch_output_pc(Q, K, V, B, N, H, M, D, scale, chunk, pmax, pden, pnum, Y, out_dtype, tmask, nullptr,
                                f16in, redo, stream, record);
    FLARE_REQUIRE(!f16in, "chunk_output_mfma: fp16 inputs need the producer/consumer kernel");
    FLARE_REQUIRE(tmask == nullptr, "chunk_output_mfma: token masks need the producer/consumer kernel");
    FLARE_REQUIRE(chunk % T == 0, "chunk_output_mfma: chunk must be a multiple of %d", T);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_OUT_MFMA(MM, DD, NWW)                                                                    \
    hipLaunchKernelGGL((chunk_output_mfma<MM, DD, NWW>), grid, dim3(64 * NWW), 0, stream,             \
                       (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                       pmax, pden, pnum, Y, out_dtype, redo)
    if (M == 128 && D == 64) FLARE_OUT_MFMA(128, 64, 4);
    else if (M == 128 && D == 128) FLARE_OUT_MFMA(128, 128, 4);
    else if (M == 256 && D == 64) FLARE_OUT_MFMA(256, 64, 4);
    else FLARE_OUT_MFMA(256, 128, 8);
#undef FLARE_OUT_MFMA
    return check_launch("chunk_output_mfma");
}

}  // namespace flare
