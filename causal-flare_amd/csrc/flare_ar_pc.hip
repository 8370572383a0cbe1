// flare_ar_pc.hip -- phase 3 of the chunked causal FLARE forward on gfx950 with
// wave-specialised producer and consumer waves (bf16 inputs, shared
// encoder/decoder weights, M in {128, 256}, D in {64, 128}).
//
// One workgroup of 2 NPW waves replays one chunk of one (b,h) in 32-token
// subtiles.  Waves 0 .. NPW-1 (producers) own M/NPW latents each; the other NPW
// waves (consumers) own D/NPW value columns each and the numerator
// U[M][their columns] in registers.  In
// iteration j the producers turn subtile j into its softmax operands while the
// consumers fold subtile j-1 into the output and the state, so that on every
// SIMD one VALU-heavy producer wave runs beside one MFMA-heavy consumer wave.
// The operands cross through double-buffered LDS with one barrier per
// iteration; producers never wait for one another.
//
// Notation (log2 domain, S = scale log2(e) k_t . q_m):
//   R[m]      lazy reference of latent m (moves when a score passes it by more
//             than kLazy, or den passes kDenMax; otherwise fixed)
//   E[t,m]    = 2^(S - R)                d_t[m] = d0[m] + sum_{tau<=t} E[tau,m]
//   alpha     = softmax over all M latents of S[t,:] (the decoder weights)
//   W2[t,m]   = alpha[t,m] / d_t[m]      G[t,tau] = sum_m W2[t,m] E[tau,m]
//   y_t       = sum_m W2[t,m] U[m] + sum_{tau<=t} G[t,tau] v_tau,   then U += E^T V
// Per subtile each producer forms S for its latents, E (fp16 E^T to LDS) and
// the cumulative den (an MFMA of E16 against a triangular ones matrix), and
// publishes its partial (max, sum) of the token softmax; the producers
// meet at an LDS counter (consumers never wait there) and each scales its own
// weights by f_w(t) = 2^(lm_w(t) - lse_t).  alpha = E 2^(R - Rmax) 2^(Rmax - lm_w)
// f_w reuses E (no second exponential) while Rmax - lm_w stays in range.  The
// producers then write W1 (fp16: W2, or W2 d0 when the group moved a reference,
// in which case the consumer reads out z0 = U / d0) and their partial G_w
// (fp32).  Consumers read out, sum the partial G, and update U.  This is the
// tokenwise recurrence of the reference (training.py:1282-1393,
// reference.py:446-496) regrouped into 16x16x32 contractions; operand
// precision is that of the single-role kernel in flare_ar_mfma.hip, except
// that G = W2 E uses the fp16 E of the numerator update on the common path.
#include <type_traits>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {
namespace mfma {

// Producer meetings of chunk_output_pc that gave up waiting (a fault counter that
// the host reads with flare_device_faults; it should stay 0).
__device__ unsigned int g_meet_timeouts = 0;
// Sleeps (s_sleep 1, about 64 clocks each) a producer waits at a meeting before it
// gives up: about 28 ms, far beyond any legitimate wait (a few microseconds).
constexpr int kMeetSpinLimit = 1 << 20;
int g_spin_limit = kMeetSpinLimit;

template <int M, int D, int NPW>
struct PCLayout {
    static constexpr int NP = NPW;           // producer waves
    static constexpr int NCW = NPW;          // consumer waves
    static constexpr int NT = 64 * (NP + NCW);
    static constexpr int MP = M / NP;        // latents per producer
    static constexpr int MTP = MP / 16;      // latent tiles per producer
    static constexpr int MBP = MP / 32;      // 32-latent k-blocks per producer group
    static constexpr int MTA = M / 16;
    static constexpr int DC = D / NCW;       // value columns per consumer
    static constexpr int DTC = DC / 16;
    static constexpr int KS = D / 32;        // k-steps of the scores
    static constexpr int KC = D / 8;         // 16-byte chunks of a K row
    static constexpr int WP = M + 8;         // padded row of q[t][m] (fp16)
    static constexpr int EP = T + 8;         // padded row of E^T[m][tau], V^T[d][tau] (16-bit)
    static constexpr int GP = 16 + 4;        // padded row of a 16x16 fp32 partial-G tile
    static constexpr float kVCap = 2048.0f;      // bound on |V'| and |z'| (fp16 operands)
    static constexpr float kLazyE = 256.0f;      // 2^kLazy: an E above it moves the reference
    static constexpr float kFactorMax = 100.0f;  // largest Rmax - lm (log2) for the factorised p
    static_assert(MTP % 2 == 0, "each producer needs an even number of latent tiles");
    static_assert(DC % 16 == 0, "value columns per consumer must be a multiple of 16");
};

// SEP: separate decoder weights.  alpha [B*H, N, M] (fp16) then holds the
// decoder softmax, written by decoder_alpha_mfma; the producers read it in place
// of the token softmax of the shared scores (no meeting, no factorised p).
template <int M, int D, int NPW, bool SEP, bool F16>
__global__ __launch_bounds__(128 * NPW, 4 / NPW) void chunk_output_pc(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, const float* __restrict__ pmax, const float* __restrict__ pden,
    const float* __restrict__ pnum, void* __restrict__ Y, int out_dtype, const int32_t* __restrict__ tmask,
    const f16* __restrict__ alpha, int* __restrict__ redo, int spin_limit) {
    using L = PCLayout<M, D, NPW>;
    // K rows of the even / odd subtiles (swizzled); two arrays rather than one so
    // that reads of one never wait on the DMA that fills the other
    __shared__ __attribute__((aligned(16))) bf16 ksl0[T * D];
    __shared__ __attribute__((aligned(16))) bf16 ksl1[T * D];
    __shared__ __attribute__((aligned(16))) f16 etl[2][M * L::EP];              // E^T[m][tau]
    __shared__ __attribute__((aligned(16))) f16 wl[2][T * L::WP];               // q or q d0, [t][m]
    __shared__ __attribute__((aligned(16))) float gpl[2][L::NP * 3 * 16 * L::GP];  // partial G, 3 causal tiles
    __shared__ __attribute__((aligned(16))) float2 lsep[2][L::NP * T];          // producers' (lm_w, sum p) per token
    __shared__ __attribute__((aligned(16))) float gaml[2][M];                   // rescale factor (moved groups)
    __shared__ __attribute__((aligned(16))) float d0l[2][M];                    // den at the subtile start
    __shared__ int movedl[2][L::NP];
    __shared__ __attribute__((aligned(16))) f16 vtl[D * L::EP];                 // V^T, consumer-private rows
    __shared__ __attribute__((aligned(16))) f16 tril[2 * 64 * 8];               // triangular B operand per lane
    __shared__ __attribute__((aligned(16))) float arl[M];                       // 2^(R - Rmax) per latent
    __shared__ int psync;                                                       // producer arrivals (monotonic)
    __shared__ int redol;                                                       // a reference jumped past kJumpMax

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const int NS = (t_end - t_begin + T - 1) / T;
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    const size_t pbase = ((size_t)bh * NC + c_idx) * M;

    if (w < L::NP) {
        // =========================== producer ===========================
        const int mp0 = w * L::MP;
        // Q rows of this wave's latents as MFMA A operands (rows m, k = d)
        bf16x8 qa[L::MTP][L::KS];
#pragma unroll
        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
            for (int kq = 0; kq < L::KS; ++kq)
                qa[mi][kq] = load8<bf16x8>(Q + ((size_t)h * M + mp0 + 16 * mi + c) * D + 32 * kq + 8 * g);
        // Upper-triangular ones as the B operand of the cumulative sums over the
        // subtile, per lane in LDS: tri[ti][e] = 1 when tau = 8 g + e <= t = 16 ti + c.
        if (w == 0) {
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                f16x8 tr;
#pragma unroll
                for (int e = 0; e < 8; ++e) tr[e] = (f16)(8 * g + e <= 16 * ti + c ? 1.0f : 0.0f);
                *reinterpret_cast<f16x8*>(tril + (ti * 64 + lane) * 8) = tr;
            }
        }
        // reference starts at the prefix's log-sum-exp: den = 1, U = z
        float R[L::MTP][4], dn[L::MTP][4];
        bool dnbig = false;
        bool rinf = false;   // some latent of this lane has no reference yet (R = -inf)
#pragma unroll
        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = mp0 + 16 * mi + 4 * g + r;
                const float pd = pden[pbase + m];
                R[mi][r] = pd > 0.0f ? pmax[pbase + m] * kLog2e + __log2f(pd) : kNegInf;
                dn[mi][r] = pd > 0.0f ? 1.0f : 0.0f;
                rinf |= R[mi][r] == kNegInf;
            }
        // Rmax = max_m R over the wave's latents, ar = 2^(R - Rmax); refreshed when a reference moves
        float Rmax;
        auto refresh_ar = [&]() {
            float mx = kNegInf;
#pragma unroll
            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, R[mi][r]);
            Rmax = rows_max4(row_max16(mx));
            if (c == 0)
#pragma unroll
                for (int mi = 0; mi < L::MTP; ++mi) {
                    f32x4 a;
#pragma unroll
                    for (int r = 0; r < 4; ++r) a[r] = Rmax == kNegInf ? 0.0f : exp2f_fast(R[mi][r] - Rmax);
                    *reinterpret_cast<f32x4*>(arl + mp0 + 16 * mi + 4 * g) = a;
                }
        };
        refresh_ar();
        if (tid == 0) {
            psync = 0;
            redol = 0;
        }
        // The producers meet (consumers never take part): each adds one arrival
        // and waits for the count of meeting n (1, 2, ...), once per subtile.  Every
        // producer runs the same subtiles (j < NS), so the count always arrives; the
        // wait is still bounded: past spin_limit sleeps the wave gives up, counts a
        // fault in g_meet_timeouts and flags the chunk for the tokenwise replay,
        // which rewrites its outputs.
        auto meet = [&](int n) {
            if (lane == 0) __hip_atomic_fetch_add(&psync, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            int spins = 0;
            while (__hip_atomic_load(&psync, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < L::NP * n) {
                if (spins++ >= spin_limit) {
                    redol = 1;
                    if (lane == 0) atomicAdd(&g_meet_timeouts, 1u);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        };
        rows_to_lds<D, 64 * L::NP>(ksl0, K, row0, stride, t_begin, N, tid, lane);
        FLARE_WAIT_VMCNT(0);
        __syncthreads();   // B0: K rows of subtile 0 and the lane tables visible
        // One subtile per call.  The buffer parity is a compile-time constant, so each LDS
        // buffer below is one fixed array; the next subtile's K rows go by DMA
        // (global_load_lds) into the other K array while this one is read.
        auto subtile = [&](auto parity, int j) {
            constexpr int buf = decltype(parity)::value;
            const bf16* kj = buf ? ksl1 : ksl0;
            bf16* knext = buf ? ksl0 : ksl1;
            // Lane-derived values (LDS addresses above all) are rebuilt from an opaque
            // copy of the lane id each subtile instead of being held across the loop.
            int lq = lane;
            asm volatile("" : "+v"(lq));
            const int c = lq & 15, g = lq >> 4;
            if (j < NS) {
                const int t0 = t_begin + T * j;
                // token mask of this lane's tokens (loaded before the DMA, so waiting for it
                // leaves the DMA in flight); a masked token has S = -inf everywhere
                bool keep[2] = {true, true};
                if (tmask != nullptr) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int t = t0 + 16 * ti + c;
                        keep[ti] = t >= t_end || tmask[(size_t)b * N + t] != 0;
                    }
                }
                // decoder weights of this lane's tokens and latents (separate decoder only),
                // issued before the DMA for the same reason as the mask
                f16x4 af[L::MTP][2];
                if constexpr (SEP) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int t = t0 + 16 * ti + c;
                        const bool ok = t < t_end;
                        const f16* arow = alpha + ((size_t)bh * N + (ok ? t : t0)) * M + mp0 + 4 * g;
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
                            af[mi][ti] = ok ? load4<f16x4>(arow + 16 * mi) : f16x4{0, 0, 0, 0};
                    }
                }
                if (j + 1 < NS) rows_to_lds<D, 64 * L::NP>(knext, K, row0, stride, t0 + T, N, 64 * w + lq, lq);
                // ---- raw scores A = Q K^T for this wave's latents (S = scale2 A):
                //      acc[mi][ti][r] = A[t = 16 ti + c][m = 16 mi + 4 g + r], -inf for invalid tokens
                const bool ragged = t0 + T > t_end;
                f32x4 acc[L::MTP][2];
#pragma unroll
                for (int mi = 0; mi < L::MTP; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kq = 0; kq < L::KS; ++kq) {
                    bf16x8 kb[2];
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int row = 16 * ti + c;
                        kb[ti] = load8<bf16x8>(kj + row * D + 8 * swz<D>(row, 4 * kq + g));
                    }
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) acc[mi][ti] = mma_in<F16>(qa[mi][kq], kb[ti], acc[mi][ti]);
                }
                if (ragged || tmask != nullptr) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
                        if (t0 + 16 * ti + c >= t_end || !keep[ti])
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi) acc[mi][ti] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
                }
                // one tile of the same scores again (general path only)
                auto scores = [&](int mi, int ti) {
                    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
                    const int row = 16 * ti + c;
#pragma unroll
                    for (int kq = 0; kq < L::KS; ++kq)
                        a = mma_in<F16>(qa[mi][kq], load8<bf16x8>(kj + row * D + 8 * swz<D>(row, 4 * kq + g)), a);
                    if ((ragged && t0 + row >= t_end) || !keep[ti]) a = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
                    return a;
                };
                // ---- E = 2^(S - R) against the current references; a reference moves
                //      (slow path, rare) when some E exceeds 2^kLazy or a den passed kDenMax
                float e[L::MTP][2][4];
                float emax = 0.0f;
#pragma unroll
                for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        e[mi][0][r] = exp2f_fast(fmaf(acc[mi][0][r], scale2, -R[mi][r]));
                        e[mi][1][r] = exp2f_fast(fmaf(acc[mi][1][r], scale2, -R[mi][r]));
                        emax = fmaxf(emax, fmaxf(e[mi][0][r], e[mi][1][r]));
                    }
                // token max over this wave's latents (log2 units; -inf for invalid tokens)
                float lm[2] = {0.0f, 0.0f};
                if constexpr (!SEP) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        float mx = kNegInf;
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
                            mx = max3_raw(mx, max3_raw(acc[mi][ti][0], acc[mi][ti][1], acc[mi][ti][2]), acc[mi][ti][3]);
                        lm[ti] = rows_max4(mx) * scale2;
                    }
                }
                dnbig |= rinf;   // some latent has no reference yet (fully masked so far): general path
                const bool moved = __any((emax > L::kLazyE) | dnbig);
                if (moved) {
                    float gam[L::MTP][4];
                    bool jump = false;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float mx = row_max16(fmaxf(acc[mi][0][r], acc[mi][1][r])) * scale2;
                            float Rn = mx > R[mi][r] + kLazy ? mx : R[mi][r];
                            // The running max of this latent at the subtile's first valid token:
                            // R, or (no reference yet) the smallest valid score.  Tokens whose
                            // running max lies more than kJumpMax below the new reference would
                            // see their den underflow against it: such a chunk is replayed
                            // tokenwise by the fp32 kernel afterwards.
                            const float s0 = acc[mi][0][r] * scale2, s1 = acc[mi][1][r] * scale2;
                            const float mn = -row_max16(fmaxf(s0 == kNegInf ? kNegInf : -s0, s1 == kNegInf ? kNegInf : -s1));
                            const float base = R[mi][r] == kNegInf ? mn : R[mi][r];
                            jump |= Rn - base > kJumpMax;
                            float g1 = exp2f_fast(R[mi][r] - Rn);                  // 0 when R = -inf
                            const float dd = dn[mi][r] * g1;
                            if (dd > kDenMax) {
                                Rn += __log2f(dd);
                                g1 = exp2f_fast(R[mi][r] - Rn);
                            }
                            gam[mi][r] = Rn == R[mi][r] ? 1.0f : g1;
                            R[mi][r] = Rn;
                            dn[mi][r] *= gam[mi][r];     // E is recomputed on the general path
                        }
                    if (jump) redol = 1;
                    refresh_ar();
                    rinf = false;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) rinf |= R[mi][r] == kNegInf;
                    // rescale factor and den at the subtile start: lanes c = 0..3 store rows r = c
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
                        float gsel = gam[mi][0], dsel = dn[mi][0];
#pragma unroll
                        for (int r = 1; r < 4; ++r) {
                            gsel = c == r ? gam[mi][r] : gsel;
                            dsel = c == r ? dn[mi][r] : dsel;
                        }
                        if (c < 4) {
                            gaml[buf][mp0 + 16 * mi + 4 * g + c] = gsel;
                            d0l[buf][mp0 + 16 * mi + 4 * g + c] = dsel;
                        }
                    }
                }
                // The factorised decoder weight p = E 2^(R - Rmax) 2^(Rmax - lm) needs
                // Rmax - lm in the fp32 range; else (extreme spreads) p = 2^(S - lm) directly.
                const bool slow = SEP ? moved
                                      : moved || __any((lm[0] > kNegInf) & (Rmax - lm[0] > L::kFactorMax)) ||
                                            __any((lm[1] > kNegInf) & (Rmax - lm[1] > L::kFactorMax));
                float bt[2] = {0.0f, 0.0f}, fw[2] = {0.0f, 0.0f};
                if constexpr (!SEP) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) bt[ti] = lm[ti] == kNegInf ? 0.0f : exp2f_fast(Rmax - lm[ti]);
                    // ---- the token softmax over all M latents: each producer publishes (lm_w, sum_m p)
                    //      per token, the four meet at an LDS counter, and each folds
                    //      f_w(t) = 2^(lm_w - lse_t) into its own weights (alpha = p f_w)
                    {
                        float lsum[2] = {0.0f, 0.0f};
                        if (!slow) {
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi) {
                                const f32x4 ar = *reinterpret_cast<const f32x4*>(arl + mp0 + 16 * mi + 4 * g);
#pragma unroll
                                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                                    for (int r = 0; r < 4; ++r) lsum[ti] = fmaf(e[mi][ti][r], ar[r], lsum[ti]);
                            }
                            lsum[0] *= bt[0];
                            lsum[1] *= bt[1];
                        } else {
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                                for (int ti = 0; ti < 2; ++ti) {
                                    const f32x4 sc = scores(mi, ti);
#pragma unroll
                                    for (int r = 0; r < 4; ++r)
                                        lsum[ti] += lm[ti] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[r], scale2, -lm[ti]));
                                }
                        }
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) {
                            const float l = rows_sum4(lsum[ti]);
                            if (g == 0) lsep[buf][w * T + 16 * ti + c] = float2{lm[ti], l};
                        }
                    }
                    meet(j + 1);
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int t = 16 * ti + c;
                        float2 pr[L::NP];
                        float mm = kNegInf;
#pragma unroll
                        for (int w2 = 0; w2 < L::NP; ++w2) {
                            pr[w2] = lsep[buf][w2 * T + t];
                            mm = fmaxf(mm, pr[w2].x);
                        }
                        float ss = 0.0f;
#pragma unroll
                        for (int w2 = 0; w2 < L::NP; ++w2) ss += pr[w2].y * exp2f_fast(pr[w2].x - mm);
                        fw[ti] = (lm[ti] == kNegInf) ? 0.0f : exp2f_fast(lm[ti] - mm) * __builtin_amdgcn_rcpf(ss);
                        bt[ti] *= fw[ti];
                    }
                }
                f16* et = etl[buf];
                f16* wq = wl[buf];
                f32x4 gacc[3];    // G_w^T tiles (t tile, tau tile) = (0,0), (1,0), (1,1)
#pragma unroll
                for (int q3 = 0; q3 < 3; ++q3) gacc[q3] = f32x4{0.f, 0.f, 0.f, 0.f};
                // E^T of latent tile mi (fp16) to LDS, and the cumulative den over the subtile
                // d_t = d0 + sum_{tau<=t} E16 by MFMA against tri with d0 as the accumulator's
                // start (the same fp16 E as the numerator update); dcum[ti][r] is d_t for
                // t = 16 ti + c, m = 16 mi + 4 g + r.
                auto cumulate = [&](int mi, const float (&em)[2][4], f16x4 (&e16)[2], f32x4 (&dcum)[2]) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        e16[ti] = __builtin_convertvector((f32x4{em[ti][0], em[ti][1], em[ti][2], em[ti][3]}), f16x4);
#pragma unroll
                        for (int r = 0; r < 4; ++r) et[(mp0 + 16 * mi + 4 * g + r) * L::EP + 16 * ti + c] = e16[ti][r];
                    }
                    const f16x8 ea = load8<f16x8>(et + (mp0 + 16 * mi + c) * L::EP + 8 * g);
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
                        dcum[ti] = mma(ea, load8<f16x8>(tril + (ti * 64 + lane) * 8),
                                       f32x4{dn[mi][0], dn[mi][1], dn[mi][2], dn[mi][3]});
                };
                dnbig = false;
                if (!slow) {
                    // ---- common path: W2 = alpha / d_t <= 1 (d_t >= d0 >= 1), so W2 and E go to
                    //      MFMA as fp16 (W2 split hi + lo); W1 = W2
#pragma unroll
                    for (int kk = 0; kk < L::MBP; ++kk) {
                        f16x4 whi[2][2], wlo[2][2], e16[2][2];
#pragma unroll
                        for (int jb = 0; jb < 2; ++jb) {
                            const int mi = 2 * kk + jb;
                            f32x4 dcum[2];
                            cumulate(mi, e[mi], e16[jb], dcum);
                            const f32x4 ar = *reinterpret_cast<const f32x4*>(arl + mp0 + 16 * mi + 4 * g);
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti) {
                                float q[4];
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    const float p = SEP ? (float)af[mi][ti][r] : e[mi][ti][r] * (ar[r] * bt[ti]);   // alpha
                                    q[r] = p * __builtin_amdgcn_rcpf(dcum[ti][r]);
                                }
                                split_f16x4(q, whi[jb][ti], wlo[jb][ti]);
                                *reinterpret_cast<f16x4*>(wq + (16 * ti + c) * L::WP + mp0 + 16 * mi + 4 * g) = whi[jb][ti];
                            }
#pragma unroll
                            for (int r = 0; r < 4; ++r) {      // den at the subtile end (column t = 31)
                                dn[mi][r] = row_bcast15(dcum[1][r]);
                                dnbig |= dn[mi][r] > kDenMax;
                            }
                        }
#pragma unroll
                        for (int q3 = 0; q3 < 3; ++q3) {
                            const int ti = q3 == 0 ? 0 : 1, ui = q3 == 2 ? 1 : 0;
                            const f16x8 ea = cat8<f16x8>(e16[0][ui], e16[1][ui]);
                            gacc[q3] = mma(ea, cat8<f16x8>(whi[0][ti], whi[1][ti]), gacc[q3]);
                            gacc[q3] = mma(ea, cat8<f16x8>(wlo[0][ti], wlo[1][ti]), gacc[q3]);
                        }
                    }
                } else {
                    // ---- general path: alpha = 2^(S - lm) f_w, guarded 1 / d_t, W1 = W2 d0 when a reference
                    //      moved (the consumer then reads out z0 = U / d0), hi/lo bf16 splits for G
#pragma unroll
                    for (int kk = 0; kk < L::MBP; ++kk) {
                        bf16x4 ehi[2][2], elo[2][2], whi[2][2], wlo[2][2];
#pragma unroll
                        for (int jb = 0; jb < 2; ++jb) {
                            const int mi = 2 * kk + jb;
                            // scores and E of the tile again: keeps acc and e dead on this path
                            const f32x4 sc[2] = {scores(mi, 0), scores(mi, 1)};
                            float em[2][4];
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    em[ti][r] = R[mi][r] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[ti][r], scale2, -R[mi][r]));
                            // E^T (fp16) to LDS; the cumulative den in fp32 (DPP scans over the token
                            // lanes): here E may lie far below the fp16 range
                            f32x4 dcum[2];
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                et[(mp0 + 16 * mi + 4 * g + r) * L::EP + c] = (f16)em[0][r];
                                et[(mp0 + 16 * mi + 4 * g + r) * L::EP + 16 + c] = (f16)em[1][r];
                                const float c0 = row_scan16(em[0][r]);
                                dcum[0][r] = c0;
                                dcum[1][r] = row_bcast15(c0) + row_scan16(em[1][r]);
                            }
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti) {
                                float q[4];
                                f16x4 w1;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    const float dt = dn[mi][r] + dcum[ti][r];
                                    const float p = SEP ? (float)af[mi][ti][r]
                                                        : lm[ti] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[ti][r], scale2, -lm[ti])) * fw[ti];
                                    q[r] = dt > 0.0f ? p / dt : 0.0f;
                                    w1[r] = (f16)(moved ? q[r] * dn[mi][r] : q[r]);
                                }
                                split_bf16x4(em[ti][0], em[ti][1], em[ti][2], em[ti][3], ehi[jb][ti], elo[jb][ti]);
                                split_bf16x4(q[0], q[1], q[2], q[3], whi[jb][ti], wlo[jb][ti]);
                                *reinterpret_cast<f16x4*>(wq + (16 * ti + c) * L::WP + mp0 + 16 * mi + 4 * g) = w1;
                            }
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                dn[mi][r] += row_bcast15(dcum[1][r]);
                                dnbig |= dn[mi][r] > kDenMax;
                            }
                        }
#pragma unroll
                        for (int q3 = 0; q3 < 3; ++q3) {
                            const int ti = q3 == 0 ? 0 : 1, ui = q3 == 2 ? 1 : 0;
                            const bf16x8 wh = cat8<bf16x8>(whi[0][ti], whi[1][ti]);
                            const bf16x8 wo = cat8<bf16x8>(wlo[0][ti], wlo[1][ti]);
                            const bf16x8 e_h = cat8<bf16x8>(ehi[0][ui], ehi[1][ui]);
                            const bf16x8 e_o = cat8<bf16x8>(elo[0][ui], elo[1][ui]);
                            gacc[q3] = mma(e_h, wh, gacc[q3]);
                            gacc[q3] = mma(e_o, wh, gacc[q3]);
                            gacc[q3] = mma(e_h, wo, gacc[q3]);
                        }
                    }
                }
                if (lane == 0) movedl[buf][w] = moved ? 1 : 0;
                // G_w[t][tau] rows t = 16 ti + c, cols tau = 16 ui + 4 g .. + 3
#pragma unroll
                for (int q3 = 0; q3 < 3; ++q3)
                    *reinterpret_cast<f32x4*>(gpl[buf] + ((w * 3 + q3) * 16 + c) * L::GP + 4 * g) = gacc[q3];
                FLARE_WAIT_VMCNT(0);     // this wave's K rows of the next subtile have landed
            }
            __syncthreads();   // hand-off: subtile j's operands visible, subtile j-1's consumed
        };
        for (int j = 0; j <= NS; j += 2) {
            subtile(std::integral_constant<int, 0>{}, j);
            if (j + 1 <= NS) subtile(std::integral_constant<int, 1>{}, j + 1);
        }
    } else {
        // =========================== consumer ===========================
        const int cw = w - L::NP;
        const int dc0 = cw * L::DC;
        f32x4 U[L::MTA][L::DTC];
#pragma unroll
        for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pd = pden[pbase + 16 * mi + 4 * g + r];
                const float ip = pd > 0.0f ? 1.0f / pd : 0.0f;
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
                    U[mi][di][r] = pnum[(pbase + 16 * mi + 4 * g + r) * D + dc0 + 16 * di + c] * ip;
            }
        // The wave keeps V' = V vs and U' = U vs with vs a power of two <= 1 chosen so
        // that |V'| and the prefix's |z'| stay below kVCap: every fp16 operand below is
        // then in range (|U'| <= kDenMax kVCap, |z0'| <= kVCap); y is scaled back at the store.
        float vs = 1.0f;
        {
            float zmax = 0.0f;
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
#pragma unroll
                    for (int r = 0; r < 4; ++r) zmax = fmaxf(zmax, fabsf(U[mi][di][r]));
            zmax = wave_max_dpp(zmax);
            if (zmax > L::kVCap && __builtin_isfinite(zmax)) {
                int e;
                frexpf(zmax / L::kVCap, &e);
                vs = ldexpf(1.0f, -e);
#pragma unroll
                for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) U[mi][di] *= vs;
            }
        }
        VTile<L::DC, 64, F16> vt;
        vt.load(V, row0, stride, t_begin, t_end, dc0, lane);
        __syncthreads();   // B0
        for (int it = 0; it <= NS; ++it) {
            if (it > 0) {
                const int j = it - 1;
                const int buf = j & 1;
                const int t0 = t_begin + T * j;
                int mv[L::NP];     // read ahead of this wave's V^T stores (LDS requests stay in order)
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2) mv[w2] = movedl[buf][w2];
                float vlane = vt.absmax(lane) * vs;
                vlane = __builtin_isfinite(vlane) ? vlane : 0.0f;   // inf / nan propagate unscaled
                if (__any(vlane > L::kVCap)) {      // rare: rescale the wave's columns
                    const float vmax = wave_max_dpp(vlane);
                    {
                        int e;
                        frexpf(vmax / L::kVCap, &e);
                        const float f = ldexpf(1.0f, -e);
                        vs *= f;
#pragma unroll
                        for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                            for (int di = 0; di < L::DTC; ++di) U[mi][di] *= f;
                    }
                }
                if (vs == 1.0f) vt.template store_f16_scaled<L::EP>(vtl, dc0, lane, 1.0f);
                else vt.template store_f16_scaled<L::EP>(vtl, dc0, lane, vs);
                // ---- readout at the subtile start: y = sum_m W1[t,m] U[m]; for the latents of a
                //      producer group that moved a reference, z0 = U / d0 against W1 = W2 d0
                auto normalise = [&](int w2, bool back) {
#pragma unroll
                    for (int mt = 0; mt < L::MTP; ++mt) {
                        const int mi = w2 * L::MTP + mt;
                        const f32x4 da = *reinterpret_cast<const f32x4*>(d0l[buf] + 16 * mi + 4 * g);
                        f32x4 gm;
                        if (back) {
                            gm = da;
                        } else {
                            const f32x4 ga = *reinterpret_cast<const f32x4*>(gaml[buf] + 16 * mi + 4 * g);
#pragma unroll
                            for (int r = 0; r < 4; ++r) gm[r] = da[r] > 0.0f ? ga[r] / da[r] : 0.0f;
                        }
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) U[mi][di] *= gm;
                    }
                };
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2)
                    if (mv[w2]) normalise(w2, false);
                f32x4 yt[L::DTC][2];
#pragma unroll
                for (int di = 0; di < L::DTC; ++di) yt[di][0] = yt[di][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                const f16* wq = wl[buf];
#pragma unroll
                for (int kk = 0; kk < L::MTA / 2; ++kk) {
                    f16x8 wb[2];
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const f16* wr = wq + (16 * ti + c) * L::WP + 32 * kk;
                        wb[ti] = cat8<f16x8>(load4<f16x4>(wr + 4 * g), load4<f16x4>(wr + 16 + 4 * g));
                    }
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) {
                        f16x8 za;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            za[r] = (f16)U[2 * kk][di][r];
                            za[4 + r] = (f16)U[2 * kk + 1][di][r];
                        }
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) yt[di][ti] = mma(za, wb[ti], yt[di][ti]);
                    }
                }
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2)
                    if (mv[w2]) normalise(w2, true);    // back from z0 to the (rescaled) numerator
                vt.load(V, row0, stride, t0 + T, t_end, dc0, lane);   // the next subtile's V
                // ---- G^T B operands: t = 16 ti + c, tau = 8 g .. 8 g + 7 (hi + lo, fp16)
                f16x8 gh[2], go[2];
                {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {    // sum the producers' partial tiles here
                        const int t = 16 * ti + c;
                        const int ui = g >> 1;     // tau tile
                        float ga[8];
#pragma unroll
                        for (int e2 = 0; e2 < 8; ++e2) ga[e2] = 0.0f;
                        if (ui <= ti) {
                            const int q3 = ti + ui;     // (0,0) -> 0, (1,0) -> 1, (1,1) -> 2
#pragma unroll
                            for (int w2 = 0; w2 < L::NP; ++w2) {
                                const float* src = gpl[buf] + ((w2 * 3 + q3) * 16 + c) * L::GP + 8 * (g & 1);
                                const f32x4 a0 = *reinterpret_cast<const f32x4*>(src);
                                const f32x4 a1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
                                for (int e2 = 0; e2 < 4; ++e2) {
                                    ga[e2] += a0[e2];
                                    ga[4 + e2] += a1[e2];
                                }
                            }
#pragma unroll
                            for (int e2 = 0; e2 < 8; ++e2)
                                if (8 * g + e2 > t) ga[e2] = 0.0f;
                        }
#pragma unroll
                        for (int e2 = 0; e2 < 8; e2 += 2) {
                            f16x2 hh, ll;
                            split_f16_pair(ga[e2], ga[e2 + 1], hh, ll);
                            gh[ti][e2] = hh[0];
                            gh[ti][e2 + 1] = hh[1];
                            go[ti][e2] = ll[0];
                            go[ti][e2 + 1] = ll[1];
                        }
                    }
                }
                const f16* et = etl[buf];
                {
                    // ---- + V'^T G^T (fp16), then U' += E^T V' (fp16 x fp16)
                    f16x8 va[L::DTC];
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) va[di] = load8<f16x8>(vtl + (dc0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) {
                            yt[di][ti] = mma(va[di], gh[ti], yt[di][ti]);
                            yt[di][ti] = mma(va[di], go[ti], yt[di][ti]);
                        }
#pragma unroll
                    for (int mi = 0; mi < L::MTA; ++mi) {
                        const f16x8 ea = load8<f16x8>(et + (16 * mi + c) * L::EP + 8 * g);
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) U[mi][di] = mma(ea, va[di], U[mi][di]);
                    }
                }
                // ---- Y[b, t, h, d] for this wave's value columns
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const int t = t0 + 16 * ti + c;
                    if (t < t_end) {
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di)
                            store4(Y, row0 + (size_t)t * stride + dc0 + 16 * di + 4 * g,
                                   vs == 1.0f ? yt[di][ti] : yt[di][ti] * (1.0f / vs), out_dtype);
                    }
                }
            }
            __syncthreads();   // hand-off
        }
    }
    if (redo != nullptr) {
        __syncthreads();
        if (tid == 0) redo[(size_t)bh * NC + c_idx] = redol;
    }
}

// ---------------------------------------------------------------------------
// Phase 1 with the same wave roles: chunk summaries (max, den, num) of one chunk
// of one (b,h), the reference's flare_chunk_prepare (training.py:914-1018).
// Producers form S = K Q^T with tokens as rows (lane: 4 tokens of one latent),
// keep the lazy reference R, the true max and den per latent, and write
// E^T (fp16, 8-byte stores) for the subtile; consumers fold it into
// U[M][their columns] += E^T V.  Same hand-off, K DMA and V scaling as the
// output kernel above.  The summary is returned relative to the true chunk
// max: (max, den 2^(R - max), U 2^(R - max)) in natural-log units.
// ---------------------------------------------------------------------------
template <int M, int D, int NPW, bool F16>
__global__ __launch_bounds__(128 * NPW, 4 / NPW) void chunk_prepare_pc(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, float* __restrict__ cmax, float* __restrict__ cden, float* __restrict__ cnum,
    const int32_t* __restrict__ tmask) {
    using L = PCLayout<M, D, NPW>;
    // K rows of subtiles j = 0, 1, 2 mod 3: fetched by DMA two subtiles ahead
    __shared__ __attribute__((aligned(16))) bf16 ksl0[T * D];
    __shared__ __attribute__((aligned(16))) bf16 ksl1[T * D];
    __shared__ __attribute__((aligned(16))) bf16 ksl2[T * D];
    __shared__ __attribute__((aligned(16))) f16 etl[2][M * L::EP];              // E^T[m][tau]
    __shared__ __attribute__((aligned(16))) float gaml[2][M];                   // rescale factor (moved groups)
    __shared__ int movedl[2][L::NP];
    __shared__ __attribute__((aligned(16))) f16 vtl[D * L::EP];                 // V^T, consumer-private rows
    __shared__ __attribute__((aligned(16))) float fl[M];                        // 2^(R - max) at the end

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const int NS = (t_end - t_begin + T - 1) / T;
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    const size_t sbase = ((size_t)bh * NC + c_idx) * M;

    if (w < L::NP) {
        // =========================== producer ===========================
        const int mp0 = w * L::MP;
        // Q rows of this wave's latents as MFMA B operands (n = m, k = d)
        bf16x8 qb[L::MTP][L::KS];
#pragma unroll
        for (int mt = 0; mt < L::MTP; ++mt)
#pragma unroll
            for (int kq = 0; kq < L::KS; ++kq)
                qb[mt][kq] = load8<bf16x8>(Q + ((size_t)h * M + mp0 + 16 * mt + c) * D + 32 * kq + 8 * g);
        // per latent m = mp0 + 16 mt + c (replicated over g): reference R and true max rt
        // (log2 units); dl is this lane's part of den
        float R[L::MTP], rt[L::MTP], dl[L::MTP];
#pragma unroll
        for (int mt = 0; mt < L::MTP; ++mt) {
            R[mt] = kNegInf;
            rt[mt] = kNegInf;
            dl[mt] = 0.0f;
        }
        constexpr int NKL = rows_to_lds_count<D, 64 * L::NP>();   // DMA loads per lane per subtile
        rows_to_lds<D, 64 * L::NP>(ksl0, K, row0, stride, t_begin, N, tid, lane);
        if (NS > 1) rows_to_lds<D, 64 * L::NP>(ksl1, K, row0, stride, t_begin + T, N, tid, lane);
        FLARE_WAIT_VMCNT(0);
        lds_barrier();   // B0
        // one subtile per call; j mod 3 is a compile-time constant so that each K
        // buffer is one fixed array
        auto subtile = [&](auto phase, int j) {
            constexpr int k3 = decltype(phase)::value;
            constexpr int buf = k3 & 1;     // unused when j is odd/even mixed below
            (void)buf;
            const bf16* kj = k3 == 0 ? ksl0 : (k3 == 1 ? ksl1 : ksl2);
            bf16* kfar = k3 == 0 ? ksl2 : (k3 == 1 ? ksl0 : ksl1);
            int lq = lane;
            asm volatile("" : "+v"(lq));
            const int c = lq & 15, g = lq >> 4;
            if (j < NS) {
                const int buf = j & 1;
                const int t0 = t_begin + T * j;
                const bool far = j + 2 < NS;
                // token mask of this lane's tokens t = 16 ti + 4 g + r (loaded before the DMA)
                bool keep[2][4] = {{true, true, true, true}, {true, true, true, true}};
                if (tmask != nullptr) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int t = t0 + 16 * ti + 4 * g + r;
                            keep[ti][r] = t >= t_end || tmask[(size_t)b * N + t] != 0;
                        }
                }
                if (far) rows_to_lds<D, 64 * L::NP>(kfar, K, row0, stride, t0 + 2 * T, N, 64 * w + lq, lq);
                // ---- A = K Q^T, tokens as rows: acc[mt][ti][r] = A[t = 16 ti + 4 g + r][m = 16 mt + c]
                f32x4 acc[L::MTP][2];
#pragma unroll
                for (int mt = 0; mt < L::MTP; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kq = 0; kq < L::KS; ++kq) {
                    bf16x8 ka[2];
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int row = 16 * ti + c;
                        ka[ti] = load8<bf16x8>(kj + row * D + 8 * swz<D>(row, 4 * kq + g));
                    }
#pragma unroll
                    for (int mt = 0; mt < L::MTP; ++mt)
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) acc[mt][ti] = mma_in<F16>(ka[ti], qb[mt][kq], acc[mt][ti]);
                }
                if (t0 + T > t_end || tmask != nullptr) {      // the ragged last subtile, masked tokens
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (t0 + 16 * ti + 4 * g + r >= t_end || !keep[ti][r])
#pragma unroll
                                for (int mt = 0; mt < L::MTP; ++mt) acc[mt][ti][r] = kNegInf;
                }
                // ---- lazy reference: checked per lane, moved (to the exact max over the latent) rarely
                float mx[L::MTP];
                bool need = false;
#pragma unroll
                for (int mt = 0; mt < L::MTP; ++mt) {
                    float x = max3_raw(acc[mt][0][0], acc[mt][0][1], acc[mt][0][2]);
                    x = max3_raw(x, acc[mt][0][3], acc[mt][1][0]);
                    x = max3_raw(x, acc[mt][1][1], acc[mt][1][2]);
                    mx[mt] = fmaxf(x, acc[mt][1][3]) * scale2;
                    rt[mt] = max3_raw(rt[mt], mx[mt], mx[mt]);
                    need |= mx[mt] > R[mt] + kLazy;
                }
                const bool moved = __any(need);
                if (moved) {
#pragma unroll
                    for (int mt = 0; mt < L::MTP; ++mt) {
                        const float m4 = rows_max4(mx[mt]);
                        const bool mv = m4 > R[mt] + kLazy;
                        const float Rn = mv ? m4 : R[mt];
                        const float gam = mv ? exp2f_fast(R[mt] - Rn) : 1.0f;     // 0 when R = -inf
                        R[mt] = Rn;
                        dl[mt] *= gam;
                        if (g == 0) gaml[buf][mp0 + 16 * mt + c] = gam;
                    }
                }
                if (lane == 0) movedl[buf][w] = moved ? 1 : 0;
                // ---- E = 2^(S - R): den partial, and E^T (fp16) to LDS, four tokens per store.
                //      A latent with no reference yet (every token so far masked) has E = 0.
                f16* et = etl[buf];
#pragma unroll
                for (int mt = 0; mt < L::MTP; ++mt) {
                    const float nR = R[mt] == kNegInf ? kNegInf : -R[mt];
                    float es = 0.0f;
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        f32x4 e;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            e[r] = exp2f_fast(fmaf(acc[mt][ti][r], scale2, nR));
                            es = (ti == 0 && r == 0) ? e[r] : es + e[r];   // e >= 0: 0 + e = e
                        }
                        *reinterpret_cast<f16x4*>(et + (mp0 + 16 * mt + c) * L::EP + 16 * ti + 4 * g) =
                            __builtin_convertvector(e, f16x4);
                    }
                    dl[mt] += es;
                }
                // this wave's K rows of the next subtile have landed (those of j + 2 may not)
                if (far) FLARE_WAIT_VMCNT(NKL);
                else FLARE_WAIT_VMCNT(0);
            }
            lds_barrier();   // hand-off: subtile j's E^T visible, subtile j-1's consumed
        };
        for (int j = 0; j <= NS; j += 3) {
            subtile(std::integral_constant<int, 0>{}, j);
            if (j + 1 <= NS) subtile(std::integral_constant<int, 1>{}, j + 1);
            if (j + 2 <= NS) subtile(std::integral_constant<int, 2>{}, j + 2);
        }
        // ---- the summary relative to the true chunk max
#pragma unroll
        for (int mt = 0; mt < L::MTP; ++mt) {
            const float Rt = rows_max4(rt[mt]);
            const float den = rows_sum4(dl[mt]);
            const float f = Rt == kNegInf ? 0.0f : exp2f_fast(R[mt] - Rt);    // <= 1
            if (g == 0) {
                const int m = mp0 + 16 * mt + c;
                cmax[sbase + m] = Rt * kLn2;
                cden[sbase + m] = den * f;
                fl[m] = f;
            }
        }
        lds_barrier();   // fl visible
    } else {
        // =========================== consumer ===========================
        const int cw = w - L::NP;
        const int dc0 = cw * L::DC;
        f32x4 U[L::MTA][L::DTC];
#pragma unroll
        for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
            for (int di = 0; di < L::DTC; ++di) U[mi][di] = f32x4{0.f, 0.f, 0.f, 0.f};
        float vs = 1.0f;     // V' = V vs, U' = U vs (powers of two keep |V'| <= kVCap)
        // V of subtiles j (vt) and j + 1 (vn) in registers: fetched two subtiles ahead
        VTile<L::DC, 64, F16> vt, vn;
        vt.load(V, row0, stride, t_begin, t_end, dc0, lane);
        vn.load(V, row0, stride, t_begin + T, t_end, dc0, lane);
        lds_barrier();   // B0
        for (int it = 0; it <= NS; ++it) {
            if (it > 0) {
                const int j = it - 1;
                const int buf = j & 1;
                const int t0 = t_begin + T * j;
                int mv[L::NP];
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2) mv[w2] = movedl[buf][w2];
                float vlane = vt.absmax(lane) * vs;
                vlane = __builtin_isfinite(vlane) ? vlane : 0.0f;
                if (__any(vlane > L::kVCap)) {
                    int e;
                    frexpf(wave_max_dpp(vlane) / L::kVCap, &e);
                    const float f = ldexpf(1.0f, -e);
                    vs *= f;
#pragma unroll
                    for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) U[mi][di] *= f;
                }
                if (vs == 1.0f) vt.template store_f16_scaled<L::EP>(vtl, dc0, lane, 1.0f);
                else vt.template store_f16_scaled<L::EP>(vtl, dc0, lane, vs);
                vt = vn;
                vn.load(V, row0, stride, t0 + 2 * T, t_end, dc0, lane);   // V of subtile j + 2
                // rescale the rows of groups that moved a reference
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2)
                    if (mv[w2]) {
#pragma unroll
                        for (int mt = 0; mt < L::MTP; ++mt) {
                            const int mi = w2 * L::MTP + mt;
                            const f32x4 ga = *reinterpret_cast<const f32x4*>(gaml[buf] + 16 * mi + 4 * g);
#pragma unroll
                            for (int di = 0; di < L::DTC; ++di) U[mi][di] *= ga;
                        }
                    }
                // ---- U' += E^T V' (fp16 x fp16)
                const f16* et = etl[buf];
                f16x8 va[L::DTC];
#pragma unroll
                for (int di = 0; di < L::DTC; ++di) va[di] = load8<f16x8>(vtl + (dc0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
                for (int mi = 0; mi < L::MTA; ++mi) {
                    const f16x8 ea = load8<f16x8>(et + (16 * mi + c) * L::EP + 8 * g);
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) U[mi][di] = mma(ea, va[di], U[mi][di]);
                }
            }
            lds_barrier();   // hand-off
        }
        lds_barrier();   // the producers' fl
        const float iv = 1.0f / vs;
#pragma unroll
        for (int mi = 0; mi < L::MTA; ++mi) {
            const f32x4 fa = *reinterpret_cast<const f32x4*>(fl + 16 * mi + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
                    cnum[(sbase + 16 * mi + 4 * g + r) * D + dc0 + 16 * di + c] = U[mi][di][r] * fa[r] * iv;
        }
    }
}

// ---------------------------------------------------------------------------
// Decoder weights for separate decoder tensors (reference flare_chunk_decoder_lse,
// training.py:1106-1188, and the exp(a - lse) of flare_chunk_fwd):
//   alpha[bh][t][m] = softmax over m of scale qd_t . kd_m   (fp16; 0 for a masked token),
// and, when lse is given, LSE_dec[bh][t] = log sum_m exp(scale qd_t . kd_m).
// grid (ceil(N / 128), B*H), 4 waves; wave w takes tokens 32 w .. 32 w + 31 of the
// block, with Kd rows as the A operand and the token rows as B.
// ---------------------------------------------------------------------------
template <int M, int D, bool F16>
__global__ __launch_bounds__(256) void decoder_alpha_mfma(const bf16* __restrict__ Qd, const bf16* __restrict__ Kd,
                                                          int N, int H, float scale2,
                                                          const int32_t* __restrict__ tmask, f16* __restrict__ alpha,
                                                          float* __restrict__ lse) {
    constexpr int MT = M / 16, KS = D / 32;
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = lane & 15, g = lane >> 4;
    const int tb = blockIdx.x * 128 + 32 * w;
    bf16x8 bq[2][KS];
    bool valid[2];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
        const int t = tb + 16 * ti + c;
        valid[ti] = t < N && (tmask == nullptr || tmask[(size_t)b * N + t] != 0);
        const bf16* row = Qd + (((size_t)b * N + min(t, N - 1)) * H + h) * D;
#pragma unroll
        for (int kq = 0; kq < KS; ++kq) bq[ti][kq] = t < N ? load8<bf16x8>(row + 32 * kq + 8 * g) : zero8();
    }
    f32x4 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kq = 0; kq < KS; ++kq) {
            const bf16x8 a = load8<bf16x8>(Kd + ((size_t)h * M + 16 * mt + c) * D + 32 * kq + 8 * g);
            acc[mt][0] = mma_in<F16>(a, bq[0][kq], acc[mt][0]);
            acc[mt][1] = mma_in<F16>(a, bq[1][kq], acc[mt][1]);
        }
    }
    // acc[mt][ti][r] = a[m = 16 mt + 4 g + r][t = tb + 16 ti + c]
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
        float mx = kNegInf;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[mt][ti][r] *= scale2;
                mx = fmaxf(mx, acc[mt][ti][r]);
            }
        mx = rows_max4(mx);
        float sum = 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[mt][ti][r] = exp2f_fast(acc[mt][ti][r] - mx);
                sum += acc[mt][ti][r];
            }
        sum = rows_sum4(sum);
        const float inv = valid[ti] ? 1.0f / sum : 0.0f;
        const int t = tb + 16 * ti + c;
        if (lse != nullptr && g == 0 && t < N) lse[(size_t)bh * N + t] = valid[ti] ? (mx + __log2f(sum)) * kLn2 : kNegInf;
        if (t < N) {
            f16* dst = alpha + ((size_t)bh * N + t) * M + 4 * g;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f16x4 o;
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = (f16)(acc[mt][ti][r] * inv);
                *reinterpret_cast<f16x4*>(dst + 16 * mt) = o;
            }
        }
    }
}

}  // namespace mfma

using namespace mfma;

int launch_decoder_alpha(const void* Qd, const void* Kd, int64_t B, int64_t N, int64_t H, int64_t M, int64_t D,
                         float scale, const int32_t* tmask, void* alpha, float* lse, bool f16in, hipStream_t stream) {
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "decoder_alpha_mfma: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    dim3 grid((unsigned)((N + 127) / 128), (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_DEC_ALPHA_T(MM, DD, F)                                                                     \
    hipLaunchKernelGGL((decoder_alpha_mfma<MM, DD, F>), grid, dim3(256), 0, stream, (const bf16*)Qd,      \
                       (const bf16*)Kd, (int)N, (int)H, s2, tmask, (f16*)alpha, lse)
#define FLARE_DEC_ALPHA(MM, DD)                        \
    do {                                               \
        if (f16in) FLARE_DEC_ALPHA_T(MM, DD, true);    \
        else FLARE_DEC_ALPHA_T(MM, DD, false);         \
    } while (0)
    if (M == 128 && D == 64) FLARE_DEC_ALPHA(128, 64);
    else if (M == 128 && D == 128) FLARE_DEC_ALPHA(128, 128);
    else if (M == 256 && D == 64) FLARE_DEC_ALPHA(256, 64);
    else FLARE_DEC_ALPHA(256, 128);
#undef FLARE_DEC_ALPHA
#undef FLARE_DEC_ALPHA_T
    return check_launch("decoder_alpha_mfma");
}

int launch_output_pc(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* pmax, const float* pden,
                     const float* pnum, void* Y, int out_dtype, const int32_t* tmask, const void* alpha,
                     bool f16in, int* redo, hipStream_t stream, bool record, float power) {
    FLARE_REQUIRE(chunk % T == 0, "chunk_output_pc: chunk must be a multiple of %d", T);
    FLARE_REQUIRE(power <= 0.0f || output_tr_enabled(), "chunk_output_pc: the stablemax encoder runs on chunk_output_tr");
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "chunk_output_pc: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    if (output_tr_enabled())
        return launch_output_tr(Q, K, V, B, N, H, M, D, scale, chunk, pmax, pden, pnum, Y, out_dtype, tmask, alpha,
                                f16in, redo, g_spin_limit, stream, record, power);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_OUT_PC_SEP(MM, DD, NW, SP, F)                                                                  \
    hipLaunchKernelGGL((chunk_output_pc<MM, DD, NW, SP, F>), grid, dim3(128 * NW), 0, stream, (const bf16*)Q, \
                       (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, pmax, pden, pnum, Y,    \
                       out_dtype, tmask, (const f16*)alpha, redo, g_spin_limit)
#define FLARE_OUT_PC(MM, DD, NW)                                  \
    do {                                                          \
        if (f16in) {                                              \
            if (alpha) FLARE_OUT_PC_SEP(MM, DD, NW, true, true);  \
            else FLARE_OUT_PC_SEP(MM, DD, NW, false, true);       \
        } else {                                                  \
            if (alpha) FLARE_OUT_PC_SEP(MM, DD, NW, true, false); \
            else FLARE_OUT_PC_SEP(MM, DD, NW, false, false);      \
        }                                                         \
    } while (0)
    // The 128 x 64 bank runs 2 + 2 waves (72 KiB of LDS: two workgroups share a CU);
    // the larger banks 4 + 4 (one workgroup fills a CU).
    if (M == 128 && D == 64) FLARE_OUT_PC(128, 64, 2);
    else if (M == 128 && D == 128) FLARE_OUT_PC(128, 128, 4);
    else if (M == 256 && D == 64) FLARE_OUT_PC(256, 64, 4);
    else FLARE_OUT_PC(256, 128, 4);
#undef FLARE_OUT_PC
#undef FLARE_OUT_PC_SEP
    return check_launch("chunk_output_pc");
}

}  // namespace flare

namespace flare {
using namespace mfma;

int launch_prepare_pc(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                      int64_t D, float scale, int64_t chunk, float* cmax, float* cden, float* cnum,
                      const int32_t* tmask, bool f16in, hipStream_t stream) {
    if (prepare_tr_enabled())
        return launch_prepare_tr(Q, K, V, B, N, H, M, D, scale, chunk, cmax, cden, cnum, tmask, f16in, stream);
    FLARE_REQUIRE(chunk % T == 0, "chunk_prepare_pc: chunk must be a multiple of %d", T);
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "chunk_prepare_pc: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_PREP_PC_T(MM, DD, NW, F)                                                                       \
    hipLaunchKernelGGL((chunk_prepare_pc<MM, DD, NW, F>), grid, dim3(128 * NW), 0, stream, (const bf16*)Q,    \
                       (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, cmax, cden, cnum, tmask)
#define FLARE_PREP_PC(MM, DD, NW)                         \
    do {                                                  \
        if (f16in) FLARE_PREP_PC_T(MM, DD, NW, true);     \
        else FLARE_PREP_PC_T(MM, DD, NW, false);          \
    } while (0)
    if (M == 128 && D == 64) FLARE_PREP_PC(128, 64, 2);
    else if (M == 128 && D == 128) FLARE_PREP_PC(128, 128, 4);
    else if (M == 256 && D == 64) FLARE_PREP_PC(256, 64, 4);
    else FLARE_PREP_PC(256, 128, 4);
#undef FLARE_PREP_PC
#undef FLARE_PREP_PC_T
    return check_launch("chunk_prepare_pc");
}

}  // namespace flare

extern "C" {

int flare_device_faults(void* stream, uint32_t* count, int reset) {
    FLARE_REQUIRE(count != nullptr, "device_faults: null pointer");
    hipStream_t st = (hipStream_t)stream;
    unsigned int v = 0;
    if (hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(flare::mfma::g_meet_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost,
                                 st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        flare::set_error("device_faults: %s", hipGetErrorString(hipGetLastError()));
        return FLARE_ERR_LAUNCH;
    }
    unsigned int vt = 0;
    if (flare::meet_timeouts_tr(st, &vt, reset != 0) != FLARE_OK) {
        flare::set_error("device_faults: %s", hipGetErrorString(hipGetLastError()));
        return FLARE_ERR_LAUNCH;
    }
    *count = v + vt;
    if (reset) {
        const unsigned int z = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(flare::mfma::g_meet_timeouts), &z, sizeof(z), 0, hipMemcpyHostToDevice,
                                   st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            flare::set_error("device_faults: %s", hipGetErrorString(hipGetLastError()));
            return FLARE_ERR_LAUNCH;
        }
    }
    return FLARE_OK;
}

int flare_set_meet_spin_limit(int limit) {
    FLARE_REQUIRE(limit >= 0, "set_meet_spin_limit: limit must be >= 0");
    flare::mfma::g_spin_limit = limit;
    return FLARE_OK;
}

}  // extern "C"
