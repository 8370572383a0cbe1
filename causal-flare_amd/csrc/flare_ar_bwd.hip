// flare_ar_bwd.hip -- backward of the chunked causal FLARE forward (scalar-fp32 kernels).
//
// Replaces the reference's _chunked_flare_lse_backward_impl
// (causal_flare/autoregressive/training.py:4369-4918): given dY, the forward's
// inputs and its output Y, produce dQ, dK, dV and, for separate decoder
// weights, dQ_dec and dK_dec.
//
// Per (b, h) and latent m, with encoder scores s_tm = scale k_t.q_m, decoder
// scores a_tm = scale qd_t.kd_m, alpha_t = softmax_m(a_t), running den
// D_tm = sum_{tau<=t} e^{s_tau m} = e^{L_tm}, z_tm = U_tm / D_tm and
// y_t = sum_m alpha_tm z_tm, the gradients with g_t = dY_t are
//     gz_tm  = g_t . z_tm                     gy_t = g_t . y_t
//     da_tm  = alpha_tm (gz_tm - gy_t)
//     ds_tm  = sum_{t >= tau} e^{s_tau m - L_tm} alpha_tm (g_t . v_tau - gz_tm)
//     dv_tau = sum_{t >= tau} sum_m e^{s_tau m - L_tm} alpha_tm g_t
// and dQ, dK, dQ_dec, dK_dec are contractions of ds and da with K, Q, Qd, Kd.
// Every factor e^{s_tau - L_t} (t >= tau) is <= 1: D_t contains e^{s_tau}.
//
// The sequence is cut into chunks of kBT tokens.  Inside a chunk the pairs
// (tau, t) are summed exactly; later chunks enter through a reverse scan:
//     X_c,m = sum_{t > end_c} e^{Lend_c - L_tm} alpha_tm g_t      (Dv vector)
//     Y_c,m = sum_{t > end_c} e^{Lend_c - L_tm} alpha_tm gz_tm
// with Lend_c = L at the last token of chunk c, so that for tau in chunk c the
// later-chunk terms are e^{s_tau - Lend_c} (v_tau . X_c - Y_c) in ds and
// sum_m e^{s_tau - Lend_c} X_c in dv; both factors stay <= 1.  The chunk's
// starting state (max, den, num) comes from the forward's own prepare and
// prefix kernels run at chunk kBT.
//
// Kernels, in launch order:
//   bwd_stats    s, L, alpha per (t, m)                   grid (NC, BH)
//   bwd_gz       gz per (t, m), into C                    grid (NC, BH)
//   bwd_gy       gy = dY . Y per token                    grid (tokens)
//   bwd_summary  per-chunk terms of X, Y                  grid (NC, BH)
//   bwd_carry    reverse scan over chunks -> X_c, Y_c     grid (BH M Dv/4)
//   bwd_dv       dV                                        grid (NC, BH)
//   bwd_ds       ds (written over s)                      grid (NC, BH)
//   bwd_dk       dK, dQ_dec per token                     grid (N/32, BH)
//   bwd_dq       dQ, dK_dec partial sums per token group  grid (NG, BH, Dk/64)
//   bwd_reduce   sum of the partials over (b, group)
#include <stdio.h>

#include <type_traits>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {

constexpr int kBT = 32;        // tokens per backward chunk
constexpr int kBNT = 256;      // threads per workgroup; thread m owns latent m (M <= 256)
constexpr int kBSlab = 64;     // value / key columns per LDS slab
constexpr int kBP = 65;        // padded pitch of [kBT][64] LDS tiles read as scalars
constexpr int kBTok = 16;      // tokens per tile in the token-row kernels
constexpr int kBGroup = kBwdGroup;   // tokens per partial sum of dQ / dK_dec

__device__ __forceinline__ size_t tok_index(int b, int t, int h, int N, int H, int D) {
    return (((size_t)b * N + t) * H + h) * D;
}

constexpr float kBLog2e = 1.4426950408889634f;
constexpr int kGT = 68;        // pitch of the transposed GV tile and of 16-byte-read tiles

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// ---------------------------------------------------------------------------
// bwd_stats: per chunk, scores s2 = s log2(e) (encoder), L2 = log2 of the
// running den from the chunk's starting state, the decoder weights alpha and
// LA = L2 - log2(alpha), so that e^{s_tau - L_t} alpha_t = exp2(s2_tau - LA_t).
// S, L and LA hold log2-domain values: every later factor is one exp2.
// power > 0 (stablemax encoder): s2 = log2 s(a) with s(a) = (1 + |a|)^(+-p), the
// encoder weight in place of e^a; the decoder keeps the raw scores.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float stablemax_log2(float a, float p) {
    return a >= 0.0f ? p * __log2f(1.0f + a) : -p * __log2f(1.0f - a);
}

template <typename T, bool MF>
__global__ __launch_bounds__(kBNT) void bwd_stats_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ Qd, const T* __restrict__ Kd,
    int N, int H, int M, int Dk, float scale, bool shared, const float* __restrict__ pmax,
    const float* __restrict__ pden, float* __restrict__ S, float* __restrict__ L, float* __restrict__ AL,
    float* __restrict__ LA, float power) {
    __shared__ float kt[kBTok * 256];
    __shared__ float qdt[kBTok * 256];
    __shared__ float at[kBTok * 256];
    __shared__ float lse[kBTok];
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, tid = threadIdx.x, m = tid;
    const bool act = m < M;
    const int t0 = c * kBT, nt = min(kBT, N - t0);
    float mx = kNegInf, dn = 0.0f;      // running max (log2 units) and den relative to it
    if (act) {
        mx = pmax[((size_t)bh * NC + c) * M + m] * kBLog2e;
        dn = pden[((size_t)bh * NC + c) * M + m];
    }
    const T* qrow = Q + ((size_t)h * M + (act ? m : 0)) * Dk;
    const T* kdrow = Kd + ((size_t)h * M + (act ? m : 0)) * Dk;
    // MF (bf16 inputs with whole 16-latent / 32-column tiles): the scores on the
    // MFMA (exact: bf16 products, fp32 sums), written to LDS as [token][m]
    // (encoder in at, decoder in kt) for the thread of latent m
    constexpr bool kBf16 = std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value;   // 16-bit inputs
    constexpr bool mf = kBf16 && MF;
    for (int i0 = 0; i0 < nt; i0 += kBTok) {
        const int ni = min(kBTok, nt - i0);
        __syncthreads();
        if constexpr (mf) {
            {
                using namespace mfma;
                const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
                const bool ok = cl < ni;
                const size_t trow = tok_index(b, t0 + i0 + min(cl, ni - 1), h, N, H, Dk) + 8 * g4;
                const bf16* kr = reinterpret_cast<const bf16*>(K) + trow;
                const bf16* qdr = reinterpret_cast<const bf16*>(Qd) + trow;
                for (int mt = w; mt < M / 16; mt += kBNT / 64) {
                    const size_t lrow = ((size_t)h * M + 16 * mt + cl) * Dk + 8 * g4;
                    const bf16* qr = reinterpret_cast<const bf16*>(Q) + lrow;
                    const bf16* kdr = reinterpret_cast<const bf16*>(Kd) + lrow;
                    f32x4 se = f32x4{0.f, 0.f, 0.f, 0.f}, sd = f32x4{0.f, 0.f, 0.f, 0.f};
                    for (int k0 = 0; k0 < Dk; k0 += 32) {
                        se = mma_in<std::is_same<T, __half>::value>(load8<bf16x8>(qr + k0), ok ? load8<bf16x8>(kr + k0) : zero8(), se);
                        if (!shared) sd = mma_in<std::is_same<T, __half>::value>(load8<bf16x8>(kdr + k0), ok ? load8<bf16x8>(qdr + k0) : zero8(), sd);
                    }
                    // D[m = 16 mt + 4 g + r][token cl]
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        at[cl * M + 16 * mt + 4 * g4 + r] = se[r];
                        if (!shared) kt[cl * M + 16 * mt + 4 * g4 + r] = sd[r];
                    }
                }
            }
        } else {
            for (int e = tid; e < kBTok * Dk; e += kBNT) {
                const int i = e / Dk, d = e % Dk;
                const size_t gi = tok_index(b, t0 + i0 + i, h, N, H, Dk) + d;
                kt[e] = i < ni ? to_f32(K[gi]) : 0.0f;
                if (!shared) qdt[e] = i < ni ? to_f32(Qd[gi]) : 0.0f;
            }
        }
        __syncthreads();
        float lv[kBTok];
        if (act) {
            float as[kBTok], aa[kBTok];
#pragma unroll
            for (int i = 0; i < kBTok; ++i) as[i] = aa[i] = 0.0f;
            if constexpr (mf) {
#pragma unroll
                for (int i = 0; i < kBTok; ++i) {
                    as[i] = at[i * M + m];
                    if (!shared) aa[i] = kt[i * M + m];
                }
            }
            for (int d = 0; d < (mf ? 0 : Dk); d += 4) {
                const float q0 = to_f32(qrow[d]), q1 = to_f32(qrow[d + 1]), q2 = to_f32(qrow[d + 2]),
                            q3 = to_f32(qrow[d + 3]);
#pragma unroll
                for (int i = 0; i < kBTok; ++i) {
                    const float4 kr = ld4(kt + i * Dk + d);
                    as[i] += kr.x * q0 + kr.y * q1 + kr.z * q2 + kr.w * q3;
                }
                if (!shared) {
                    const float k0 = to_f32(kdrow[d]), k1 = to_f32(kdrow[d + 1]), k2 = to_f32(kdrow[d + 2]),
                                k3 = to_f32(kdrow[d + 3]);
#pragma unroll
                    for (int i = 0; i < kBTok; ++i) {
                        const float4 qr = ld4(qdt + i * Dk + d);
                        aa[i] += qr.x * k0 + qr.y * k1 + qr.z * k2 + qr.w * k3;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kBTok; ++i) {
                if (i < ni) {
                    const float s = as[i] * scale;
                    const float s2 = power > 0.0f ? stablemax_log2(s, power) : s * kBLog2e;
                    const float mn = fmaxf(mx, s2);
                    dn = dn * ex2(mx - mn) + ex2(s2 - mn);     // mx = -inf before the first token: ex2 -> 0
                    mx = mn;
                    const size_t o = ((size_t)bh * N + t0 + i0 + i) * M + m;
                    S[o] = s2;
                    lv[i] = mx + __log2f(dn);
                    L[o] = lv[i];
                    at[i * M + m] = shared ? s : aa[i] * scale;
                }
            }
        }
        __syncthreads();
        {   // decoder log-sum-exp per token: wavefront w handles tokens w, w+4, ...
            const int w = tid >> 6, lane = tid & 63;
            for (int i = w; i < ni; i += kBNT / 64) {
                float v = kNegInf;
                for (int mm = lane; mm < M; mm += 64) v = fmaxf(v, at[i * M + mm]);
                v = wave_max(v);
                float sm = 0.0f;
                for (int mm = lane; mm < M; mm += 64) sm += __expf(at[i * M + mm] - v);
                sm = wave_sum(sm);
                if (lane == 0) lse[i] = v + __logf(sm);
            }
        }
        __syncthreads();
        if (act) {
#pragma unroll
            for (int i = 0; i < kBTok; ++i) {
                if (i < ni) {
                    const size_t o = ((size_t)bh * N + t0 + i0 + i) * M + m;
                    const float la = at[i * M + m] - lse[i];     // log alpha
                    if (AL != nullptr) AL[o] = __expf(la);
                    LA[o] = lv[i] - la * kBLog2e;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Shared by bwd_gz and bwd_ds: GV[t][tau] = g_t . v_tau over one chunk, from
// column slabs staged in LDS, kept transposed (gvt[tau][t], pitch kGT) so that
// a row of t values is read 16 bytes at a time.  Thread (t = tid / kGVQ,
// tau = kGVJ (tid % kGVQ) + j) owns kGVJ entries.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void stage_slab(float* dst, const T* __restrict__ src, int b, int t0, int nt, int h,
                                           int N, int H, int D, int d0, int ds, int pitch) {
    for (int e = threadIdx.x; e < kBT * kBSlab; e += kBNT) {
        const int i = e / kBSlab, d = e % kBSlab;
        dst[i * pitch + d] = (i < nt && d < ds) ? to_f32(src[tok_index(b, t0 + i, h, N, H, D) + d0 + d]) : 0.0f;
    }
}

constexpr int kGVJ = kBT * kBT / kBNT;   // GV entries per thread
constexpr int kGVQ = kBT / kGVJ;         // threads per GV row

__device__ __forceinline__ void gv_accumulate(float (&gv)[kGVJ], const float* gs, const float* vs, int ds) {
    const int t = threadIdx.x / kGVQ, tq = (threadIdx.x % kGVQ) * kGVJ;
    for (int d = 0; d < ds; d += 4) {
        const float4 g4 = ld4(gs + t * kGT + d);
#pragma unroll
        for (int j = 0; j < kGVJ; ++j) {
            const float4 v4 = ld4(vs + (tq + j) * kGT + d);
            gv[j] += g4.x * v4.x + g4.y * v4.y + g4.z * v4.z + g4.w * v4.w;
        }
    }
}

__device__ __forceinline__ void gv_store(const float (&gv)[kGVJ], float* gvt) {
    const int t = threadIdx.x / kGVQ, tq = (threadIdx.x % kGVQ) * kGVJ;
#pragma unroll
    for (int j = 0; j < kGVJ; ++j) gvt[(tq + j) * kGT + t] = gv[j];
}

// 16-bit inputs, Dv a multiple of 32: GV on the MFMA straight from the token rows
// (exact products, fp32 sums), one 16 x 16 tile of (t, tau) per wave, stored
// transposed into gvt; the tile t < 16 <= tau, which no t >= tau reads, is zeroed.
template <bool F16>
__device__ __forceinline__ void gv_mfma(const mfma::bf16* __restrict__ dY, const mfma::bf16* __restrict__ V, int b,
                                        int t0, int nt, int h, int N, int H, int Dv, float* gvt) {
    using namespace mfma;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g4 = lane >> 4, cl = lane & 15;
    const int ti = w >> 1, tj = w & 1;
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
    if (ti >= tj) {
        const int t = 16 * ti + cl, tau = 16 * tj + cl;
        const bf16* grow = dY + tok_index(b, t0 + min(t, nt - 1), h, N, H, Dv) + 8 * g4;
        const bf16* vrow = V + tok_index(b, t0 + min(tau, nt - 1), h, N, H, Dv) + 8 * g4;
#pragma unroll 4
        for (int k0 = 0; k0 < Dv; k0 += 32)
            d = mma_in<F16>(t < nt ? load8<bf16x8>(grow + k0) : zero8(), tau < nt ? load8<bf16x8>(vrow + k0) : zero8(), d);
    }
    // D[t = 16 ti + 4 g4 + r][tau = 16 tj + cl]
    *reinterpret_cast<float4*>(gvt + (16 * tj + cl) * kGT + 16 * ti + 4 * g4) = make_float4(d[0], d[1], d[2], d[3]);
}

// D[m][t] += sum_d P[m][d] r[t][d] over one 16 x 16 tile for an fp32 row of P (the
// chunk's state rows, split into bf16 hi + lo) and a 16-bit token row r: each group of
// four 32-column steps issues all its loads before its MFMAs, so that a wave waits for
// the state once per 128 columns rather than once per 32.
template <bool F16>
__device__ __forceinline__ mfma::f32x4 state_row_mma(const float* __restrict__ prow, const mfma::bf16* __restrict__ rrow,
                                                    bool tok_ok, int Dv, mfma::f32x4 d2) {
    using namespace mfma;
    int k0 = 0;
    for (; k0 + 128 <= Dv; k0 += 128) {
        float4 p[8];
        bf16x8 rb[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            p[2 * kk] = ld4(prow + k0 + 32 * kk);
            p[2 * kk + 1] = ld4(prow + k0 + 32 * kk + 4);
            rb[kk] = tok_ok ? load8<bf16x8>(rrow + k0 + 32 * kk) : zero8();
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const float pv[8] = {p[2 * kk].x, p[2 * kk].y, p[2 * kk].z, p[2 * kk].w,
                                 p[2 * kk + 1].x, p[2 * kk + 1].y, p[2 * kk + 1].z, p[2 * kk + 1].w};
            bf16x8 ph, pl;
#pragma unroll
            for (int e = 0; e < 8; ++e) SPLIT2(bf16, pv[e], ph[e], pl[e]);
            d2 = mma_split<F16>(ph, pl, rb[kk], d2);
        }
    }
    for (; k0 < Dv; k0 += 32) {
        const float4 p0 = ld4(prow + k0), p1 = ld4(prow + k0 + 4);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        bf16x8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; ++e) SPLIT2(bf16, pv[e], ph[e], pl[e]);
        d2 = mma_split<F16>(ph, pl, tok_ok ? load8<bf16x8>(rrow + k0) : zero8(), d2);
    }
    return d2;
}

// ---------------------------------------------------------------------------
// bwd_gz: gz_tm (stored in C; alpha_tm gz_tm is formed where needed) with
//   gz_tm = e^{pm_m - L_tm} (g_t . pu_m) + sum_{tau <= t} e^{s_tau m - L_tm} (g_t . v_tau)
// (pm, pu: the chunk's starting max and numerator, pu relative to pm).
// Thread m; the pair sum runs over 16-token blocks of t: blocks wholly after
// tau need no causal test, the diagonal block selects t >= tau.  L of tokens
// past the sequence end is +inf, which zeroes their factors.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBNT) void bwd_gz_kernel(
    const T* __restrict__ V, const T* __restrict__ dY, int N, int H, int M, int Dv,
    const float* __restrict__ pmax, const float* __restrict__ pnum, const float* __restrict__ S,
    const float* __restrict__ L, float* __restrict__ C) {
    __shared__ __attribute__((aligned(16))) float gvt[kBT * kGT];
    // dY and V slabs; afterwards (bf16) g_t . pu_m of one 16-token half as [m][17]
    __shared__ __attribute__((aligned(16))) float gsv[2 * kBT * kGT];
    static_assert(2 * kBT * kGT >= 256 * 17, "g . pu half tile must fit in the slab staging");
    float* gs = gsv;
    float* vs = gsv + kBT * kGT;
    constexpr bool kBf16 = std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value;   // 16-bit inputs
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, tid = threadIdx.x, m = tid;
    const bool act = m < M;
    const int t0 = c * kBT, nt = min(kBT, N - t0);
    const size_t rbase = ((size_t)bh * N + t0) * M;
    // bf16 inputs with whole 16-latent / 32-column tiles: g . pu on the MFMA
    const bool mf = kBf16 && M % 16 == 0 && Dv % 32 == 0;
    float gv[kGVJ];
#pragma unroll
    for (int j = 0; j < kGVJ; ++j) gv[j] = 0.0f;
    float acc[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) acc[t] = 0.0f;
    const float* pu = pnum + (((size_t)bh * NC + c) * M + (act ? m : 0)) * Dv;
    if constexpr (kBf16) {
        if (mf)
            gv_mfma<std::is_same<T, __half>::value>(reinterpret_cast<const mfma::bf16*>(dY),
                                                    reinterpret_cast<const mfma::bf16*>(V), b, t0, nt, h, N, H, Dv, gvt);
    }
    for (int d0 = 0; d0 < (mf ? 0 : Dv); d0 += kBSlab) {
        const int ds = min(kBSlab, Dv - d0);
        __syncthreads();
        stage_slab(gs, dY, b, t0, nt, h, N, H, Dv, d0, ds, kGT);
        stage_slab(vs, V, b, t0, nt, h, N, H, Dv, d0, ds, kGT);
        __syncthreads();
        gv_accumulate(gv, gs, vs, ds);
        if (act) {
            for (int d = 0; d < ds; d += 4) {
                const float4 p = ld4(pu + d0 + d);
#pragma unroll
                for (int t = 0; t < kBT; ++t) {
                    const float4 g4 = ld4(gs + t * kGT + d);
                    acc[t] += g4.x * p.x + g4.y * p.y + g4.z * p.z + g4.w * p.w;
                }
            }
        }
    }
    if constexpr (kBf16) {
        if (mf) {
            // D[m][t] = sum_d pu[m][d] g[t][d] per 16-token half: A = pu rows (fp32 as
            // bf16 hi + lo), B = dY rows; through LDS to the thread of latent m
            using namespace mfma;
            const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
            for (int ti = 0; ti < kBT / 16; ++ti) {
                __syncthreads();   // the slabs (or the previous half) are consumed
                const int t = 16 * ti + cl;
                const bf16* grow = reinterpret_cast<const bf16*>(dY) + tok_index(b, t0 + min(t, nt - 1), h, N, H, Dv) + 8 * g4;
                for (int mt = w; mt < M / 16; mt += kBNT / 64) {
                    f32x4 d2 = f32x4{0.f, 0.f, 0.f, 0.f};
                    const float* prow = pnum + (((size_t)bh * NC + c) * M + 16 * mt + cl) * Dv + 8 * g4;
                    d2 = state_row_mma<std::is_same<T, __half>::value>(prow, grow, t < nt, Dv, d2);
#pragma unroll
                    for (int r = 0; r < 4; ++r) gsv[(16 * mt + 4 * g4 + r) * 17 + cl] = d2[r];
                }
                __syncthreads();
                if (act) {
#pragma unroll
                    for (int u = 0; u < 16; ++u) acc[16 * ti + u] = gsv[m * 17 + u];
                }
            }
        }
    }
    if (!mf) gv_store(gv, gvt);
    __syncthreads();
    if (!act) return;
    const float pm = pmax[((size_t)bh * NC + c) * M + m];
    const float pm2 = pm * kBLog2e;
    float lt[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) {
        lt[t] = t < nt ? L[rbase + (size_t)t * M + m] : __builtin_huge_valf();
        acc[t] = pm == kNegInf ? 0.0f : ex2(pm2 - lt[t]) * acc[t];
    }
    // the chunk's scores of latent m, all loaded before the pair sums (one wait, not one
    // per token)
    const float* scol = S + rbase + m;
    float sv[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) sv[t] = t < nt ? scol[(size_t)t * M] : 0.0f;
#pragma unroll
    for (int tb = 0; tb < kBT / 16; ++tb) {
        if (16 * tb >= nt) break;
        // tau < 16 tb: every t of the block is >= tau
#pragma unroll
        for (int tau = 0; tau < 16 * tb; ++tau) {
            const float s = sv[tau];
            const float* gr = gvt + tau * kGT + 16 * tb;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 g4 = ld4(gr + 4 * q);
                const int t = 16 * tb + 4 * q;
                acc[t] += g4.x * ex2(s - lt[t]);
                acc[t + 1] += g4.y * ex2(s - lt[t + 1]);
                acc[t + 2] += g4.z * ex2(s - lt[t + 2]);
                acc[t + 3] += g4.w * ex2(s - lt[t + 3]);
            }
        }
        // the diagonal block: tau in [16 tb, min(nt, 16 tb + 16))
#pragma unroll
        for (int du = 0; du < 16; ++du) {
            const int tau = 16 * tb + du;
            if (tau >= nt) break;
            const float s = sv[tau];
            const float* gr = gvt + tau * kGT + 16 * tb;
#pragma unroll
            for (int u = du; u < 16; ++u) {
                const int t = 16 * tb + u;
                acc[t] += ex2(s - lt[t]) * gr[u];
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kBT; ++t)
        if (t < nt) C[rbase + (size_t)t * M + m] = acc[t];
}

// ---------------------------------------------------------------------------
// bwd_gy: gy_t = dY_t . Y_t per (b, t, h); one wavefront per token row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_gy_kernel(const T* __restrict__ dY, const T* __restrict__ Y, int N,
                                                     int H, int Dv, int64_t rows, float* __restrict__ gy) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const T* a = dY + row * Dv;
    const T* y = Y + row * Dv;
    float sum = 0.0f;
    for (int d = lane; d < Dv; d += 64) sum += to_f32(a[d]) * to_f32(y[d]);
    sum = wave_sum(sum);
    if (lane == 0) {
        const int h = (int)(row % H);
        const int64_t bt = row / H;
        const int b = (int)(bt / N), t = (int)(bt % N);
        gy[((int64_t)b * H + h) * N + t] = sum;
    }
}

// 16-bit inputs with Dv / 8 a power of two <= 64: lpr = Dv / 8 lanes per row, each
// with one 16-byte load of dY and of Y, and a shuffle reduction over the row's lanes.
template <typename T>
__global__ __launch_bounds__(256) void bwd_gy_vec_kernel(const T* __restrict__ dY, const T* __restrict__ Y, int N,
                                                         int H, int Dv, int64_t rows, float* __restrict__ gy) {
    const int lpr = Dv >> 3;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gid / lpr;
    const int sub = (int)(gid % lpr);
    float sum = 0.0f;
    if (row < rows) {
        union { uint4 raw; T el[8]; } a, y;
        a.raw = *reinterpret_cast<const uint4*>(dY + row * Dv + 8 * sub);
        y.raw = *reinterpret_cast<const uint4*>(Y + row * Dv + 8 * sub);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += to_f32(a.el[e]) * to_f32(y.el[e]);
    }
    for (int off = lpr >> 1; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (row < rows && sub == 0) {
        const int h = (int)(row % H);
        const int64_t bt = row / H;
        const int b = (int)(bt / N), t = (int)(bt % N);
        gy[((int64_t)b * H + h) * N + t] = sum;
    }
}

// ---------------------------------------------------------------------------
// Register-blocked accumulation shared by bwd_summary and bwd_dq:
// acc[i][j] += a[8 mi + i] * b[8 di + j] for one token row of each operand.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void outer8(float (&acc)[8][8], const float* a, const float* b) {
    const float4 a0 = ld4(a), a1 = ld4(a + 4), b0 = ld4(b), b1 = ld4(b + 4);
    const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] += av[i] * bv[j];
}

// ---------------------------------------------------------------------------
// bwd_summary: chunk c's own terms of the reverse scan, relative to
// Lpre = L at the last token of chunk c-1 (chunk 0 has none):
//   a_c,m = sum_{t in c} w_tm g_t,  b_c,m = sum_{t in c} w_tm gz_tm,
//   w_tm = e^{Lpre_m - L_tm} alpha_tm = 2^(Lpre_m - LA_tm)  (gz is stored in C).
// a overwrites the chunk's starting numerator, b its starting den.
// Thread (mi = tid % 32, di = tid / 32) owns a[8 mi .. +8][d0 + 8 di .. +8].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBNT) void bwd_summary_kernel(
    const T* __restrict__ dY, int N, int H, int M, int Dv, const float* __restrict__ L,
    const float* __restrict__ LA, const float* __restrict__ C, float* __restrict__ a_out,
    float* __restrict__ b_out) {
    __shared__ __attribute__((aligned(16))) float wl[kBT * 256];
    __shared__ __attribute__((aligned(16))) float gs[kBT * kGT];
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    if (c == 0) return;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int t0 = c * kBT, nt = min(kBT, N - t0);
    const size_t rbase = ((size_t)bh * N + t0) * M;
    const float* lpre = L + rbase - M;
    for (int e = tid; e < nt * M; e += kBNT) wl[e] = ex2(lpre[e % M] - LA[rbase + e]);
    const size_t sbase = ((size_t)bh * NC + c) * M;
    if (tid < M) {
        float sum = 0.0f;
        for (int t = 0; t < nt; ++t) {
            const size_t o = rbase + (size_t)t * M + tid;
            sum += ex2(lpre[tid] - LA[o]) * C[o];
        }
        b_out[sbase + tid] = sum;
    }
    const int mi = tid & 31, di = tid >> 5;
    const bool act = 8 * mi < M;
    for (int d0 = 0; d0 < Dv; d0 += kBSlab) {
        const int ds = min(kBSlab, Dv - d0);
        __syncthreads();
        stage_slab(gs, dY, b, t0, nt, h, N, H, Dv, d0, ds, kGT);
        __syncthreads();
        if (!act || 8 * di >= ds) continue;
        float acc[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
        for (int t = 0; t < nt; ++t) outer8(acc, wl + t * M + 8 * mi, gs + t * kGT + 8 * di);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float* dst = a_out + (sbase + 8 * mi + i) * Dv + d0 + 8 * di;
            *reinterpret_cast<float4*>(dst) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
        }
    }
}

// ---------------------------------------------------------------------------
// bwd_carry: reverse scan over chunks, in place.  Slot c of (a, b) receives
// (X_c, Y_c); X_{NC-1} = 0 and X_{c-1} = a_c + e^{Lend_{c-1} - Lend_c} X_c.
// Thread per (bh, m, four value columns); chunks are read kScanB at a time.
// ---------------------------------------------------------------------------
constexpr int kScanB = 8;

__global__ __launch_bounds__(256) void bwd_carry_kernel(float* __restrict__ a, float* __restrict__ bsum,
                                                        const float* __restrict__ L, int N, int NC, int M,
                                                        int Dv, int64_t rows) {
    const int D4 = Dv >> 2;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * D4) return;
    const int64_t row = gid / D4;
    const int j = (int)(gid % D4);
    const int64_t bh = row / M;
    const int m = (int)(row % M);
    float4* a4 = reinterpret_cast<float4*>(a);
    auto lend = [&](int c) { return L[((size_t)bh * N + min(N, (c + 1) * kBT) - 1) * M + m]; };
    float4 X = make_float4(0.f, 0.f, 0.f, 0.f);
    float Y = 0.0f;
    float lnext = lend(NC - 1);
    for (int c1 = NC - 1; c1 >= 0; c1 -= kScanB) {
        float4 av[kScanB];
        float bv[kScanB], lv[kScanB];
#pragma unroll
        for (int i = 0; i < kScanB; ++i) {
            const int c = c1 - i;
            const size_t si = (size_t)bh * NC * M + (size_t)max(c, 0) * M + m;
            av[i] = c > 0 ? a4[si * D4 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
            bv[i] = c > 0 ? bsum[si] : 0.0f;
            lv[i] = c > 0 ? lend(c - 1) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kScanB; ++i) {
            const int c = c1 - i;
            if (c < 0) break;
            const size_t si = (size_t)bh * NC * M + (size_t)c * M + m;
            a4[si * D4 + j] = X;
            if (j == 0) bsum[si] = Y;
            if (c > 0) {
                const float f = ex2(lv[i] - lnext);
                X.x = av[i].x + f * X.x;
                X.y = av[i].y + f * X.y;
                X.z = av[i].z + f * X.z;
                X.w = av[i].w + f * X.w;
                Y = bv[i] + f * Y;
                lnext = lv[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// bwd_dv: dv_tau = sum_{t >= tau} G[tau][t] g_t + sum_m e^{s_tau m - Lend_m} X_m,
// G[tau][t] = sum_m e^{s_tau m - L_tm} alpha_tm = sum_m exp2(s2_tau m - LA_tm).
// G covers the causal 16 x 16 blocks (ib <= jb) of the chunk: thread
// (u = tid % 16, v = tid / 16) owns pair (16 ib + u, 16 jb + v) of each, over
// latent slabs of 64 staged in LDS.  The output, for value slabs of 64
// (Dv <= 64 NSL), is accumulated by thread (col, rg) owning
// dv[tau = rg + 4 r][64 sl + col]; the X term runs over latent slabs of 64.
// NSL = 2 serves Dv <= 128 with a quarter of the accumulator registers of NSL = 8.
// ---------------------------------------------------------------------------
constexpr int kMaxVSlab = 8;
constexpr int kTB = kBT / 16;                         // 16-token blocks per chunk
constexpr int kBlockPairs = kTB * (kTB + 1) / 2;      // causal block pairs (ib <= jb)
constexpr int kRT = kBT / 4;                          // output tokens per thread
struct BlockPairs {
    int ib[kBlockPairs], jb[kBlockPairs];
};
constexpr BlockPairs block_pairs() {
    BlockPairs p{};
    int k = 0;
    for (int i = 0; i < kTB; ++i)
        for (int j = i; j < kTB; ++j) {
            p.ib[k] = i;
            p.jb[k] = j;
            ++k;
        }
    return p;
}

template <typename T, int NSL>
__global__ __launch_bounds__(kBNT) void bwd_dv_kernel(
    const T* __restrict__ dY, int N, int H, int M, int Dv, const float* __restrict__ S,
    const float* __restrict__ L, const float* __restrict__ LA, const float* __restrict__ X, T* __restrict__ dV) {
    __shared__ __attribute__((aligned(16))) float uni[2 * kBT * kGT];   // s / LA latent slabs, then e^{s - Lend}
    __shared__ __attribute__((aligned(16))) float gl[kBT * kGT];        // G[tau][t]
    __shared__ float gs[kBT * kBP];                                      // dY slab
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int t0 = c * kBT, nt = min(kBT, N - t0);
    const bool carry = c + 1 < NC;
    const size_t rbase = ((size_t)bh * N + t0) * M;
    float* ss = uni;
    float* ls = uni + kBT * kGT;
    constexpr BlockPairs kP = block_pairs();
    constexpr int kNB = kBlockPairs;
    const int u = tid & 15, v = tid >> 4;
    for (int e = tid; e < kBT * kGT; e += kBNT) gl[e] = 0.0f;
    // bf16 / fp16 inputs, M in {128, 256}: G = E' W^T on the MFMA with the chunk's first-token
    // L as per-latent reference c, E' = 2^(s - c) and W = 2^(c - LA) <= 1 (L grows
    // along the chunk and LA >= L), one exponential per (token, latent) instead of one
    // per pair.  A chunk whose scores pass c by more than 2^64 (E' near the fp32
    // range) redoes G pair by pair below.
    bool exact = true;
    if constexpr (!std::is_same<T, float>::value) {
        if (M % 128 == 0) {
            using namespace mfma;
            __shared__ int big_any;
            if (tid == 0) big_any = 0;
            const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
            f32x4 gp[3] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            bool big = false;
            const int mw = M / 4;
            for (int m0 = w * mw; m0 < (w + 1) * mw; m0 += 32) {
                const float4 c0 = ld4(L + rbase + m0 + 8 * g4), c1 = ld4(L + rbase + m0 + 8 * g4 + 4);
                const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                bf16x8 eh[2], el[2], wh[2], wl[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int row = 16 * q + cl;
                    float ev[8], wv[8];
                    if (row < nt) {
                        const size_t o = rbase + (size_t)row * M + m0 + 8 * g4;
                        const float4 s0 = ld4(S + o), s1 = ld4(S + o + 4), a0 = ld4(LA + o), a1 = ld4(LA + o + 4);
                        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
                        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            big |= sv[e] - cv[e] > 64.0f;
                            ev[e] = ex2(sv[e] - cv[e]);
                            wv[e] = ex2(cv[e] - av[e]);
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) ev[e] = wv[e] = 0.0f;
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        SPLIT2(bf16, ev[e], eh[q][e], el[q][e]);
                        SPLIT2(bf16, wv[e], wh[q][e], wl[q][e]);
                    }
                }
                // causal tile pairs (tau tile, t tile): (0, 0), (0, 1), (1, 1)
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const int ti = k == 2 ? 1 : 0, tj = k == 0 ? 0 : 1;
                    gp[k] = mma(eh[ti], wh[tj], gp[k]);
                    gp[k] = mma(eh[ti], wl[tj], gp[k]);
                    gp[k] = mma(el[ti], wh[tj], gp[k]);
                }
            }
            if (__any(big) && lane == 0) big_any = 1;
            // partial G of each wave (rows tau = 4 g + r, columns t = cl) -> summed in LDS
            float* gpart = uni;   // [4 waves][3 tiles][16][16]
#pragma unroll
            for (int k = 0; k < 3; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) gpart[((w * 3 + k) * 16 + 4 * g4 + r) * 16 + cl] = gp[k][r];
            __syncthreads();
            for (int e = tid; e < 3 * 256; e += kBNT) {
                const int k = e >> 8, i = (e >> 4) & 15, j = e & 15;
                const int tau = 16 * (k == 2 ? 1 : 0) + i, t = 16 * (k == 0 ? 0 : 1) + j;
                float sum = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < 4; ++w2) sum += gpart[((w2 * 3 + k) * 16 + i) * 16 + j];
                gl[tau * kGT + t] = t >= tau ? sum : 0.0f;
            }
            __syncthreads();
            exact = big_any != 0;
        }
    }
    float g[kNB];
#pragma unroll
    for (int k = 0; k < kNB; ++k) g[k] = 0.0f;
    for (int m0 = 0; m0 < (exact ? M : 0); m0 += 64) {
        const int mc = min(64, M - m0);
        __syncthreads();
        for (int e = tid; e < kBT * 64; e += kBNT) {
            const int i = e >> 6, mm = e & 63;
            const bool ok = i < nt && mm < mc;
            const size_t o = rbase + (size_t)i * M + m0 + mm;
            ss[i * kGT + mm] = ok ? S[o] : kNegInf;
            ls[i * kGT + mm] = ok ? LA[o] : __builtin_huge_valf();
        }
        __syncthreads();
        for (int mm = 0; mm < mc; mm += 4) {
            float4 s4[kTB], l4[kTB];
#pragma unroll
            for (int q = 0; q < kTB; ++q) {
                s4[q] = ld4(ss + (16 * q + u) * kGT + mm);
                l4[q] = ld4(ls + (16 * q + v) * kGT + mm);
            }
#pragma unroll
            for (int k = 0; k < kNB; ++k) {
                const float4 sv = s4[kP.ib[k]], lv = l4[kP.jb[k]];
                g[k] += ex2(sv.x - lv.x) + ex2(sv.y - lv.y) + ex2(sv.z - lv.z) + ex2(sv.w - lv.w);
            }
        }
    }
    if (exact) {
#pragma unroll
        for (int k = 0; k < kNB; ++k) {
            const int tau = 16 * kP.ib[k] + u, t = 16 * kP.jb[k] + v;
            gl[tau * kGT + t] = (t >= tau) ? g[k] : 0.0f;
        }
    }
    const int col = tid & 63, rg = tid >> 6;
    float acc[NSL][kRT];
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
        for (int r = 0; r < kRT; ++r) acc[sl][r] = 0.0f;
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
        if (sl * kBSlab >= Dv) break;
        __syncthreads();
        stage_slab(gs, dY, b, t0, nt, h, N, H, Dv, sl * kBSlab, min(kBSlab, Dv - sl * kBSlab), kBP);
        __syncthreads();
        // G rows are zero past nt and gs rows are zero-filled, so whole groups of 4 tokens are safe
        for (int t = 0; t < nt; t += 4) {
            const float g0 = gs[t * kBP + col], g1 = gs[(t + 1) * kBP + col], g2 = gs[(t + 2) * kBP + col],
                        g3 = gs[(t + 3) * kBP + col];
#pragma unroll
            for (int r = 0; r < kRT; ++r) {
                const float4 q4 = ld4(gl + (rg + 4 * r) * kGT + t);
                acc[sl][r] += q4.x * g0 + q4.y * g1 + q4.z * g2 + q4.w * g3;
            }
        }
    }
    if (carry) {
        // e^{s_tau m - Lend_m}, Lend = L at the chunk's last token, per latent slab
        const float* lend = L + rbase + (size_t)(nt - 1) * M;
        const float* xb = X + ((size_t)bh * NC + c) * M * Dv;
        constexpr bool kBf16 = !std::is_same<T, float>::value;   // 16-bit inputs (operands here are fp32 intermediates)
        bool done = false;
        if constexpr (kBf16) {
            if (M % 32 == 0 && (Dv == 64 || Dv == 128)) {
                // bf16 inputs: P X on the MFMA, P = e^{s - Lend} <= 1 and X both fp32 as
                // bf16 hi + lo (three products); D[tau][d] through LDS (uni) to acc
                using namespace mfma;
                const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
                constexpr int kNjw = 2;                  // value tiles per wave (Dv <= 128)
                f32x4 xa[kNjw][2];
#pragma unroll
                for (int q = 0; q < kNjw; ++q) xa[q][0] = xa[q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int m0 = 0; m0 < M; m0 += 32) {
                    const float4 l0 = ld4(lend + m0 + 8 * g4), l1 = ld4(lend + m0 + 8 * g4 + 4);
                    const float lv[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
                    bf16x8 ph[2], pl[2];
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int tau = 16 * ti + cl;
                        float sv[8];
                        if (tau < nt) {
                            const float* srow = S + rbase + (size_t)tau * M + m0 + 8 * g4;
                            const float4 s0 = ld4(srow), s1 = ld4(srow + 4);
                            sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
                            sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
#pragma unroll
                            for (int e = 0; e < 8; ++e) sv[e] = ex2(sv[e] - lv[e]);
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e) sv[e] = 0.0f;
                        }
#pragma unroll
                        for (int e = 0; e < 8; ++e) SPLIT2(bf16, sv[e], ph[ti][e], pl[ti][e]);
                    }
#pragma unroll
                    for (int q = 0; q < kNjw; ++q) {
                        const int nj = w + 4 * q;
                        if (16 * nj >= Dv) break;
                        bf16x8 xh, xl;
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            SPLIT2(bf16, xb[(size_t)(m0 + 8 * g4 + e) * Dv + 16 * nj + cl], xh[e], xl[e]);
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) {
                            xa[q][ti] = mma(ph[ti], xh, xa[q][ti]);
                            xa[q][ti] = mma(ph[ti], xl, xa[q][ti]);
                            xa[q][ti] = mma(pl[ti], xh, xa[q][ti]);
                        }
                    }
                }
                __syncthreads();   // uni is free (its last readers were before the slab loop)
#pragma unroll
                for (int q = 0; q < kNjw; ++q) {
                    const int nj = w + 4 * q;
                    if (16 * nj >= Dv) break;
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r) uni[(16 * ti + 4 * g4 + r) * Dv + 16 * nj + cl] = xa[q][ti][r];
                }
                __syncthreads();
#pragma unroll
                for (int sl = 0; sl < NSL; ++sl) {
                    if (sl * kBSlab >= Dv) break;
#pragma unroll
                    for (int r = 0; r < kRT; ++r) acc[sl][r] += uni[(rg + 4 * r) * Dv + sl * kBSlab + col];
                }
                done = true;
            }
        }
        for (int m0 = 0; m0 < (done ? 0 : M); m0 += 64) {
            const int mc = min(64, M - m0);
            __syncthreads();
            for (int e = tid; e < kBT * 64; e += kBNT) {
                const int i = e >> 6, mm = e & 63;
                uni[i * kGT + mm] = (i < nt && mm < mc) ? ex2(S[rbase + (size_t)i * M + m0 + mm] - lend[m0 + mm]) : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int sl = 0; sl < NSL; ++sl) {
                if (sl * kBSlab >= Dv) break;
                if (sl * kBSlab + col >= Dv) continue;
                const float* xr = xb + (size_t)m0 * Dv + sl * kBSlab + col;
                for (int mm = 0; mm < mc; mm += 4) {
                    const float x0 = xr[(size_t)mm * Dv], x1 = xr[(size_t)(mm + 1) * Dv],
                                x2 = xr[(size_t)(mm + 2) * Dv], x3 = xr[(size_t)(mm + 3) * Dv];
#pragma unroll
                    for (int r = 0; r < kRT; ++r) {
                        const float4 q4 = ld4(uni + (rg + 4 * r) * kGT + mm);
                        acc[sl][r] += q4.x * x0 + q4.y * x1 + q4.z * x2 + q4.w * x3;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
        if (sl * kBSlab >= Dv) break;
        const int d = sl * kBSlab + col;
        if (d >= Dv) continue;
#pragma unroll
        for (int r = 0; r < kRT; ++r) {
            const int tk = rg + 4 * r;
            if (tk < nt) dV[tok_index(b, t0 + tk, h, N, H, Dv) + d] = from_f32<T>(acc[sl][r]);
        }
    }
}

// ---------------------------------------------------------------------------
// bwd_ds: ds_tau m = e^{s - Lend}(v_tau . X_m - Y_m)
//                  + sum_{t >= tau} e^{s_tau m - L_tm} alpha_tm GV[t][tau]
//                  - e^{s_tau m - L_tau m} R_tau m,
// R_tau = sum_{t >= tau} e^{L_tau - L_t} c_t = c_tau + e^{L_tau - L_tau+1} R_tau+1,
// c_t = alpha_t gz_t = 2^(L_t - LA_t) gz_t (C holds gz), written over s.  dsum (shared
// weights): da_tau m = alpha (gz - gy_tau) is added (after the stablemax factor, which
// belongs to ds alone), so that the contractions read ds + da from one array.  Thread m.  The first and last terms are formed in one
// reverse pass over the chunk and kept in registers, with the chunk's scores; the pair sum, exp2(s2_tau - LA_t) GV[t][tau],
// runs per tau over 16-token blocks of t as in bwd_gz.  power > 0 (stablemax,
// s2 = log2 s(a)): the gradient with respect to a is the one with respect to
// log s(a) times d log s / da = p / (1 + |a|) = p 2^(-|s2| / p).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBNT) void bwd_ds_kernel(
    const T* __restrict__ V, const T* __restrict__ dY, int N, int H, int M, int Dv, float* __restrict__ S,
    float* __restrict__ L, const float* __restrict__ LA, const float* __restrict__ C,
    const float* __restrict__ X, const float* __restrict__ Ysum, float power, const float* __restrict__ gy,
    bool dsum) {
    __shared__ __attribute__((aligned(16))) float gvt[kBT * kGT];
    // dY and V slabs; afterwards (bf16) v_t . X_m of one 16-token half as [m][17]
    __shared__ __attribute__((aligned(16))) float gsv[2 * kBT * kGT];
    float* gs = gsv;
    float* vs = gsv + kBT * kGT;
    constexpr bool kBf16 = std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value;   // 16-bit inputs
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, tid = threadIdx.x, m = tid;
    const bool act = m < M;
    const int t0 = c * kBT, nt = min(kBT, N - t0);
    const bool carry = c + 1 < NC;
    const size_t rbase = ((size_t)bh * N + t0) * M;
    // bf16 inputs with whole 16-latent / 32-column tiles: v . X on the MFMA
    const bool mf = kBf16 && M % 16 == 0 && Dv % 32 == 0;
    float gv[kGVJ];
#pragma unroll
    for (int j = 0; j < kGVJ; ++j) gv[j] = 0.0f;
    float acc[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) acc[t] = 0.0f;
    const float* xr = X + (((size_t)bh * NC + c) * M + (act ? m : 0)) * Dv;
    if constexpr (kBf16) {
        if (mf)
            gv_mfma<std::is_same<T, __half>::value>(reinterpret_cast<const mfma::bf16*>(dY),
                                                    reinterpret_cast<const mfma::bf16*>(V), b, t0, nt, h, N, H, Dv, gvt);
    }
    for (int d0 = 0; d0 < (mf ? 0 : Dv); d0 += kBSlab) {
        const int ds = min(kBSlab, Dv - d0);
        __syncthreads();
        stage_slab(gs, dY, b, t0, nt, h, N, H, Dv, d0, ds, kGT);
        stage_slab(vs, V, b, t0, nt, h, N, H, Dv, d0, ds, kGT);
        __syncthreads();
        gv_accumulate(gv, gs, vs, ds);
        if (act && carry) {
            for (int d = 0; d < ds; d += 4) {
                const float4 p = ld4(xr + d0 + d);
#pragma unroll
                for (int t = 0; t < kBT; ++t) {
                    const float4 v4 = ld4(vs + t * kGT + d);
                    acc[t] += v4.x * p.x + v4.y * p.y + v4.z * p.z + v4.w * p.w;
                }
            }
        }
    }
    if constexpr (kBf16) {
        if (mf && carry) {
            // D[m][t] = sum_d X[m][d] v[t][d] per 16-token half: A = X rows (fp32 as bf16
            // hi + lo), B = V rows; through LDS to the thread of latent m
            using namespace mfma;
            const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
            for (int ti = 0; ti < kBT / 16; ++ti) {
                __syncthreads();   // the slabs (or the previous half) are consumed
                const int t = 16 * ti + cl;
                const bf16* vrow = reinterpret_cast<const bf16*>(V) + tok_index(b, t0 + min(t, nt - 1), h, N, H, Dv) + 8 * g4;
                for (int mt = w; mt < M / 16; mt += kBNT / 64) {
                    f32x4 d2 = f32x4{0.f, 0.f, 0.f, 0.f};
                    const float* xrow = X + (((size_t)bh * NC + c) * M + 16 * mt + cl) * Dv + 8 * g4;
                    d2 = state_row_mma<std::is_same<T, __half>::value>(xrow, vrow, t < nt, Dv, d2);
#pragma unroll
                    for (int r = 0; r < 4; ++r) gsv[(16 * mt + 4 * g4 + r) * 17 + cl] = d2[r];
                }
                __syncthreads();
                if (act) {
#pragma unroll
                    for (int u = 0; u < 16; ++u) acc[16 * ti + u] = gsv[m * 17 + u];
                }
            }
        }
    }
    if (!mf) gv_store(gv, gvt);
    __syncthreads();
    if (!act) return;
    float* scol = S + rbase + m;
    float* lcol = L + rbase + m;
    const float* ccol = C + rbase + m;
    const float lend = lcol[(size_t)(nt - 1) * M];
    const float ysum = carry ? Ysum[((size_t)bh * NC + c) * M + m] : 0.0f;
    float R = 0.0f, lnext = 0.0f;
    // the scores of latent m, and the first and last terms of its ds (in acc, whose
    // v . X it replaces), kept in registers for the pair sums below
    float sv[kBT], la[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) {
        sv[t] = t < nt ? scol[(size_t)t * M] : 0.0f;
        la[t] = t < nt ? LA[rbase + (size_t)t * M + m] : __builtin_huge_valf();
    }
#pragma unroll
    for (int t = kBT - 1; t >= 0; --t) {
        if (t < nt) {
            const size_t o = (size_t)t * M;
            const float l = lcol[o], s = sv[t], al = ex2(l - la[t]), gzt = ccol[o];
            R = al * gzt + (t + 1 < nt ? ex2(l - lnext) * R : 0.0f);
            lnext = l;
            float park = -ex2(s - l) * R;
            if (carry) park += ex2(s - lend) * (acc[t] - ysum);
            if (dsum && power == 0.0f) park += al * (gzt - gy[(size_t)bh * N + t0 + t]);
            acc[t] = park;
        }
    }
#pragma unroll
    for (int tau = 0; tau < kBT; ++tau) {
        if (tau >= nt) break;
        const float s = sv[tau];
        const float* gr = gvt + tau * kGT;
        const int tb0 = tau >> 4;
        float sum = 0.0f;
#pragma unroll
        for (int tb = 0; tb < kBT / 16; ++tb) {
            if (tb == tb0) {
#pragma unroll
                for (int uu = 0; uu < 16; ++uu) {
                    const int t = 16 * tb + uu;
                    const float e = ex2(s - la[t]) * gr[t];
                    sum += t >= tau ? e : 0.0f;
                }
            } else if (tb > tb0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int t = 16 * tb + 4 * q;
                    const float4 g4 = ld4(gr + t);
                    sum += ex2(s - la[t]) * g4.x + ex2(s - la[t + 1]) * g4.y + ex2(s - la[t + 2]) * g4.z +
                           ex2(s - la[t + 3]) * g4.w;
                }
            }
        }
        const size_t o = (size_t)tau * M;
        const float dlog = acc[tau] + sum;
        float dsv = dlog;
        if (power > 0.0f) {
            dsv = dlog * (power * ex2(-fabsf(s) / power));
            if (dsum) dsv += ex2(lcol[o] - la[tau]) * (ccol[o] - gy[(size_t)bh * N + t0 + tau]);
        }
        scol[o] = dsv;
    }
}

// ---------------------------------------------------------------------------
// bwd_dk: per token, dK_t = scale sum_m (ds_tm Q_m [+ da_tm Kd_m when Qd = K])
// and dQd_t = scale sum_m da_tm Kd_m (separate Qd); da_tm = alpha_tm (gz_tm - gy_t)
// (score_grad_da).  dsum (shared weights only): DS already holds ds + da.
// Thread (col, tg) owns tokens tg + 4 r (r < kDkTok / 4) and columns col + 64 k.
// ---------------------------------------------------------------------------
constexpr int kDkTok = 32;     // tokens per bwd_dk workgroup

template <typename T>
__global__ __launch_bounds__(kBNT) void bwd_dk_kernel(
    const T* __restrict__ Q, const T* __restrict__ Kd, int N, int H, int M, int Dk, float scale, bool sep_q,
    const float* __restrict__ DS, const float* __restrict__ AL, const float* __restrict__ C,
    const float* __restrict__ gy, bool cgz, bool dsum, T* __restrict__ dK, T* __restrict__ dQd) {
    __shared__ __attribute__((aligned(16))) float dsl[kDkTok * 256];
    __shared__ __attribute__((aligned(16))) float dal[kDkTok * 256];
    const int bh = blockIdx.y, b = bh / H, h = bh % H, tid = threadIdx.x;
    const int t0 = blockIdx.x * kDkTok, nt = min(kDkTok, N - t0);
    const size_t rbase = ((size_t)bh * N + t0) * M;
    for (int e = tid; e < kDkTok * M; e += kBNT) {
        const int i = e / M;
        const bool ok = i < nt;
        dsl[e] = ok ? DS[rbase + e] : 0.0f;
        dal[e] = ok && !dsum ? score_grad_da(C[rbase + e], AL[rbase + e], gy[(size_t)bh * N + t0 + i], cgz) : 0.0f;
    }
    __syncthreads();
    const int col = tid & 63, tg = tid >> 6;
    constexpr int R = kDkTok / 4;
    for (int d0 = 0; d0 < Dk; d0 += 64) {
        const int d = d0 + col;
        if (d >= Dk) break;
        float ak[R], aq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) ak[r] = aq[r] = 0.0f;
        const T* qc = Q + (size_t)h * M * Dk + d;
        const T* kc = Kd + (size_t)h * M * Dk + d;
        for (int m = 0; m < M; m += 4) {
            const float q0 = to_f32(qc[(size_t)m * Dk]), q1 = to_f32(qc[(size_t)(m + 1) * Dk]),
                        q2 = to_f32(qc[(size_t)(m + 2) * Dk]), q3 = to_f32(qc[(size_t)(m + 3) * Dk]);
            const float k0 = to_f32(kc[(size_t)m * Dk]), k1 = to_f32(kc[(size_t)(m + 1) * Dk]),
                        k2 = to_f32(kc[(size_t)(m + 2) * Dk]), k3 = to_f32(kc[(size_t)(m + 3) * Dk]);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int i = tg + 4 * r;
                const float4 s4 = ld4(dsl + i * M + m), a4 = ld4(dal + i * M + m);
                ak[r] += s4.x * q0 + s4.y * q1 + s4.z * q2 + s4.w * q3;
                aq[r] += a4.x * k0 + a4.y * k1 + a4.z * k2 + a4.w * k3;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = tg + 4 * r;
            if (i >= nt) continue;
            const size_t o = tok_index(b, t0 + i, h, N, H, Dk) + d;
            if (sep_q) {
                dK[o] = from_f32<T>(scale * ak[r]);
                dQd[o] = from_f32<T>(scale * aq[r]);
            } else {
                dK[o] = from_f32<T>(scale * (ak[r] + aq[r]));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// bwd_dq: partial sums over a group of kBGroup tokens of
//   P1_m = sum_t ds_tm k_t (+ da_tm qd_t when Kd = Q),  P2_m = sum_t da_tm qd_t.
// grid (NG, BH, ceil(Dk/64)); thread (mi = tid % 32, di = tid / 32) owns the
// 8 x 8 tile m = 8 mi .., d = d0 + 8 di ..
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBNT) void bwd_dq_kernel(
    const T* __restrict__ K, const T* __restrict__ Qd, int N, int H, int M, int Dk, bool sep_k,
    const float* __restrict__ DS, const float* __restrict__ AL, const float* __restrict__ C,
    const float* __restrict__ gy, bool cgz, bool dsum, float* __restrict__ P1, float* __restrict__ P2) {
    __shared__ __attribute__((aligned(16))) float dsl[kBTok * 256];
    __shared__ __attribute__((aligned(16))) float dal[kBTok * 256];
    __shared__ __attribute__((aligned(16))) float kt[kBTok * kGT];
    __shared__ __attribute__((aligned(16))) float qt[kBTok * kGT];
    const int g = blockIdx.x, NG = gridDim.x, bh = blockIdx.y, b = bh / H, h = bh % H, tid = threadIdx.x;
    const int d0 = blockIdx.z * 64;
    const int mi = tid & 31, di = tid >> 5;
    const bool act = 8 * mi < M && d0 + 8 * di < Dk;
    float a1[8][8], a2[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) a1[i][j] = a2[i][j] = 0.0f;
    const int tg0 = g * kBGroup, tg1 = min(N, tg0 + kBGroup);
    for (int t0 = tg0; t0 < tg1; t0 += kBTok) {
        const int nt = min(kBTok, tg1 - t0);
        const size_t rbase = ((size_t)bh * N + t0) * M;
        __syncthreads();
        for (int e = tid; e < kBTok * M; e += kBNT) {
            const int i = e / M;
            const bool ok = i < nt;
            dsl[e] = ok ? DS[rbase + e] : 0.0f;
            dal[e] = ok && !dsum ? score_grad_da(C[rbase + e], AL[rbase + e], gy[(size_t)bh * N + t0 + i], cgz) : 0.0f;
        }
        for (int e = tid; e < kBTok * 64; e += kBNT) {
            const int i = e >> 6, dd = e & 63, d = d0 + dd;
            const bool ok = i < nt && d < Dk;
            const size_t o = tok_index(b, t0 + i, h, N, H, Dk) + d;
            kt[i * kGT + dd] = ok ? to_f32(K[o]) : 0.0f;
            qt[i * kGT + dd] = ok ? to_f32(Qd[o]) : 0.0f;
        }
        __syncthreads();
        if (act) {
            for (int i = 0; i < nt; ++i) {
                outer8(a1, dsl + i * M + 8 * mi, kt + i * kGT + 8 * di);
                outer8(a2, dal + i * M + 8 * mi, qt + i * kGT + 8 * di);
            }
        }
    }
    if (!act) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const size_t o = (((size_t)bh * NG + g) * M + 8 * mi + i) * Dk + d0 + 8 * di;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (sep_k) {
                P1[o + j] = a1[i][j];
                P2[o + j] = a2[i][j];
            } else {
                P1[o + j] = a1[i][j] + a2[i][j];
            }
        }
    }
}

// out[h][m][d] = scale * sum over (b, group) of P[(b H + h)][group][m][d]
template <typename T>
__global__ __launch_bounds__(256) void bwd_reduce_kernel(const float* __restrict__ P, int B, int H, int NG,
                                                         int MD, float scale, T* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (int64_t)H * MD) return;
    const int h = (int)(gid / MD), e = (int)(gid % MD);
    float sum = 0.0f;
    for (int b = 0; b < B; ++b)
        for (int g = 0; g < NG; ++g) sum += P[(((size_t)b * H + h) * NG + g) * MD + e];
    out[gid] = from_f32<T>(scale * sum);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// dQ, dK, dQ_dec, dK_dec from the score gradients (ds in DS; da = C - AL gy):
// shared by the token-causal and the block-causal backward.
template <typename T>
static int launch_contract(const T* q, const T* k, const T* qd, const T* kd, bool sep_q, bool sep_k, int64_t B,
                           int64_t N, int64_t H, int64_t M, int64_t Dk, float scale, const float* DS, const float* AL,
                           const float* C, const float* gy, bool cgz, bool dsum, void* dQ, void* dK, void* dQd,
                           void* dKd, float* P1, float* P2, hipStream_t st) {
    const int64_t BH = B * H, NG = (N + kBGroup - 1) / kBGroup;
    int rc;
    constexpr bool kHalf = std::is_same<T, __half>::value;
    constexpr bool k16 = std::is_same<T, __hip_bfloat16>::value || kHalf;
    if (k16 && bwd_dk_mfma_supported(M, Dk)) {
        if ((rc = launch_dk_mfma(q, kd, sep_q, sep_k, B, N, H, M, Dk, scale, DS, AL, C, gy, cgz, dsum, dK, dQd, kHalf, st)))
            return rc;
    } else {
        hipLaunchKernelGGL(bwd_dk_kernel<T>, dim3((unsigned)((N + kDkTok - 1) / kDkTok), (unsigned)BH), dim3(kBNT),
                           0, st, q, kd, (int)N, (int)H, (int)M, (int)Dk, scale, sep_q, DS, AL, C, gy,
                           cgz, dsum, static_cast<T*>(dK), static_cast<T*>(dQd));
        if ((rc = check_launch("bwd_dk_kernel"))) return rc;
    }
    if (k16 && bwd_dq_mfma_supported(M, Dk)) {
        if ((rc = launch_dq_mfma(k, qd, sep_q, sep_k, B, N, H, M, Dk, DS, AL, C, gy, cgz, dsum, P1, P2, kHalf, st))) return rc;
    } else {
        hipLaunchKernelGGL(bwd_dq_kernel<T>, dim3((unsigned)NG, (unsigned)BH, (unsigned)((Dk + 63) / 64)),
                           dim3(kBNT), 0, st, k, qd, (int)N, (int)H, (int)M, (int)Dk, sep_k, DS, AL, C, gy, cgz, dsum, P1, P2);
        if ((rc = check_launch("bwd_dq_kernel"))) return rc;
    }
    const int64_t red = H * M * Dk;
    hipLaunchKernelGGL(bwd_reduce_kernel<T>, dim3((unsigned)((red + 255) / 256)), dim3(256), 0, st, P1, (int)B,
                       (int)H, (int)NG, (int)(M * Dk), scale, static_cast<T*>(dQ));
    if ((rc = check_launch("bwd_reduce_kernel"))) return rc;
    if (sep_k) {
        hipLaunchKernelGGL(bwd_reduce_kernel<T>, dim3((unsigned)((red + 255) / 256)), dim3(256), 0, st, P2,
                           (int)B, (int)H, (int)NG, (int)(M * Dk), scale, static_cast<T*>(dKd));
        if ((rc = check_launch("bwd_reduce_kernel"))) return rc;
    }
    return FLARE_OK;
}

template <typename T>
static int launch_gy(const T* dy, const T* y, int64_t B, int64_t N, int64_t H, int64_t Dv, float* gy, hipStream_t st) {
    const int64_t rows = B * N * H;
    const int64_t lpr = Dv / 8;
    const bool aligned = ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    if (!std::is_same<T, float>::value && aligned && Dv % 8 == 0 && lpr <= 64 && (lpr & (lpr - 1)) == 0) {
        const int64_t threads = rows * lpr;
        hipLaunchKernelGGL(bwd_gy_vec_kernel<T>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, dy, y,
                           (int)N, (int)H, (int)Dv, rows, gy);
        return check_launch("bwd_gy_vec_kernel");
    }
    hipLaunchKernelGGL(bwd_gy_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, dy, y, (int)N, (int)H,
                       (int)Dv, rows, gy);
    return check_launch("bwd_gy_kernel");
}

size_t bwd_partial_floats(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk) {
    return (size_t)B * H * ((N + kBGroup - 1) / kBGroup) * M * Dk;
}

int launch_bwd_gy(const void* dY, const void* Y, int dtype, int64_t B, int64_t N, int64_t H, int64_t Dv, float* gy,
                  hipStream_t st) {
    if (dtype == FLARE_BF16)
        return launch_gy((const __hip_bfloat16*)dY, (const __hip_bfloat16*)Y, B, N, H, Dv, gy, st);
    if (dtype == FLARE_F16) return launch_gy((const __half*)dY, (const __half*)Y, B, N, H, Dv, gy, st);
    return launch_gy((const float*)dY, (const float*)Y, B, N, H, Dv, gy, st);
}

int launch_bwd_contract(const void* Q, const void* K, const void* Qdec, const void* Kdec, int dtype, int64_t B,
                        int64_t N, int64_t H, int64_t M, int64_t Dk, float scale, const float* DS, const float* AL,
                        const float* C, const float* gy, bool cgz, bool dsum, void* dQ, void* dK, void* dQdec,
                        void* dKdec, float* P1, float* P2, hipStream_t st) {
    const bool sep_q = Qdec != nullptr, sep_k = Kdec != nullptr;
#define FLARE_CONTRACT(TY)                                                                                       \
    return launch_contract((const TY*)Q, (const TY*)K, (const TY*)(sep_q ? Qdec : K), (const TY*)(sep_k ? Kdec : Q), \
                           sep_q, sep_k, B, N, H, M, Dk, scale, DS, AL, C, gy, cgz, dsum, dQ, dK, dQdec, dKdec, P1, \
                           P2, st)
    if (dtype == FLARE_BF16) FLARE_CONTRACT(__hip_bfloat16);
    if (dtype == FLARE_F16) FLARE_CONTRACT(__half);
    FLARE_CONTRACT(float);
#undef FLARE_CONTRACT
}

// The chunk starting states come from one walk over long chunks (chunk_prepare_tr's EMIT
// instance) where the shapes allow it: the summaries and scan of those long chunks first.
static bool bwd_states_walk(int dtype, int64_t M, int64_t Dk, int64_t Dv) {
    return (dtype == FLARE_BF16 || dtype == FLARE_F16) && (mfma_phase_mask() & 1) && output_pc_enabled() &&
           output_tr_enabled() && mfma_prepare_supported(dtype, M, Dk, Dv) && (M == 128 || M == 256);
}

// The walk's chunk: the forward's own, or FLARE_BWD_WALK_CHUNK tokens (rounded up to a
// multiple of 64; read at every call, for tests of walks over many tiles and A/B runs).
static int64_t bwd_walk_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv) {
    const char* e = getenv("FLARE_BWD_WALK_CHUNK");
    if (e && atoll(e) > 0) return ((atoll(e) + 63) / 64) * 64;
    return default_chunk(B, N, H, M, Dv);
}

struct BwdLayout {
    int64_t NC, NG, seg, NCS;
    size_t off_pm, off_pd, off_pn, off_s, off_l, off_al, off_la, off_c, off_gy, off_p1, off_p2, off_gm, off_gd,
        off_gn, total;
    BwdLayout(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv) {
        NC = (N + kBT - 1) / kBT;
        NG = (N + kBGroup - 1) / kBGroup;
        seg = bwd_walk_chunk(B, N, H, M, Dv);   // the walk's chunk (a multiple of 64)
        NCS = (N + seg - 1) / seg;
        const size_t BH = (size_t)B * H;
        size_t o = 0;
        auto take = [&](size_t floats) {
            const size_t at = o;
            o += ((floats * sizeof(float) + 255) / 256) * 256;
            return at;
        };
        off_pm = take(BH * NC * M);
        off_pd = take(BH * NC * M);
        off_pn = take(BH * NC * M * Dv);
        off_s = take(BH * N * M);
        off_l = take(BH * N * M);
        off_al = take(BH * N * M);
        off_la = take(BH * N * M);
        off_c = take(BH * N * M);
        off_gy = take(BH * N);
        off_p1 = take(BH * NG * M * Dk);
        off_p2 = take(BH * NG * M * Dk);
        off_gm = take(BH * NCS * M);
        off_gd = take(BH * NCS * M);
        off_gn = take(BH * NCS * M * Dv);
        total = o + 256;
    }
};

template <typename T>
static int run_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec, int dtype,
                        int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                        const void* Yp, const void* dYp, void* dQ, void* dK, void* dV, void* dQd, void* dKd,
                        char* ws, const BwdLayout& lay, hipStream_t st, float power) {
    const bool sep_q = Qdec != nullptr, sep_k = Kdec != nullptr;
    const bool shared = !sep_q && !sep_k;
    float* pm = reinterpret_cast<float*>(ws + lay.off_pm);
    float* pd = reinterpret_cast<float*>(ws + lay.off_pd);
    float* pn = reinterpret_cast<float*>(ws + lay.off_pn);
    float* S = reinterpret_cast<float*>(ws + lay.off_s);
    float* L = reinterpret_cast<float*>(ws + lay.off_l);
    float* AL = reinterpret_cast<float*>(ws + lay.off_al);
    float* LA = reinterpret_cast<float*>(ws + lay.off_la);
    float* C = reinterpret_cast<float*>(ws + lay.off_c);
    float* gy = reinterpret_cast<float*>(ws + lay.off_gy);
    float* P1 = reinterpret_cast<float*>(ws + lay.off_p1);
    float* P2 = reinterpret_cast<float*>(ws + lay.off_p2);
    const int64_t NC = lay.NC, NG = lay.NG, BH = B * H;
    const T* q = static_cast<const T*>(Q);
    const T* k = static_cast<const T*>(K);
    const T* v = static_cast<const T*>(V);
    const T* qd = sep_q ? static_cast<const T*>(Qdec) : k;
    const T* kd = sep_k ? static_cast<const T*>(Kdec) : q;
    const T* y = static_cast<const T*>(Yp);
    const T* dy = static_cast<const T*>(dYp);
    int rc;
    // chunk starting states at the backward's chunk length: from a walk over long chunks
    // (their summaries and scan first), else the prepare and scan at 32 tokens
    if (bwd_states_walk(dtype, M, Dk, Dv)) {
        float* gm = reinterpret_cast<float*>(ws + lay.off_gm);
        float* gd = reinterpret_cast<float*>(ws + lay.off_gd);
        float* gn = reinterpret_cast<float*>(ws + lay.off_gn);
        if ((rc = launch_prepare_public(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, lay.seg, gm, gd, gn, st, power)))
            return rc;
        if ((rc = launch_prefix_public(gm, gd, gn, BH, lay.NCS, M, Dv, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, st)))
            return rc;
        if ((rc = launch_states_tr(Q, K, V, B, N, H, M, Dk, scale, lay.seg, gm, gd, gn, pm, pd, pn,
                                   dtype == FLARE_F16, st, power)))
            return rc;
    } else {
        if ((rc = launch_prepare_public(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, kBT, pm, pd, pn, st, power)))
            return rc;
        if ((rc = launch_prefix_public(pm, pd, pn, BH, NC, M, Dv, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, st)))
            return rc;
    }
    const dim3 gc((unsigned)NC, (unsigned)BH);
    // shared weights: bwd_ds adds da to ds, and the contractions read that one array (not
    // C, alpha and gy); alpha is then read by no kernel and not written
    const bool dsum = !sep_q && !sep_k;
    float* const ALw = dsum ? nullptr : AL;
    bool stats_mfma = false;
    if constexpr (std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) {
        stats_mfma = M % 16 == 0 && Dk % 32 == 0;
        if (stats_mfma)
            hipLaunchKernelGGL((bwd_stats_kernel<T, true>), gc, dim3(kBNT), 0, st, q, k, qd, kd, (int)N, (int)H,
                               (int)M, (int)Dk, scale, shared, pm, pd, S, L, ALw, LA, power);
    }
    if (!stats_mfma)
        hipLaunchKernelGGL((bwd_stats_kernel<T, false>), gc, dim3(kBNT), 0, st, q, k, qd, kd, (int)N, (int)H, (int)M,
                           (int)Dk, scale, shared, pm, pd, S, L, ALw, LA, power);
    if ((rc = check_launch("bwd_stats_kernel"))) return rc;
    hipLaunchKernelGGL(bwd_gz_kernel<T>, gc, dim3(kBNT), 0, st, v, dy, (int)N, (int)H, (int)M, (int)Dv, pm, pn, S,
                       L, C);
    if ((rc = check_launch("bwd_gz_kernel"))) return rc;
    if ((rc = launch_gy(dy, y, B, N, H, Dv, gy, st))) return rc;
    static_assert(kBT == 32, "the MFMA chunk summary assumes 32-token chunks");
    if ((std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) &&
        bwd_summary_mfma_supported(M, Dv)) {
        if ((rc = launch_summary_mfma(dy, B, N, H, M, Dv, L, LA, C, pn, pd, std::is_same<T, __half>::value, st)))
            return rc;
    } else {
        hipLaunchKernelGGL(bwd_summary_kernel<T>, gc, dim3(kBNT), 0, st, dy,
                           (int)N, (int)H, (int)M, (int)Dv, L, LA, C, pn, pd);
        if ((rc = check_launch("bwd_summary_kernel"))) return rc;
    }
    const int64_t cthreads = BH * M * (Dv / 4);
    hipLaunchKernelGGL(bwd_carry_kernel, dim3((unsigned)((cthreads + 255) / 256)), dim3(256), 0, st, pn, pd, L,
                       (int)N, (int)NC, (int)M, (int)Dv, BH * M);
    if ((rc = check_launch("bwd_carry_kernel"))) return rc;
    auto* dv_kernel = Dv <= 2 * kBSlab ? bwd_dv_kernel<T, 2> : bwd_dv_kernel<T, kMaxVSlab>;
    hipLaunchKernelGGL(dv_kernel, gc, dim3(kBNT), 0, st, dy, (int)N, (int)H, (int)M, (int)Dv, S, L, LA, pn, static_cast<T*>(dV));
    if ((rc = check_launch("bwd_dv_kernel"))) return rc;
    hipLaunchKernelGGL(bwd_ds_kernel<T>, gc, dim3(kBNT), 0, st, v, dy, (int)N, (int)H, (int)M, (int)Dv, S, L, LA,
                       C, pn, pd, power, gy, dsum);
    if ((rc = check_launch("bwd_ds_kernel"))) return rc;
    return launch_contract(q, k, qd, kd, sep_q, sep_k, B, N, H, M, Dk, scale, S, AL, C, gy, true, dsum, dQ, dK, dQd,
                           dKd, P1, P2, st);
}

bool ar_backward_supported(int64_t M, int64_t Dk, int64_t Dv) {
    return M % 16 == 0 && M >= 16 && M <= 256 && Dk % 16 == 0 && Dk >= 16 && Dk <= 256 && Dv % 16 == 0 &&
           Dv >= 16 && Dv <= 512;
}

size_t ar_backward_workspace(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv) {
    return BwdLayout(B, N, H, M, Dk, Dv).total;
}

int ar_backward_run(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec, int dtype,
                    int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale, const void* Y,
                    const void* dY, void* dQ, void* dK, void* dV, void* dQdec, void* dKdec, void* workspace,
                    size_t workspace_bytes, hipStream_t st, float power) {
    const BwdLayout lay(B, N, H, M, Dk, Dv);
    FLARE_REQUIRE(workspace && workspace_bytes >= lay.total,
                  "flare_ar_backward: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                  lay.total);
    FLARE_REQUIRE((((uintptr_t)workspace) & 255) == 0, "flare_ar_backward: workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
#define FLARE_BWD(TY)                                                                                          \
    return run_backward<TY>(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, Y, dY, dQ, dK, dV, dQdec, \
                            dKdec, ws, lay, st, power)
    if (dtype == FLARE_BF16) FLARE_BWD(__hip_bfloat16);
    if (dtype == FLARE_F16) FLARE_BWD(__half);
    FLARE_BWD(float);
#undef FLARE_BWD
}

}  // namespace flare

using namespace flare;

extern "C" {

size_t flare_ar_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv) {
    return ar_backward_workspace(B, N, H, M, Dk, Dv);
}

int flare_ar_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec, int dtype,
                      int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                      const void* Y, const void* dY, void* dQ, void* dK, void* dV, void* dQdec, void* dKdec,
                      void* workspace, size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y && dY && dQ && dK && dV, "flare_ar_backward: null tensor pointer");
    FLARE_REQUIRE(dtype == FLARE_F32 || dtype == FLARE_BF16 || dtype == FLARE_F16,
                  "flare_ar_backward: unknown dtype code %d", dtype);
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0, "flare_ar_backward: empty problem (B=%lld N=%lld H=%lld)",
                  (long long)B, (long long)N, (long long)H);
    FLARE_REQUIRE(M % 16 == 0 && M >= 16 && M <= 256,
                  "flare_ar_backward: M=%lld must be a multiple of 16 in [16, 256]", (long long)M);
    FLARE_REQUIRE(Dk % 16 == 0 && Dk >= 16 && Dk <= 256,
                  "flare_ar_backward: D_score=%lld must be a multiple of 16 in [16, 256]", (long long)Dk);
    FLARE_REQUIRE(Dv % 16 == 0 && Dv >= 16 && Dv <= 512,
                  "flare_ar_backward: D_value=%lld must be a multiple of 16 in [16, 512]", (long long)Dv);
    FLARE_REQUIRE(!Qdec || dQdec, "flare_ar_backward: Qdec given without dQdec");
    FLARE_REQUIRE(!Kdec || dKdec, "flare_ar_backward: Kdec given without dKdec");
    return ar_backward_run(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, Y, dY, dQ, dK, dV, dQdec, dKdec,
                           workspace, workspace_bytes, static_cast<hipStream_t>(stream), 0.0f);
}

}  // extern "C"
