// flare_semi_bwd.hip -- backward of the block-causal (semi-autoregressive)
// forward (scalar-fp32 kernels).
//
// Replaces the reference's _semi_autoregressive_backward_impl
// (causal_flare/semi_autoregressive/training.py:3768-3988), the autograd
// backward of SemiAutoRegressiveFLARE (:3990-4080).  Token t of block g reads
// the encoder state after the last token of block g:
//   z_g,m = U_g,m / D_g,m,  D_g,m = sum_{tau in blocks <= g} e^{s_tau m} = e^{L_g,m},
//   y_t   = sum_m alpha_tm z_g(t),m.
// With g_t = dY_t:
//   gz_tm = g_t . z_g(t),m    gy_t = g_t . y_t    da_tm = alpha_tm (gz_tm - gy_t)
//   dz_g,m = sum_{t in g} alpha_tm g_t,   c_g,m = sum_{t in g} alpha_tm gz_tm
//   X_g = dz_g + e^{L_g - L_g+1} X_g+1,   Y_g = c_g + e^{L_g - L_g+1} Y_g+1   (reverse scan)
//   ds_tau m = e^{s_tau m - L_g} (v_tau . X_g,m - Y_g,m),  dv_tau = sum_m e^{s_tau m - L_g} X_g,m
// for tau in block g; every factor is <= 1.  dQ, dK, dQ_dec and dK_dec follow
// from ds and da with the token-causal backward's contraction kernels.  The
// states after each block come from the forward's prepare and prefix kernels
// run at chunk = block.
//
// Kernels, in launch order:
//   semi_bwd_tok    s, alpha, c = alpha gz per (t, m)        grid (NB, BH)
//   semi_bwd_dz     dz_g and c_g per block                   grid (NB, BH)
//   semi_bwd_carry  reverse scan over blocks -> X_g, Y_g     grid (BH M Dv/4)
//   semi_bwd_dv     dV                                        grid (NB, BH, Dv/64)
//   semi_bwd_ds     ds (written over s)                      grid (NB, BH)
//   then gy and the dQ / dK contractions (flare_ar_bwd.hip)
#include <stdio.h>

#include <type_traits>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {

constexpr int kSNT = 256;      // threads per workgroup; thread m owns latent m (M <= 256)
constexpr int kSTok = 16;      // tokens per LDS tile
constexpr float kSLog2e = 1.4426950408889634f;

__device__ __forceinline__ float sexp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ size_t stok(int b, int t, int h, int N, int H, int D) {
    return (((size_t)b * N + t) * H + h) * D;
}

// State after block g (exclusive prefix of block g + 1, or the final state).
struct BlockStates {
    const float *pm, *pd, *pn, *fm, *fd, *fu;
    int NB, M, Dv;
    __device__ __forceinline__ void get(int bh, int g, int m, float& mx, float& dn, const float*& num) const {
        if (g + 1 < NB) {
            const size_t r = ((size_t)bh * NB + g + 1) * M + m;
            mx = pm[r];
            dn = pd[r];
            num = pn + r * Dv;
        } else {
            const size_t r = (size_t)bh * M + m;
            mx = fm[r];
            dn = fd[r];
            num = fu + r * Dv;
        }
    }
    // log2 of the den after block g
    __device__ __forceinline__ float log2den(int bh, int g, int m) const {
        float mx, dn;
        const float* num;
        get(bh, g, m, mx, dn, num);
        return mx * kSLog2e + __log2f(dn);
    }
};

// ---------------------------------------------------------------------------
// semi_bwd_tok: s2 = scale log2(e) k.q, alpha = softmax_m(a), c = alpha gz with
// gz_tm = dY_t . z_g,m.  Thread m; tokens in tiles of kSTok.  MF (bf16 inputs,
// whole 16-latent / 32-column tiles): the scores (exact) and dY . num (num as
// bf16 hi + lo) on the MFMA, handed to the thread of latent m through LDS.
// ---------------------------------------------------------------------------
template <typename T, bool MF>
__global__ __launch_bounds__(kSNT) void semi_bwd_tok_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ Qd, const T* __restrict__ Kd,
    const T* __restrict__ dY, int N, int H, int M, int Dk, int Dv, int blk, float scale, bool shared, BlockStates st,
    float* __restrict__ S, float* __restrict__ AL, float* __restrict__ C) {
    __shared__ __attribute__((aligned(16))) float kt[kSTok * 256];
    __shared__ __attribute__((aligned(16))) float qdt[kSTok * 256];
    __shared__ float at[kSTok * 256];
    __shared__ __attribute__((aligned(16))) float gt[kSTok * 512];
    __shared__ float lse[kSTok];
    const int g = blockIdx.x, bh = blockIdx.y;
    const int b = bh / H, h = bh % H, tid = threadIdx.x, m = tid;
    const bool act = m < M;
    float zmx = 0.0f, zdn = 1.0f;
    const float* znum = nullptr;
    if (act) st.get(bh, g, m, zmx, zdn, znum);
    const float zinv = 1.0f / zdn;
    const T* qrow = Q + ((size_t)h * M + (act ? m : 0)) * Dk;
    const T* kdrow = Kd + ((size_t)h * M + (act ? m : 0)) * Dk;
    const int tb0 = g * blk;
    for (int i0 = 0; i0 < blk; i0 += kSTok) {
        const int ni = min(kSTok, blk - i0);
        const int t0 = tb0 + i0;
        __syncthreads();
        if constexpr (MF) {
            // D[m][token] for the encoder scores (at), decoder scores (kt) and dY . num (gt),
            // each as [token][m]
            using namespace mfma;
            const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
            const bool ok = cl < ni;
            const size_t krow = stok(b, t0 + min(cl, ni - 1), h, N, H, Dk) + 8 * g4;
            const size_t grow = stok(b, t0 + min(cl, ni - 1), h, N, H, Dv) + 8 * g4;
            for (int mt = w; mt < M / 16; mt += kSNT / 64) {
                const size_t lrow = ((size_t)h * M + 16 * mt + cl) * Dk + 8 * g4;
                f32x4 se = f32x4{0.f, 0.f, 0.f, 0.f}, sd = f32x4{0.f, 0.f, 0.f, 0.f}, gzz = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int k0 = 0; k0 < Dk; k0 += 32) {
                    se = mma_in<std::is_same<T, __half>::value>(load8<bf16x8>(reinterpret_cast<const bf16*>(Q) + lrow + k0),
                             ok ? load8<bf16x8>(reinterpret_cast<const bf16*>(K) + krow + k0) : zero8(), se);
                    if (!shared)
                        sd = mma_in<std::is_same<T, __half>::value>(load8<bf16x8>(reinterpret_cast<const bf16*>(Kd) + lrow + k0),
                                 ok ? load8<bf16x8>(reinterpret_cast<const bf16*>(Qd) + krow + k0) : zero8(), sd);
                }
                float zm, zd;
                const float* zr;
                st.get(bh, g, 16 * mt + cl, zm, zd, zr);
                for (int k0 = 0; k0 < Dv; k0 += 32) {
                    const float4 p0 = *reinterpret_cast<const float4*>(zr + k0 + 8 * g4);
                    const float4 p1 = *reinterpret_cast<const float4*>(zr + k0 + 8 * g4 + 4);
                    const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                    bf16x8 ph, pl;
#pragma unroll
                    for (int e = 0; e < 8; ++e) SPLIT2(bf16, pv[e], ph[e], pl[e]);
                    const bf16x8 gb = ok ? load8<bf16x8>(reinterpret_cast<const bf16*>(dY) + grow + k0) : zero8();
                    gzz = mma_split<std::is_same<T, __half>::value>(ph, pl, gb, gzz);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int mm = 16 * mt + 4 * g4 + r;
                    at[cl * M + mm] = se[r];
                    if (!shared) kt[cl * M + mm] = sd[r];
                    gt[cl * M + mm] = gzz[r];
                }
            }
        } else {
            for (int e = tid; e < kSTok * Dk; e += kSNT) {
                const int i = e / Dk, d = e % Dk;
                const size_t gi = stok(b, t0 + i, h, N, H, Dk) + d;
                kt[e] = i < ni ? to_f32(K[gi]) : 0.0f;
                if (!shared) qdt[e] = i < ni ? to_f32(Qd[gi]) : 0.0f;
            }
            for (int e = tid; e < kSTok * Dv; e += kSNT) {
                const int i = e / Dv, d = e % Dv;
                gt[e] = i < ni ? to_f32(dY[stok(b, t0 + i, h, N, H, Dv) + d]) : 0.0f;
            }
        }
        __syncthreads();
        float as[kSTok], aa[kSTok], gzm[kSTok];
#pragma unroll
        for (int i = 0; i < kSTok; ++i) as[i] = aa[i] = gzm[i] = 0.0f;
        if constexpr (MF) {
            if (act) {
#pragma unroll
                for (int i = 0; i < kSTok; ++i) {
                    as[i] = at[i * M + m];
                    if (!shared) aa[i] = kt[i * M + m];
                    gzm[i] = gt[i * M + m];
                }
            }
        }
        if (act) {
            for (int d = 0; d < (MF ? 0 : Dk); d += 4) {
                const float q0 = to_f32(qrow[d]), q1 = to_f32(qrow[d + 1]), q2 = to_f32(qrow[d + 2]),
                            q3 = to_f32(qrow[d + 3]);
#pragma unroll
                for (int i = 0; i < kSTok; ++i) {
                    const float4 kr = *reinterpret_cast<const float4*>(kt + i * Dk + d);
                    as[i] += kr.x * q0 + kr.y * q1 + kr.z * q2 + kr.w * q3;
                }
                if (!shared) {
                    const float k0 = to_f32(kdrow[d]), k1 = to_f32(kdrow[d + 1]), k2 = to_f32(kdrow[d + 2]),
                                k3 = to_f32(kdrow[d + 3]);
#pragma unroll
                    for (int i = 0; i < kSTok; ++i) {
                        const float4 qr = *reinterpret_cast<const float4*>(qdt + i * Dk + d);
                        aa[i] += qr.x * k0 + qr.y * k1 + qr.z * k2 + qr.w * k3;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kSTok; ++i) {
                if (i < ni) {
                    const float s = as[i] * scale;
                    S[((size_t)bh * N + t0 + i) * M + m] = s * kSLog2e;
                    at[i * M + m] = shared ? s : aa[i] * scale;
                }
            }
        }
        __syncthreads();
        {   // decoder log-sum-exp per token: wavefront w handles tokens w, w+4, ...
            const int w = tid >> 6, lane = tid & 63;
            for (int i = w; i < ni; i += kSNT / 64) {
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
        if (!act) continue;
        float gz[kSTok];
#pragma unroll
        for (int i = 0; i < kSTok; ++i) gz[i] = gzm[i];
        for (int d = 0; d < (MF ? 0 : Dv); d += 4) {
            const float4 u = *reinterpret_cast<const float4*>(znum + d);
#pragma unroll
            for (int i = 0; i < kSTok; ++i) {
                const float4 gg = *reinterpret_cast<const float4*>(gt + i * Dv + d);
                gz[i] += gg.x * u.x + gg.y * u.y + gg.z * u.z + gg.w * u.w;
            }
        }
#pragma unroll
        for (int i = 0; i < kSTok; ++i) {
            if (i < ni) {
                const size_t o = ((size_t)bh * N + t0 + i) * M + m;
                const float al = __expf(at[i * M + m] - lse[i]);
                AL[o] = al;
                C[o] = al * gz[i] * zinv;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// semi_bwd_dz: dz_g[m][d] = sum_{t in g} alpha_tm g_t[d] and c_g[m] = sum_t c_tm.
// Per value slab of 64, thread (mi = tid % 32, di = tid / 32) owns the 8 x 8
// tile m = 8 mi .., d = 8 di ..; tokens in tiles of kSTok.
// ---------------------------------------------------------------------------
constexpr int kSGP = 68;

template <typename T>
__global__ __launch_bounds__(kSNT) void semi_bwd_dz_kernel(const T* __restrict__ dY, int N, int H, int M, int Dv,
                                                           int blk, int NB, const float* __restrict__ AL,
                                                           const float* __restrict__ C, float* __restrict__ X,
                                                           float* __restrict__ Yb) {
    __shared__ __attribute__((aligned(16))) float alt[kSTok * 256];
    __shared__ __attribute__((aligned(16))) float gs[kSTok * kSGP];
    const int g = blockIdx.x, bh = blockIdx.y;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int tb0 = g * blk;
    const size_t sbase = ((size_t)bh * NB + g) * M;
    if (tid < M) {
        float sum = 0.0f;
        for (int t = 0; t < blk; ++t) sum += C[((size_t)bh * N + tb0 + t) * M + tid];
        Yb[sbase + tid] = sum;
    }
    const int mi = tid & 31, di = tid >> 5;
    const bool act = 8 * mi < M;
    for (int d0 = 0; d0 < Dv; d0 += 64) {
        const int ds = min(64, Dv - d0);
        float acc[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
        for (int i0 = 0; i0 < blk; i0 += kSTok) {
            const int ni = min(kSTok, blk - i0);
            __syncthreads();
            for (int e = tid; e < kSTok * M; e += kSNT) {
                const int i = e / M;
                alt[e] = i < ni ? AL[((size_t)bh * N + tb0 + i0) * M + e] : 0.0f;
            }
            for (int e = tid; e < kSTok * 64; e += kSNT) {
                const int i = e >> 6, d = e & 63;
                gs[i * kSGP + d] = (i < ni && d < ds) ? to_f32(dY[stok(b, tb0 + i0 + i, h, N, H, Dv) + d0 + d]) : 0.0f;
            }
            __syncthreads();
            if (!act || 8 * di >= ds) continue;
            for (int i = 0; i < ni; ++i) {
                const float4 a0 = *reinterpret_cast<const float4*>(alt + i * M + 8 * mi);
                const float4 a1 = *reinterpret_cast<const float4*>(alt + i * M + 8 * mi + 4);
                const float4 b0 = *reinterpret_cast<const float4*>(gs + i * kSGP + 8 * di);
                const float4 b1 = *reinterpret_cast<const float4*>(gs + i * kSGP + 8 * di + 4);
                const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < 8; ++c) acc[r][c] += av[r] * bv[c];
            }
        }
        if (act && 8 * di < ds) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                float* dst = X + (sbase + 8 * mi + r) * Dv + d0 + 8 * di;
                *reinterpret_cast<float4*>(dst) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
                *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[r][4], acc[r][5], acc[r][6], acc[r][7]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// semi_bwd_carry: in place, X_g = dz_g + e^{L_g - L_g+1} X_g+1 (and Y_g alike),
// from the last block down.  Thread per (bh, m, four value columns); blocks are
// read kSScanB at a time.
// ---------------------------------------------------------------------------
constexpr int kSScanB = 8;

__global__ __launch_bounds__(256) void semi_bwd_carry_kernel(float* __restrict__ X, float* __restrict__ Yb,
                                                             BlockStates st, int NB, int M, int Dv, int64_t rows) {
    const int D4 = Dv >> 2;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * D4) return;
    const int64_t row = gid / D4;
    const int j = (int)(gid % D4);
    const int bh = (int)(row / M), m = (int)(row % M);
    float4* x4 = reinterpret_cast<float4*>(X);
    float4 xc = make_float4(0.f, 0.f, 0.f, 0.f);
    float yc = 0.0f;
    float lnext = 0.0f;
    for (int g1 = NB - 1; g1 >= 0; g1 -= kSScanB) {
        float4 xv[kSScanB];
        float yv[kSScanB], lv[kSScanB];
#pragma unroll
        for (int i = 0; i < kSScanB; ++i) {
            const int g = g1 - i;
            const size_t si = ((size_t)bh * NB + max(g, 0)) * M + m;
            xv[i] = g >= 0 ? x4[si * D4 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
            yv[i] = g >= 0 ? Yb[si] : 0.0f;
            lv[i] = g >= 0 ? st.log2den(bh, g, m) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kSScanB; ++i) {
            const int g = g1 - i;
            if (g < 0) break;
            const float f = g == NB - 1 ? 0.0f : sexp2(lv[i] - lnext);
            xc.x = xv[i].x + f * xc.x;
            xc.y = xv[i].y + f * xc.y;
            xc.z = xv[i].z + f * xc.z;
            xc.w = xv[i].w + f * xc.w;
            yc = yv[i] + f * yc;
            lnext = lv[i];
            const size_t si = ((size_t)bh * NB + g) * M + m;
            x4[si * D4 + j] = xc;
            if (j == 0) Yb[si] = yc;
        }
    }
}

// ---------------------------------------------------------------------------
// semi_bwd_dv: dv_tau[d] = sum_m e^{s_tau m - L_g,m} X_g,m[d].  grid (NB, BH,
// ceil(Dv / 64)); thread (col, rg) owns dv[tau = rg + 4 r][d0 + col] of each
// token tile, whose factors are staged in LDS.
// ---------------------------------------------------------------------------
template <typename T, bool MF>
__global__ __launch_bounds__(kSNT) void semi_bwd_dv_kernel(int N, int H, int M, int Dv, int blk, int NB,
                                                           const float* __restrict__ S, BlockStates st,
                                                           const float* __restrict__ X, T* __restrict__ dV) {
    __shared__ __attribute__((aligned(16))) float pt[kSTok * 256];
    __shared__ float lg[256];
    const int g = blockIdx.x, bh = blockIdx.y, d0 = blockIdx.z * 64;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int tb0 = g * blk;
    if (tid < M) lg[tid] = st.log2den(bh, g, tid);
    if constexpr (MF) {
        // 16-bit inputs, M % 32 == 0, whole 64-column slabs: D[token][d] = sum_m P X on the
        // MFMA, P = 2^(s - L_g) and X both fp32 as bf16 hi + lo (three products); wave w
        // owns columns d0 + 16 w ..
        using namespace mfma;
        __syncthreads();   // lg visible
        const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
        const float* xb = X + ((size_t)bh * NB + g) * M * Dv + d0 + 16 * w + cl;
        for (int i0 = 0; i0 < blk; i0 += 16) {
            const int tok = tb0 + i0 + cl;
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int m0 = 0; m0 < M; m0 += 32) {
                const float* srow = S + ((size_t)bh * N + tok) * M + m0 + 8 * g4;
                bf16x8 ph, pl, xh, xl;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    SPLIT2(bf16, sexp2(srow[e] - lg[m0 + 8 * g4 + e]), ph[e], pl[e]);
                    SPLIT2(bf16, xb[(size_t)(m0 + 8 * g4 + e) * Dv], xh[e], xl[e]);
                }
                acc = mma(ph, xh, acc);
                acc = mma(ph, xl, acc);
                acc = mma(pl, xh, acc);
            }
            // rows: tokens i0 + 4 g + r, column d0 + 16 w + cl
#pragma unroll
            for (int r = 0; r < 4; ++r)
                dV[stok(b, tb0 + i0 + 4 * g4 + r, h, N, H, Dv) + d0 + 16 * w + cl] = from_f32<T>(acc[r]);
        }
        return;
    }
    const int col = tid & 63, rg = tid >> 6;
    const bool act = d0 + col < Dv;
    const float* xr = X + ((size_t)bh * NB + g) * M * Dv + d0 + col;
    for (int i0 = 0; i0 < blk; i0 += kSTok) {
        const int ni = min(kSTok, blk - i0);
        __syncthreads();
        for (int e = tid; e < kSTok * M; e += kSNT) {
            const int i = e / M, m = e % M;
            pt[e] = i < ni ? sexp2(S[((size_t)bh * N + tb0 + i0) * M + e] - lg[m]) : 0.0f;
        }
        __syncthreads();
        if (!act) continue;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int m = 0; m < M; m += 4) {
            const float x0 = xr[(size_t)m * Dv], x1 = xr[(size_t)(m + 1) * Dv], x2 = xr[(size_t)(m + 2) * Dv],
                        x3 = xr[(size_t)(m + 3) * Dv];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 p = *reinterpret_cast<const float4*>(pt + (rg + 4 * r) * M + m);
                acc[r] += p.x * x0 + p.y * x1 + p.z * x2 + p.w * x3;
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = rg + 4 * r;
            if (i < ni) dV[stok(b, tb0 + i0 + i, h, N, H, Dv) + d0 + col] = from_f32<T>(acc[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// semi_bwd_ds: ds_tau m = e^{s_tau m - L_g,m} (v_tau . X_g,m - Y_g,m), written
// over s.  Thread m; value tiles of kSTok tokens staged in LDS.
// ---------------------------------------------------------------------------
template <typename T, bool MF>
__global__ __launch_bounds__(kSNT) void semi_bwd_ds_kernel(const T* __restrict__ V, int N, int H, int M, int Dv,
                                                           int blk, int NB, float* __restrict__ S, BlockStates st,
                                                           const float* __restrict__ X,
                                                           const float* __restrict__ Yb, const float* __restrict__ AL,
                                                           const float* __restrict__ C, const float* __restrict__ gy,
                                                           bool dsum) {
    __shared__ __attribute__((aligned(16))) float vt[kSTok * 512];
    const int g = blockIdx.x, bh = blockIdx.y;
    const int b = bh / H, h = bh % H, tid = threadIdx.x, m = tid;
    const bool act = m < M;
    const int tb0 = g * blk;
    const size_t sbase = ((size_t)bh * NB + g) * M + (act ? m : 0);
    const float lgm = act ? st.log2den(bh, g, m) : 0.0f;
    const float ym = act ? Yb[sbase] : 0.0f;
    const float* xr = X + sbase * Dv;
    for (int i0 = 0; i0 < blk; i0 += kSTok) {
        const int ni = min(kSTok, blk - i0);
        __syncthreads();
        if constexpr (MF) {
            // D[m][token] = X[m] . v_token (X as bf16 hi + lo, V exact) to LDS as [token][m]
            using namespace mfma;
            const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
            const bool ok = cl < ni;
            const bf16* vrow = reinterpret_cast<const bf16*>(V) + stok(b, tb0 + i0 + min(cl, ni - 1), h, N, H, Dv) + 8 * g4;
            for (int mt = w; mt < M / 16; mt += kSNT / 64) {
                const float* xrow = X + (((size_t)bh * NB + g) * M + 16 * mt + cl) * Dv + 8 * g4;
                f32x4 d2 = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int k0 = 0; k0 < Dv; k0 += 32) {
                    const float4 p0 = *reinterpret_cast<const float4*>(xrow + k0);
                    const float4 p1 = *reinterpret_cast<const float4*>(xrow + k0 + 4);
                    const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                    bf16x8 ph, pl;
#pragma unroll
                    for (int e = 0; e < 8; ++e) SPLIT2(bf16, pv[e], ph[e], pl[e]);
                    const bf16x8 vb = ok ? load8<bf16x8>(vrow + k0) : zero8();
                    d2 = mma_split<std::is_same<T, __half>::value>(ph, pl, vb, d2);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) vt[cl * M + 16 * mt + 4 * g4 + r] = d2[r];
            }
        } else {
            for (int e = tid; e < kSTok * Dv; e += kSNT) {
                const int i = e / Dv, d = e % Dv;
                vt[e] = i < ni ? to_f32(V[stok(b, tb0 + i0 + i, h, N, H, Dv) + d]) : 0.0f;
            }
        }
        __syncthreads();
        if (!act) continue;
        float vx[kSTok];
#pragma unroll
        for (int i = 0; i < kSTok; ++i) vx[i] = MF ? vt[i * M + m] : 0.0f;
        for (int d = 0; d < (MF ? 0 : Dv); d += 4) {
            const float4 x = *reinterpret_cast<const float4*>(xr + d);
#pragma unroll
            for (int i = 0; i < kSTok; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(vt + i * Dv + d);
                vx[i] += v.x * x.x + v.y * x.y + v.z * x.z + v.w * x.w;
            }
        }
#pragma unroll
        for (int i = 0; i < kSTok; ++i) {
            if (i < ni) {
                const size_t o = ((size_t)bh * N + tb0 + i0 + i) * M + m;
                const float da = dsum ? C[o] - AL[o] * gy[(size_t)bh * N + tb0 + i0 + i] : 0.0f;
                S[o] = sexp2(S[o] - lgm) * (vx[i] - ym) + da;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct SemiBwdLayout {
    int64_t NB;
    size_t off_bm, off_bd, off_bn, off_fm, off_fd, off_fu, off_s, off_al, off_c, off_gy, off_x, off_y, off_p1,
        off_p2, total;
    SemiBwdLayout(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, int64_t block) {
        NB = N / block;
        const size_t BH = (size_t)B * H;
        size_t o = 0;
        auto take = [&](size_t floats) {
            const size_t at = o;
            o += ((floats * sizeof(float) + 255) / 256) * 256;
            return at;
        };
        off_bm = take(BH * NB * M);
        off_bd = take(BH * NB * M);
        off_bn = take(BH * NB * M * Dv);
        off_fm = take(BH * M);
        off_fd = take(BH * M);
        off_fu = take(BH * M * Dv);
        off_s = take(BH * N * M);
        off_al = take(BH * N * M);
        off_c = take(BH * N * M);
        off_gy = take(BH * N);
        off_x = take(BH * NB * M * Dv);
        off_y = take(BH * NB * M);
        off_p1 = take(bwd_partial_floats(B, N, H, M, Dk));
        off_p2 = take(bwd_partial_floats(B, N, H, M, Dk));
        total = o + 256;
    }
};

template <typename T>
static int run_semi_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                             int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                             float scale, int64_t block, const void* Y, const void* dY, void* dQ, void* dK, void* dV,
                             void* dQd, void* dKd, char* ws, const SemiBwdLayout& lay, hipStream_t s) {
    auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
    float *bm = F(lay.off_bm), *bd = F(lay.off_bd), *bn = F(lay.off_bn), *fm = F(lay.off_fm), *fd = F(lay.off_fd),
          *fu = F(lay.off_fu), *S = F(lay.off_s), *AL = F(lay.off_al), *C = F(lay.off_c), *gy = F(lay.off_gy),
          *X = F(lay.off_x), *Yb = F(lay.off_y), *P1 = F(lay.off_p1), *P2 = F(lay.off_p2);
    const int64_t NB = lay.NB, BH = B * H;
    const bool shared = Qdec == nullptr && Kdec == nullptr;
    const T* q = static_cast<const T*>(Q);
    const T* k = static_cast<const T*>(K);
    const T* qd = Qdec ? static_cast<const T*>(Qdec) : k;
    const T* kd = Kdec ? static_cast<const T*>(Kdec) : q;
    int rc;
    if ((rc = launch_prepare_public(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, block, bm, bd, bn, s))) return rc;
    if ((rc = launch_prefix_public(bm, bd, bn, BH, NB, M, Dv, nullptr, nullptr, nullptr, fm, fd, fu, s))) return rc;
    const BlockStates st{bm, bd, bn, fm, fd, fu, (int)NB, (int)M, (int)Dv};
    const dim3 gb((unsigned)NB, (unsigned)BH);
    bool tok_mfma = false;
    if constexpr (std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) {
        tok_mfma = M % 16 == 0 && Dk % 32 == 0 && Dv % 32 == 0;
        if (tok_mfma)
            hipLaunchKernelGGL((semi_bwd_tok_kernel<T, true>), gb, dim3(kSNT), 0, s, q, k, qd, kd,
                               static_cast<const T*>(dY), (int)N, (int)H, (int)M, (int)Dk, (int)Dv, (int)block, scale,
                               shared, st, S, AL, C);
    }
    if (!tok_mfma)
        hipLaunchKernelGGL((semi_bwd_tok_kernel<T, false>), gb, dim3(kSNT), 0, s, q, k, qd, kd,
                           static_cast<const T*>(dY), (int)N, (int)H, (int)M, (int)Dk, (int)Dv, (int)block, scale,
                           shared, st, S, AL, C);
    if ((rc = check_launch("semi_bwd_tok_kernel"))) return rc;
    if ((std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) &&
        bwd_summary_mfma_supported(M, Dv)) {
        if ((rc = launch_semi_dz_mfma(dY, B, N, H, M, Dv, block, AL, C, X, Yb, std::is_same<T, __half>::value, s)))
            return rc;
    } else {
        hipLaunchKernelGGL(semi_bwd_dz_kernel<T>, gb, dim3(kSNT), 0, s, static_cast<const T*>(dY), (int)N, (int)H,
                           (int)M, (int)Dv, (int)block, (int)NB, AL, C, X, Yb);
        if ((rc = check_launch("semi_bwd_dz_kernel"))) return rc;
    }
    const int64_t cthreads = BH * M * (Dv / 4);
    hipLaunchKernelGGL(semi_bwd_carry_kernel, dim3((unsigned)((cthreads + 255) / 256)), dim3(256), 0, s, X, Yb, st,
                       (int)NB, (int)M, (int)Dv, BH * M);
    if ((rc = check_launch("semi_bwd_carry_kernel"))) return rc;
    const dim3 gdv((unsigned)NB, (unsigned)BH, (unsigned)((Dv + 63) / 64));
    bool dv_mfma = false;
    if constexpr (std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) {
        dv_mfma = M % 32 == 0 && Dv % 64 == 0;
        if (dv_mfma)
            hipLaunchKernelGGL((semi_bwd_dv_kernel<T, true>), gdv, dim3(kSNT), 0, s, (int)N, (int)H, (int)M, (int)Dv,
                               (int)block, (int)NB, S, st, X, static_cast<T*>(dV));
    }
    if (!dv_mfma)
        hipLaunchKernelGGL((semi_bwd_dv_kernel<T, false>), gdv, dim3(kSNT), 0, s, (int)N, (int)H, (int)M, (int)Dv,
                           (int)block, (int)NB, S, st, X, static_cast<T*>(dV));
    if ((rc = check_launch("semi_bwd_dv_kernel"))) return rc;
    // shared weights: semi_bwd_ds adds da = c - alpha gy to ds, and the contractions read
    // that one array (not C, alpha and gy)
    const bool dsum = shared;
    if ((rc = launch_bwd_gy(dY, Y, dtype, B, N, H, Dv, gy, s))) return rc;
    bool ds_mfma = false;
    if constexpr (std::is_same<T, __hip_bfloat16>::value || std::is_same<T, __half>::value) {
        ds_mfma = M % 16 == 0 && Dv % 32 == 0;
        if (ds_mfma)
            hipLaunchKernelGGL((semi_bwd_ds_kernel<T, true>), gb, dim3(kSNT), 0, s, static_cast<const T*>(V), (int)N,
                               (int)H, (int)M, (int)Dv, (int)block, (int)NB, S, st, X, Yb, AL, C, gy, dsum);
    }
    if (!ds_mfma)
        hipLaunchKernelGGL((semi_bwd_ds_kernel<T, false>), gb, dim3(kSNT), 0, s, static_cast<const T*>(V), (int)N,
                           (int)H, (int)M, (int)Dv, (int)block, (int)NB, S, st, X, Yb, AL, C, gy, dsum);
    if ((rc = check_launch("semi_bwd_ds_kernel"))) return rc;
    return launch_bwd_contract(Q, K, Qdec, Kdec, dtype, B, N, H, M, Dk, scale, S, AL, C, gy, false, dsum, dQ, dK, dQd,
                               dKd, P1, P2, s);
}

}  // namespace flare

using namespace flare;

extern "C" {

size_t flare_semi_ar_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                                             int64_t block) {
    if (block <= 0) return 0;
    return SemiBwdLayout(B, N, H, M, Dk, Dv, block).total;
}

int flare_semi_ar_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                           int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                           float scale, int64_t block, const void* Y, const void* dY, void* dQ, void* dK, void* dV,
                           void* dQdec, void* dKdec, void* workspace, size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y && dY && dQ && dK && dV, "flare_semi_ar_backward: null tensor pointer");
    FLARE_REQUIRE(dtype == FLARE_F32 || dtype == FLARE_BF16 || dtype == FLARE_F16,
                  "flare_semi_ar_backward: unknown dtype code %d", dtype);
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0, "flare_semi_ar_backward: empty problem (B=%lld N=%lld H=%lld)",
                  (long long)B, (long long)N, (long long)H);
    FLARE_REQUIRE(block > 0 && block % 16 == 0 && N % block == 0,
                  "flare_semi_ar_backward: need block %% 16 == 0 and N %% block == 0 (N=%lld, block=%lld)",
                  (long long)N, (long long)block);
    FLARE_REQUIRE(M % 16 == 0 && M >= 16 && M <= 256,
                  "flare_semi_ar_backward: M=%lld must be a multiple of 16 in [16, 256]", (long long)M);
    FLARE_REQUIRE(Dk % 16 == 0 && Dk >= 16 && Dk <= 256,
                  "flare_semi_ar_backward: D_score=%lld must be a multiple of 16 in [16, 256]", (long long)Dk);
    FLARE_REQUIRE(Dv % 16 == 0 && Dv >= 16 && Dv <= 512,
                  "flare_semi_ar_backward: D_value=%lld must be a multiple of 16 in [16, 512]", (long long)Dv);
    FLARE_REQUIRE(!Qdec || dQdec, "flare_semi_ar_backward: Qdec given without dQdec");
    FLARE_REQUIRE(!Kdec || dKdec, "flare_semi_ar_backward: Kdec given without dKdec");
    const SemiBwdLayout lay(B, N, H, M, Dk, Dv, block);
    FLARE_REQUIRE(workspace && workspace_bytes >= lay.total,
                  "flare_semi_ar_backward: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                  lay.total);
    FLARE_REQUIRE((((uintptr_t)workspace) & 255) == 0, "flare_semi_ar_backward: workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
#define FLARE_SEMI_BWD(TY)                                                                                        \
    return run_semi_backward<TY>(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, block, Y, dY, dQ, dK, dV, \
                                 dQdec, dKdec, ws, lay, st)
    if (dtype == FLARE_BF16) FLARE_SEMI_BWD(__hip_bfloat16);
    if (dtype == FLARE_F16) FLARE_SEMI_BWD(__half);
    FLARE_SEMI_BWD(float);
#undef FLARE_SEMI_BWD
}

}  // extern "C"
