// flare_bwd_mfma.hip -- bf16 MFMA contractions of the FLARE backward on gfx950.
//
// dK (and dQ_dec) are contractions over the latent bank of the score gradients
// ds and da = alpha (gz - gy) (fp32, [B*H, N, M]; C holds alpha gz or gz, see score_grad_da;
// dsum: DS already holds ds + da, for the shared-weight instances, which read no C or alpha) with the bf16 latent tensors:
//     dK_t   = scale sum_m (ds_tm Q_m  [+ da_tm Kd_m when Qd = K])
//     dQd_t  = scale sum_m  da_tm Kd_m                  (separate Qd)
// (the per-token loop of bwd_dk in flare_ar_bwd.hip, which stays the fp32 /
// fp16 path).  Here each fp32 gradient is split into bf16 hi + lo parts, so
// that hi x Q + lo x Q carries about 16 mantissa bits of the gradient while Q
// enters exactly; the products accumulate in fp32 on the 16x16x32 bf16 MFMA.
#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {
namespace mfma {

constexpr int kDkMfmaTok = 128;     // tokens per workgroup (32 per wave)
constexpr int kDkMaxM = 256;
constexpr int kDkLP = kDkMaxM + 8;  // padded row of the transposed latent tensors in LDS

// A operand (rows = 16 tokens, k = 8 latents of this lane) of one fp32 row as bf16 hi and lo.
__device__ __forceinline__ void split8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) SPLIT2(bf16, x[e], hi[e], lo[e]);
}

// TWO_B: a second latent tensor Kd (transposed in LDS) multiplies da
// TWO_OUT: da goes to a second output dQd instead of into dK
template <int DK, bool TWO_B, bool TWO_OUT, bool F16>
__global__ __launch_bounds__(256) void bwd_dk_mfma(const bf16* __restrict__ Q, const bf16* __restrict__ Kd, int N,
                                                   int H, int M, float scale, const float* __restrict__ DS,
                                                   const float* __restrict__ AL, const float* __restrict__ C,
                                                   const float* __restrict__ gy, bool cgz, bool dsum,
                                                   __hip_bfloat16* __restrict__ dK,
                                                   __hip_bfloat16* __restrict__ dQd) {
    constexpr int NJ = DK / 16;
    __shared__ __attribute__((aligned(16))) bf16 qt[DK * kDkLP];                 // Q^T[d][m]
    __shared__ __attribute__((aligned(16))) bf16 kt[TWO_B ? DK * kDkLP : 8];     // Kd^T[d][m]
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    // ---- latent tensors of head h, transposed (8 values of one row per thread step)
    for (int e = tid; e < M * DK / 8; e += 256) {
        const int m = e / (DK / 8), d8 = e % (DK / 8);
        const bf16x8 qv = load8<bf16x8>(Q + ((size_t)h * M + m) * DK + 8 * d8);
#pragma unroll
        for (int i = 0; i < 8; ++i) qt[(8 * d8 + i) * kDkLP + m] = qv[i];
        if constexpr (TWO_B) {
            const bf16x8 kv = load8<bf16x8>(Kd + ((size_t)h * M + m) * DK + 8 * d8);
#pragma unroll
            for (int i = 0; i < 8; ++i) kt[(8 * d8 + i) * kDkLP + m] = kv[i];
        }
    }
    __syncthreads();
    const int tw0 = blockIdx.x * kDkMfmaTok + 32 * w;
    f32x4 acc[2][NJ], acc2[TWO_OUT ? 2 : 1][TWO_OUT ? NJ : 1];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            acc[ti][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (TWO_OUT) acc2[ti][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    float gyt[2];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
        const int t = tw0 + 16 * ti + c;
        gyt[ti] = t < N ? gy[(size_t)bh * N + t] : 0.0f;
    }
    for (int m0 = 0; m0 < M; m0 += 32) {
        bf16x8 bq[NJ], bk[TWO_B ? NJ : 1];
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            bq[nj] = load8<bf16x8>(qt + (16 * nj + c) * kDkLP + m0 + 8 * g);
            if constexpr (TWO_B) bk[nj] = load8<bf16x8>(kt + (16 * nj + c) * kDkLP + m0 + 8 * g);
        }
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const int t = tw0 + 16 * ti + c;
            float ds[8], da[8];
            if (t < N) {
                const size_t o = ((size_t)bh * N + t) * M + m0 + 8 * g;
                const f32x4 s0 = *reinterpret_cast<const f32x4*>(DS + o), s1 = *reinterpret_cast<const f32x4*>(DS + o + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ds[e] = s0[e];
                    ds[4 + e] = s1[e];
                    da[e] = da[4 + e] = 0.0f;
                }
                if (!(dsum && !TWO_B && !TWO_OUT)) {
                    const f32x4 c0 = *reinterpret_cast<const f32x4*>(C + o), c1 = *reinterpret_cast<const f32x4*>(C + o + 4);
                    const f32x4 a0 = *reinterpret_cast<const f32x4*>(AL + o), a1 = *reinterpret_cast<const f32x4*>(AL + o + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        da[e] = score_grad_da(c0[e], a0[e], gyt[ti], cgz);
                        da[4 + e] = score_grad_da(c1[e], a1[e], gyt[ti], cgz);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) ds[e] = da[e] = 0.0f;
            }
            if constexpr (!TWO_B && !TWO_OUT) {   // dK = (ds + da) Q
#pragma unroll
                for (int e = 0; e < 8; ++e) ds[e] += da[e];
            }
            bf16x8 sh, sl;
            split8(ds, sh, sl);
#pragma unroll
            for (int nj = 0; nj < NJ; ++nj) {
                acc[ti][nj] = mma_split<F16>(sh, sl, bq[nj], acc[ti][nj]);
            }
            if constexpr (TWO_B || TWO_OUT) {
                bf16x8 ah, alo;
                split8(da, ah, alo);
#pragma unroll
                for (int nj = 0; nj < NJ; ++nj) {
                    const bf16x8 bb = TWO_B ? bk[nj] : bq[nj];
                    if constexpr (TWO_OUT) {
                        acc2[ti][nj] = mma_split<F16>(ah, alo, bb, acc2[ti][nj]);
                    } else {
                        acc[ti][nj] = mma_split<F16>(ah, alo, bb, acc[ti][nj]);
                    }
                }
            }
        }
    }
    // ---- rows 4 g + r of each token tile, column 16 nj + c
    const size_t stride = (size_t)H * DK;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tw0 + 16 * ti + 4 * g + r;
            if (t >= N) continue;
            const size_t o = ((size_t)b * N + t) * stride + (size_t)h * DK + c;
#pragma unroll
            for (int nj = 0; nj < NJ; ++nj) {
                // outputs in the input dtype (the pointers are bf16-typed 16-bit storage)
                if constexpr (F16) {
                    reinterpret_cast<f16*>(dK)[o + 16 * nj] = (f16)(scale * acc[ti][nj][r]);
                    if constexpr (TWO_OUT) reinterpret_cast<f16*>(dQd)[o + 16 * nj] = (f16)(scale * acc2[ti][nj][r]);
                } else {
                    dK[o + 16 * nj] = __float2bfloat16(scale * acc[ti][nj][r]);
                    if constexpr (TWO_OUT) dQd[o + 16 * nj] = __float2bfloat16(scale * acc2[ti][nj][r]);
                }
            }
        }
}

// dQ / dK_dec partial sums over a group of kDqGroup tokens (the bf16 MFMA form
// of bwd_dq in flare_ar_bwd.hip):
//     P1_m = sum_t ds_tm k_t (+ da_tm qd_t when Kd = Q),   P2_m = sum_t da_tm qd_t
// The contraction runs over tokens, the row index of both ds and K, so each
// 32-token subtile is staged transposed in LDS: ds^T (bf16 hi and lo) and K^T.
// Wave w owns latent rows [w M / 4, (w + 1) M / 4) and the DKS value columns of
// blockIdx.z.
constexpr int kDqGroup = kBwdGroup;
constexpr int kDqTP = 32 + 8;       // padded row of the transposed subtiles

template <int MW, int DKS, bool TWO_A, bool TWO_B, bool TWO_OUT, bool F16>
__global__ __launch_bounds__(256) void bwd_dq_mfma(const bf16* __restrict__ K, const bf16* __restrict__ Qd, int N,
                                                   int H, int Dk, const float* __restrict__ DS,
                                                   const float* __restrict__ AL, const float* __restrict__ C,
                                                   const float* __restrict__ gy, bool cgz, bool dsum,
                                                   float* __restrict__ P1,
                                                   float* __restrict__ P2) {
    constexpr int M = 64 * MW, NJ = DKS / 16;
    __shared__ __attribute__((aligned(16))) bf16 sh[M * kDqTP], sl[M * kDqTP];                    // ds^T hi, lo
    __shared__ __attribute__((aligned(16))) bf16 ah[TWO_A ? M * kDqTP : 8], alo[TWO_A ? M * kDqTP : 8];   // da^T
    __shared__ __attribute__((aligned(16))) bf16 kt[DKS * kDqTP];                                   // K^T
    __shared__ __attribute__((aligned(16))) bf16 qt[TWO_B ? DKS * kDqTP : 8];                       // Qd^T
    const int grp = blockIdx.x, NG = gridDim.x, bh = blockIdx.y, b = bh / H, h = bh % H;
    const int d0 = blockIdx.z * DKS;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int mw0 = w * 16 * MW;
    f32x4 acc[MW][NJ], acc2[TWO_OUT ? MW : 1][TWO_OUT ? NJ : 1];
#pragma unroll
    for (int mi = 0; mi < MW; ++mi)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            acc[mi][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (TWO_OUT) acc2[mi][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    const int tg0 = grp * kDqGroup, tg1 = min(N, tg0 + kDqGroup);
    const size_t stride = (size_t)H * Dk;
    for (int t0 = tg0; t0 < tg1; t0 += 32) {
        __syncthreads();   // the previous subtile's operands are consumed
        // ---- ds (and da) rows -> transposed hi / lo; lanes run over m (coalesced loads)
        for (int e = tid; e < M * 8; e += 256) {
            const int m = e % M, tq = e / M;
            float x[4], y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + 4 * tq + i;
                if (t < tg1) {
                    const size_t o = ((size_t)bh * N + t) * M + m;
                    x[i] = DS[o];
                    y[i] = (dsum && !TWO_A) ? 0.0f : score_grad_da(C[o], AL[o], gy[(size_t)bh * N + t], cgz);
                } else {
                    x[i] = y[i] = 0.0f;
                }
            }
            bf16x4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) SPLIT2(bf16, TWO_A ? x[i] : x[i] + y[i], hi[i], lo[i]);
            *reinterpret_cast<bf16x4*>(sh + m * kDqTP + 4 * tq) = hi;
            *reinterpret_cast<bf16x4*>(sl + m * kDqTP + 4 * tq) = lo;
            if constexpr (TWO_A) {
#pragma unroll
                for (int i = 0; i < 4; ++i) SPLIT2(bf16, y[i], hi[i], lo[i]);
                *reinterpret_cast<bf16x4*>(ah + m * kDqTP + 4 * tq) = hi;
                *reinterpret_cast<bf16x4*>(alo + m * kDqTP + 4 * tq) = lo;
            }
        }
        // ---- K (and Qd) columns d0 .. d0 + DKS -> transposed
        for (int e = tid; e < DKS * 8; e += 256) {
            const int d = e % DKS, tq = e / DKS;
            bf16x4 kv, qv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + 4 * tq + i;
                const size_t o = ((size_t)b * N + t) * stride + (size_t)h * Dk + d0 + d;
                kv[i] = t < tg1 ? K[o] : (bf16)0.0f;
                if constexpr (TWO_B) qv[i] = t < tg1 ? Qd[o] : (bf16)0.0f;
            }
            *reinterpret_cast<bf16x4*>(kt + d * kDqTP + 4 * tq) = kv;
            if constexpr (TWO_B) *reinterpret_cast<bf16x4*>(qt + d * kDqTP + 4 * tq) = qv;
        }
        __syncthreads();
        // ---- D[m][d] += A[m][t] B[t][d]: A = ds^T rows (hi, lo), B = K^T rows
        bf16x8 bk[NJ], bq[TWO_B ? NJ : 1];
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            bk[nj] = load8<bf16x8>(kt + (16 * nj + c) * kDqTP + 8 * g);
            if constexpr (TWO_B) bq[nj] = load8<bf16x8>(qt + (16 * nj + c) * kDqTP + 8 * g);
        }
#pragma unroll
        for (int mi = 0; mi < MW; ++mi) {
            const int row = (mw0 + 16 * mi + c) * kDqTP + 8 * g;
            const bf16x8 a0 = load8<bf16x8>(sh + row), a1 = load8<bf16x8>(sl + row);
#pragma unroll
            for (int nj = 0; nj < NJ; ++nj) {
                acc[mi][nj] = mma_split<F16>(a0, a1, bk[nj], acc[mi][nj]);
            }
            if constexpr (TWO_A) {
                const bf16x8 e0 = load8<bf16x8>(ah + row), e1 = load8<bf16x8>(alo + row);
#pragma unroll
                for (int nj = 0; nj < NJ; ++nj) {
                    const bf16x8 bb = TWO_B ? bq[nj] : bk[nj];
                    if constexpr (TWO_OUT) {
                        acc2[mi][nj] = mma_split<F16>(e0, e1, bb, acc2[mi][nj]);
                    } else {
                        acc[mi][nj] = mma_split<F16>(e0, e1, bb, acc[mi][nj]);
                    }
                }
            }
        }
    }
    // ---- partials: row m = mw0 + 16 mi + 4 g + r, column d0 + 16 nj + c
#pragma unroll
    for (int mi = 0; mi < MW; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t o = (((size_t)bh * NG + grp) * M + mw0 + 16 * mi + 4 * g + r) * Dk + d0 + c;
#pragma unroll
            for (int nj = 0; nj < NJ; ++nj) {
                P1[o + 16 * nj] = acc[mi][nj][r];
                if constexpr (TWO_OUT) P2[o + 16 * nj] = acc2[mi][nj][r];
            }
        }
}

// Per-chunk terms of the backward's reverse scan (the bf16 MFMA form of
// bwd_summary in flare_ar_bwd.hip), for chunks c >= 1 of 32 tokens:
//     a_c[m][:] = sum_t w_tm g_t,   b_c[m] = sum_t w_tm c_tm,
//     w_tm = 2^(Lpre_m - L_tm) alpha_tm = 2^(Lpre_m - LA_tm)
// (Lpre = L at the last token of chunk c-1; C holds gz).
// a is a contraction over tokens: each lane forms its own A operand (latent
// row m, tokens 8 g .. 8 g + 7) from LA as bf16 hi and lo; g^T (dY, exact) is
// staged transposed in LDS.  b sums the lanes' 8-token parts.
template <int MW, int DV, bool F16>
__global__ __launch_bounds__(256) void bwd_summary_mfma(const bf16* __restrict__ dY, int N, int H,
                                                        const float* __restrict__ L, const float* __restrict__ LA,
                                                        const float* __restrict__ C, float* __restrict__ a_out,
                                                        float* __restrict__ b_out) {
    constexpr int M = 64 * MW, NJ = DV / 16;
    __shared__ __attribute__((aligned(16))) bf16 gt[DV * kDqTP];                  // g^T
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    if (c == 0) return;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, g = lane >> 4, cl = lane & 15;
    const int t0 = c * 32, nt = min(32, N - t0);
    const size_t rbase = ((size_t)bh * N + t0) * M;
    const size_t sbase = ((size_t)bh * NC + c) * M;
    const size_t stride = (size_t)H * DV;
    for (int e = tid; e < DV * 8; e += 256) {
        const int d = e % DV, tq = e / DV;
        bf16x4 gv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 4 * tq + i;
            gv[i] = t < nt ? dY[((size_t)b * N + t0 + t) * stride + (size_t)h * DV + d] : (bf16)0.0f;
        }
        *reinterpret_cast<bf16x4*>(gt + d * kDqTP + 4 * tq) = gv;
    }
    const int mw0 = w * 16 * MW;
    bf16x8 ah[MW], alo[MW];
#pragma unroll
    for (int mi = 0; mi < MW; ++mi) {
        const int m = mw0 + 16 * mi + cl;
        const float lp = L[rbase - M + m];
        float bsum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = 8 * g + e;
            float wv = 0.0f;
            if (t < nt) {
                const size_t o = rbase + (size_t)t * M + m;
                wv = __builtin_amdgcn_exp2f(lp - LA[o]);
                bsum += wv * C[o];
            }
            SPLIT2(bf16, wv, ah[mi][e], alo[mi][e]);
        }
        bsum += __shfl_xor(bsum, 16);
        bsum += __shfl_xor(bsum, 32);
        if (g == 0) b_out[sbase + m] = bsum;
    }
    __syncthreads();
    if constexpr (F16) {
        // fp16 dY: each B tile split into its exact bf16 pair once, for all MW row tiles
        // (the products of mma_split<true>, in its order)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            const f16x8 bf = __builtin_bit_cast(f16x8, load8<bf16x8>(gt + (16 * nj + cl) * kDqTP + 8 * g));
            bf16x8 bh, bl;
#pragma unroll
            for (int e = 0; e < 8; ++e) SPLIT2(bf16, (float)bf[e], bh[e], bl[e]);
#pragma unroll
            for (int mi = 0; mi < MW; ++mi) {
                f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
                acc = mma(ah[mi], bh, acc);
                acc = mma(alo[mi], bh, acc);
                acc = mma(ah[mi], bl, acc);
#pragma unroll
                for (int r = 0; r < 4; ++r) a_out[(sbase + mw0 + 16 * mi + 4 * g + r) * DV + 16 * nj + cl] = acc[r];
            }
        }
        return;
    }
    bf16x8 bg[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) bg[nj] = load8<bf16x8>(gt + (16 * nj + cl) * kDqTP + 8 * g);
#pragma unroll
    for (int mi = 0; mi < MW; ++mi) {
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
            acc = mma_split<false>(ah[mi], alo[mi], bg[nj], acc);
            // rows m = mw0 + 16 mi + 4 g + r, column 16 nj + cl
#pragma unroll
            for (int r = 0; r < 4; ++r) a_out[(sbase + mw0 + 16 * mi + 4 * g + r) * DV + 16 * nj + cl] = acc[r];
        }
    }
}

// Block sums of the block-causal backward (the bf16 MFMA form of semi_bwd_dz in
// flare_semi_bwd.hip): dz_g[m][:] = sum_{t in g} alpha_tm g_t and Yb_g[m] = sum_t c_tm,
// over the block's tokens in 32-token steps (alpha^T as bf16 hi + lo, g^T exact),
// staged transposed in LDS as in bwd_summary_mfma.
template <int MW, int DV, bool F16>
__global__ __launch_bounds__(256) void semi_dz_mfma(const bf16* __restrict__ dY, int N, int H, int blk,
                                                    const float* __restrict__ AL, const float* __restrict__ C,
                                                    float* __restrict__ X, float* __restrict__ Yb) {
    constexpr int M = 64 * MW, NJ = DV / 16;
    __shared__ __attribute__((aligned(16))) bf16 ah[M * kDqTP], alo[M * kDqTP];   // alpha^T hi, lo
    __shared__ __attribute__((aligned(16))) bf16 gt[DV * kDqTP];                  // g^T
    const int g = blockIdx.x, bh = blockIdx.y, NB = gridDim.x;
    const int b = bh / H, h = bh % H, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, g4 = lane >> 4, cl = lane & 15;
    const int tb0 = g * blk;
    const size_t sbase = ((size_t)bh * NB + g) * M;
    const size_t stride = (size_t)H * DV;
    const int mw0 = w * 16 * MW;
    f32x4 acc[MW][NJ];
#pragma unroll
    for (int mi = 0; mi < MW; ++mi)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) acc[mi][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ysum = 0.0f;
    for (int k0 = 0; k0 < blk; k0 += 32) {
        const int nk = min(32, blk - k0);
        __syncthreads();   // the previous step's operands are consumed
        if (tid < M) {
            const int m = tid;
#pragma unroll
            for (int t8 = 0; t8 < 4; ++t8) {
                bf16x8 hi, lo;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int t = 8 * t8 + e;
                    float av = 0.0f;
                    if (t < nk) {
                        const size_t o = ((size_t)bh * N + tb0 + k0 + t) * M + m;
                        av = AL[o];
                        ysum += C[o];
                    }
                    SPLIT2(bf16, av, hi[e], lo[e]);
                }
                *reinterpret_cast<bf16x8*>(ah + m * kDqTP + 8 * t8) = hi;
                *reinterpret_cast<bf16x8*>(alo + m * kDqTP + 8 * t8) = lo;
            }
        }
        for (int e = tid; e < DV * 8; e += 256) {
            const int d = e % DV, tq = e / DV;
            bf16x4 gv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * tq + i;
                gv[i] = t < nk ? dY[((size_t)b * N + tb0 + k0 + t) * stride + (size_t)h * DV + d] : (bf16)0.0f;
            }
            *reinterpret_cast<bf16x4*>(gt + d * kDqTP + 4 * tq) = gv;
        }
        __syncthreads();
        bf16x8 bg[NJ];
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj) bg[nj] = load8<bf16x8>(gt + (16 * nj + cl) * kDqTP + 8 * g4);
#pragma unroll
        for (int mi = 0; mi < MW; ++mi) {
            const int row = (mw0 + 16 * mi + cl) * kDqTP + 8 * g4;
            const bf16x8 a0 = load8<bf16x8>(ah + row), a1 = load8<bf16x8>(alo + row);
#pragma unroll
            for (int nj = 0; nj < NJ; ++nj) {
                acc[mi][nj] = mma_split<F16>(a0, a1, bg[nj], acc[mi][nj]);
            }
        }
    }
    if (tid < M) Yb[sbase + tid] = ysum;
#pragma unroll
    for (int mi = 0; mi < MW; ++mi)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
            for (int r = 0; r < 4; ++r) X[(sbase + mw0 + 16 * mi + 4 * g4 + r) * DV + 16 * nj + cl] = acc[mi][nj][r];
}

}  // namespace mfma

int launch_semi_dz_mfma(const void* dY, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, int64_t blk,
                        const float* AL, const float* C, float* X, float* Yb, bool f16in, hipStream_t st) {
    using namespace mfma;
    FLARE_REQUIRE(bwd_summary_mfma_supported(M, Dv) && blk % 16 == 0 && N % blk == 0,
                  "semi_dz_mfma: unsupported M=%lld Dv=%lld block=%lld", (long long)M, (long long)Dv, (long long)blk);
    dim3 grid((unsigned)(N / blk), (unsigned)(B * H));
#define FLARE_DZ_T(MW, DD, F)                                                                              \
    hipLaunchKernelGGL((semi_dz_mfma<MW, DD, F>), grid, dim3(256), 0, st, (const bf16*)dY, (int)N, (int)H, \
                       (int)blk, AL, C, X, Yb)
#define FLARE_DZ(MW, DD)                        \
    do {                                        \
        if (f16in) FLARE_DZ_T(MW, DD, true);    \
        else FLARE_DZ_T(MW, DD, false);         \
    } while (0)
#define FLARE_DZ_D(MW)              \
    if (Dv == 64) FLARE_DZ(MW, 64); \
    else FLARE_DZ(MW, 128);
    if (M == 64) { FLARE_DZ_D(1) }
    else if (M == 128) { FLARE_DZ_D(2) }
    else { FLARE_DZ_D(4) }
#undef FLARE_DZ_D
#undef FLARE_DZ
#undef FLARE_DZ_T
    return check_launch("semi_dz_mfma");
}

bool bwd_summary_mfma_supported(int64_t M, int64_t Dv) {
    return (M == 64 || M == 128 || M == 256) && (Dv == 64 || Dv == 128);
}

int launch_summary_mfma(const void* dY, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, const float* L,
                        const float* LA, const float* C, float* a_out, float* b_out, bool f16in, hipStream_t st) {
    using namespace mfma;
    FLARE_REQUIRE(bwd_summary_mfma_supported(M, Dv), "bwd_summary_mfma: unsupported M=%lld Dv=%lld",
                  (long long)M, (long long)Dv);
    dim3 grid((unsigned)((N + 31) / 32), (unsigned)(B * H));
#define FLARE_SUM_T(MW, DD, F)                                                                              \
    hipLaunchKernelGGL((bwd_summary_mfma<MW, DD, F>), grid, dim3(256), 0, st, (const bf16*)dY, (int)N, (int)H, \
                       L, LA, C, a_out, b_out)
#define FLARE_SUM(MW, DD)                        \
    do {                                         \
        if (f16in) FLARE_SUM_T(MW, DD, true);    \
        else FLARE_SUM_T(MW, DD, false);         \
    } while (0)
#define FLARE_SUM_D(MW)              \
    if (Dv == 64) FLARE_SUM(MW, 64); \
    else FLARE_SUM(MW, 128);
    if (M == 64) { FLARE_SUM_D(1) }
    else if (M == 128) { FLARE_SUM_D(2) }
    else { FLARE_SUM_D(4) }
#undef FLARE_SUM_D
#undef FLARE_SUM
#undef FLARE_SUM_T
    return check_launch("bwd_summary_mfma");
}

bool bwd_dq_mfma_supported(int64_t M, int64_t Dk) {
    return (M == 64 || M == 128 || M == 256) && (Dk == 64 || Dk == 128);
}

// partial sums per group of 512 tokens into P1 (and P2 when sep_k), as bwd_dq_kernel
int launch_dq_mfma(const void* K, const void* Qd, bool sep_q, bool sep_k, int64_t B, int64_t N, int64_t H,
                   int64_t M, int64_t Dk, const float* DS, const float* AL, const float* C, const float* gy,
                   bool cgz, bool dsum, float* P1, float* P2, bool f16in, hipStream_t st) {
    using namespace mfma;
    FLARE_REQUIRE(bwd_dq_mfma_supported(M, Dk), "bwd_dq_mfma: unsupported M=%lld Dk=%lld", (long long)M,
                  (long long)Dk);
    const int64_t NG = (N + kDqGroup - 1) / kDqGroup;
    // two accumulator sets (sep_k) keep 64 columns per workgroup
    const int dks = sep_k ? 64 : (int)Dk;
    dim3 grid((unsigned)NG, (unsigned)(B * H), (unsigned)(Dk / dks));
#define FLARE_DQ_T(MW, DKS, TA, TB, TO, F)                                                                     \
    hipLaunchKernelGGL((bwd_dq_mfma<MW, DKS, TA, TB, TO, F>), grid, dim3(256), 0, st, (const bf16*)K,         \
                       (const bf16*)Qd, (int)N, (int)H, (int)Dk, DS, AL, C, gy, cgz, dsum, P1, P2)
#define FLARE_DQ(MW, DKS, TA, TB, TO)                          \
    do {                                                       \
        if (f16in) FLARE_DQ_T(MW, DKS, TA, TB, TO, true);      \
        else FLARE_DQ_T(MW, DKS, TA, TB, TO, false);           \
    } while (0)
#define FLARE_DQ_MODES(MW, DKS)                                                          \
    if (sep_k) {                                                                        \
        if (sep_q) FLARE_DQ(MW, 64, true, true, true);                                  \
        else FLARE_DQ(MW, 64, true, false, true);                                       \
    } else {                                                                            \
        if (sep_q) FLARE_DQ(MW, DKS, true, true, false);                                \
        else FLARE_DQ(MW, DKS, false, false, false);                                    \
    }
#define FLARE_DQ_D(MW)                     \
    if (Dk == 64) { FLARE_DQ_MODES(MW, 64) } \
    else { FLARE_DQ_MODES(MW, 128) }
    if (M == 64) { FLARE_DQ_D(1) }
    else if (M == 128) { FLARE_DQ_D(2) }
    else { FLARE_DQ_D(4) }
#undef FLARE_DQ_D
#undef FLARE_DQ_MODES
#undef FLARE_DQ
#undef FLARE_DQ_T
    return check_launch("bwd_dq_mfma");
}

bool bwd_dk_mfma_supported(int64_t M, int64_t Dk) {
    return M % 32 == 0 && M <= mfma::kDkMaxM && (Dk == 64 || Dk == 128);
}

// sep_q: dQd is its own output; sep_k: Kd is not Q (Q / Kd as in bwd_dk_kernel)
int launch_dk_mfma(const void* Q, const void* Kd, bool sep_q, bool sep_k, int64_t B, int64_t N, int64_t H,
                   int64_t M, int64_t Dk, float scale, const float* DS, const float* AL, const float* C,
                   const float* gy, bool cgz, bool dsum, void* dK, void* dQd, bool f16in, hipStream_t st) {
    using namespace mfma;
    FLARE_REQUIRE(bwd_dk_mfma_supported(M, Dk), "bwd_dk_mfma: unsupported M=%lld Dk=%lld", (long long)M,
                  (long long)Dk);
    dim3 grid((unsigned)((N + kDkMfmaTok - 1) / kDkMfmaTok), (unsigned)(B * H));
#define FLARE_DK_T(DD, TB, TO, F)                                                                              \
    hipLaunchKernelGGL((bwd_dk_mfma<DD, TB, TO, F>), grid, dim3(256), 0, st, (const bf16*)Q, (const bf16*)Kd,  \
                       (int)N, (int)H, (int)M, scale, DS, AL, C, gy, cgz, dsum, (__hip_bfloat16*)dK, (__hip_bfloat16*)dQd)
#define FLARE_DK(DD, TB, TO)                          \
    do {                                              \
        if (f16in) FLARE_DK_T(DD, TB, TO, true);      \
        else FLARE_DK_T(DD, TB, TO, false);           \
    } while (0)
#define FLARE_DK_MODES(DD)                                          \
    if (sep_q) {                                                   \
        if (sep_k) FLARE_DK(DD, true, true);                       \
        else FLARE_DK(DD, false, true);                            \
    } else {                                                       \
        if (sep_k) FLARE_DK(DD, true, false);                      \
        else FLARE_DK(DD, false, false);                           \
    }
    if (Dk == 64) { FLARE_DK_MODES(64) }
    else { FLARE_DK_MODES(128) }
#undef FLARE_DK_MODES
#undef FLARE_DK
#undef FLARE_DK_T
    return check_launch("bwd_dk_mfma");
}

}  // namespace flare
