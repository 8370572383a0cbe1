// flare_bwd_mfma.hip -- bf16 MFMA contractions of the FLARE backward on gfx950.
//
// dK (and dQ_dec) are contractions over the latent bank of the score gradients
// ds and da = c - alpha gy (fp32, [B*H, N, M]) with the bf16 latent tensors:
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
template <int DK, bool TWO_B, bool TWO_OUT>
__global__ __launch_bounds__(256) void bwd_dk_mfma(const bf16* __restrict__ Q, const bf16* __restrict__ Kd, int N,
                                                   int H, int M, float scale, const float* __restrict__ DS,
                                                   const float* __restrict__ AL, const float* __restrict__ C,
                                                   const float* __restrict__ gy, __hip_bfloat16* __restrict__ dK,
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
                const f32x4 c0 = *reinterpret_cast<const f32x4*>(C + o), c1 = *reinterpret_cast<const f32x4*>(C + o + 4);
                const f32x4 a0 = *reinterpret_cast<const f32x4*>(AL + o), a1 = *reinterpret_cast<const f32x4*>(AL + o + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ds[e] = s0[e];
                    ds[4 + e] = s1[e];
                    da[e] = c0[e] - a0[e] * gyt[ti];
                    da[4 + e] = c1[e] - a1[e] * gyt[ti];
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
                acc[ti][nj] = mma(sh, bq[nj], acc[ti][nj]);
                acc[ti][nj] = mma(sl, bq[nj], acc[ti][nj]);
            }
            if constexpr (TWO_B || TWO_OUT) {
                bf16x8 ah, alo;
                split8(da, ah, alo);
#pragma unroll
                for (int nj = 0; nj < NJ; ++nj) {
                    const bf16x8 bb = TWO_B ? bk[nj] : bq[nj];
                    if constexpr (TWO_OUT) {
                        acc2[ti][nj] = mma(ah, bb, acc2[ti][nj]);
                        acc2[ti][nj] = mma(alo, bb, acc2[ti][nj]);
                    } else {
                        acc[ti][nj] = mma(ah, bb, acc[ti][nj]);
                        acc[ti][nj] = mma(alo, bb, acc[ti][nj]);
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
                dK[o + 16 * nj] = __float2bfloat16(scale * acc[ti][nj][r]);
                if constexpr (TWO_OUT) dQd[o + 16 * nj] = __float2bfloat16(scale * acc2[ti][nj][r]);
            }
        }
}

}  // namespace mfma

bool bwd_dk_mfma_supported(int64_t M, int64_t Dk) {
    return M % 32 == 0 && M <= mfma::kDkMaxM && (Dk == 64 || Dk == 128);
}

// sep_q: dQd is its own output; sep_k: Kd is not Q (Q / Kd as in bwd_dk_kernel)
int launch_dk_mfma(const void* Q, const void* Kd, bool sep_q, bool sep_k, int64_t B, int64_t N, int64_t H,
                   int64_t M, int64_t Dk, float scale, const float* DS, const float* AL, const float* C,
                   const float* gy, void* dK, void* dQd, hipStream_t st) {
    using namespace mfma;
    FLARE_REQUIRE(bwd_dk_mfma_supported(M, Dk), "bwd_dk_mfma: unsupported M=%lld Dk=%lld", (long long)M,
                  (long long)Dk);
    dim3 grid((unsigned)((N + kDkMfmaTok - 1) / kDkMfmaTok), (unsigned)(B * H));
#define FLARE_DK(DD, TB, TO)                                                                                   \
    hipLaunchKernelGGL((bwd_dk_mfma<DD, TB, TO>), grid, dim3(256), 0, st, (const bf16*)Q, (const bf16*)Kd,     \
                       (int)N, (int)H, (int)M, scale, DS, AL, C, gy, (__hip_bfloat16*)dK, (__hip_bfloat16*)dQd)
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
    return check_launch("bwd_dk_mfma");
}

}  // namespace flare
