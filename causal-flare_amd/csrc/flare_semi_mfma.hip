// flare_semi_mfma.hip -- bf16-input MFMA readout of the block-causal
// (semi-autoregressive) causal FLARE forward on gfx950.
//
// Token t of block g reads the encoder state after the last token of block g
// (causal_flare/semi_autoregressive/reference.py:452-503):
//   z_g[m]  = U_g[m] / d_g[m]                 (inclusive over blocks <= g)
//   y_t     = sum_m alpha[t,m] z_g[m],        alpha = softmax_m(S[t,:])
// so, unlike the token-causal readout, there is no within-block correction
// term.  One workgroup replays one chunk (a whole number of blocks) of one
// (b,h), starting from the chunk's exclusive prefix (phases 1 and 2 of the
// chunked forward).  Per block of NSUB 32-token subtiles:
//   for each subtile: S^T = Q K^T, lazy reference max R, E = 2^(S - R),
//                     d += sum E, U += E^T V (fp16 x fp16),
//                     alpha cached in LDS (fp16), LSE_dec written
//   at block end:     LSE_enc = R + log2(d) (natural log units), then
//                     Y^T = z^T alpha^T for the block's tokens (fp16 x fp16;
//                     |z| <= max|v| and alpha <= 1, both fp16-safe)
// The score / maxima / den work is split over waves by latent; U and y by
// value column, as in chunk_output_mfma (flare_ar_mfma.hip).
#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {
namespace mfma {

template <int M, int D, int NW, int NSUB>
struct SemiLayout {
    static constexpr int NT = 64 * NW;
    static constexpr int MW = M / NW;        // latents per wave (scores)
    static constexpr int MT = MW / 16;       // latent tiles per wave
    static constexpr int MTA = M / 16;       // latent tiles of the bank
    static constexpr int MB = M / 32;        // 32-latent k-blocks of the readout
    static constexpr int DW = D / NW;        // value columns per wave
    static constexpr int DTW = DW / 16;      // value tiles per wave
    static constexpr int KS = D / 32;        // k-steps of the scores
    static constexpr int AP = M + 8;         // padded row of alpha[t][m]
    static constexpr int EP = T + 8;         // padded row of E^T[m][tau] and V^T[d][tau]
    static constexpr int QP = D + 8;         // padded row of Q in LDS
    static constexpr int BLOCK = NSUB * T;
    static_assert(MT % 2 == 0 && DW % 16 == 0, "unsupported wave split");
};

// SEP: separate decoder tensors; alpha [B*H, N, M] (fp16, from decoder_alpha_mfma,
// which also writes LSE_dec) replaces the softmax of the shared scores.
// GA: alpha of the block lives in global memory (the [B*H, N, M] buffer) instead of
// LDS, for blocks whose alpha does not fit next to the Q bank: written there from
// the shared scores (or, with SEP, read as the decoder pass left it) and staged into
// LDS one subtile at a time for the readout; the block is nsub = block / 32
// subtiles at run time and NSUB is unused.
template <int M, int D, int NW, int NSUB, bool SEP, bool GA, bool F16>
// (at least 3 workgroups per CU where the registers allow it: the 128 x 64 instances with
// the block's softmax in LDS for blocks up to 64 fit in 168 VGPRs; the compiler keeps the
// larger instances at their own count)
__global__ __launch_bounds__(64 * NW, 3) void semi_output_mfma(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N, int H,
    float scale2, int chunk, const float* __restrict__ pmax, const float* __restrict__ pden,
    const float* __restrict__ pnum, void* __restrict__ Y, int out_dtype, float* __restrict__ lse_dec,
    float* __restrict__ lse_enc, f16* __restrict__ alpha, int nsub_ga) {
    using L = SemiLayout<M, D, NW, NSUB>;
    __shared__ __attribute__((aligned(16))) f16 al[(GA ? 1 : NSUB) * T * L::AP];   // alpha[t][m] of the block
    __shared__ __attribute__((aligned(16))) f16 etl[M * L::EP];         // E^T[m][tau]
    __shared__ __attribute__((aligned(16))) f16 vtl[D * L::EP];         // V^T[d][tau] (bf16 if moved)
    __shared__ __attribute__((aligned(16))) float lsep[NW * T * 2];     // (max, sum) per wave/token
    __shared__ __attribute__((aligned(16))) float gaml[M];              // rescale factor per latent
    __shared__ __attribute__((aligned(16))) float invd[M];              // 1 / d at block end
    __shared__ int moved[NW];
    __shared__ __attribute__((aligned(16))) bf16 qs[M * L::QP];

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int nsub = GA ? nsub_ga : NSUB;
    const int blockT = nsub * T;
    const int NB = N / blockT;
    // alpha row of token blk + jt in global memory (GA)
    auto grow = [&](int blk, int jt) -> f16* { return alpha + ((size_t)bh * N + blk + jt) * M; };
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int mw0 = w * L::MW;
    const int dw0 = w * L::DW;

    for (int vi = tid; vi < M * D / 8; vi += L::NT) {
        const int m = vi / (D / 8), d8 = vi % (D / 8);
        *reinterpret_cast<bf16x8*>(qs + m * L::QP + 8 * d8) = load8<bf16x8>(Q + ((size_t)h * M + m) * D + 8 * d8);
    }
    const size_t pbase = ((size_t)bh * NC + c_idx) * M;
    // R is the same on the 16 lanes of a latent's row; dn[mi][r] is this lane's partial den
    // (its tokens' E, the prefix's den on lane c = 0), summed over the row at block ends
    float R[L::MT][4], dn[L::MT][4];
#pragma unroll
    for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mw0 + 16 * mi + 4 * g + r;
            R[mi][r] = pmax[pbase + m] * kLog2e;
            dn[mi][r] = c == 0 ? pden[pbase + m] : 0.0f;   // this lane's share of the den
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
    const int t_end = min(N, t_begin + chunk);      // chunk and N are whole blocks
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    VTile<L::DW, 64, F16> vt;
    vt.load(V, row0, stride, t_begin, t_end, dw0, lane);
    bf16x8 kb[2][L::KS];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int ks = 0; ks < L::KS; ++ks)
            kb[ti][ks] = load8<bf16x8>(K + row0 + (size_t)(t_begin + 16 * ti + c) * stride + 32 * ks + 8 * g);

    for (int blk0 = t_begin; blk0 < t_end; blk0 += blockT) {
        for (int j = 0; j < nsub; ++j) {
            const int t0 = blk0 + j * T;
            // (fp16 inputs are always in the fp16 range: no bf16 fallback)
            const bool vbig = __any(vt.template store_f16<L::EP>(vtl, dw0, lane)) && !F16;
            vt.load(V, row0, stride, t0 + T, t_end, dw0, lane);
            // ---- S^T = Q K^T (log2 domain); prefetch the next subtile's K rows
            float s[L::MT][2][4];
            {
                f32x4 acc[L::MT][2];
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < L::KS; ++ks)
#pragma unroll
                    for (int mi = 0; mi < L::MT; ++mi) {
                        const bf16x8 qa = load8<bf16x8>(qs + (mw0 + 16 * mi + c) * L::QP + 32 * ks + 8 * g);
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) acc[mi][ti] = mma_in<F16>(qa, kb[ti][ks], acc[mi][ti]);
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
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[mi][ti][r] = acc[mi][ti][r] * scale2;
            }
            // ---- lazy reference max (checked per lane; moved rarely), E (fp16 -> LDS), den
            bool need = false;
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) need |= fmaxf(s[mi][0][r], s[mi][1][r]) > R[mi][r] + kLazy;
            const bool wave_moved = __any(need);
            if (wave_moved) {
                asm volatile("");   // a branch: reference moves are rare
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float mx = row_max16(fmaxf(s[mi][0][r], s[mi][1][r]));
                        const bool mv = mx > R[mi][r] + kLazy;
                        const float Rn = mv ? mx : R[mi][r];
                        const float gam = mv ? exp2f_fast(R[mi][r] - Rn) : 1.0f;   // 0 when R = -inf
                        R[mi][r] = Rn;
                        dn[mi][r] *= gam;
                        if (c == 0) gaml[mw0 + 16 * mi + 4 * g + r] = gam;
                    }
            }
#pragma unroll
            for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e0 = exp2f_fast(s[mi][0][r] - R[mi][r]);
                    const float e1 = exp2f_fast(s[mi][1][r] - R[mi][r]);
                    dn[mi][r] += e0 + e1;
                    f16* er = etl + (mw0 + 16 * mi + 4 * g + r) * L::EP;
                    er[c] = (f16)e0;
                    er[16 + c] = (f16)e1;
                }
            if (lane == 0) moved[w] = wave_moved ? 1 : 0;
            // ---- decoder log-sum-exp partials per token; the exponentials against the wave's
            //      maximum lm are kept for alpha = 2^(s - lm) 2^(lm - lse)
            float ex[L::MT][2][4], lmv[2];
#pragma unroll
            for (int ti = 0; ti < (SEP ? 0 : 2); ++ti) {
                float lm = kNegInf;
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) lm = fmaxf(lm, s[mi][ti][r]);
                lm = rows_max4(lm);
                float ls = 0.0f;
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        ex[mi][ti][r] = exp2f_fast(s[mi][ti][r] - lm);
                        ls += ex[mi][ti][r];
                    }
                ls = rows_sum4(ls);
                lmv[ti] = lm;
                if (g == 0) {
                    lsep[(w * T + 16 * ti + c) * 2 + 0] = lm;
                    lsep[(w * T + 16 * ti + c) * 2 + 1] = ls;
                }
            }
            __syncthreads();   // S1: lse partials, E^T, rescale factors, moved flags visible
            // ---- alpha = softmax over the bank (fp16 -> LDS), LSE_dec; separate decoder
            //      tensors: alpha copied from the decoder pass
            if constexpr (SEP && !GA) {
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const int t = 16 * ti + c;
                    const f16* arow = alpha + ((size_t)bh * N + t0 + t) * M + mw0 + 4 * g;
#pragma unroll
                    for (int mi = 0; mi < L::MT; ++mi)
                        *reinterpret_cast<f16x4*>(al + (j * T + t) * L::AP + mw0 + 16 * mi + 4 * g) =
                            load4<f16x4>(arow + 16 * mi);
                }
            }
#pragma unroll
            for (int ti = 0; ti < (SEP ? 0 : 2); ++ti) {
                const int t = 16 * ti + c;
                float mm = kNegInf;
#pragma unroll
                for (int w2 = 0; w2 < NW; ++w2) mm = fmaxf(mm, lsep[(w2 * T + t) * 2]);
                float ss = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < NW; ++w2) ss += lsep[(w2 * T + t) * 2 + 1] * exp2f_fast(lsep[(w2 * T + t) * 2] - mm);
                const float lse2 = mm + __log2f(ss);
                if (lse_dec && w == 0 && g == 0) lse_dec[(size_t)bh * N + t0 + t] = lse2 * kLn2;
                const float sc = exp2f_fast(lmv[ti] - lse2);   // <= 1
#pragma unroll
                for (int mi = 0; mi < L::MT; ++mi) {
                    f16x4 a4;
#pragma unroll
                    for (int r = 0; r < 4; ++r) a4[r] = (f16)(ex[mi][ti][r] * sc);
                    f16* dst = GA ? grow(blk0, j * T + t) : al + (j * T + t) * L::AP;
                    *reinterpret_cast<f16x4*>(dst + mw0 + 16 * mi + 4 * g) = a4;
                }
            }
            // ---- numerator: move to new reference maxima (rare), then U += E^T V
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi) {
                if (moved[(16 * mi) / L::MW]) {   // the rows of a wave that moved its references
                    const f32x4 gm = *reinterpret_cast<const f32x4*>(gaml + 16 * mi + 4 * g);
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                        for (int r = 0; r < 4; ++r) U[mi][di][r] *= gm[r];
                }
            }
            if (!vbig) {
                f16x8 va[L::DTW];
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) va[di] = load8<f16x8>(vtl + (dw0 + 16 * di + c) * L::EP + 8 * g);
#pragma unroll
                for (int mi = 0; mi < L::MTA; ++mi) {
                    const f16x8 ea = load8<f16x8>(etl + (16 * mi + c) * L::EP + 8 * g);
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di) U[mi][di] = mma(ea, va[di], U[mi][di]);
                }
            } else {   // a value outside the fp16 range: bf16 V, exact hi/lo split of E
                bf16* vtb = reinterpret_cast<bf16*>(vtl);
                stage_vt_bf16<L::EP>(vtb, V, row0, stride, t0, t_end, dw0, L::DW, lane, 64);
                bf16x8 va[L::DTW];
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) va[di] = load8<bf16x8>(vtb + (dw0 + 16 * di + c) * L::EP + 8 * g);
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
            __syncthreads();   // S2: E^T, V^T and the lse table are rewritten next subtile
        }
        // ---- block end: LSE_enc and 1/d for the readout
        const int gblk = blk0 / blockT;
#pragma unroll
        for (int mi = 0; mi < L::MT; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = mw0 + 16 * mi + 4 * g + r;
                const float den = row_sum16(dn[mi][r]);
                if (c == 0) {
                    invd[m] = __builtin_amdgcn_rcpf(den);
                    if (lse_enc) lse_enc[((size_t)bh * NB + gblk) * M + m] = (R[mi][r] + __log2f(den)) * kLn2;
                }
            }
        __syncthreads();   // S3: 1/d visible
        // ---- Y^T = z^T alpha^T, z = U / d (fp16 x fp16)
        f16x8 za[L::MB][L::DTW];
#pragma unroll
        for (int kk = 0; kk < L::MB; ++kk) {
            const f32x4 ilo = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 4 * g);
            const f32x4 ihi = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 16 + 4 * g);
#pragma unroll
            for (int di = 0; di < L::DTW; ++di)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    za[kk][di][r] = (f16)(U[2 * kk][di][r] * ilo[r]);
                    za[kk][di][4 + r] = (f16)(U[2 * kk + 1][di][r] * ihi[r]);
                }
        }
        bool bad = false;
        for (int j = 0; j < nsub; ++j) {
            if constexpr (GA) {   // subtile j's alpha rows -> LDS (every wave reads all of them)
                __syncthreads();
                for (int vi = tid; vi < T * M / 8; vi += L::NT) {
                    const int t = vi / (M / 8), m8 = vi % (M / 8);
                    *reinterpret_cast<f16x8*>(al + t * L::AP + 8 * m8) = load8<f16x8>(grow(blk0, j * T + t) + 8 * m8);
                }
                __syncthreads();
            }
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) {
                f32x4 yacc[L::DTW];
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) yacc[di] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < L::MB; ++kk) {
                    const f16* ar = al + ((GA ? 0 : j * T) + 16 * ti + c) * L::AP + 32 * kk;
                    const f16x8 ab = cat8<f16x8>(load4<f16x4>(ar + 4 * g), load4<f16x4>(ar + 16 + 4 * g));
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di) yacc[di] = mma(za[kk][di], ab, yacc[di]);
                }
                const int t = blk0 + j * T + 16 * ti + c;
#pragma unroll
                for (int di = 0; di < L::DTW; ++di) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(yacc[di][r]);
                    store4(Y, row0 + (size_t)t * stride + dw0 + 16 * di + 4 * g, yacc[di], out_dtype);
                }
            }
        }
        if (__any(bad)) {
            // |z| <= max|v| overflowed fp16 (|v| > 65504 somewhere): redo the block's readout in bf16
            for (int j = 0; j < nsub; ++j)
                for (int ti = 0; ti < 2; ++ti) {
                    f32x4 yacc[L::DTW];
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di) yacc[di] = f32x4{0.f, 0.f, 0.f, 0.f};
                    for (int kk = 0; kk < L::MB; ++kk) {
                        // (wave-divergent branch: no staging barrier; GA reads global rows)
                        const f16* ar = (GA ? grow(blk0, j * T + 16 * ti + c) : al + (j * T + 16 * ti + c) * L::AP) + 32 * kk;
                        bf16x8 ab;
#pragma unroll
                        for (int e2 = 0; e2 < 4; ++e2) {
                            ab[e2] = (bf16)(float)ar[4 * g + e2];
                            ab[4 + e2] = (bf16)(float)ar[16 + 4 * g + e2];
                        }
                        const f32x4 ilo = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 4 * g);
                        const f32x4 ihi = *reinterpret_cast<const f32x4*>(invd + 32 * kk + 16 + 4 * g);
#pragma unroll
                        for (int di = 0; di < L::DTW; ++di) {
                            bf16x8 zb;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                zb[r] = (bf16)(U[2 * kk][di][r] * ilo[r]);
                                zb[4 + r] = (bf16)(U[2 * kk + 1][di][r] * ihi[r]);
                            }
                            yacc[di] = mma(zb, ab, yacc[di]);
                        }
                    }
                    const int t = blk0 + j * T + 16 * ti + c;
#pragma unroll
                    for (int di = 0; di < L::DTW; ++di)
                        store4(Y, row0 + (size_t)t * stride + dw0 + 16 * di + 4 * g, yacc[di], out_dtype);
                }
        }
        __syncthreads();   // S4: alpha and 1/d are rewritten by the next block
    }
}

}  // namespace mfma

using namespace mfma;

// shared: true also for separate decoder tensors served through decoder_alpha_mfma
bool mfma_semi_supported(int dtype, int out_dtype, bool shared, int64_t M, int64_t Dk, int64_t Dv,
                         int64_t block) {
    const bool shape = shared && Dk == Dv && (Dk == 64 || Dk == 128) && (M == 128 || M == 256);
    const bool bf = dtype == FLARE_BF16 && (out_dtype == FLARE_BF16 || out_dtype == FLARE_F32);
    const bool hf = dtype == FLARE_F16 && (out_dtype == FLARE_F16 || out_dtype == FLARE_F32);
    if (!(shape && (bf || hf))) return false;
    return block % 32 == 0;
}

bool semi_alpha_in_lds(int64_t M, int64_t block) {
    return block == 32 || block == 64 || (block == 128 && M == 128);
}

int launch_semi_output_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                            int64_t M, int64_t D, float scale, int64_t chunk, int64_t block,
                            const float* pmax, const float* pden, const float* pnum, void* Y, int out_dtype,
                            float* lse_dec, float* lse_enc, void* alpha, bool sep, bool f16in, hipStream_t stream) {
    FLARE_REQUIRE(chunk % block == 0 && N % block == 0, "semi_output_mfma: chunk and N must be whole blocks");
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
    const bool ga = !semi_alpha_in_lds(M, block);
    FLARE_REQUIRE(block % T == 0 && (!ga || alpha) && (!sep || alpha),
                  "semi_output_mfma: block=%lld needs whole subtiles and an alpha buffer", (long long)block);
#define FLARE_SEMI_MFMA_SEP(MM, DD, NWW, NS, SP, G)                                                        \
    do {                                                                                                   \
        if (f16in) FLARE_SEMI_MFMA_T(MM, DD, NWW, NS, SP, G, true);                                        \
        else FLARE_SEMI_MFMA_T(MM, DD, NWW, NS, SP, G, false);                                             \
    } while (0)
#define FLARE_SEMI_MFMA_T(MM, DD, NWW, NS, SP, G, F)                                                       \
    hipLaunchKernelGGL((semi_output_mfma<MM, DD, NWW, NS, SP, G, F>), grid, dim3(64 * NWW), 0, stream,    \
                       (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk,     \
                       pmax, pden, pnum, Y, out_dtype, lse_dec, lse_enc, (f16*)alpha, (int)(block / T))
#define FLARE_SEMI_MFMA(MM, DD, NWW, NS)                                \
    do {                                                               \
        if (sep) FLARE_SEMI_MFMA_SEP(MM, DD, NWW, NS, true, false);    \
        else FLARE_SEMI_MFMA_SEP(MM, DD, NWW, NS, false, false);       \
    } while (0)
#define FLARE_SEMI_GA(MM, DD, NWW)                                      \
    do {                                                               \
        if (sep) FLARE_SEMI_MFMA_SEP(MM, DD, NWW, 1, true, true);      \
        else FLARE_SEMI_MFMA_SEP(MM, DD, NWW, 1, false, true);         \
    } while (0)
#define FLARE_SEMI_BLOCKS(MM, DD, NWW)                       \
    if (ga) FLARE_SEMI_GA(MM, DD, NWW);                      \
    else if (block == 32) FLARE_SEMI_MFMA(MM, DD, NWW, 1);   \
    else FLARE_SEMI_MFMA(MM, DD, NWW, 2);
    if (ga) {
        if (M == 128 && D == 64) FLARE_SEMI_GA(128, 64, 4);
        else if (M == 128 && D == 128) FLARE_SEMI_GA(128, 128, 4);
        else if (M == 256 && D == 64) FLARE_SEMI_GA(256, 64, 4);
        else FLARE_SEMI_GA(256, 128, 8);
    } else if (M == 128 && D == 64) {
        if (block == 128) FLARE_SEMI_MFMA(128, 64, 4, 4);
        else { FLARE_SEMI_BLOCKS(128, 64, 4) }
    } else if (M == 128 && D == 128) {
        if (block == 128) FLARE_SEMI_MFMA(128, 128, 4, 4);
        else { FLARE_SEMI_BLOCKS(128, 128, 4) }
    } else if (M == 256 && D == 64) {
        FLARE_SEMI_BLOCKS(256, 64, 4)
    } else {
        FLARE_SEMI_BLOCKS(256, 128, 8)
    }
#undef FLARE_SEMI_BLOCKS
#undef FLARE_SEMI_GA
#undef FLARE_SEMI_MFMA
#undef FLARE_SEMI_MFMA_SEP
#undef FLARE_SEMI_MFMA_T
    return check_launch("semi_output_mfma");
}

}  // namespace flare
