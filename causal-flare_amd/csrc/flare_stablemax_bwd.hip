// flare_stablemax_bwd.hip -- backward of the stablemax causal FLARE forward on gfx950
// (reference FLAREAutoregressiveStablemaxTriton.backward, autoregressive/
// stablemax_triton.py:1981-2420; PyTorch form stablemax.py:482-635).
//
// Per (b,h), latent m and token t, with E = s(a) the stablemax transform of the
// encoder score a = scale k_t . q_m, D_t = sum_{tau<=t} E_tau, z_t = sum E_tau v_tau / D_t,
// alpha_t = softmax_m(scale qd_t . kd_m) and g_t = dY_t:
//
//   gz_tm = g_t . z_tm,  w_tm = alpha_tm / D_tm,
//   X_tau,m = sum_{t >= tau} w_tm g_t,   Y_tau,m = sum_{t >= tau} w_tm gz_tm,
//   dE_tau,m = v_tau . X_tau,m - Y_tau,m,   da_tau,m = dE_tau,m s'(a_tau,m),
//   dv_tau = sum_m E_tau,m X_tau,m,   dA_tm (decoder) = alpha_tm (gz_tm - g_t . y_t).
//
// The sums over t >= tau are cut at chunks of CT tokens: phase 1 (stablemax_bwd_forward)
// replays each chunk from its exclusive prefix (den, num) -- the forward's own prepare and
// prefix kernels in stablemax mode, at chunk CT -- and writes alpha, w, gz per token plus
// the chunk totals of w g and w gz; phase 2 turns those into exclusive suffix sums over
// chunks; phase 3 (stablemax_bwd_tokens) finishes X and Y inside each chunk and writes
// da (as the score gradient DS) and dv.  The contractions with Q, K, Q_dec and K_dec are
// the token-causal backward's (launch_bwd_contract, with AL = alpha and C = alpha gz).
// Everything is fp32 on VALU lanes; thread m of a 256-thread workgroup owns latent m.
//
// Shapes with M, Dk and Dv multiples of 16 (ar_backward_supported) take the softmax
// backward instead (flare_ar_bwd.hip, with its MFMA contractions): its formulas hold
// with e^a replaced by s(a) -- the scores become log2 s(a), and the score gradient
// picks up d log s / da = p / (1 + |a|).  The kernels here serve the other shapes.
#include "flare_common.h"
#include "flare_internal.h"

namespace flare {

constexpr int kSBT = 256;     // threads; M <= kSBT
constexpr int kSBC = 16;      // largest chunk (tokens per workgroup)

// s'(x) = p s(x) / (1 + |x|): p (1 + x)^(p - 1) for x >= 0, p (1 - x)^(-p - 1) below
__device__ __forceinline__ float stablemax_grad_from(float x, float sx, float p) {
    return p * sx / (x >= 0.0f ? 1.0f + x : 1.0f - x);
}

struct SbSmem {
    int CT, Dk, Dv, M;
    bool sep;
    // phase 1: k, qd (separate decoder), v, g rows; GV[t][tau]; per-token reductions
    __host__ __device__ size_t floats1() const {
        return (size_t)CT * Dk * (sep ? 2 : 1) + (size_t)2 * CT * Dv + (size_t)CT * CT + 8 * kSBC;
    }
    // phase 3: k, v, g rows; GV; E and w rows over the latents; Gw[tau][t]
    __host__ __device__ size_t floats3() const {
        return (size_t)CT * Dk + (size_t)2 * CT * Dv + (size_t)2 * CT * CT + (size_t)2 * CT * M;
    }
};

// Rows [t0, t0 + nt) of a [B, N, H, D] tensor for head h into LDS (fp32), zero past nt.
template <typename T>
__device__ __forceinline__ void load_rows(const T* X, int b, int N, int H, int h, int D, int t0, int nt, int CT,
                                          float* dst) {
    for (int e = threadIdx.x; e < CT * D; e += kSBT) {
        const int i = e / D, d = e % D;
        dst[e] = i < nt ? to_f32(X[(((size_t)b * N + t0 + i) * H + h) * D + d]) : 0.0f;
    }
}

// Encoder (and decoder) scores of latent m for the chunk's tokens.
template <typename T>
__device__ __forceinline__ void latent_scores(const T* qrow, const T* kdrow, const float* ks, const float* qds,
                                              int Dk, int CT, float scale, bool sep, float* a, float* A) {
#pragma unroll
    for (int i = 0; i < kSBC; ++i) a[i] = A[i] = 0.0f;
    for (int d = 0; d < Dk; ++d) {
        const float qv = to_f32(qrow[d]);
        const float kv = sep ? to_f32(kdrow[d]) : 0.0f;
#pragma unroll
        for (int i = 0; i < kSBC; ++i) {
            if (i < CT) {
                a[i] += ks[i * Dk + d] * qv;
                if (sep) A[i] += qds[i * Dk + d] * kv;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        a[i] *= scale;
        A[i] = sep ? A[i] * scale : a[i];
    }
}

// ---------------------------------------------------------------------------
// Phase 1.  grid = (NC, B*H).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kSBT) void stablemax_bwd_forward(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, const T* __restrict__ Qd,
    const T* __restrict__ Kd, const T* __restrict__ dY, int N, int H, int M, int Dk, int Dv, float scale,
    float power, int CT, const float* __restrict__ pmax, const float* __restrict__ pden,
    const float* __restrict__ pnum, float* __restrict__ AL,
    float* __restrict__ Cc, float* __restrict__ Wt, float* __restrict__ GZ, float* __restrict__ Sx,
    float* __restrict__ Sy) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const bool sep = Qd != nullptr;               // decoder query rows of their own (else K's)
    const bool dec = sep || Kd != nullptr;         // decoder scores of their own
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, m = threadIdx.x;
    const int t0 = c * CT, nt = min(CT, N - t0);
    float* ks = sm;
    float* qds = ks + CT * Dk;
    float* vs = qds + (sep ? CT * Dk : 0);
    float* gs = vs + CT * Dv;
    float* GV = gs + CT * Dv;
    float* red = GV + CT * CT;     // [4 waves][kSBC]... reused per reduction
    load_rows(K, b, N, H, h, Dk, t0, nt, CT, ks);
    if (sep) load_rows(Qd, b, N, H, h, Dk, t0, nt, CT, qds);
    load_rows(V, b, N, H, h, Dv, t0, nt, CT, vs);
    load_rows(dY, b, N, H, h, Dv, t0, nt, CT, gs);
    __syncthreads();
    // g_t . v_tau for the chunk's token pairs
    for (int e = threadIdx.x; e < CT * CT; e += kSBT) {
        const int t = e / CT, tau = e % CT;
        float acc = 0.0f;
        for (int d = 0; d < Dv; ++d) acc += gs[t * Dv + d] * vs[tau * Dv + d];
        GV[e] = acc;
    }
    const bool on = m < M;
    float a[kSBC], A[kSBC];
    if (on) {
        latent_scores(Q + ((size_t)h * M + m) * Dk, (Kd ? Kd : Q) + ((size_t)h * M + m) * Dk, ks, sep ? qds : ks, Dk,
                      CT, scale, dec, a, A);
    } else {
#pragma unroll
        for (int i = 0; i < kSBC; ++i) a[i] = A[i] = kNegInf;
    }
    // decoder softmax over the latents, per token: wave partials then the 4 waves
    const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
    float alpha[kSBC];
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        if (i < CT) {
            const float mx = wave_max(A[i]);
            if (ln == 0) red[wv * kSBC + i] = mx;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        if (i < CT) {
            const float mx = fmaxf(fmaxf(red[i], red[kSBC + i]), fmaxf(red[2 * kSBC + i], red[3 * kSBC + i]));
            alpha[i] = on ? __expf(A[i] - mx) : 0.0f;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        if (i < CT) {
            const float sum = wave_sum(alpha[i]);
            if (ln == 0) red[wv * kSBC + i] = sum;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        if (i < CT) alpha[i] /= red[i] + red[kSBC + i] + red[2 * kSBC + i] + red[3 * kSBC + i];
    }
    if (!on) return;     // (no barrier below)
    const size_t pb = ((size_t)bh * NC + c) * M + m;
    // E, the cumulative den from the chunk's prefix, and g_t . U0_m from its numerator row
    // (summaries written by the MFMA prepare carry a reference max: absolute sums here)
    const float ps = __expf(pmax[pb]);
    float E[kSBC], Dt[kSBC], gu[kSBC];
    float dcur = pden[pb] * ps;
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        E[i] = i < nt ? stablemax_transform(a[i], power) : 0.0f;
        dcur += E[i];
        Dt[i] = dcur;
        gu[i] = 0.0f;
    }
    const float* u0 = pnum + pb * Dv;
    for (int d = 0; d < Dv; ++d) {
        const float u = u0[d] * ps;
#pragma unroll
        for (int i = 0; i < kSBC; ++i)
            if (i < CT) gu[i] += u * gs[i * Dv + d];
    }
    float w[kSBC], gz[kSBC];
    float sy = 0.0f;
#pragma unroll
    for (int i = 0; i < kSBC; ++i) {
        float acc = gu[i];
#pragma unroll
        for (int tau = 0; tau <= i; ++tau) acc += E[tau] * GV[i * CT + tau];
        const bool ok = i < nt;
        gz[i] = ok ? acc / Dt[i] : 0.0f;
        w[i] = ok ? alpha[i] / Dt[i] : 0.0f;
        sy += w[i] * gz[i];
        if (ok) {
            const size_t o = ((size_t)bh * N + t0 + i) * M + m;
            AL[o] = alpha[i];
            Cc[o] = alpha[i] * gz[i];
            Wt[o] = w[i];
            GZ[o] = gz[i];
        }
    }
    Sy[pb] = sy;
    float* sx = Sx + pb * Dv;
    for (int d = 0; d < Dv; ++d) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kSBC; ++i)
            if (i < CT) acc += w[i] * gs[i * Dv + d];
        sx[d] = acc;
    }
}

// ---------------------------------------------------------------------------
// Phase 2.  Exclusive suffix sums over chunks, in place: one thread per (b*h, m, column)
// of Sx and one per (b*h, m) of Sy.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stablemax_bwd_suffix(float* __restrict__ Sx, float* __restrict__ Sy, int BH,
                                                            int NC, int M, int Dv) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nx = (int64_t)BH * M * Dv;
    if (gid < nx) {
        const int64_t bh = gid / ((int64_t)M * Dv), r = gid % ((int64_t)M * Dv);
        float acc = 0.0f;
        for (int c = NC - 1; c >= 0; --c) {
            float& x = Sx[((size_t)bh * NC + c) * M * Dv + r];
            const float v = x;
            x = acc;
            acc += v;
        }
    } else if (gid < nx + (int64_t)BH * M) {
        const int64_t g2 = gid - nx, bh = g2 / M, m = g2 % M;
        float acc = 0.0f;
        for (int c = NC - 1; c >= 0; --c) {
            float& y = Sy[((size_t)bh * NC + c) * M + m];
            const float v = y;
            y = acc;
            acc += v;
        }
    }
}

// ---------------------------------------------------------------------------
// Phase 3.  grid = (NC, B*H).  dS (the encoder score gradient) and dV.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kSBT) void stablemax_bwd_tokens(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, const T* __restrict__ dY, int N,
    int H, int M, int Dk, int Dv, float scale, float power, int CT, const float* __restrict__ Wt,
    const float* __restrict__ GZ, const float* __restrict__ Sx, const float* __restrict__ Sy,
    float* __restrict__ DS, T* __restrict__ dV) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int c = blockIdx.x, bh = blockIdx.y, NC = gridDim.x;
    const int b = bh / H, h = bh % H, m = threadIdx.x;
    const int t0 = c * CT, nt = min(CT, N - t0);
    float* ks = sm;
    float* vs = ks + CT * Dk;
    float* gs = vs + CT * Dv;
    float* GV = gs + CT * Dv;
    float* Gw = GV + CT * CT;
    float* Es = Gw + CT * CT;     // [CT][M]
    float* Ws = Es + CT * M;      // [CT][M]
    load_rows(K, b, N, H, h, Dk, t0, nt, CT, ks);
    load_rows(V, b, N, H, h, Dv, t0, nt, CT, vs);
    load_rows(dY, b, N, H, h, Dv, t0, nt, CT, gs);
    __syncthreads();
    for (int e = threadIdx.x; e < CT * CT; e += kSBT) {
        const int t = e / CT, tau = e % CT;
        float acc = 0.0f;
        for (int d = 0; d < Dv; ++d) acc += gs[t * Dv + d] * vs[tau * Dv + d];
        GV[e] = acc;
    }
    const bool on = m < M;
    const size_t pb = ((size_t)bh * NC + c) * M + m;
    float E[kSBC], sp[kSBC], w[kSBC], gz[kSBC], xv[kSBC];
    {
        float a[kSBC], A[kSBC];
        latent_scores(Q + ((size_t)h * (on ? M : 1) + (on ? m : 0)) * Dk, Q, ks, ks, Dk, CT, scale, false, a, A);
#pragma unroll
        for (int i = 0; i < kSBC; ++i) {
            const bool ok = on && i < nt;
            E[i] = ok ? stablemax_transform(a[i], power) : 0.0f;
            sp[i] = ok ? stablemax_grad_from(a[i], E[i], power) : 0.0f;
            const size_t o = ((size_t)bh * N + t0 + (ok ? i : 0)) * M + (on ? m : 0);
            w[i] = ok ? Wt[o] : 0.0f;
            gz[i] = ok ? GZ[o] : 0.0f;
            xv[i] = 0.0f;
            if (on && i < CT) {
                Es[i * M + m] = E[i];
                Ws[i * M + m] = w[i];
            }
        }
    }
    if (on) {
        // v_tau . Xc_m (the later chunks' part of X)
        const float* xc = Sx + pb * Dv;
        for (int d = 0; d < Dv; ++d) {
            const float x = xc[d];
#pragma unroll
            for (int i = 0; i < kSBC; ++i)
                if (i < CT) xv[i] += x * vs[i * Dv + d];
        }
    }
    __syncthreads();   // GV, Es and Ws complete
    if (on) {
        float ysum = Sy[pb];
        float ds_[kSBC];
#pragma unroll
        for (int i = kSBC - 1; i >= 0; --i) {
            ds_[i] = 0.0f;
            if (i < CT) {
                ysum += w[i] * gz[i];
                float x = xv[i];
#pragma unroll
                for (int t = i; t < kSBC; ++t)
                    if (t < CT) x += w[t] * GV[t * CT + i];
                ds_[i] = (x - ysum) * sp[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kSBC; ++i)
            if (i < nt) DS[((size_t)bh * N + t0 + i) * M + m] = ds_[i];
    }
    // Gw[tau][t] = sum_m E_tau,m w_tm for t >= tau
    for (int e = threadIdx.x; e < CT * CT; e += kSBT) {
        const int tau = e / CT, t = e % CT;
        float acc = 0.0f;
        if (t >= tau)
            for (int mm = 0; mm < M; ++mm) acc += Es[tau * M + mm] * Ws[t * M + mm];
        Gw[e] = acc;
    }
    __syncthreads();
    // dv_tau[d] = sum_m E_tau,m Xc_m[d] + sum_{t >= tau} Gw[tau][t] g_t[d]
    for (int d = threadIdx.x; d < Dv; d += kSBT) {
        float acc[kSBC];
#pragma unroll
        for (int i = 0; i < kSBC; ++i) acc[i] = 0.0f;
        const float* xcol = Sx + ((size_t)bh * NC + c) * M * Dv + d;
        for (int mm = 0; mm < M; ++mm) {
            const float x = xcol[(size_t)mm * Dv];
#pragma unroll
            for (int i = 0; i < kSBC; ++i)
                if (i < CT) acc[i] += Es[i * M + mm] * x;
        }
#pragma unroll
        for (int i = 0; i < kSBC; ++i) {
            if (i < nt) {
                float v = acc[i];
                for (int t = i; t < CT; ++t) v += Gw[i * CT + t] * gs[t * Dv + d];
                dV[(((size_t)b * N + t0 + i) * H + h) * Dv + d] = from_f32<T>(v);
            }
        }
    }
}

// Workspace: prefix (max, den, num) at chunk CT, alpha, alpha gz, w, gz, DS [B*H, N, M],
// chunk totals Sx [B*H, NC, M, Dv] and Sy [B*H, NC, M], g . y [B*H, N], and the
// contraction partials.
struct SbLayout {
    int64_t NC;
    size_t off_pm, off_pd, off_pn, off_al, off_c, off_w, off_gz, off_ds, off_sx, off_sy, off_gy, off_p1, off_p2,
        total;
    SbLayout(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, int CT) {
        NC = (N + CT - 1) / CT;
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
        off_al = take(BH * N * M);
        off_c = take(BH * N * M);
        off_w = take(BH * N * M);
        off_gz = take(BH * N * M);
        off_ds = take(BH * N * M);
        off_sx = take(BH * NC * M * Dv);
        off_sy = take(BH * NC * M);
        off_gy = take(BH * N);
        off_p1 = take(bwd_partial_floats(B, N, H, M, Dk));
        off_p2 = take(bwd_partial_floats(B, N, H, M, Dk));
        total = o + 256;
    }
};

// Tokens per chunk: 16 when phase 3's LDS rows fit in 60 KiB, else 8.
static int stablemax_bwd_chunk(int64_t M, int64_t Dk, int64_t Dv, bool sep) {
    SbSmem s{kSBC, (int)Dk, (int)Dv, (int)M, sep};
    const size_t lim = 60 * 1024 / sizeof(float);
    return (s.floats1() <= lim && s.floats3() <= lim) ? kSBC : kSBC / 2;
}

template <typename T>
static int run_stablemax_backward(const void* Q, const void* K, const void* V, const void* Qd, const void* Kd,
                                  int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                                  float scale, float power, const void* Y, const void* dY, void* dQ, void* dK,
                                  void* dV, void* dQd, void* dKd, char* ws, const SbLayout& lay, int CT,
                                  hipStream_t st) {
    auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
    const int64_t NC = lay.NC, BH = B * H;
    int rc = launch_prepare_public(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, CT, F(lay.off_pm), F(lay.off_pd),
                                   F(lay.off_pn), st, power);
    if (rc) return rc;
    // (the stablemax summaries carry max 0, so the scan's merges are plain sums)
    rc = launch_prefix_public(F(lay.off_pm), F(lay.off_pd), F(lay.off_pn), BH, NC, M, Dv, nullptr, nullptr, nullptr,
                              nullptr, nullptr, nullptr, st);
    if (rc) return rc;
    SbSmem s{CT, (int)Dk, (int)Dv, (int)M, Qd != nullptr};
    dim3 grid((unsigned)NC, (unsigned)BH);
    hipLaunchKernelGGL(stablemax_bwd_forward<T>, grid, dim3(kSBT), s.floats1() * sizeof(float), st, (const T*)Q,
                       (const T*)K, (const T*)V, (const T*)Qd, (const T*)Kd, (const T*)dY, (int)N, (int)H, (int)M,
                       (int)Dk, (int)Dv, scale, power, CT, F(lay.off_pm), F(lay.off_pd), F(lay.off_pn), F(lay.off_al),
                       F(lay.off_c), F(lay.off_w), F(lay.off_gz), F(lay.off_sx), F(lay.off_sy));
    if ((rc = check_launch("stablemax_bwd_forward"))) return rc;
    const int64_t threads = BH * M * Dv + BH * M;
    hipLaunchKernelGGL(stablemax_bwd_suffix, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       F(lay.off_sx), F(lay.off_sy), (int)BH, (int)NC, (int)M, (int)Dv);
    if ((rc = check_launch("stablemax_bwd_suffix"))) return rc;
    hipLaunchKernelGGL(stablemax_bwd_tokens<T>, grid, dim3(kSBT), s.floats3() * sizeof(float), st, (const T*)Q,
                       (const T*)K, (const T*)V, (const T*)dY, (int)N, (int)H, (int)M, (int)Dk, (int)Dv, scale, power, CT,
                       F(lay.off_w), F(lay.off_gz), F(lay.off_sx), F(lay.off_sy), F(lay.off_ds), (T*)dV);
    if ((rc = check_launch("stablemax_bwd_tokens"))) return rc;
    if ((rc = launch_bwd_gy(dY, Y, dtype, B, N, H, Dv, F(lay.off_gy), st))) return rc;
    return launch_bwd_contract(Q, K, Qd, Kd, dtype, B, N, H, M, Dk, scale, F(lay.off_ds), F(lay.off_al),
                               F(lay.off_c), F(lay.off_gy), false, false, dQ, dK, dQd, dKd, F(lay.off_p1), F(lay.off_p2), st);
}

}  // namespace flare

using namespace flare;

extern "C" {

size_t flare_stablemax_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk,
                                               int64_t Dv, int separate_decoder) {
    if (ar_backward_supported(M, Dk, Dv)) return ar_backward_workspace(B, N, H, M, Dk, Dv);
    const int CT = stablemax_bwd_chunk(M, Dk, Dv, separate_decoder != 0);
    return SbLayout(B, N, H, M, Dk, Dv, CT).total;
}

int flare_stablemax_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                             int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                             float scale, float power, const void* Y, const void* dY, void* dQ, void* dK,
                             void* dV, void* dQdec, void* dKdec, void* workspace, size_t workspace_bytes,
                             void* stream) {
    FLARE_REQUIRE(Q && K && V && Y && dY && dQ && dK && dV, "stablemax_backward: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0, "stablemax_backward: sizes must be positive");
    FLARE_REQUIRE(M <= kSBT && Dk <= 256 && Dv <= 256,
                  "stablemax_backward: supports M <= %d, D_score <= 256 and D_value <= 256 (got M=%lld Dk=%lld Dv=%lld)",
                  kSBT, (long long)M, (long long)Dk, (long long)Dv);
    FLARE_REQUIRE(power > 0.0f && power < 1e30f, "stablemax_backward: power must be positive and finite");
    FLARE_REQUIRE((Qdec == nullptr) == (dQdec == nullptr) && (Kdec == nullptr) == (dKdec == nullptr),
                  "stablemax_backward: a separate decoder tensor needs its gradient buffer");
    hipStream_t st = (hipStream_t)stream;
    FLARE_REQUIRE(dtype == FLARE_F32 || dtype == FLARE_BF16 || dtype == FLARE_F16,
                  "stablemax_backward: unknown dtype code %d", dtype);
    if (ar_backward_supported(M, Dk, Dv)) {
        const size_t need = ar_backward_workspace(B, N, H, M, Dk, Dv);
        if (!workspace || workspace_bytes < need) {
            set_error("stablemax_backward: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
            return FLARE_ERR_WORKSPACE;
        }
        return ar_backward_run(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, Y, dY, dQ, dK, dV, dQdec,
                               dKdec, workspace, workspace_bytes, st, power);
    }
    const int CT = stablemax_bwd_chunk(M, Dk, Dv, Qdec != nullptr);
    const SbLayout lay(B, N, H, M, Dk, Dv, CT);
    if (!workspace || workspace_bytes < lay.total) {
        set_error("stablemax_backward: workspace of %zu bytes needed, %zu given", lay.total, workspace_bytes);
        return FLARE_ERR_WORKSPACE;
    }
    char* ws = (char*)workspace;
#define FLARE_SB(TY)                                                                                              \
    return run_stablemax_backward<TY>(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, power, Y, dY, dQ, dK, \
                                      dV, dQdec, dKdec, ws, lay, CT, st)
    if (dtype == FLARE_BF16) FLARE_SB(__hip_bfloat16);
    if (dtype == FLARE_F16) FLARE_SB(__half);
    FLARE_SB(float);
#undef FLARE_SB
}

}  // extern "C"
