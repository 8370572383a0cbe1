// flare_decode.hip -- one recurrent decode step of causal FLARE for every (b,h).
//
// Follows flare_recurrent_step_kernel (causal_flare/autoregressive/inference.py:358-489):
//   s = scale * Q k                         (encoder scores, [M])
//   (m, d, u) <- inf-safe update with (s, v) (in place, fp32)
//   z = u / d_safe;  alpha = softmax_M(a);  y = sum_m alpha_m z_m
// with a = s when the decoder shares the encoder weights.
//
// The step is HBM-bound: per (b,h) it reads and writes the fp32 state
// (8M + 4*M*Dv bytes each way).  One 256-thread workgroup owns one (b,h), so
// the per-latent scalars never leave the workgroup (no cross-workgroup race on
// m/d); the numerator u is streamed with 16-byte loads/stores, consecutive
// threads covering consecutive addresses of a row.
#include "flare_common.h"

namespace flare {

constexpr int kDecNT = 256;
constexpr int kDecBatchRows = 8;   // float4 rows loaded before any is stored
constexpr int kDecKPT = 2;         // k / v elements per thread in the fast step (Dk, Dv <= 512)

__device__ __forceinline__ void store_out_dec(void* Y, size_t idx, float v, int out_dtype) {
    if (out_dtype == FLARE_BF16) reinterpret_cast<__hip_bfloat16*>(Y)[idx] = __float2bfloat16(v);
    else if (out_dtype == FLARE_F16) reinterpret_cast<__half*>(Y)[idx] = __float2half(v);
    else reinterpret_cast<float*>(Y)[idx] = v;
}

template <typename T>
__global__ __launch_bounds__(kDecNT) void decode_step_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ Qdec, const T* __restrict__ Kdec, const int32_t* __restrict__ mask,
    int H, int M, int Dk, int Dv, float scale, bool shared, float* __restrict__ mst,
    float* __restrict__ dst, float* __restrict__ ust, void* __restrict__ Y, int out_dtype) {
    extern __shared__ float smem[];
    float* kv = smem;                 // [Dk]
    float* qd = kv + Dk;              // [Dk]
    float* vv = qd + Dk;              // [Dv]
    float* av = vv + Dv;              // [M] decoder scores
    float* gam = av + M;              // [M]
    float* eta = gam + M;             // [M]
    float* wts = eta + M;             // [M]
    float* red = wts + M;             // [8]
    float4* ypart = reinterpret_cast<float4*>(smem + ((2 * Dk + Dv + 4 * M + 8 + 3) & ~3));  // [RG][NT4]

    const int bh = blockIdx.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x;
    const bool valid = mask == nullptr || mask[b] != 0;
    const size_t kvoff = (size_t)bh * Dk;

    if (!valid) {
        // s = -inf for every latent: gamma = 1, eta = 0, so the state is unchanged
        // and y = 0 (inference.py:395-397, 476-478).
        for (int j = tid; j < Dv; j += kDecNT) store_out_dec(Y, (size_t)bh * Dv + j, 0.0f, out_dtype);
        return;
    }
    for (int j = tid; j < Dk; j += kDecNT) {
        kv[j] = to_f32(K[kvoff + j]);
        if (!shared) qd[j] = to_f32(Qdec[kvoff + j]);
    }
    for (int j = tid; j < Dv; j += kDecNT) vv[j] = to_f32(V[(size_t)bh * Dv + j]);
    __syncthreads();

    // Scores and the per-latent scalar update; thread-per-latent dot products
    // (Q[h] is shared by every batch row and stays in L2).
    const T* qh = Q + (size_t)h * M * Dk;
    const T* kdh = shared ? qh : Kdec + (size_t)h * M * Dk;
    float amax = kNegInf;
    for (int m = tid; m < M; m += kDecNT) {
        const T* qrow = qh + (size_t)m * Dk;
        float acc = 0.0f;
        for (int d = 0; d < Dk; ++d) acc += to_f32(qrow[d]) * kv[d];
        const float s = acc * scale;
        float a = s;
        if (!shared) {
            const T* krow = kdh + (size_t)m * Dk;
            float acc2 = 0.0f;
            for (int d = 0; d < Dk; ++d) acc2 += to_f32(krow[d]) * qd[d];
            a = acc2 * scale;
        }
        const size_t si = (size_t)bh * M + m;
        const MergeScales ts = token_scales(mst[si], s);
        const float dn = dst[si] * ts.sa + ts.sb;
        mst[si] = ts.m_new;
        dst[si] = dn;
        gam[m] = ts.sa;
        eta[m] = ts.sb;
        wts[m] = dn > 0.0f ? dn : 1.0f;   // d_safe, turned into weights below
        av[m] = a;
        amax = fmaxf(amax, a);
    }
    amax = block_max<kDecNT>(amax, red);
    float asum = 0.0f;
    for (int m = tid; m < M; m += kDecNT) asum += __expf(av[m] - amax);
    asum = block_sum<kDecNT>(asum, red);
    const float inv = 1.0f / asum;
    for (int m = tid; m < M; m += kDecNT) wts[m] = __expf(av[m] - amax) * inv / wts[m];
    __syncthreads();

    // Numerator update and readout, 16 bytes per access.
    const int D4 = Dv >> 2;
    int NT4 = 1;
    while (NT4 * 2 <= D4 && NT4 * 2 <= kDecNT) NT4 *= 2;
    const int RG = kDecNT / NT4;
    const int jt = tid % NT4, rg = tid / NT4;
    float4* u4 = reinterpret_cast<float4*>(ust + (size_t)bh * M * Dv);
    const float4* v4 = reinterpret_cast<const float4*>(vv);
    for (int j0 = 0; j0 < D4; j0 += NT4) {
        const int j4 = j0 + jt;
        const bool act = j4 < D4;
        float4 y4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (act) {
            const float4 vj = v4[j4];
            for (int mb = rg; mb < M; mb += RG * kDecBatchRows) {
                float4 buf[kDecBatchRows];
#pragma unroll
                for (int r = 0; r < kDecBatchRows; ++r) {
                    const int m = mb + r * RG;
                    if (m < M) buf[r] = u4[(size_t)m * D4 + j4];
                }
#pragma unroll
                for (int r = 0; r < kDecBatchRows; ++r) {
                    const int m = mb + r * RG;
                    if (m < M) {
                        const float g = gam[m], e = eta[m], w = wts[m];
                        float4 x = buf[r];
                        x.x = x.x * g + e * vj.x;
                        x.y = x.y * g + e * vj.y;
                        x.z = x.z * g + e * vj.z;
                        x.w = x.w * g + e * vj.w;
                        u4[(size_t)m * D4 + j4] = x;
                        y4.x += w * x.x;
                        y4.y += w * x.y;
                        y4.z += w * x.z;
                        y4.w += w * x.w;
                    }
                }
            }
        }
        ypart[rg * NT4 + jt] = y4;
        __syncthreads();
        if (tid < NT4 && j0 + tid < D4) {
            float4 acc = ypart[tid];
            for (int g2 = 1; g2 < RG; ++g2) {
                const float4 p = ypart[g2 * NT4 + tid];
                acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
            }
            const size_t yo = (size_t)bh * Dv + 4 * (j0 + tid);
            store_out_dec(Y, yo + 0, acc.x, out_dtype);
            store_out_dec(Y, yo + 1, acc.y, out_dtype);
            store_out_dec(Y, yo + 2, acc.z, out_dtype);
            store_out_dec(Y, yo + 3, acc.w, out_dtype);
        }
        __syncthreads();
    }
}

// Fast step for the common shapes: M = RG * ROWS latents and Dv = 4 * NT4 value
// columns with RG = 256 / NT4, so every thread owns ROWS rows of one float4
// column of u.  Every workgroup of the grid runs its (b,h) at once, so the step
// is one short chain per workgroup: all reads are issued at the start, the
// small ones (k, the Q row of thread m, m / d, v) ahead of the u rows, since
// loads complete in issue order; thread m then forms its score from k read
// straight from global memory (the same 16 bytes in every thread, scalar
// loads), so no barrier stands before the scores.  Three barriers follow: the
// merge scales and per-wave softmax partials published, the weights
// published, the y partials published.
template <typename T, int ROWS, int NT4>
__global__ __launch_bounds__(kDecNT) void decode_step_fast(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ Qdec, const T* __restrict__ Kdec, const int32_t* __restrict__ mask,
    int H, int M, int Dk, int Dv, float scale, bool shared, float* __restrict__ mst,
    float* __restrict__ dst, float* __restrict__ ust, void* __restrict__ Y, int out_dtype) {
    constexpr int RG = kDecNT / NT4;
    constexpr int NWV = kDecNT / 64;
    constexpr int CH = 16 / sizeof(T);   // Q elements per 16-byte load
    constexpr int QPF = 8;               // 16-byte pieces of the Q row prefetched
    extern __shared__ float smem[];
    float* vv = smem;                 // [Dv]
    float* av = vv + Dv;              // [M] decoder scores
    float* gam = av + M;              // [M]
    float* eta = gam + M;             // [M]
    float* wts = eta + M;             // [M]
    float* red = wts + M;             // [2 NWV] per-wave (max, sum) of the decoder softmax
    float4* ypart = reinterpret_cast<float4*>(smem + ((Dv + 4 * M + 8 + 3) & ~3));  // [RG][NT4]

    const int bh = blockIdx.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int jt = tid % NT4, rg = tid / NT4;
    if (mask != nullptr && mask[b] == 0) {
        for (int j = tid; j < Dv; j += kDecNT) store_out_dec(Y, (size_t)bh * Dv + j, 0.0f, out_dtype);
        return;
    }
    // ---- every read of the step, issued up front, the small ones first: loads return
    //      in issue order, so the scores wait only for k, q and m / d while the u rows
    //      (the bulk of the step's traffic) are still in flight.  Thread m reads k (and
    //      the token's decoder query) straight from global memory, the same 16-byte
    //      pieces for every thread, so no barrier stands before the scores.
    //      (Clamped indices, no branches: a branch around a load makes the compiler
    //      wait for it.)
    const size_t kvoff = (size_t)bh * Dk;
    const T* qdsrc = shared ? K : Qdec;
    const int npieces = Dk / CH;
    typedef unsigned u32v4 __attribute__((ext_vector_type(4)));
    const u32v4* k4 = reinterpret_cast<const u32v4*>(K + kvoff);
    const u32v4* qd4 = reinterpret_cast<const u32v4*>(qdsrc + kvoff);
    u32v4 kpf[QPF], qdpf[QPF], qpf[QPF];
    const T* qrow = Q + ((size_t)h * M + min(tid, M - 1)) * Dk;
#pragma unroll
    for (int p = 0; p < QPF; ++p) {
        kpf[p] = k4[min(p, npieces - 1)];
        qpf[p] = reinterpret_cast<const u32v4*>(qrow)[min(p, npieces - 1)];
    }
    if (!shared) {
#pragma unroll
        for (int p = 0; p < QPF; ++p) qdpf[p] = qd4[min(p, npieces - 1)];
    }
    const size_t si = (size_t)bh * M + tid;
    const bool own = tid < M;
    const size_t sc = (size_t)bh * M + min(tid, M - 1);
    float m_old = mst[sc];
    float d_old = dst[sc];
    float vr[kDecKPT];
#pragma unroll
    for (int i = 0; i < kDecKPT; ++i) vr[i] = to_f32(V[(size_t)bh * Dv + min(tid + i * kDecNT, Dv - 1)]);
    float4* u4 = reinterpret_cast<float4*>(ust + (size_t)bh * M * Dv);
    float4 ur[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) ur[r] = u4[(size_t)(rg + r * RG) * NT4 + jt];
    // every load above is issued before the scores wait for k and q (the empty asm
    // statements keep the compiler from moving that wait, or the dot product, above the
    // u loads)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int p = 0; p < QPF; ++p) asm volatile("" : "+v"(kpf[p]), "+v"(qpf[p]));
    asm volatile("" : "+v"(m_old), "+v"(d_old));

    // ---- scores (thread m); the decoder softmax partials of each wave
    auto dot = [&](u32v4 x, u32v4 y) {
        union { u32v4 raw; T el[CH]; } xa, ya;
        xa.raw = x;
        ya.raw = y;
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < CH; ++e) acc += to_f32(xa.el[e]) * to_f32(ya.el[e]);
        return acc;
    };
    float a = kNegInf;
    if (own) {
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < QPF; ++p)
            if (p < npieces) acc += dot(qpf[p], kpf[p]);
        for (int p = QPF; p < npieces; ++p) acc += dot(reinterpret_cast<const u32v4*>(qrow)[p], k4[p]);
        const float s = acc * scale;
        a = s;
        if (!shared) {
            const u32v4* kd4 = reinterpret_cast<const u32v4*>(Kdec + ((size_t)h * M + tid) * Dk);
            float acc2 = 0.0f;
            for (int p = 0; p < npieces; ++p) acc2 += dot(kd4[p], p < QPF ? qdpf[p] : qd4[p]);
            a = acc2 * scale;
        }
        const MergeScales ts = token_scales(m_old, s);
        const float dn = d_old * ts.sa + ts.sb;
        mst[si] = ts.m_new;
        dst[si] = dn;
        gam[tid] = ts.sa;
        eta[tid] = ts.sb;
        wts[tid] = dn > 0.0f ? dn : 1.0f;
        av[tid] = a;
    }
#pragma unroll
    for (int i = 0; i < kDecKPT; ++i) vv[min(tid + i * kDecNT, Dv - 1)] = vr[i];   // (past the end: the last value again)
    const float wmax = wave_max(a);
    const float wsum = wave_sum(own && wmax != kNegInf ? __expf(a - wmax) : 0.0f);
    if (lane == 0) {
        red[2 * wv] = wmax;
        red[2 * wv + 1] = wsum;
    }
    __syncthreads();   // (1) v, the merge scales and the softmax partials visible
    float amax = kNegInf;
#pragma unroll
    for (int i = 0; i < NWV; ++i) amax = fmaxf(amax, red[2 * i]);
    float asum = 0.0f;
#pragma unroll
    for (int i = 0; i < NWV; ++i)
        if (red[2 * i] != kNegInf) asum += red[2 * i + 1] * __expf(red[2 * i] - amax);
    if (own) wts[tid] = __expf(a - amax) / (asum * wts[tid]);
    __syncthreads();   // (2) weights visible

    // ---- numerator update and readout from the prefetched rows
    const float4 vj = reinterpret_cast<const float4*>(vv)[jt];
    float4 y4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int m = rg + r * RG;
        const float g = gam[m], e = eta[m], w = wts[m];
        float4 x = ur[r];
        x.x = x.x * g + e * vj.x;
        x.y = x.y * g + e * vj.y;
        x.z = x.z * g + e * vj.z;
        x.w = x.w * g + e * vj.w;
        u4[(size_t)m * NT4 + jt] = x;
        y4.x += w * x.x;
        y4.y += w * x.y;
        y4.z += w * x.z;
        y4.w += w * x.w;
    }
    ypart[rg * NT4 + jt] = y4;
    __syncthreads();   // (3) y partials visible
    if (tid < NT4) {
        float4 acc = ypart[tid];
        for (int g2 = 1; g2 < RG; ++g2) {
            const float4 p = ypart[g2 * NT4 + tid];
            acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
        }
        const size_t yo = (size_t)bh * Dv + 4 * tid;
        store_out_dec(Y, yo + 0, acc.x, out_dtype);
        store_out_dec(Y, yo + 1, acc.y, out_dtype);
        store_out_dec(Y, yo + 2, acc.z, out_dtype);
        store_out_dec(Y, yo + 3, acc.w, out_dtype);
    }
}

}  // namespace flare

using namespace flare;

extern "C" int flare_decode_step(const void* Q, const void* K, const void* V, const void* Qdec,
                                 const void* Kdec, const int32_t* mask, int dtype, int64_t B,
                                 int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                                 float* m, float* d, float* u, void* y, int out_dtype,
                                 void* stream) {
    FLARE_REQUIRE(Q && K && V && m && d && u && y, "decode_step: null pointer");
    FLARE_REQUIRE(B > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0, "decode_step: sizes must be positive");
    FLARE_REQUIRE(Dv % 4 == 0, "decode_step: Dv=%lld must be a multiple of 4", (long long)Dv);
    FLARE_REQUIRE(((uintptr_t)u & 15) == 0, "decode_step: u must be 16-byte aligned");
    const bool shared = Qdec == nullptr && Kdec == nullptr;
    const void* qd = Qdec ? Qdec : K;
    const void* kd = Kdec ? Kdec : Q;
    int NT4 = 1;
    while (NT4 * 2 <= Dv / 4 && NT4 * 2 <= kDecNT) NT4 *= 2;
    const size_t sm = sizeof(float) * (2 * Dk + Dv + 4 * M + 8 + 3) + sizeof(float4) * kDecNT;
    FLARE_REQUIRE(sm <= 64 * 1024, "decode_step: shape too large for LDS");
    (void)NT4;
    hipStream_t s = (hipStream_t)stream;
    // fast path: M = (256 / NT4) * ROWS with Dv = 4 * NT4, M <= 256, Dk a multiple of 16 bytes
    {
        const int64_t D4 = Dv / 4;
        const int64_t esz = dtype == FLARE_F32 ? 4 : 2;
        const bool pow2 = D4 > 0 && D4 <= kDecNT && (D4 & (D4 - 1)) == 0;
        const int64_t RG = pow2 ? kDecNT / D4 : 0;
        const int64_t rows = RG ? M / RG : 0;
        const bool aligned = ((uintptr_t)Q & 15) == 0 && ((uintptr_t)K & 15) == 0 &&
                             (!Kdec || ((uintptr_t)Kdec & 15) == 0) && (!Qdec || ((uintptr_t)Qdec & 15) == 0);
        if (pow2 && M <= kDecNT && rows * RG == M && (Dk * esz) % 16 == 0 && aligned &&
            Dk <= kDecKPT * kDecNT && Dv <= kDecKPT * kDecNT &&
            (rows == 1 || rows == 2 || rows == 4 || rows == 8 || rows == 16)) {
#define FLARE_DEC_FAST(TY, RW, N4)                                                                         \
    hipLaunchKernelGGL((decode_step_fast<TY, RW, N4>), dim3((unsigned)(B * H)), dim3(kDecNT), sm, s,        \
                       (const TY*)Q, (const TY*)K, (const TY*)V, (const TY*)qd, (const TY*)kd, mask, (int)H, \
                       (int)M, (int)Dk, (int)Dv, scale, shared, m, d, u, y, out_dtype)
#define FLARE_DEC_ROWS(TY, N4)                                   \
    switch (rows) {                                              \
        case 1: FLARE_DEC_FAST(TY, 1, N4); break;                \
        case 2: FLARE_DEC_FAST(TY, 2, N4); break;                \
        case 4: FLARE_DEC_FAST(TY, 4, N4); break;                \
        case 8: FLARE_DEC_FAST(TY, 8, N4); break;                \
        default: FLARE_DEC_FAST(TY, 16, N4); break;              \
    }
#define FLARE_DEC_N4(TY)                                         \
    switch (D4) {                                                \
        case 1: FLARE_DEC_ROWS(TY, 1) break;                     \
        case 2: FLARE_DEC_ROWS(TY, 2) break;                     \
        case 4: FLARE_DEC_ROWS(TY, 4) break;                     \
        case 8: FLARE_DEC_ROWS(TY, 8) break;                     \
        case 16: FLARE_DEC_ROWS(TY, 16) break;                   \
        case 32: FLARE_DEC_ROWS(TY, 32) break;                   \
        case 64: FLARE_DEC_ROWS(TY, 64) break;                   \
        case 128: FLARE_DEC_ROWS(TY, 128) break;                 \
        default: FLARE_DEC_ROWS(TY, 256) break;                  \
    }
            if (dtype == FLARE_BF16) { FLARE_DEC_N4(__hip_bfloat16) }
            else if (dtype == FLARE_F16) { FLARE_DEC_N4(__half) }
            else { FLARE_DEC_N4(float) }
#undef FLARE_DEC_N4
#undef FLARE_DEC_ROWS
#undef FLARE_DEC_FAST
            return check_launch("decode_step_fast");
        }
    }
#define FLARE_DEC(TY)                                                                          \
    hipLaunchKernelGGL(decode_step_kernel<TY>, dim3((unsigned)(B * H)), dim3(kDecNT), sm, s,     \
                       (const TY*)Q, (const TY*)K, (const TY*)V, (const TY*)qd, (const TY*)kd,   \
                       mask, (int)H, (int)M, (int)Dk, (int)Dv, scale, shared, m, d, u, y,        \
                       out_dtype)
    if (dtype == FLARE_BF16) FLARE_DEC(__hip_bfloat16);
    else if (dtype == FLARE_F16) FLARE_DEC(__half);
    else FLARE_DEC(float);
#undef FLARE_DEC
    return check_launch("decode_step_kernel");
}
