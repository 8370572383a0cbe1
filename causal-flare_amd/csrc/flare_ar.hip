// flare_ar.hip -- chunked causal FLARE forward / prefill (scalar-fp32 kernels).
//
// Three phases, the structure of causal_flare/autoregressive/training.py:
//   1. chunk_prepare_kernel  per-chunk (max, den, num) summaries   (:914-1018)
//   2. chunk_prefix_kernel   exclusive scan over chunks + initial / final
//                            state merges                          (:1021-1103,
//                            inference.py:753-814)
//   3. chunk_output_kernel   tokenwise replay from the chunk prefix and the
//                            latent softmax readout                 (:1106-1392)
// All arithmetic is fp32 on CUDA-core-equivalent VALU lanes; inputs may be
// fp32, bf16 or fp16.  These kernels serve every dtype and shape; the bf16/fp16
// MFMA kernels in flare_ar_mfma.hip take over the shapes they support.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_replay.h"

namespace flare {

constexpr int kPrepTT = 16;     // tokens per LDS tile in the prepare kernel
constexpr int kPrepMT = 64;     // latents per prepare workgroup
constexpr int kPrepCols = 64;   // max value columns per prepare thread (Dv <= 256)


// ---------------------------------------------------------------------------
// Phase 1.  grid = (NC, B*H, ceil(M/64)), 256 threads.  Thread (ml, g) owns
// latent m0+ml and value columns g, g+4, g+8, ...
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kNT) void chunk_prepare_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, int N, int H,
    int M, int Dk, int Dv, float scale, int chunk, float* __restrict__ cmax,
    float* __restrict__ cden, float* __restrict__ cnum, const int32_t* __restrict__ tmask, float power) {
    // power > 0: the stablemax encoder (E = stablemax_transform(s), no running max:
    // the summary's max stays 0, so the prefix merges are plain sums)
    extern __shared__ float smem[];
    float* k_tile = smem;                       // [TT][Dk]
    float* v_tile = k_tile + kPrepTT * Dk;      // [TT][Dv]
    float* s_tile = v_tile + kPrepTT * Dv;      // [TT][64]

    const int c = blockIdx.x, bh = blockIdx.y, mbase = blockIdx.z * kPrepMT;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, ml = tid & 63, g = tid >> 6;
    const int m = mbase + ml;
    const T* q_h = Q + (size_t)h * M * Dk;

    float mx = power > 0.0f ? 0.0f : kNegInf, den = 0.0f;
    float num[kPrepCols];
#pragma unroll
    for (int i = 0; i < kPrepCols; ++i) num[i] = 0.0f;

    const int t_begin = c * chunk;
    const int t_end = min(N, t_begin + chunk);
    for (int t0 = t_begin; t0 < t_end; t0 += kPrepTT) {
        const int nt = min(kPrepTT, t_end - t0);
        for (int e = tid; e < kPrepTT * Dk; e += kNT) {
            const int i = e / Dk, d = e % Dk;
            k_tile[e] = i < nt ? to_f32(K[(((size_t)b * N + t0 + i) * H + h) * Dk + d]) : 0.0f;
        }
        for (int e = tid; e < kPrepTT * Dv; e += kNT) {
            const int i = e / Dv, d = e % Dv;
            v_tile[e] = i < nt ? to_f32(V[(((size_t)b * N + t0 + i) * H + h) * Dv + d]) : 0.0f;
        }
        __syncthreads();
        for (int p = tid; p < kPrepTT * kPrepMT; p += kNT) {
            const int i = p / kPrepMT, mm = mbase + p % kPrepMT;
            float s = kNegInf;     // also for a masked token: it adds nothing to the summary
            if (i < nt && mm < M && (tmask == nullptr || tmask[(size_t)b * N + t0 + i] != 0)) {
                const T* qrow = q_h + (size_t)mm * Dk;
                const float* kr = k_tile + i * Dk;
                float acc = 0.0f;
                for (int d = 0; d < Dk; ++d) acc += kr[d] * to_f32(qrow[d]);
                s = acc * scale;
            }
            s_tile[p] = s;
        }
        __syncthreads();
        for (int i = 0; i < nt; ++i) {
            const float s = s_tile[i * kPrepMT + ml];
            if (s == kNegInf) continue;     // a masked token (no update; keeps mx = -inf safe)
            const float m_new = power > 0.0f ? mx : fmaxf(mx, s);
            const float r = power > 0.0f ? 1.0f : __expf(mx - m_new);     // mx = -inf on the first token -> 0
            const float e = power > 0.0f ? stablemax_transform(s, power) : __expf(s - m_new);
            den = den * r + e;
            const float* vr = v_tile + i * Dv;
#pragma unroll
            for (int k = 0; k < kPrepCols; ++k) {
                const int col = g + 4 * k;
                if (col < Dv) num[k] = num[k] * r + e * vr[col];
            }
            mx = m_new;
        }
        __syncthreads();
    }
    if (m < M) {
        const size_t sidx = ((size_t)bh * NC + c) * M + m;
        if (g == 0) {
            cmax[sidx] = mx;
            cden[sidx] = den;
        }
        float* nrow = cnum + sidx * Dv;
#pragma unroll
        for (int k = 0; k < kPrepCols; ++k) {
            const int col = g + 4 * k;
            if (col < Dv) nrow[col] = num[k];
        }
    }
}

// ---------------------------------------------------------------------------
// Phase 2.  One thread per (b*h, latent, 4 value columns); 256-thread
// workgroups.  A bandwidth kernel: every summary is read once and overwritten
// in place by the exclusive prefix with 16-byte accesses.  The (max, den) pair
// of a latent is re-derived by each of its Dv/4 threads (cheap, keeps the
// kernel free of cross-thread traffic).  Chunks are loaded kScanBatch at a time
// before their serial merges run, so one memory latency covers kScanBatch
// merges.
// ---------------------------------------------------------------------------
constexpr int kScanBatch = 16;   // chunk summaries loaded before the first merge (config 3 has 16 chunks)

__global__ __launch_bounds__(256) void chunk_prefix_kernel(
    float* __restrict__ cmax, float* __restrict__ cden, float* __restrict__ cnum, int NC, int M,
    int Dv, int rows, const float* __restrict__ m0, const float* __restrict__ d0,
    const float* __restrict__ u0, float* __restrict__ m_fin, float* __restrict__ d_fin,
    float* __restrict__ u_fin) {
    const int D4 = Dv >> 2;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * D4) return;
    const int row = gid / D4, j = gid % D4;    // row = bh * M + m, value columns 4j .. 4j+3
    const int bh = row / M, m = row % M;
    float mc = m0 ? m0[row] : kNegInf;
    float dc = d0 ? d0[row] : 0.0f;
    float4 uc = u0 ? reinterpret_cast<const float4*>(u0)[(size_t)row * D4 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
    const size_t base = (size_t)bh * NC * M + m;          // summary index of chunk 0
    float4* num4 = reinterpret_cast<float4*>(cnum);
    for (int c0 = 0; c0 < NC; c0 += kScanBatch) {
        float bm[kScanBatch], bd[kScanBatch];
        float4 bu[kScanBatch];
#pragma unroll
        for (int i = 0; i < kScanBatch; ++i) {
            const bool in = c0 + i < NC;
            const size_t si = base + (size_t)(c0 + i) * M;
            bm[i] = in ? cmax[si] : kNegInf;
            bd[i] = in ? cden[si] : 0.0f;
            bu[i] = in ? num4[si * D4 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < kScanBatch; ++i) {
            if (c0 + i >= NC) break;
            const size_t si = base + (size_t)(c0 + i) * M;
            if (j == 0) {
                cmax[si] = mc;
                cden[si] = dc;
            }
            num4[si * D4 + j] = uc;
            const MergeScales ms = merge_scales(mc, bm[i]);
            dc = dc * ms.sa + bd[i] * ms.sb;
            uc.x = uc.x * ms.sa + bu[i].x * ms.sb;
            uc.y = uc.y * ms.sa + bu[i].y * ms.sb;
            uc.z = uc.z * ms.sa + bu[i].z * ms.sb;
            uc.w = uc.w * ms.sa + bu[i].w * ms.sb;
            mc = ms.m_new;
        }
    }
    if (m_fin) {
        if (j == 0) {
            m_fin[row] = mc;
            d_fin[row] = dc;
        }
        reinterpret_cast<float4*>(u_fin)[(size_t)row * D4 + j] = uc;
    }
}

template <typename T, int ROWS>
__global__ __launch_bounds__(kNT) void chunk_output_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ Qdec, const T* __restrict__ Kdec, int N, int H, int M, int Dk, int Dv,
    int DT, int TT, float scale, int chunk, bool shared, const float* __restrict__ pmax,
    const float* __restrict__ pden, const float* __restrict__ pnum, void* __restrict__ Y,
    int out_dtype, float* __restrict__ lse_dec, const int32_t* __restrict__ tmask, const int* __restrict__ only,
    float power) {
    // only: when given, [B*H, NC] flags; chunks whose flag is 0 are left alone (the
    // tokenwise replay of the chunks an MFMA output kernel could not resolve).  A
    // narrow flag replays 32-token subtiles j1 .. j2 of the chunk only, from the
    // state at subtile j1's start (which then stands in the chunk's prefix slot).
    // power > 0: the stablemax encoder (den += stablemax_transform(s), no rescale);
    // the decoder weights stay a softmax over the latents.
    int flag = kRedoWhole;
    if (only != nullptr) {
        flag = only[(size_t)blockIdx.y * gridDim.x + blockIdx.x];
        if (flag == 0) return;
    }
    extern __shared__ __attribute__((aligned(16))) float smem[];
    output_chunk_replay<T, ROWS>(Q, K, V, Qdec, Kdec, N, H, M, Dk, Dv, DT, TT, scale, chunk, shared, pmax, pden,
                                 pnum, Y, out_dtype, lse_dec, tmask, power, smem, blockIdx.x, blockIdx.y,
                                 blockIdx.z * DT, gridDim.x, threadIdx.x, flag);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int launch_prepare(const void* Q, const void* K, const void* V, int dtype, int64_t B,
                          int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                          int64_t chunk, float* cmax, float* cden, float* cnum,
                          hipStream_t stream, const int32_t* tmask = nullptr, float power = 0.0f) {
    if (power > 0.0f && (mfma_phase_mask() & 1) && chunk % 32 == 0 && tmask == nullptr &&
        mfma_prepare_supported(dtype, M, Dk, Dv) && (M == 128 || M == 256) && (Dk == 64 || Dk == 128))
        return launch_prepare_tr(Q, K, V, B, N, H, M, Dk, scale, chunk, cmax, cden, cnum, nullptr, dtype == FLARE_F16,
                                 stream, power);
    if (power <= 0.0f && (mfma_phase_mask() & 1) && chunk % 32 == 0 && mfma_prepare_supported(dtype, M, Dk, Dv)) {
        if (output_pc_enabled() && (M == 128 || M == 256))
            return launch_prepare_pc(Q, K, V, B, N, H, M, Dk, scale, chunk, cmax, cden, cnum, tmask,
                                     dtype == FLARE_F16, stream);
        if (tmask == nullptr)
            return launch_prepare_mfma(Q, K, V, B, N, H, M, Dk, scale, chunk, cmax, cden, cnum, dtype == FLARE_F16,
                                       stream);
    }
    FLARE_REQUIRE(Dv <= 4 * kPrepCols, "chunk_prepare: Dv=%lld exceeds %d", (long long)Dv, 4 * kPrepCols);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H), (unsigned)((M + kPrepMT - 1) / kPrepMT));
    const size_t sm = sizeof(float) * (kPrepTT * (Dk + Dv) + kPrepTT * kPrepMT);
    FLARE_REQUIRE(sm <= 64 * 1024, "chunk_prepare: Dk+Dv too large for LDS");
#define FLARE_PREP(TY)                                                                          \
    hipLaunchKernelGGL(chunk_prepare_kernel<TY>, grid, dim3(kNT), sm, stream,                   \
                       (const TY*)Q, (const TY*)K, (const TY*)V, (int)N, (int)H, (int)M,         \
                       (int)Dk, (int)Dv, scale, (int)chunk, cmax, cden, cnum, tmask, power)
    if (dtype == FLARE_BF16) FLARE_PREP(__hip_bfloat16);
    else if (dtype == FLARE_F16) FLARE_PREP(__half);
    else FLARE_PREP(float);
#undef FLARE_PREP
    return check_launch("chunk_prepare_kernel");
}

static int launch_prefix(float* cmax, float* cden, float* cnum, int64_t BH, int64_t NC, int64_t M,
                         int64_t Dv, const float* m0, const float* d0, const float* u0,
                         float* m_fin, float* d_fin, float* u_fin, hipStream_t stream) {
    FLARE_REQUIRE(Dv % 4 == 0, "chunk_prefix: Dv=%lld must be a multiple of 4", (long long)Dv);
    FLARE_REQUIRE((((uintptr_t)cnum) & 15) == 0 && (!u0 || (((uintptr_t)u0) & 15) == 0) &&
                  (!u_fin || (((uintptr_t)u_fin) & 15) == 0), "chunk_prefix: numerators must be 16-byte aligned");
    FLARE_REQUIRE((m0 && d0 && u0) || (!m0 && !d0 && !u0), "chunk_prefix: give all of m0/d0/u0 or none");
    FLARE_REQUIRE((m_fin && d_fin && u_fin) || (!m_fin && !d_fin && !u_fin),
                  "chunk_prefix: give all of m_fin/d_fin/u_fin or none");
    const int64_t threads = BH * M * (Dv / 4);
    hipLaunchKernelGGL(chunk_prefix_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, cmax,
                       cden, cnum, (int)NC, (int)M, (int)Dv, (int)(BH * M), m0, d0, u0, m_fin, d_fin, u_fin);
    return check_launch("chunk_prefix_kernel");
}

static int launch_output(const void* Q, const void* K, const void* V, const void* Qdec,
                         const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                         int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* pmax,
                         const float* pden, const float* pnum, void* Y, int out_dtype,
                         float* lse_dec, hipStream_t stream, const int32_t* tmask = nullptr,
                         void* alpha_ws = nullptr, int* redo = nullptr, float power = 0.0f,
                         bool record = false) {
    // record: pmax / pden / pnum are this call's own scratch (the forward's workspace), so
    // the output kernel may overwrite a chunk's slot with a replay record
    const bool shared = Qdec == nullptr && Kdec == nullptr;
    // A launch of the scalar kernel restricted to the chunks flagged in `only` (or all).
    auto scalar = [&](const int* only) -> int {
        const int DT = replay_dt((int)M, (int)Dv);
        FLARE_REQUIRE(DT > 0,
                      "chunk_output: unsupported M=%lld Dv=%lld (Dv must be a multiple of 16, M*16 <= 16384)",
                      (long long)M, (long long)Dv);
        const int R = kNT / DT;
        const int64_t rows = (M + R - 1) / R;
        const int rows_t = replay_rows((int)M, DT);   // the ROWS instance
        OutSmem lay{16, (int)Dk, DT, (int)M, R, R * rows_t, shared};
        while (lay.floats() * sizeof(float) > 64 * 1024 && lay.TT > 1) lay.TT /= 2;
        FLARE_REQUIRE(lay.floats() * sizeof(float) <= 64 * 1024, "chunk_output: shape too large for LDS");
        const int TT = lay.TT;
        const int64_t NC = (N + chunk - 1) / chunk;
        dim3 grid((unsigned)NC, (unsigned)(B * H), (unsigned)(Dv / DT));
        const size_t sm = lay.floats() * sizeof(float);
        // Missing decoder tensors default to the encoder ones (K as Qdec, Q as Kdec).
        const void* qd = Qdec ? Qdec : K;
        const void* kd = Kdec ? Kdec : Q;
#define FLARE_OUT(TY, RW)                                                                       \
    hipLaunchKernelGGL((chunk_output_kernel<TY, RW>), grid, dim3(kNT), sm, stream, (const TY*)Q, \
                       (const TY*)K, (const TY*)V, (const TY*)qd, (const TY*)kd, (int)N, (int)H,  \
                       (int)M, (int)Dk, (int)Dv, DT, TT, scale, (int)chunk, shared, pmax, pden,   \
                       pnum, Y, out_dtype, lse_dec, tmask, only, power)
#define FLARE_OUT_ROWS(TY)                   \
    if (rows <= 8) FLARE_OUT(TY, 8);         \
    else if (rows <= 16) FLARE_OUT(TY, 16);  \
    else if (rows <= 32) FLARE_OUT(TY, 32);  \
    else FLARE_OUT(TY, 64);
        if (dtype == FLARE_BF16) { FLARE_OUT_ROWS(__hip_bfloat16) }
        else if (dtype == FLARE_F16) { FLARE_OUT_ROWS(__half) }
        else { FLARE_OUT_ROWS(float) }
#undef FLARE_OUT_ROWS
#undef FLARE_OUT
        return check_launch("chunk_output_kernel");
    };
    // the stablemax encoder on the MFMA output kernel: the decoder softmax first (as for
    // separate decoder tensors; the encoder weights are not a softmax), then chunk_output_tr
    // with the stablemax transform of the scores; flagged chunks replay in fp32
    if (power > 0.0f && (mfma_phase_mask() & 2) && chunk % 32 == 0 && lse_dec == nullptr && redo != nullptr &&
        alpha_ws != nullptr && tmask == nullptr && output_pc_enabled() && output_tr_enabled() &&
        mfma_output_supported(dtype, out_dtype, true, M, Dk, Dv)) {
        int rc = launch_decoder_alpha(Qdec ? Qdec : K, Kdec ? Kdec : Q, B, N, H, M, Dk, scale, nullptr, alpha_ws,
                                      nullptr, dtype == FLARE_F16, stream);
        if (rc) return rc;
        rc = launch_output_pc(Q, K, V, B, N, H, M, Dk, scale, chunk, pmax, pden, pnum, Y, out_dtype, nullptr, alpha_ws,
                              dtype == FLARE_F16, redo, stream, false, power);
        if (rc) return rc;
        return scalar(redo);
    }
    // the MFMA kernels run with the redo flags (the chunks they hand back to the scalar kernel)
    if (power <= 0.0f && (mfma_phase_mask() & 2) && chunk % 32 == 0 && lse_dec == nullptr && redo != nullptr) {
        int rc = -1;
        if (mfma_output_supported(dtype, out_dtype, shared, M, Dk, Dv) && (tmask == nullptr || output_pc_enabled())) {
            rc = launch_output_mfma(Q, K, V, B, N, H, M, Dk, scale, chunk, pmax, pden, pnum, Y, out_dtype,
                                    tmask, dtype == FLARE_F16, redo, stream, record);
        } else if (!shared && alpha_ws != nullptr && output_pc_enabled() &&
                   mfma_output_supported(dtype, out_dtype, true, M, Dk, Dv)) {
            // separate decoder tensors: the decoder softmax first (alpha_ws, [B*H, N, M] fp16),
            // then the producer/consumer kernel reading it
            rc = launch_decoder_alpha(Qdec ? Qdec : K, Kdec ? Kdec : Q, B, N, H, M, Dk, scale, tmask,
                                      alpha_ws, nullptr, dtype == FLARE_F16, stream);
            if (rc) return rc;
            rc = launch_output_pc(Q, K, V, B, N, H, M, Dk, scale, chunk, pmax, pden, pnum, Y, out_dtype, tmask,
                                  alpha_ws, dtype == FLARE_F16, redo, stream);
        }
        if (rc >= 0) {
            if (rc) return rc;
            // chunks where a latent's reference jumped past what the MFMA kernel resolves
            // (a score more than kJumpMax above the running max within one subtile) are
            // replayed tokenwise in fp32 (every other chunk's workgroup returns at once),
            // by chunk_output_tr itself where it can
            if (shared && output_tr_replays_inline(M, Dv, false)) return 0;
            return scalar(redo);
        }
    }
    return scalar(nullptr);
}

int launch_prepare_public(const void* Q, const void* K, const void* V, int dtype, int64_t B,
                          int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                          int64_t chunk, float* cmax, float* cden, float* cnum, hipStream_t stream, float power) {
    return launch_prepare(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, chunk, cmax, cden, cnum, stream, nullptr, power);
}

int launch_prefix_public(float* cmax, float* cden, float* cnum, int64_t BH, int64_t NC, int64_t M, int64_t Dv,
                         const float* m0, const float* d0, const float* u0, float* m_fin, float* d_fin,
                         float* u_fin, hipStream_t stream) {
    return launch_prefix(cmax, cden, cnum, BH, NC, M, Dv, m0, d0, u0, m_fin, d_fin, u_fin, stream);
}

int64_t default_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv) {
    // One round of chunk workgroups over the device: about one (chunk, b, h)
    // per resident workgroup slot.  Longer chunks mean fewer, cheaper summaries (phase 2
    // and the summary traffic of phases 1 and 3 shrink with them); each chunk
    // is a multiple of 64 tokens, between 64 and 8192.
    static int cus = 0;
    if (cus <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    const int64_t BH = B * H;
    // the output kernel fills a compute unit with one workgroup, except for the
    // small banks (M * Dv below 128 x 128), where two share it
    const int64_t per_cu = (M * Dv >= 128 * 128) ? 1 : 2;
    const int64_t target_chunks = (per_cu * cus + BH - 1) / BH;
    int64_t c = (N + target_chunks - 1) / target_chunks;
    c = ((c + 63) / 64) * 64;
    if (c < 64) c = 64;
    if (c > 8192) c = 8192;
    return c;
}

}  // namespace flare

using namespace flare;

extern "C" {

int flare_chunk_prepare(const void* Q, const void* K, const void* V, int dtype, int64_t B,
                        int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                        int64_t chunk, float* chunk_max, float* chunk_den, float* chunk_num,
                        void* stream) {
    FLARE_REQUIRE(Q && K && V && chunk_max && chunk_den && chunk_num, "chunk_prepare: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0 && chunk > 0,
                  "chunk_prepare: sizes must be positive");
    return launch_prepare(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, chunk, chunk_max, chunk_den,
                          chunk_num, (hipStream_t)stream);
}

int flare_chunk_prefix(float* chunk_max, float* chunk_den, float* chunk_num, int64_t BH,
                       int64_t NC, int64_t M, int64_t Dv, const float* m0, const float* d0,
                       const float* u0, float* m_fin, float* d_fin, float* u_fin, void* stream) {
    FLARE_REQUIRE(chunk_max && chunk_den && chunk_num, "chunk_prefix: null pointer");
    FLARE_REQUIRE(BH > 0 && NC > 0 && M > 0 && Dv > 0, "chunk_prefix: sizes must be positive");
    return launch_prefix(chunk_max, chunk_den, chunk_num, BH, NC, M, Dv, m0, d0, u0, m_fin, d_fin,
                         u_fin, (hipStream_t)stream);
}

int flare_chunk_output(const void* Q, const void* K, const void* V, const void* Qdec,
                       const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                       int64_t Dk, int64_t Dv, float scale, int64_t chunk,
                       const float* prefix_max, const float* prefix_den, const float* prefix_num,
                       void* Y, int out_dtype, float* lse_dec, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y && prefix_max && prefix_den && prefix_num, "chunk_output: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0 && chunk > 0,
                  "chunk_output: sizes must be positive");
    // the MFMA output kernels report the chunks they hand back to the scalar kernel in
    // [B*H, NC] flags: a stream-ordered allocation of them for this call.  If it fails the
    // call fails (the MFMA kernels need the flags; there is no silent fallback).  The
    // prefix arrays are the caller's, so replays here always cover whole chunks.
    hipStream_t st = (hipStream_t)stream;
    int* redo = nullptr;
    const int64_t NC = (N + chunk - 1) / chunk;
    if (lse_dec == nullptr) {
        const hipError_t e = hipMallocAsync((void**)&redo, (size_t)B * H * NC * sizeof(int), st);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error("chunk_output: hipMallocAsync of %lld redo flags failed: %s", (long long)(B * H * NC),
                      hipGetErrorString(e));
            return FLARE_ERR_LAUNCH;
        }
    }
    const int rc = launch_output(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, chunk, prefix_max,
                                 prefix_den, prefix_num, Y, out_dtype, lse_dec, st, nullptr, nullptr, redo);
    if (redo != nullptr) (void)hipFreeAsync(redo, st);
    return rc;
}

int64_t flare_ar_default_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv) {
    return default_chunk(B, N, H, M, Dv);
}

int flare_forward_kernel_resources(int dtype, int64_t M, int64_t Dk, int64_t Dv, int shared, int64_t chunk,
                                   int phase, int32_t* out) {
    FLARE_REQUIRE(out != nullptr && phase >= 0 && phase <= 2, "kernel_resources: bad arguments");
    hipFuncAttributes attr{};
    int threads = 0;
    const bool f16in = dtype == FLARE_F16;
    const bool tile_shape = Dk == Dv && (M == 128 || M == 256) && (Dk == 64 || Dk == 128);
    if (phase == 1) {
        FLARE_REQUIRE(hipFuncGetAttributes(&attr, (const void*)chunk_prefix_kernel) == hipSuccess,
                      "kernel_resources: hipFuncGetAttributes failed");
        threads = 256;
    } else if (phase == 0) {
        // the kernel launch_prepare picks for this call: chunk_prepare_tr, or none reported
        FLARE_REQUIRE((mfma_phase_mask() & 1) && chunk % 32 == 0 && mfma_prepare_supported(dtype, M, Dk, Dv) &&
                          output_pc_enabled() && prepare_tr_enabled() && tile_shape,
                      "kernel_resources: this call does not run chunk_prepare_tr");
        const int rc = prepare_tr_attributes(M, Dk, f16in, &attr, &threads);
        if (rc) return rc;
    } else {
        FLARE_REQUIRE((mfma_phase_mask() & 2) && chunk % 32 == 0 &&
                          mfma_output_supported(dtype, dtype, true, M, Dk, Dv) && output_pc_enabled() &&
                          output_tr_enabled() && tile_shape,
                      "kernel_resources: this call does not run chunk_output_tr");
        const int rc = output_tr_attributes(M, Dk, shared == 0, f16in, &attr, &threads);
        if (rc) return rc;
    }
    out[0] = threads / 64;
    out[1] = attr.numRegs;
    out[2] = (int32_t)attr.localSizeBytes;
    out[3] = (int32_t)attr.sharedSizeBytes;
    return FLARE_OK;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Bytes of the chunk summaries (max, den, num) and the per-chunk redo flags of the
// output kernel ([B*H, NC] ints), each 256-byte aligned.
static size_t summary_bytes(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, int64_t chunk) {
    const int64_t NC = (N + chunk - 1) / chunk;
    const size_t per = (size_t)B * H * NC * M;
    return 2 * align256(per * sizeof(float)) + align256(per * Dv * sizeof(float)) +
           align256((size_t)B * H * NC * sizeof(int));
}

size_t flare_ar_forward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                       int64_t chunk) {
    if (chunk <= 0) chunk = default_chunk(B, N, H, M, Dv);
    return summary_bytes(B, N, H, M, Dv, chunk);
}

size_t flare_ar_forward_workspace_size_sep(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                           int64_t chunk) {
    if (chunk <= 0) chunk = default_chunk(B, N, H, M, Dv);
    return summary_bytes(B, N, H, M, Dv, chunk) + align256((size_t)B * H * N * M * 2);
}

int flare_ar_forward(const void* Q, const void* K, const void* V, const void* Qdec,
                     const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                     const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                     void* Y, int out_dtype, void* workspace, size_t workspace_bytes,
                     void* stream) {
    return flare_ar_forward_masked(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, chunk, m0, d0, u0,
                                   m_fin, d_fin, u_fin, Y, out_dtype, nullptr, workspace, workspace_bytes, stream);
}

int flare_stablemax_forward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                            int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                            float scale, int64_t chunk, float power, void* Y, int out_dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y, "stablemax_forward: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0,
                  "stablemax_forward: sizes must be positive");
    FLARE_REQUIRE(power > 0.0f && power < 1e30f, "stablemax_forward: power must be positive and finite");
    if (chunk <= 0) chunk = default_chunk(B, N, H, M, Dv);
    const size_t need = flare_ar_forward_workspace_size(B, N, H, M, Dv, chunk);
    if (!workspace || workspace_bytes < need) {
        set_error("stablemax_forward: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return FLARE_ERR_WORKSPACE;
    }
    const int64_t NC = (N + chunk - 1) / chunk;
    const size_t per = (size_t)B * H * NC * M;
    char* ws = (char*)workspace;
    float* cmax = (float*)ws;
    float* cden = (float*)(ws + align256(per * sizeof(float)));
    float* cnum = (float*)(ws + 2 * align256(per * sizeof(float)));
    int* redo = (int*)(ws + 2 * align256(per * sizeof(float)) + align256(per * Dv * sizeof(float)));
    // with room for the decoder softmax (flare_ar_forward_workspace_size_sep), the MFMA
    // kernels for bf16 / fp16 inputs of their shapes
    void* alpha_ws = workspace_bytes >= flare_ar_forward_workspace_size_sep(B, N, H, M, Dv, chunk)
                         ? (void*)(ws + summary_bytes(B, N, H, M, Dv, chunk)) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    int rc = launch_prepare(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, chunk, cmax, cden, cnum, s, nullptr, power);
    if (rc) return rc;
    // the scan's online-softmax merges: plain sums for the scalar prepare's summaries (max 0),
    // reference-scaled ones for the MFMA prepare's
    rc = launch_prefix(cmax, cden, cnum, B * H, NC, M, Dv, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, s);
    if (rc) return rc;
    return launch_output(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, chunk, cmax, cden, cnum, Y,
                         out_dtype, nullptr, s, nullptr, alpha_ws, alpha_ws ? redo : nullptr, power);
}

int flare_ar_forward_masked(const void* Q, const void* K, const void* V, const void* Qdec,
                            const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                            int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                            const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                            void* Y, int out_dtype, const int32_t* token_mask, void* workspace,
                            size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y, "ar_forward: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0, "ar_forward: sizes must be positive");
    if (chunk <= 0) chunk = default_chunk(B, N, H, M, Dv);
    const size_t need = flare_ar_forward_workspace_size(B, N, H, M, Dv, chunk);
    if (!workspace || workspace_bytes < need) {
        set_error("ar_forward: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return FLARE_ERR_WORKSPACE;
    }
    // room for the decoder softmax of separate decoder tensors (MFMA path)
    void* alpha_ws = nullptr;
    if ((Qdec || Kdec) && workspace_bytes >= flare_ar_forward_workspace_size_sep(B, N, H, M, Dv, chunk))
        alpha_ws = (char*)workspace + summary_bytes(B, N, H, M, Dv, chunk);
    const int64_t NC = (N + chunk - 1) / chunk;
    const size_t per = (size_t)B * H * NC * M;
    char* ws = (char*)workspace;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    float* cmax = (float*)ws;
    float* cden = (float*)(ws + align(per * sizeof(float)));
    float* cnum = (float*)(ws + 2 * align(per * sizeof(float)));
    int* redo = (int*)(ws + 2 * align(per * sizeof(float)) + align(per * Dv * sizeof(float)));
    hipStream_t s = (hipStream_t)stream;
    int rc = launch_prepare(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, chunk, cmax, cden, cnum, s, token_mask);
    if (rc) return rc;
    rc = launch_prefix(cmax, cden, cnum, B * H, NC, M, Dv, m0, d0, u0, m_fin, d_fin, u_fin, s);
    if (rc) return rc;
    return launch_output(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, chunk, cmax, cden,
                         cnum, Y, out_dtype, nullptr, s, token_mask, alpha_ws, redo, 0.0f, true);
}

// ---------------------------------------------------------------------------
// flare_ar_forward_noalloc: flare_ar_forward_masked on a fixed device scratch
// array instead of a caller workspace, for callers that cannot allocate.
// ---------------------------------------------------------------------------
}  // extern "C"

namespace flare {
// The workspace of flare_ar_forward_noalloc: chunk summaries, the output kernel's
// redo flags and (separate decoder tensors) the decoder softmax.  One copy per
// GPU, held until the process ends; every call on a GPU shares it.
constexpr size_t kScratchBytes = (size_t)64 << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
// Per device: the device address of `scratch`, and the order of the calls that use it
// (an event recorded after the last call's kernels, on the stream they ran on).
struct ScratchSlot {
    void* ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool pending = false;
};
static ScratchSlot g_scratch[kMaxDevices];
// Held from the device lookup to the end of a call's enqueue: calls from several host
// threads enqueue one after the other, so the event order below is the call order.
static std::mutex g_scratch_mu;

// The current device's slot, set up once per device (symbol address, order event).
static int scratch_slot(ScratchSlot** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("ar_forward_noalloc: no usable current device");
        return FLARE_ERR_LAUNCH;
    }
    ScratchSlot& sl = g_scratch[dev];
    if (sl.ptr == nullptr) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("ar_forward_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return FLARE_ERR_LAUNCH;
        }
        e = hipEventCreateWithFlags(&sl.done, hipEventDisableTiming);
        if (e != hipSuccess) {
            set_error("ar_forward_noalloc: hipEventCreateWithFlags failed: %s", hipGetErrorString(e));
            return FLARE_ERR_LAUNCH;
        }
        sl.ptr = p;
    }
    *out = &sl;
    return FLARE_OK;
}
}  // namespace flare

extern "C" {

size_t flare_ar_forward_noalloc_max_bytes(void) { return flare::kScratchBytes; }

int flare_ar_forward_noalloc(const void* Q, const void* K, const void* V, const void* Qdec,
                             const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                             int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                             const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                             void* Y, int out_dtype, const int32_t* token_mask, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y, "ar_forward_noalloc: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0,
                  "ar_forward_noalloc: sizes must be positive");
    if (chunk <= 0) chunk = default_chunk(B, N, H, M, Dv);
    // the separate-decoder workspace when it fits (MFMA path), else the plain one
    size_t bytes = flare_ar_forward_workspace_size(B, N, H, M, Dv, chunk);
    FLARE_REQUIRE(bytes <= kScratchBytes,
                  "ar_forward_noalloc: needs %zu bytes of scratch, the maximum is %zu "
                  "(B*H*ceil(N/chunk)*M*(2+Dv)*4 bytes of chunk summaries)",
                  bytes, kScratchBytes);
    if (Qdec || Kdec) {
        const size_t sep = flare_ar_forward_workspace_size_sep(B, N, H, M, Dv, chunk);
        if (sep <= kScratchBytes) bytes = sep;
    }
    std::lock_guard<std::mutex> lock(flare::g_scratch_mu);
    flare::ScratchSlot* sl = nullptr;
    int rc = flare::scratch_slot(&sl);
    if (rc) return rc;
    // Calls share the scratch array: one enqueued on another stream than the previous
    // call first waits for that call's kernels (same-stream calls are in stream order).
    // Under graph capture the order is the graph's; a replay that overlaps a call on
    // another stream is not ordered by this.
    hipStream_t st = (hipStream_t)stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    FLARE_REQUIRE(hipStreamIsCapturing(st, &cap) == hipSuccess, "ar_forward_noalloc: hipStreamIsCapturing failed");
    const bool eager = cap == hipStreamCaptureStatusNone;
    if (eager && sl->pending && sl->last != st)
        FLARE_REQUIRE(hipStreamWaitEvent(st, sl->done, 0) == hipSuccess, "ar_forward_noalloc: hipStreamWaitEvent failed");
    rc = flare_ar_forward_masked(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, chunk, m0, d0, u0, m_fin,
                                 d_fin, u_fin, Y, out_dtype, token_mask, sl->ptr, bytes, stream);
    if (rc == FLARE_OK && eager) {
        FLARE_REQUIRE(hipEventRecord(sl->done, st) == hipSuccess, "ar_forward_noalloc: hipEventRecord failed");
        sl->last = st;
        sl->pending = true;
    }
    return rc;
}

}  // extern "C"
