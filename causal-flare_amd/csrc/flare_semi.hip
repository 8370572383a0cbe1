// flare_semi.hip -- block-causal (semi-autoregressive) FLARE forward, scalar-fp32 kernels.
//
// Structure of causal_flare/semi_autoregressive/training.py (and the fp32
// restatement in semi_autoregressive/reference.py:308-536):
//   1. per-block (max, den, num) summaries -- the chunk_prepare kernel of
//      flare_ar.hip with chunk = block               (training.py:540-841)
//   2. semi_scan_z_kernel: inclusive scan over blocks, LSE_enc and the
//      normalised z_block = num * exp(max - LSE_enc)  (training.py:843-951)
//   3. semi_output_kernel: per token, softmax over latents of the decoder
//      scores and y = sum_m alpha_m z_block[m]        (training.py:1113-1399)
// z_block stays fp32 here (the reference stores it in V.dtype).
#include "flare_common.h"
#include "flare_internal.h"

namespace flare {

constexpr int kSemiNT = 256;
constexpr int kSemiCols = 4;

// grid = B*H*M workgroups of one wavefront; in place: num becomes z.  The scan starts
// from the cached state (m0, d0, u0) when given (earlier blocks: max, den and numerator
// relative to the max, inference.py:66-120) and leaves the state after the last block in
// (m_fin, d_fin, u_fin) when asked.
__global__ __launch_bounds__(64) void semi_scan_z_kernel(float* __restrict__ bmax,
                                                         float* __restrict__ bden,
                                                         float* __restrict__ bnum, int NB, int M,
                                                         int Dv, float* __restrict__ lse_enc,
                                                         const float* __restrict__ m0, const float* __restrict__ d0,
                                                         const float* __restrict__ u0, float* __restrict__ m_fin,
                                                         float* __restrict__ d_fin, float* __restrict__ u_fin) {
    const int row = blockIdx.x;
    const int bh = row / M, m = row % M;
    const int lane = threadIdx.x;
    float mc = kNegInf, dc = 0.0f;
    float uc[kSemiCols];
#pragma unroll
    for (int k = 0; k < kSemiCols; ++k) uc[k] = 0.0f;
    if (m0 != nullptr) {
        mc = m0[row];
        dc = d0[row];
#pragma unroll
        for (int k = 0; k < kSemiCols; ++k)
            if (lane + 64 * k < Dv) uc[k] = u0[(size_t)row * Dv + lane + 64 * k];
    }
    for (int g = 0; g < NB; ++g) {
        const size_t si = ((size_t)bh * NB + g) * M + m;
        const float bm = bmax[si], bd = bden[si];
        const float mn = fmaxf(mc, bm);
        const float rp = __expf(mc - mn), rb = __expf(bm - mn);
        dc = dc * rp + bd * rb;
        mc = mn;
        const float lse = __logf(fmaxf(dc, 1e-20f)) + mc;
        const float w = __expf(mc - lse);
        if (lane == 0 && lse_enc) lse_enc[si] = lse;
#pragma unroll
        for (int k = 0; k < kSemiCols; ++k) {
            const int col = lane + 64 * k;
            if (col < Dv) {
                uc[k] = uc[k] * rp + bnum[si * Dv + col] * rb;
                bnum[si * Dv + col] = uc[k] * w;
            }
        }
    }
    if (m_fin != nullptr) {
        if (lane == 0) {
            m_fin[row] = mc;
            d_fin[row] = dc;
        }
#pragma unroll
        for (int k = 0; k < kSemiCols; ++k)
            if (lane + 64 * k < Dv) u_fin[(size_t)row * Dv + lane + 64 * k] = uc[k];
    }
}

// grid = (NB, B*H, Dv/DT), 256 threads.  z_block[g][:, dt0:dt0+DT] is staged in
// LDS; each token tile computes decoder scores, their log-sum-exp, and the
// readout y[i][col] = sum_m exp(a[i][m] - lse[i]) z[m][col].
template <typename T>
__global__ __launch_bounds__(kSemiNT) void semi_output_kernel(
    const T* __restrict__ Qdec, const T* __restrict__ Kdec, int N, int H, int M, int Dk, int Dv,
    int DT, int TT, int block, float scale, const float* __restrict__ z,
    void* __restrict__ Y, int out_dtype, float* __restrict__ lse_dec) {
    extern __shared__ float smem[];
    float* zt = smem;                    // [M][DT]
    float* qt = zt + M * DT;             // [TT][Dk]
    float* at = qt + TT * Dk;            // [TT][M]
    float* lse = at + TT * M;            // [TT]
    const int g = blockIdx.x, bh = blockIdx.y, dt0 = blockIdx.z * DT;
    const int NB = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x;
    const T* kd_h = Kdec + (size_t)h * M * Dk;
    const float* zg = z + ((size_t)bh * NB + g) * M * Dv;
    for (int e = tid; e < M * DT; e += kSemiNT) zt[e] = zg[(size_t)(e / DT) * Dv + dt0 + e % DT];
    for (int t0 = g * block; t0 < (g + 1) * block; t0 += TT) {
        __syncthreads();
        for (int e = tid; e < TT * Dk; e += kSemiNT) {
            const int i = e / Dk, d = e % Dk;
            qt[e] = to_f32(Qdec[(((size_t)b * N + t0 + i) * H + h) * Dk + d]);
        }
        __syncthreads();
        for (int p = tid; p < TT * M; p += kSemiNT) {
            const int i = p / M, m = p % M;
            const T* krow = kd_h + (size_t)m * Dk;
            const float* qr = qt + i * Dk;
            float acc = 0.0f;
            for (int d = 0; d < Dk; ++d) acc += qr[d] * to_f32(krow[d]);
            at[p] = acc * scale;
        }
        __syncthreads();
        {
            const int w = tid >> 6, lane = tid & 63;
            for (int i = w; i < TT; i += kSemiNT / 64) {
                float mx = kNegInf;
                for (int m = lane; m < M; m += 64) mx = fmaxf(mx, at[i * M + m]);
                mx = wave_max(mx);
                float sm = 0.0f;
                for (int m = lane; m < M; m += 64) sm += __expf(at[i * M + m] - mx);
                sm = wave_sum(sm);
                if (lane == 0) lse[i] = mx + __logf(sm);
            }
        }
        __syncthreads();
        for (int p = tid; p < TT * M; p += kSemiNT) at[p] = __expf(at[p] - lse[p / M]);
        __syncthreads();
        for (int p = tid; p < TT * DT; p += kSemiNT) {
            const int i = p / DT, c = p % DT;
            float acc = 0.0f;
            for (int m = 0; m < M; ++m) acc += at[i * M + m] * zt[m * DT + c];
            const size_t yo = (((size_t)b * N + t0 + i) * H + h) * Dv + dt0 + c;
            if (out_dtype == FLARE_BF16) reinterpret_cast<__hip_bfloat16*>(Y)[yo] = __float2bfloat16(acc);
            else if (out_dtype == FLARE_F16) reinterpret_cast<__half*>(Y)[yo] = __float2half(acc);
            else reinterpret_cast<float*>(Y)[yo] = acc;
        }
        if (lse_dec && dt0 == 0)
            for (int i = tid; i < TT; i += kSemiNT) lse_dec[(size_t)bh * N + t0 + i] = lse[i];
    }
}

}  // namespace flare

using namespace flare;

namespace {
// per-block (max, den, num) summaries; chunks of the MFMA path are whole blocks,
// so their summaries fit in the same room
size_t semi_summary_bytes(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, int64_t block) {
    const int64_t NB = N / block;
    const size_t per = (size_t)B * H * NB * M;
    return (sizeof(float) * (per * 2 + per * Dv) + 3 * 256 + 255) & ~(size_t)255;
}
// fp16 decoder softmax [B*H, N, M], placed after the summaries
size_t semi_alpha_bytes(int64_t B, int64_t N, int64_t H, int64_t M) {
    return ((size_t)B * H * N * M * 2 + 255) & ~(size_t)255;
}
}  // namespace

extern "C" {

size_t flare_semi_ar_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                    int64_t block) {
    if (block <= 0) return 0;
    // blocks whose decoder softmax does not fit in LDS keep it in the workspace
    return semi_summary_bytes(B, N, H, M, Dv, block) +
           (semi_alpha_in_lds(M, block) ? 0 : semi_alpha_bytes(B, N, H, M));
}

size_t flare_semi_ar_workspace_size_sep(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                        int64_t block) {
    if (block <= 0) return 0;
    return semi_summary_bytes(B, N, H, M, Dv, block) + semi_alpha_bytes(B, N, H, M);
}

}  // extern "C"

// The block-causal forward with an optional cached state in (m0, d0, u0: the blocks
// before this call) and out (m_fin, d_fin, u_fin: after its last block).
static int semi_forward_impl(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                             int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                             float scale, int64_t block, const float* m0, const float* d0, const float* u0,
                             float* m_fin, float* d_fin, float* u_fin, void* Y, int out_dtype, float* lse_dec,
                             float* lse_enc, void* workspace, size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE(Q && K && V && Y, "semi_ar_forward: null pointer");
    FLARE_REQUIRE(B > 0 && N > 0 && H > 0 && M > 0 && Dk > 0 && Dv > 0, "semi_ar_forward: sizes must be positive");
    FLARE_REQUIRE(block > 0 && block % 16 == 0 && N % block == 0,
                  "semi_ar_forward: need block %% 16 == 0 and N %% block == 0 (N=%lld, block=%lld)",
                  (long long)N, (long long)block);
    FLARE_REQUIRE(Dv <= 64 * kSemiCols, "semi_ar_forward: Dv=%lld exceeds %d", (long long)Dv, 64 * kSemiCols);
    const size_t need = semi_summary_bytes(B, N, H, M, Dv, block);
    if (!workspace || workspace_bytes < need) {
        set_error("semi_ar_forward: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return FLARE_ERR_WORKSPACE;
    }
    const int64_t NB = N / block;
    const size_t per = (size_t)B * H * NB * M;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    char* ws = (char*)workspace;
    float* bmax = (float*)ws;
    float* bden = (float*)(ws + align(per * sizeof(float)));
    float* bnum = (float*)(ws + 2 * align(per * sizeof(float)));
    hipStream_t s = (hipStream_t)stream;
    const bool shared = Qdec == nullptr && Kdec == nullptr;
    // separate decoder tensors, and blocks whose softmax does not fit in LDS, take the
    // MFMA path when the workspace has room for the [B*H, N, M] softmax
    // (flare_semi_ar_workspace_size_sep)
    void* alpha_ws = nullptr;
    if (workspace_bytes >= need + semi_alpha_bytes(B, N, H, M)) alpha_ws = ws + need;
    if ((mfma_phase_mask() & 3) == 3 && (shared || alpha_ws) && (semi_alpha_in_lds(M, block) || alpha_ws) &&
        mfma_semi_supported(dtype, out_dtype, true, M, Dk, Dv, block) && mfma_prepare_supported(dtype, M, Dk, Dv)) {
        if (!shared) {
            const int rc = launch_decoder_alpha(Qdec ? Qdec : K, Kdec ? Kdec : Q, B, N, H, M, Dk, scale, nullptr,
                                                alpha_ws, lse_dec, dtype == FLARE_F16, s);
            if (rc) return rc;
        }
        // Chunks of whole blocks: prefix of every chunk from phases 1-2, then the
        // block-causal MFMA readout.  The summaries fit in the workspace since
        // chunks are never shorter than blocks.
        // One round of chunk workgroups, whole blocks each: ~512 (two per compute unit),
        // or ~768 where three fit (M = 128, Dv = 64 with the block's softmax in LDS for
        // blocks up to 64, or in the workspace: <= 168 VGPRs and <= 53 KiB of LDS).
        // Measured on config 5 (B*H = 32) at two per CU, 2048 / 1024 / 512 / 256
        // workgroups take 151 / 126 / 119 / 168 us, the shorter chunks paying in summary
        // traffic; three per CU over 704 workgroups: 104 us.
        const bool three = M == 128 && Dv == 64 && block != 128;
        const int64_t target = ((three ? 768 : 512) + B * H - 1) / (B * H);
        int64_t chunk = (N + target - 1) / target;
        if (chunk > 2048) chunk = 2048;
        chunk = ((chunk + block - 1) / block) * block;
        if (chunk > N) chunk = N;
        const int64_t NC = (N + chunk - 1) / chunk;
        int rc = launch_prepare_mfma(Q, K, V, B, N, H, M, Dk, scale, chunk, bmax, bden, bnum, dtype == FLARE_F16, s);
        if (rc) return rc;
        rc = launch_prefix_public(bmax, bden, bnum, B * H, NC, M, Dv, m0, d0, u0, m_fin, d_fin, u_fin, s);
        if (rc) return rc;
        return launch_semi_output_mfma(Q, K, V, B, N, H, M, Dk, scale, chunk, block, bmax, bden, bnum, Y,
                                       out_dtype, lse_dec, lse_enc, alpha_ws, !shared, dtype == FLARE_F16, s);
    }
    int rc = launch_prepare_public(Q, K, V, dtype, B, N, H, M, Dk, Dv, scale, block, bmax, bden, bnum, s);
    if (rc) return rc;
    hipLaunchKernelGGL(semi_scan_z_kernel, dim3((unsigned)(B * H * M)), dim3(64), 0, s, bmax, bden,
                       bnum, (int)NB, (int)M, (int)Dv, lse_enc, m0, d0, u0, m_fin, d_fin, u_fin);
    rc = check_launch("semi_scan_z_kernel");
    if (rc) return rc;
    // Value tile so that z_block[g][:, tile] fits in 32 KB of LDS.
    int DT = 0;
    for (int dt = 128; dt >= 16; dt >>= 1)
        if (Dv % dt == 0 && M * dt <= 8192) { DT = dt; break; }
    FLARE_REQUIRE(DT > 0, "semi_ar_forward: unsupported M=%lld Dv=%lld", (long long)M, (long long)Dv);
    const int TT = 16;
    const size_t sm = sizeof(float) * ((size_t)M * DT + TT * Dk + TT * M + TT);
    FLARE_REQUIRE(sm <= 64 * 1024, "semi_ar_forward: shape too large for LDS");
    const void* qd = Qdec ? Qdec : K;
    const void* kd = Kdec ? Kdec : Q;
    dim3 grid((unsigned)NB, (unsigned)(B * H), (unsigned)(Dv / DT));
#define FLARE_SEMI(TY)                                                                          \
    hipLaunchKernelGGL(semi_output_kernel<TY>, grid, dim3(kSemiNT), sm, s, (const TY*)qd,          \
                       (const TY*)kd, (int)N, (int)H, (int)M, (int)Dk, (int)Dv, DT, TT,           \
                       (int)block, scale, bnum, Y, out_dtype, lse_dec)
    if (dtype == FLARE_BF16) FLARE_SEMI(__hip_bfloat16);
    else if (dtype == FLARE_F16) FLARE_SEMI(__half);
    else FLARE_SEMI(float);
#undef FLARE_SEMI
    return check_launch("semi_output_kernel");
}

extern "C" {

int flare_semi_ar_forward(const void* Q, const void* K, const void* V, const void* Qdec,
                          const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H,
                          int64_t M, int64_t Dk, int64_t Dv, float scale, int64_t block,
                          void* Y, int out_dtype, float* lse_dec, float* lse_enc,
                          void* workspace, size_t workspace_bytes, void* stream) {
    return semi_forward_impl(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, block, nullptr, nullptr,
                             nullptr, nullptr, nullptr, nullptr, Y, out_dtype, lse_dec, lse_enc, workspace,
                             workspace_bytes, stream);
}

int flare_semi_ar_forward_state(const void* Q, const void* K, const void* V, const void* Qdec,
                                const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                                int64_t Dk, int64_t Dv, float scale, int64_t block, const float* m0,
                                const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                                void* Y, int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    FLARE_REQUIRE((m0 == nullptr) == (d0 == nullptr) && (m0 == nullptr) == (u0 == nullptr),
                  "semi_ar_forward_state: give all of m0, d0, u0 or none");
    FLARE_REQUIRE((m_fin == nullptr) == (d_fin == nullptr) && (m_fin == nullptr) == (u_fin == nullptr),
                  "semi_ar_forward_state: give all of m_fin, d_fin, u_fin or none");
    return semi_forward_impl(Q, K, V, Qdec, Kdec, dtype, B, N, H, M, Dk, Dv, scale, block, m0, d0, u0, m_fin,
                             d_fin, u_fin, Y, out_dtype, nullptr, nullptr, workspace, workspace_bytes, stream);
}

}  // extern "C"
