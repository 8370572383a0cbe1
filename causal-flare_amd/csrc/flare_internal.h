// flare_internal.h -- host-side declarations shared between the library's translation units.
#pragma once
#include <stdint.h>

namespace flare {
int64_t default_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv);
}

#include <hip/hip_runtime.h>
#include <stdlib.h>

namespace flare {
// bf16 inputs, or fp16 inputs on the producer / consumer kernels (M in {128, 256});
// the launchers below take f16in = (dtype == FLARE_F16)
bool mfma_prepare_supported(int dtype, int64_t M, int64_t Dk, int64_t Dv);
bool mfma_output_supported(int dtype, int out_dtype, bool shared, int64_t M, int64_t Dk, int64_t Dv);
int launch_prepare_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                        int64_t M, int64_t D, float scale, int64_t chunk, float* cmax, float* cden,
                        float* cnum, bool f16in, hipStream_t stream);
int launch_output_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                       int64_t M, int64_t D, float scale, int64_t chunk, const float* pmax,
                       const float* pden, const float* pnum, void* Y, int out_dtype, const int32_t* tmask,
                       bool f16in, int* redo, hipStream_t stream, bool record = false);

// FLARE_DISABLE_MFMA=1 routes every shape to the scalar-fp32 kernels (A/B checks);
// FLARE_MFMA_PHASES=<bits> keeps the MFMA kernel only for phase 1 (bit 0) and/or
// phase 3 (bit 1).  Both are read once per process.
inline int mfma_phase_mask() {
    static const int mask = [] {
        const char* e = getenv("FLARE_DISABLE_MFMA");
        if (e && e[0] == '1') return 0;
        const char* p = getenv("FLARE_MFMA_PHASES");
        return p ? atoi(p) : 3;
    }();
    return mask;
}
inline bool mfma_enabled() { return mfma_phase_mask() != 0; }
// FLARE_OUTPUT_KERNEL=single selects the single-role phase-3 MFMA kernel
// instead of the producer/consumer one (A/B checks).  Read once per process.
inline bool output_pc_enabled() {
    static const bool on = [] {
        const char* e = getenv("FLARE_OUTPUT_KERNEL");
        return !(e && e[0] == 's');
    }();
    return on;
}
// FLARE_OUTPUT_KERNEL=pc keeps the earlier producer / consumer phase-3 kernel
// (partial G summed by the consumers) instead of chunk_output_tr (A/B checks).
inline bool output_tr_enabled() {
    static const bool on = [] {
        const char* e = getenv("FLARE_OUTPUT_KERNEL");
        return !(e && e[0] == 'p');
    }();
    return on;
}
int launch_output_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* pmax, const float* pden,
                     const float* pnum, void* Y, int out_dtype, const int32_t* tmask, const void* alpha,
                     bool f16in, int* redo, int spin_limit, hipStream_t stream, bool record = false,
                     float power = 0.0f);
// chunk_output_tr replays its own flagged chunks (shared decoder weights; the shapes whose
// threads make whole replay slices): the caller then launches no replay kernel.
bool output_tr_replays_inline(int64_t M, int64_t D, bool sep);
// Meetings of chunk_output_tr that gave up waiting (optionally reset to 0).
int meet_timeouts_tr(hipStream_t stream, unsigned int* count, bool reset);
int launch_prepare_pc(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                      int64_t D, float scale, int64_t chunk, float* cmax, float* cden, float* cnum,
                      const int32_t* tmask, bool f16in, hipStream_t stream);
// Phase 1 with wave-private latents (chunk_prepare_tr); FLARE_PREPARE_KERNEL=pc keeps
// the producer / consumer kernel chunk_prepare_pc instead (A/B checks).
// power > 0: the stablemax encoder (no token mask).
int launch_prepare_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                      int64_t D, float scale, int64_t chunk, float* cmax, float* cden, float* cnum,
                      const int32_t* tmask, bool f16in, hipStream_t stream, float power = 0.0f);
// Register, scratch and LDS use of the kernels the forward launches (profile=True).
// The running state at the start of every 32-token chunk, [B*H, ceil(N/32), M(, D)]
// (max in natural-log units, den and num relative to it), from one pass over chunks of
// `chunk` tokens (a multiple of 64) that start from their exclusive prefixes s0*.  The
// shapes of launch_prepare_tr.
int launch_states_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* s0max, const float* s0den,
                     const float* s0num, float* smax, float* sden, float* snum, bool f16in, hipStream_t stream,
                     float power);
int prepare_tr_attributes(int64_t M, int64_t D, bool f16in, hipFuncAttributes* attr, int* threads);
int output_tr_attributes(int64_t M, int64_t D, bool sep, bool f16in, hipFuncAttributes* attr, int* threads);
inline bool prepare_tr_enabled() {
    static const bool on = [] {
        const char* e = getenv("FLARE_PREPARE_KERNEL");
        return !(e && e[0] == 'p');
    }();
    return on;
}
// alpha: NULL for shared decoder weights; else the decoder softmax [B*H, N, M]
// (fp16) written by launch_decoder_alpha, for separate Qdec / Kdec.
// redo: NULL, or [B*H, NC] ints; the kernel writes kRedoWhole for a chunk in which
// some latent's reference jumped past kJumpMax within a subtile (else 0), and the
// caller replays those chunks with the tokenwise fp32 kernel.  record: the prefix
// arrays are the caller's own scratch, so chunk_output_tr (shared weights) may write
// the state at the first flagged subtile over a chunk's prefix slot and flag only
// the subtiles to replay (redo_narrow).
int launch_output_pc(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* pmax, const float* pden,
                     const float* pnum, void* Y, int out_dtype, const int32_t* tmask, const void* alpha,
                     bool f16in, int* redo, hipStream_t stream, bool record = false, float power = 0.0f);
int launch_decoder_alpha(const void* Qd, const void* Kd, int64_t B, int64_t N, int64_t H, int64_t M, int64_t D,
                         float scale, const int32_t* tmask, void* alpha, float* lse, bool f16in, hipStream_t stream);
}  // namespace flare

namespace flare {
bool mfma_semi_supported(int dtype, int out_dtype, bool shared, int64_t M, int64_t Dk, int64_t Dv, int64_t block);
int launch_semi_output_mfma(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H,
                            int64_t M, int64_t D, float scale, int64_t chunk, int64_t block,
                            const float* pmax, const float* pden, const float* pnum, void* Y, int out_dtype,
                            float* lse_dec, float* lse_enc, void* alpha, bool sep, bool f16in, hipStream_t stream);
// true when the semi MFMA readout keeps a block's decoder softmax in LDS; otherwise
// it needs a [B*H, N, M] fp16 alpha buffer in the workspace
bool semi_alpha_in_lds(int64_t M, int64_t block);
// tokens per partial sum of the backward's dQ / dK_dec contraction
constexpr int kBwdGroup = 512;
// bf16 MFMA form of the backward's dK / dQ_dec contraction (flare_bwd_mfma.hip)
bool bwd_dk_mfma_supported(int64_t M, int64_t Dk);
int launch_dk_mfma(const void* Q, const void* Kd, bool sep_q, bool sep_k, int64_t B, int64_t N, int64_t H,
                   int64_t M, int64_t Dk, float scale, const float* DS, const float* AL, const float* C,
                   const float* gy, bool cgz, bool dsum, void* dK, void* dQd, bool f16in, hipStream_t st);
bool bwd_summary_mfma_supported(int64_t M, int64_t Dv);
int launch_summary_mfma(const void* dY, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, const float* L,
                        const float* LA, const float* C, float* a_out, float* b_out, bool f16in, hipStream_t st);
// block sums dz_g, Yb_g of the block-causal backward (M and Dv as bwd_summary_mfma_supported)
int launch_semi_dz_mfma(const void* dY, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv, int64_t blk,
                        const float* AL, const float* C, float* X, float* Yb, bool f16in, hipStream_t st);
bool bwd_dq_mfma_supported(int64_t M, int64_t Dk);
int launch_dq_mfma(const void* K, const void* Qd, bool sep_q, bool sep_k, int64_t B, int64_t N, int64_t H,
                   int64_t M, int64_t Dk, const float* DS, const float* AL, const float* C, const float* gy,
                   bool cgz, bool dsum, float* P1, float* P2, bool f16in, hipStream_t st);
int launch_prepare_public(const void* Q, const void* K, const void* V, int dtype, int64_t B,
                          int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                          int64_t chunk, float* cmax, float* cden, float* cnum, hipStream_t stream,
                          float power = 0.0f);
int launch_prefix_public(float* cmax, float* cden, float* cnum, int64_t BH, int64_t NC, int64_t M, int64_t Dv,
                         const float* m0, const float* d0, const float* u0, float* m_fin, float* d_fin,
                         float* u_fin, hipStream_t stream);
}  // namespace flare

namespace flare {
// Shared by the token-causal and block-causal backward (flare_ar_bwd.hip).
size_t bwd_partial_floats(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk);
int launch_bwd_gy(const void* dY, const void* Y, int dtype, int64_t B, int64_t N, int64_t H, int64_t Dv, float* gy,
                  hipStream_t stream);
int launch_bwd_contract(const void* Q, const void* K, const void* Qdec, const void* Kdec, int dtype, int64_t B,
                        int64_t N, int64_t H, int64_t M, int64_t Dk, float scale, const float* DS, const float* AL,
                        const float* C, const float* gy, bool cgz, bool dsum, void* dQ, void* dK, void* dQdec,
                        void* dKdec, float* P1, float* P2, hipStream_t stream);
// The token-causal backward (shapes as ar_backward_supported).  power > 0: the
// stablemax encoder weight s(a) in place of e^a (the decoder stays a softmax).
bool ar_backward_supported(int64_t M, int64_t Dk, int64_t Dv);
size_t ar_backward_workspace(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv);
int ar_backward_run(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec, int dtype,
                    int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale, const void* Y,
                    const void* dY, void* dQ, void* dK, void* dV, void* dQdec, void* dKdec, void* workspace,
                    size_t workspace_bytes, hipStream_t stream, float power);
}  // namespace flare
