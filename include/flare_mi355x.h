/*
 * flare_mi355x.h -- C ABI of the MI355X (gfx950) causal FLARE forward library.
 *
 * Every entry point takes plain device pointers, sizes, a scale and a HIP
 * stream (passed as void*; NULL = the legacy default stream), enqueues its
 * kernels on that stream and returns without synchronising.  The return value
 * is FLARE_OK or a negative FLARE_ERR_* code; flare_last_error() then gives a
 * human-readable message (thread-local).
 *
 * Tensor layouts are the reference's (vpuri3/causal-flare), contiguous:
 *   Q     [H, M, Dk]      latent queries (encoder)
 *   K     [B, N, H, Dk]   keys        V [B, N, H, Dv] values
 *   Qdec  [B, N, H, Dk]   decoder queries (NULL -> K, the reference default)
 *   Kdec  [H, M, Dk]      decoder keys    (NULL -> Q, the reference default)
 *   Y     [B, N, H, Dv]   output, element type `out_dtype`
 *   state m, d [B, H, M] and u [B, H, M, Dv], always fp32
 * `dtype` is the element type of Q, K, V, Qdec and Kdec (one type for all).
 * Chunk summaries (chunk_max/den [B*H, NC, M], chunk_num [B*H, NC, M, Dv])
 * are fp32 and are owned by the caller.
 *
 * Each declaration names the reference interface it replaces (path:line in
 * vpuri3/causal-flare).
 */
#ifndef FLARE_MI355X_H
#define FLARE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum flare_dtype { FLARE_F32 = 0, FLARE_BF16 = 1, FLARE_F16 = 2 };

enum flare_status {
    FLARE_OK = 0,
    FLARE_ERR_INVALID = -1,     /* bad argument / unsupported shape */
    FLARE_ERR_LAUNCH = -2,      /* HIP launch or runtime error */
    FLARE_ERR_WORKSPACE = -3    /* workspace too small */
};

/* Library identification and the message of the last failed call. */
int flare_abi_version(void);
const char* flare_last_error(void);

/*
 * Phase 1 of the chunked forward: per chunk of `chunk` tokens and per latent,
 * the max score, softmax denominator and softmax-weighted value sum.
 * Replaces the Triton kernel flare_chunk_prepare
 * (causal_flare/autoregressive/training.py:914-1018) and its launcher
 * _run_chunked_prepare_phase (training.py:489-557).  NC = ceil(N / chunk).
 */
int flare_chunk_prepare(const void* Q, const void* K, const void* V, int dtype, int64_t B,
                        int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv, float scale,
                        int64_t chunk, float* chunk_max, float* chunk_den, float* chunk_num,
                        void* stream);

/*
 * Phase 2: in-place exclusive online-softmax scan over the NC chunk summaries
 * of each (b,h), optionally starting from an initial cached state (m0/d0/u0,
 * any may be NULL only if all are NULL) and optionally writing the inclusive
 * final state (m_fin/d_fin/u_fin, all or none).
 * Replaces flare_chunk_prefix (training.py:1021-1103) and, for prefill, the
 * torch merges of the initial and final states
 * (causal_flare/autoregressive/inference.py:753-814, _merge_flare_stats :194-228).
 */
int flare_chunk_prefix(float* chunk_max, float* chunk_den, float* chunk_num, int64_t BH,
                       int64_t NC, int64_t M, int64_t Dv, const float* m0, const float* d0,
                       const float* u0, float* m_fin, float* d_fin, float* u_fin, void* stream);

/*
 * Phase 3: per chunk, replay the token recurrence from the chunk's prefix
 * state and emit y_t = sum_m softmax_m(a_t)[m] * z_t[m].  Optionally writes
 * LSE_dec [B*H, N] (logsumexp_m of the decoder scores; may be NULL).
 * Replaces flare_chunk_decoder_lse + flare_chunk_fwd
 * (training.py:1106-1392) and _run_chunked_output_phase (training.py:615-728).
 */
int flare_chunk_output(const void* Q, const void* K, const void* V, const void* Qdec,
                       const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                       int64_t Dk, int64_t Dv, float scale, int64_t chunk,
                       const float* prefix_max, const float* prefix_den, const float* prefix_num,
                       void* Y, int out_dtype, float* lse_dec, void* stream);

/* Bytes of workspace flare_ar_forward needs: the fp32 chunk summaries and one
 * int per (b*h, chunk) on which the MFMA output kernel marks the chunks it
 * hands to the tokenwise fp32 replay (a latent whose score jumps more than
 * ~66 nats above its running max within one 32-token subtile). */
size_t flare_ar_forward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                       int64_t chunk);
/*
 * Workspace for separate decoder tensors (Qdec / Kdec given): the chunk
 * summaries plus the decoder softmax [B*H, N, M] (fp16), which the bf16 MFMA
 * path computes first, as the reference's flare_chunk_decoder_lse does
 * (training.py:1106-1188).  Given a smaller workspace (at least
 * flare_ar_forward_workspace_size), flare_ar_forward runs separate decoder
 * tensors on the scalar-fp32 kernels.
 */
size_t flare_ar_forward_workspace_size_sep(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                           int64_t chunk);

/*
 * Whole chunked forward / prefill: phases 1-3 on one stream.  `chunk` <= 0
 * selects the library's own chunk length.  m0/d0/u0 (initial state) and
 * m_fin/d_fin/u_fin (final state) are optional as in flare_chunk_prefix.
 * Replaces AutoRegressiveFLARE.forward (training.py:731-905) and
 * flare_autoregressive_prefill_triton's unmasked path (inference.py:697-820).
 */
int flare_ar_forward(const void* Q, const void* K, const void* V, const void* Qdec,
                     const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                     const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                     void* Y, int out_dtype, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * flare_ar_forward with a per-token mask: token_mask [B, N] (int32, nonzero =
 * keep) may be NULL.  A masked token adds nothing to the latent state and gets
 * y = 0, the semantics of the reference's masked prefill, which runs the decode
 * step token by token with attention_mask[:, t] (inference.py:663-695, masked
 * decode rows at :395-397 and :476-478); here the chunked kernels apply it.
 */
int flare_ar_forward_masked(const void* Q, const void* K, const void* V, const void* Qdec,
                            const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                            int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                            const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                            void* Y, int out_dtype, const int32_t* token_mask, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Stablemax FLARE forward, the non-write-gated path of
 * flare_autoregressive_stablemax_triton (autoregressive/stablemax_triton.py:
 * 1707-2055, 2423-2468; PyTorch form stablemax.py:482-635):
 *   y_t = sum_m softmax_m(scale qd_t . kd_m) *
 *         (sum_{tau<=t} s(a_tau,m) v_tau) / (sum_{tau<=t} s(a_tau,m)),
 *   a_tau,m = scale k_tau . q_m,  s(x) = (1+x)^power (x >= 0), (1-x)^-power (x < 0).
 * Qdec / Kdec may be NULL (K and Q).  Runs the fp32 chunk kernels with the
 * stablemax encoder; workspace of flare_ar_forward_workspace_size bytes.
 */
int flare_stablemax_forward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                            int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                            float scale, int64_t chunk, float power, void* Y, int out_dtype, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Stablemax FLARE backward, replacing FLAREAutoregressiveStablemaxTriton.backward
 * (autoregressive/stablemax_triton.py:1981-2420): gradients of sum(Y * dY) with
 * respect to Q, K, V and the separate decoder tensors.  Inputs as the forward's
 * (compute dtype `dtype`; Qdec / Kdec NULL when they are K / Q, whose gradients
 * then carry the decoder share), Y and dY [B, N, H, Dv] in `dtype`; dQ, dK, dV,
 * dQdec, dKdec in `dtype` (dQdec / dKdec NULL exactly when Qdec / Kdec are).
 * M <= 256, Dk, Dv <= 256.  Workspace of flare_stablemax_backward_workspace_size
 * bytes (separate_decoder: Qdec != NULL), 256-byte aligned.  fp32 accumulation;
 * M, Dk, Dv multiples of 16 run flare_ar_backward's kernels (bf16 / fp16
 * contractions on MFMA).
 */
size_t flare_stablemax_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk,
                                               int64_t Dv, int separate_decoder);
int flare_stablemax_backward(const void* Q, const void* K, const void* V, const void* Qdec, const void* Kdec,
                             int dtype, int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk, int64_t Dv,
                             float scale, float power, const void* Y, const void* dY, void* dQ, void* dK,
                             void* dV, void* dQdec, void* dKdec, void* workspace, size_t workspace_bytes,
                             void* stream);

/* The chunk length flare_ar_forward uses when called with chunk <= 0. */
int64_t flare_ar_default_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv);

/*
 * Resources of a forward kernel this library launches for the given call
 * (phase 0: chunk summaries, 1: prefix scan, 2: token replay), for the
 * profile=True record: out[0] waves per workgroup, out[1] VGPRs per lane,
 * out[2] scratch (spill) bytes per lane, out[3] LDS bytes per workgroup.
 * Replaces the reference's _maybe_record_kernel_resource
 * (autoregressive/training.py:4-18), which reads the same facts from Triton's
 * compiled kernels.  Phases 0 and 2 answer FLARE_ERR_INVALID when the call
 * would run another kernel than chunk_prepare_tr / chunk_output_tr.
 */
int flare_forward_kernel_resources(int dtype, int64_t M, int64_t Dk, int64_t Dv, int shared, int64_t chunk,
                                   int phase, int32_t* out);

/*
 * Backward of the chunked forward (flare_ar_forward without initial state or
 * mask): from the forward's inputs, its output Y and dY (all in `dtype`,
 * Y and dY [B, N, H, Dv]) write dQ [H, M, Dk], dK [B, N, H, Dk], dV [B, N, H, Dv]
 * and, when Qdec / Kdec are given, dQdec [B, N, H, Dk] / dKdec [H, M, Dk], all
 * in `dtype`.  A NULL Qdec (Kdec) means the decoder uses K (Q) and its gradient
 * is folded into dK (dQ).  Requires M, Dk, Dv multiples of 16 with M <= 256,
 * Dk <= 256, Dv <= 512.  Replaces _chunked_flare_lse_backward_impl
 * (training.py:4369-4918), the autograd backward of AutoRegressiveFLARE.
 */
size_t flare_ar_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk,
                                        int64_t Dv);
int flare_ar_backward(const void* Q, const void* K, const void* V, const void* Qdec,
                      const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                      int64_t Dk, int64_t Dv, float scale, const void* Y, const void* dY, void* dQ,
                      void* dK, void* dV, void* dQdec, void* dKdec, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * One recurrent decode step for every (b,h): K, V (and Qdec) are [B, H, D];
 * the fp32 state m/d/u is updated in place; y [B, H, Dv] is written in
 * `out_dtype`.  mask [B] (int32, nonzero = valid) may be NULL; an invalid
 * batch row leaves its state unchanged and gets y = 0.
 * Replaces flare_recurrent_step_kernel + flare_autoregressive_decode_triton
 * (inference.py:358-621).
 */
int flare_decode_step(const void* Q, const void* K, const void* V, const void* Qdec,
                      const void* Kdec, const int32_t* mask, int dtype, int64_t B, int64_t H,
                      int64_t M, int64_t Dk, int64_t Dv, float scale, float* m, float* d,
                      float* u, void* y, int out_dtype, void* stream);

/*
 * Block-causal (semi-autoregressive) forward: token t of block g attends to
 * every token of blocks <= g.  Writes Y, and optionally LSE_dec [B*H, N] and
 * LSE_enc [B*H, NB, M] (NB = N / block).  Requires N % block == 0 and
 * block % 16 == 0 (validated on the host side as in the reference).
 * Replaces _semi_autoregressive_forward_triton and its kernels
 * (causal_flare/semi_autoregressive/training.py:540-1399, 1836-1961).
 */
/* Workspace of flare_semi_ar_forward: per-block summaries, plus an fp16
 * [B*H, N, M] buffer for the decoder softmax when the block is too large for
 * the MFMA readout to keep it in LDS. */
size_t flare_semi_ar_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                    int64_t block);
/*
 * Backward of flare_semi_ar_forward: from the inputs, Y and dY (all in `dtype`)
 * write dQ, dK, dV and, when Qdec / Kdec are given, dQdec / dKdec, as
 * flare_ar_backward does.  Requires block % 16 == 0, N % block == 0 and M, Dk,
 * Dv multiples of 16 with M <= 256, Dk <= 256, Dv <= 512.  Replaces
 * _semi_autoregressive_backward_impl (causal_flare/semi_autoregressive/
 * training.py:3768-3988), the autograd backward of SemiAutoRegressiveFLARE.
 */
size_t flare_semi_ar_backward_workspace_size(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dk,
                                             int64_t Dv, int64_t block);
int flare_semi_ar_backward(const void* Q, const void* K, const void* V, const void* Qdec,
                           const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                           int64_t Dk, int64_t Dv, float scale, int64_t block, const void* Y,
                           const void* dY, void* dQ, void* dK, void* dV, void* dQdec, void* dKdec,
                           void* workspace, size_t workspace_bytes, void* stream);

/* As flare_ar_forward_workspace_size_sep: room for the decoder softmax of separate
 * decoder tensors, which then run on the bf16 MFMA path. */
size_t flare_semi_ar_workspace_size_sep(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv,
                                        int64_t block);
int flare_semi_ar_forward(const void* Q, const void* K, const void* V, const void* Qdec,
                          const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H,
                          int64_t M, int64_t Dk, int64_t Dv, float scale, int64_t block,
                          void* Y, int out_dtype, float* lse_dec, float* lse_enc,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Semi-autoregressive cached prefill / block decode: flare_semi_ar_forward over N
 * tokens that continue a cached latent state.  m0 / d0 [B, H, M] and u0 [B, H, M, Dv]
 * (fp32; all NULL for an empty cache) hold the earlier blocks as running max, den
 * and numerator relative to the max -- the layout of the autoregressive cache
 * (causal_flare/autoregressive/inference.py:66-120).  Every token of a block reads
 * the state after its whole block.  m_fin / d_fin / u_fin (all NULL, or all given;
 * they must not overlap m0 / d0 / u0) receive the state after the last block.  Same
 * requirements and workspace as flare_semi_ar_forward; no LSE outputs.  The
 * reference ships these entry points as stubs that raise NotImplementedError
 * (causal_flare/semi_autoregressive/inference.py:5-36,
 * flare_semi_autoregressive_prefill_trition / flare_semi_autoregressive_decode_trition).
 */
int flare_semi_ar_forward_state(const void* Q, const void* K, const void* V, const void* Qdec,
                                const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                                int64_t Dk, int64_t Dv, float scale, int64_t block, const float* m0,
                                const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                                void* Y, int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * flare_ar_forward_masked without a workspace argument: its chunk summaries, redo
 * flags and (separate decoder tensors) decoder softmax live in a fixed device
 * array of the library, one copy per GPU, held until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it calls no allocating routine.  A call whose workspace
 * (flare_ar_forward_workspace_size) exceeds flare_ar_forward_noalloc_max_bytes()
 * (64 MiB) returns FLARE_ERR_INVALID before launching anything; separate decoder
 * tensors use the MFMA path when flare_ar_forward_workspace_size_sep also fits,
 * else the scalar kernels.  Every call on a GPU shares its array.  Calls are
 * ordered on the device: a call enqueued on another stream than the previous
 * call's first waits for that call's kernels (an event recorded after them;
 * calls from several host threads enqueue under one lock).  Under HIP graph
 * capture this ordering is not recorded: a replay of a captured call that
 * overlaps another call on another stream races on the array.
 */
size_t flare_ar_forward_noalloc_max_bytes(void);
int flare_ar_forward_noalloc(const void* Q, const void* K, const void* V, const void* Qdec,
                             const void* Kdec, int dtype, int64_t B, int64_t N, int64_t H, int64_t M,
                             int64_t Dk, int64_t Dv, float scale, int64_t chunk, const float* m0,
                             const float* d0, const float* u0, float* m_fin, float* d_fin, float* u_fin,
                             void* Y, int out_dtype, const int32_t* token_mask, void* stream);

/*
 * Diagnostics (no counterpart in the reference, whose Triton kernels have no
 * bounded waits).  The producer waves of the bf16/fp16 output kernel meet once
 * per 32-token subtile at a workgroup-local counter; the wait is bounded.  A
 * wait that gives up flags its chunk for the tokenwise fp32 replay (so the
 * output stays correct) and increments a device-wide fault counter.
 * flare_device_faults synchronises `stream`, reads the counter of the current
 * device into *count and, if `reset` is nonzero, sets it to 0.
 * flare_set_meet_spin_limit sets the number of sleeps (about 64 clocks each)
 * before a wait gives up, for kernels launched afterwards by this process
 * (default 1 << 20, about 28 ms); tests use 0 to force the fault path.
 */
int flare_device_faults(void* stream, uint32_t* count, int reset);
int flare_set_meet_spin_limit(int limit);

#ifdef __cplusplus
}
#endif

#endif /* FLARE_MI355X_H */
