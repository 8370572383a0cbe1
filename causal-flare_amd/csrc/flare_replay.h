// flare_replay.h -- the tokenwise fp32 replay of one chunk of the causal FLARE
// forward (phase 3 of the scalar kernels), shared by chunk_output_kernel (the
// scalar output kernel and the replay launch after an MFMA output kernel) and by
// chunk_output_tr, which replays its own flagged chunk in place.
#pragma once

#include "flare_common.h"

namespace flare {

constexpr int kNT = 256;        // threads per workgroup of the scalar kernels (4 wavefronts)

__device__ __forceinline__ void store_out(void* Y, size_t idx, float v, int out_dtype) {
    if (out_dtype == FLARE_BF16) reinterpret_cast<__hip_bfloat16*>(Y)[idx] = __float2bfloat16(v);
    else if (out_dtype == FLARE_F16) reinterpret_cast<__half*>(Y)[idx] = __float2half(v);
    else reinterpret_cast<float*>(Y)[idx] = v;
}

// ---------------------------------------------------------------------------
// Phase 3 (chunk_output_kernel: grid = (NC, B*H, Dv/DT), 256 threads; inside
// chunk_output_tr: one 256-thread slice per DT value columns).  Thread (col, rg) owns the
// numerator entries u[m][dt0+col] for m = rg, rg+R, ... (R = 256/DT) in
// registers; per-latent max/den live in LDS.  Tokens are processed in tiles
// of TT: scores and decoder log-sum-exps for the tile first, then the
// tokenwise recurrence and the readout, two barriers per token.
// ---------------------------------------------------------------------------
// The per-token factors gam / eta / wts come first (16-byte aligned) and are padded to
// Mp = R * ROWS latents (gam 1, eta and wts 0 past M): a thread's ROWS consecutive latents
// are then read four at a time with no bounds branch.  The token rows follow, also
// 16-byte aligned when Dk is a multiple of 4.
struct OutSmem {
    int TT, Dk, DT, M, R, Mp;
    bool shared;
    __host__ __device__ constexpr size_t floats() const {
        return (size_t)3 * Mp + (size_t)TT * Dk * (shared ? 1 : 2) + (size_t)TT * DT +
               (size_t)TT * M * (shared ? 1 : 2) + (size_t)2 * M + (size_t)R * DT + TT + 8;
    }
};

// 32 consecutive elements (16-byte aligned) to fp32 through 16-byte loads.
template <typename T>
__device__ __forceinline__ void load_row32(const T* p, float* out) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 x = reinterpret_cast<const float4*>(p)[j];
            out[4 * j] = x.x;
            out[4 * j + 1] = x.y;
            out[4 * j + 2] = x.z;
            out[4 * j + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 x = reinterpret_cast<const uint4*>(p)[j];
            const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const unsigned short lo = (unsigned short)(w[e] & 0xffffu), hi = (unsigned short)(w[e] >> 16);
                out[8 * j + 2 * e] = to_f32(__builtin_bit_cast(T, lo));
                out[8 * j + 2 * e + 1] = to_f32(__builtin_bit_cast(T, hi));
            }
        }
    }
}

template <typename T, int ROWS>
__device__ __forceinline__ void output_chunk_replay(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ Qdec, const T* __restrict__ Kdec, int N, int H, int M, int Dk, int Dv,
    int DT, int TT, float scale, int chunk, bool shared, const float* __restrict__ pmax,
    const float* __restrict__ pden, const float* __restrict__ pnum, void* __restrict__ Y,
    int out_dtype, float* __restrict__ lse_dec, const int32_t* __restrict__ tmask, float power,
    float* smem, int c, int bh, int dt0, int NC, int tid, int flag) {
    // The tokenwise replay of chunk c of (b,h) = bh, value columns dt0 .. dt0 + DT, by kNT
    // threads (thread index tid) with LDS scratch smem (OutSmem::floats() floats, 16-byte
    // aligned).  flag: kRedoWhole replays the whole chunk from its prefix slot; a narrow
    // flag replays 32-token subtiles j1 .. j2 only, from the state at subtile j1's start
    // (which then stands in the chunk's prefix slot).
    // power > 0: the stablemax encoder (den += stablemax_transform(s), no rescale);
    // the decoder weights stay a softmax over the latents.
    const int R = kNT / DT;
    const int Mp = R * ROWS;
    float* gam = smem;                                      // [Mp]
    float* eta = gam + Mp;                                  // [Mp]
    float* wts = eta + Mp;                                  // [Mp]
    float* k_tile = wts + Mp;                               // [TT][Dk]
    float* qd_tile = k_tile + TT * Dk;                      // [TT][Dk] (separate decoder only)
    float* v_tile = qd_tile + (shared ? 0 : TT * Dk);       // [TT][DT]
    float* s_tile = v_tile + TT * DT;                       // [TT][M]
    float* a_tile = s_tile + TT * M;                        // [TT][M] (separate decoder only)
    float* mstate = a_tile + (shared ? 0 : TT * M);         // [M]
    float* dstate = mstate + M;
    float* ypart = dstate + M;                              // [R][DT]
    float* lse = ypart + R * DT;                            // [TT]

    const int b = bh / H, h = bh % H;
    const int col = tid % DT, rg = tid / DT;
    const int mb = rg * ROWS;     // this thread's latents mb .. mb + ROWS - 1 (value column col)
    const T* q_h = Q + (size_t)h * M * Dk;
    const T* kd_h = shared ? q_h : Kdec + (size_t)h * M * Dk;

    const size_t pbase = ((size_t)bh * NC + c) * M;
    // stablemax: the recurrence below keeps absolute sums (max 0); summaries written by the
    // MFMA prepare carry a reference max, folded in here
    for (int m = tid; m < M; m += kNT) {
        mstate[m] = power > 0.0f ? 0.0f : pmax[pbase + m];
        dstate[m] = power > 0.0f ? pden[pbase + m] * __expf(pmax[pbase + m]) : pden[pbase + m];
    }
    for (int m = M + tid; m < Mp; m += kNT) {
        gam[m] = 1.0f;
        eta[m] = 0.0f;
        wts[m] = 0.0f;
    }
    float U[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int m = mb + r;
        U[r] = m < M ? pnum[(pbase + m) * Dv + dt0 + col] * (power > 0.0f ? __expf(pmax[pbase + m]) : 1.0f) : 0.0f;
    }

    int t_begin = c * chunk;
    int t_end = min(N, t_begin + chunk);
    if (redo_is_narrow(flag)) {
        t_end = min(t_end, t_begin + 32 * (redo_j2(flag) + 1));
        t_begin += 32 * redo_j1(flag);
    }
    for (int t0 = t_begin; t0 < t_end; t0 += TT) {
        const int nt = min(TT, t_end - t0);
        __syncthreads();
        for (int e = tid; e < TT * Dk; e += kNT) {
            const int i = e / Dk, d = e % Dk;
            const size_t gi = (((size_t)b * N + t0 + i) * H + h) * Dk + d;
            k_tile[e] = i < nt ? to_f32(K[gi]) : 0.0f;
            if (!shared) qd_tile[e] = i < nt ? to_f32(Qdec[gi]) : 0.0f;
        }
        for (int e = tid; e < TT * DT; e += kNT) {
            const int i = e / DT, d = e % DT;
            v_tile[e] = i < nt ? to_f32(V[(((size_t)b * N + t0 + i) * H + h) * Dv + dt0 + d]) : 0.0f;
        }
        __syncthreads();
        // Scores of the tile: thread m holds 32 columns of its latent's Q (and K_dec) row at a
        // time and reads the TT token rows from LDS four columns at a time (the same address
        // in every lane: broadcast reads); the sums run over d in order, per token.
        for (int m = tid; m < M; m += kNT) {
            const T* qrow = q_h + (size_t)m * Dk;
            const T* kdrow = kd_h + (size_t)m * Dk;
            float acc[16], acc2[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = acc2[i] = 0.0f;
            if ((Dk & 3) == 0) {
                for (int d0 = 0; d0 < Dk; d0 += 32) {
                    float qv[32], kv[32];
                    if (d0 + 32 <= Dk && (Dk * (int)sizeof(T)) % 16 == 0) {   // 16-byte aligned pieces
                        load_row32(qrow + d0, qv);
                        if (!shared) load_row32(kdrow + d0, kv);
                    } else {
#pragma unroll
                        for (int e = 0; e < 32; ++e) {
                            qv[e] = d0 + e < Dk ? to_f32(qrow[d0 + e]) : 0.0f;
                            kv[e] = (!shared && d0 + e < Dk) ? to_f32(kdrow[d0 + e]) : 0.0f;
                        }
                    }
                    const int nd = min(32, Dk - d0);
#pragma unroll
                    for (int dd = 0; dd < 32; dd += 4) {
                        if (dd < nd) {
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                if (i < nt) {
                                    const float4 k4 = *reinterpret_cast<const float4*>(k_tile + i * Dk + d0 + dd);
                                    acc[i] += k4.x * qv[dd];
                                    acc[i] += k4.y * qv[dd + 1];
                                    acc[i] += k4.z * qv[dd + 2];
                                    acc[i] += k4.w * qv[dd + 3];
                                    if (!shared) {
                                        const float4 q4 = *reinterpret_cast<const float4*>(qd_tile + i * Dk + d0 + dd);
                                        acc2[i] += q4.x * kv[dd];
                                        acc2[i] += q4.y * kv[dd + 1];
                                        acc2[i] += q4.z * kv[dd + 2];
                                        acc2[i] += q4.w * kv[dd + 3];
                                    }
                                }
                            }
                        }
                    }
                }
            } else {
                for (int d = 0; d < Dk; ++d) {
                    const float qd1 = to_f32(qrow[d]);
                    const float kd1 = shared ? 0.0f : to_f32(kdrow[d]);
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        if (i < nt) {
                            acc[i] += k_tile[i * Dk + d] * qd1;
                            if (!shared) acc2[i] += qd_tile[i * Dk + d] * kd1;
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (i < nt) {
                    // a masked token: s = a = -inf leaves the state unchanged and gives y = 0
                    // (inference.py:395-397, 476-478)
                    const bool masked = tmask != nullptr && tmask[(size_t)b * N + t0 + i] == 0;
                    s_tile[i * M + m] = masked ? kNegInf : acc[i] * scale;
                    if (!shared) a_tile[i * M + m] = masked ? kNegInf : acc2[i] * scale;
                }
            }
        }
        __syncthreads();
        {   // decoder log-sum-exp per token: wavefront w handles tokens w, w+4, ...
            const int w = tid >> 6, lane = tid & 63;
            const float* asrc = shared ? s_tile : a_tile;
            for (int i = w; i < nt; i += kNT / 64) {
                float mxv = kNegInf;
                for (int m = lane; m < M; m += 64) mxv = fmaxf(mxv, asrc[i * M + m]);
                mxv = wave_max(mxv);
                float sm = 0.0f;
                for (int m = lane; m < M; m += 64) sm += __expf(asrc[i * M + m] - mxv);
                sm = wave_sum(sm);
                if (lane == 0) lse[i] = mxv == kNegInf ? kNegInf : mxv + __logf(sm);   // -inf: a masked token
            }
        }
        __syncthreads();
        for (int i = 0; i < nt; ++i) {
            const float li = lse[i];
            for (int m = tid; m < M; m += kNT) {
                const float s = s_tile[i * M + m];
                MergeScales ts;
                if (power > 0.0f) {
                    ts.m_new = mstate[m];
                    ts.sa = 1.0f;
                    ts.sb = stablemax_transform(s, power);
                } else {
                    ts = token_scales(mstate[m], s);
                }
                const float dn = dstate[m] * ts.sa + ts.sb;
                mstate[m] = ts.m_new;
                dstate[m] = dn;
                gam[m] = ts.sa;
                eta[m] = ts.sb;
                const float a = shared ? s : a_tile[i * M + m];
                wts[m] = li == kNegInf ? 0.0f : __expf(a - li) / (dn > 0.0f ? dn : 1.0f);
            }
            __syncthreads();
            const float vc = v_tile[i * DT + col];
            float yp = 0.0f;
#pragma unroll
            for (int r = 0; r < ROWS; r += 4) {
                // (< Mp: past M the factors keep U = 0 and add 0; the same address in every
                // lane of a wave: broadcast reads)
                const float4 g4 = *reinterpret_cast<const float4*>(gam + mb + r);
                const float4 e4 = *reinterpret_cast<const float4*>(eta + mb + r);
                const float4 w4 = *reinterpret_cast<const float4*>(wts + mb + r);
                U[r] = U[r] * g4.x + e4.x * vc;
                U[r + 1] = U[r + 1] * g4.y + e4.y * vc;
                U[r + 2] = U[r + 2] * g4.z + e4.z * vc;
                U[r + 3] = U[r + 3] * g4.w + e4.w * vc;
                yp += w4.x * U[r] + w4.y * U[r + 1] + w4.z * U[r + 2] + w4.w * U[r + 3];
            }
            ypart[rg * DT + col] = yp;
            __syncthreads();
            if (tid < DT) {
                float y = 0.0f;
                for (int g2 = 0; g2 < R; ++g2) y += ypart[g2 * DT + tid];
                const int t = t0 + i;
                store_out(Y, (((size_t)b * N + t) * H + h) * Dv + dt0 + tid, y, out_dtype);
                if (lse_dec && dt0 == 0 && tid == 0) lse_dec[(size_t)bh * N + t] = li;
            }
        }
    }
}

// Value-column tile of the replay: the largest power of two <= 128 dividing Dv with
// at most 64 numerator registers per thread (0: no such tile).
__host__ __device__ constexpr int replay_dt(int M, int Dv) {
    for (int dt = 128; dt >= 16; dt >>= 1) {
        if (Dv % dt) continue;
        const int rows = (M + (kNT / dt) - 1) / (kNT / dt);
        if (rows <= 64) return dt;
    }
    return 0;
}
// The ROWS instance for M latents over kNT / DT row groups.
__host__ __device__ constexpr int replay_rows(int M, int DT) {
    const int rows = (M + kNT / DT - 1) / (kNT / DT);
    return rows <= 8 ? 8 : rows <= 16 ? 16 : rows <= 32 ? 32 : 64;
}

}  // namespace flare
