// flare_common.h -- shared device helpers for the causal FLARE HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/flare_mi355x.h"

namespace flare {

constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------------------
// Element loads: inputs arrive as fp32, bf16 or fp16; all arithmetic is fp32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }
__device__ __forceinline__ float to_f32(__half x) { return __half2float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) { return __float2bfloat16(x); }
template <> __device__ __forceinline__ __half from_f32<__half>(float x) { return __float2half(x); }

__device__ __forceinline__ bool is_neg_inf(float x) { return x == kNegInf; }

// da_tm = alpha_tm (gz_tm - gy_t), from the stored C = alpha gz (cgz false) or C = gz
// (cgz true, the token-causal backward, whose later kernels need no alpha).
__device__ __forceinline__ float score_grad_da(float c, float al, float gy, bool cgz) {
    return cgz ? al * (c - gy) : c - al * gy;
}

// ---------------------------------------------------------------------------
// Per-chunk replay flags of the MFMA output kernels ([B*H, NC] ints), read by the
// tokenwise fp32 kernel: 0 leaves the chunk alone, kRedoWhole replays the whole
// chunk from its prefix state, and a narrow flag replays the 32-token subtiles
// j1 .. j2 only, starting from the state at subtile j1's start, which the output
// kernel then wrote over the chunk's prefix slot.
// ---------------------------------------------------------------------------
constexpr int kRedoWhole = 1;
constexpr int kRedoNarrowBit = 1 << 30;
constexpr int kRedoMaxSubtiles = 1 << 15;    // j1, j2 < kRedoMaxSubtiles
__host__ __device__ __forceinline__ int redo_narrow(int j1, int j2) { return kRedoNarrowBit | (j1 << 15) | j2; }
__host__ __device__ __forceinline__ bool redo_is_narrow(int f) { return (f & kRedoNarrowBit) != 0; }
__host__ __device__ __forceinline__ int redo_j1(int f) { return (f >> 15) & (kRedoMaxSubtiles - 1); }
__host__ __device__ __forceinline__ int redo_j2(int f) { return f & (kRedoMaxSubtiles - 1); }

// ---------------------------------------------------------------------------
// Online-softmax monoid on one latent: (max, den, num).  The inf-safe forms
// follow causal_flare/autoregressive/reference.py:160-187 (merge) and
// :461-473 (single-token update).
// ---------------------------------------------------------------------------
struct MergeScales {
    float m_new, sa, sb;
};

__device__ __forceinline__ MergeScales merge_scales(float ma, float mb) {
    MergeScales r;
    r.m_new = fmaxf(ma, mb);
    const bool a_inf = is_neg_inf(ma), b_inf = is_neg_inf(mb), n_inf = is_neg_inf(r.m_new);
    const float m_safe = n_inf ? 0.0f : r.m_new;
    r.sa = (a_inf && n_inf) ? 1.0f : (a_inf ? 0.0f : __expf(ma - m_safe));
    r.sb = (b_inf && n_inf) ? 1.0f : (b_inf ? 0.0f : __expf(mb - m_safe));
    return r;
}

// Token update: gamma rescales the old state, eta weights the new token.
__device__ __forceinline__ MergeScales token_scales(float m, float s) {
    MergeScales r;
    r.m_new = fmaxf(m, s);
    const bool m_inf = is_neg_inf(m), n_inf = is_neg_inf(r.m_new);
    const float m_safe = n_inf ? 0.0f : r.m_new;
    r.sa = (m_inf && n_inf) ? 1.0f : (m_inf ? 0.0f : __expf(m - m_safe));
    r.sb = n_inf ? 0.0f : __expf(s - m_safe);
    return r;
}

// The stablemax score transform (reference autoregressive/stablemax.py:45-52,
// stablemax_triton.py:137-170): (1 + x)^p for x >= 0 and (1 - x)^-p for x < 0,
// positive and monotone; x = -inf gives 0.  Powers 1-4 by products, others as
// exp2(p log2 base).
__device__ __forceinline__ float stablemax_transform(float x, float p) {
    const float base = x >= 0.0f ? 1.0f + x : 1.0f - x;
    float r;
    if (p == 1.0f) r = base;
    else if (p == 2.0f) r = base * base;
    else if (p == 3.0f) r = base * base * base;
    else if (p == 4.0f) {
        const float b2 = base * base;
        r = b2 * b2;
    } else r = exp2f(p * log2f(base));
    return x >= 0.0f ? r : 1.0f / r;
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) and workgroup reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Reduce across a workgroup of NT threads; `red` holds >= NT/64 floats of LDS.
// All threads receive the result.  Contains two barriers.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) r += red[i];
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// Error reporting through the C-ABI (flare_last_error()).
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int check_launch(const char* what);

}  // namespace flare

#define FLARE_REQUIRE(cond, ...)                  \
    do {                                          \
        if (!(cond)) {                            \
            ::flare::set_error(__VA_ARGS__);      \
            return FLARE_ERR_INVALID;             \
        }                                         \
    } while (0)
