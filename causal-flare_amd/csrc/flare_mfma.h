// flare_mfma.h -- device helpers shared by the gfx950 MFMA kernels: operand
// types, 16x16x32 bf16/fp16 MFMA wrappers, hi/lo splits, DPP row reductions and
// the transposed V staging used by every chunk kernel.
#pragma once

#include "flare_common.h"

namespace flare {
namespace mfma {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int T = 32;       // tokens per subtile (= the MFMA K depth)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.0f;            // log2 headroom before a reference max moves
constexpr float kDenMax = 16.0f;         // den (relative to the reference) that moves it in the output kernel
// Largest move of a latent's reference within one subtile (log2 units, ~66 nats) that the
// MFMA output kernels resolve; beyond it the earlier tokens' den would approach the fp32
// underflow against the new reference, and the chunk is replayed tokenwise in fp32.
constexpr float kJumpMax = 96.0f;

// The stablemax encoder on the MFMA kernels: a raw score x (k . q, before the scale)
// becomes log2 s(a) / scale2 with a = x scale and s(a) = (1 + a)^p (a >= 0), (1 - a)^-p
// (a < 0), so that every later `x * scale2` is log2 of the encoder weight and the lazy
// references, dens and numerators work unchanged.  -inf (a masked token) stays -inf.
__device__ __forceinline__ float smx_log2(float x, float scale2, float power) {
    const float a = x * scale2 * kLn2;
    const float l = a >= 0.0f ? power * __log2f(1.0f + a) : -power * __log2f(1.0f - a);
    return l * __builtin_amdgcn_rcpf(scale2);
}
constexpr float kF16Max = 65504.0f;
constexpr int kMaxPrepM = 256;           // largest latent bank of the prepare kernel (8 waves)

__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Input tensors (Q, K, V and the decoder tensors) travel as raw 16-bit words in
// bf16-typed storage; F16 selects the fp16 reading of those words for the MFMA
// that consumes them and for conversions to float.
template <bool F16>
__device__ __forceinline__ f32x4 mma_in(bf16x8 a, bf16x8 b, f32x4 c) {
    if constexpr (F16) return mma(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c);
    else return mma(a, b, c);
}
template <bool F16>
__device__ __forceinline__ float in_f32(bf16 x) {
    if constexpr (F16) return (float)__builtin_bit_cast(f16, x);
    else return (float)x;
}


// x = hi + lo, both halves of type TY.
#define SPLIT2(TY, x, HI, LO)              \
    do {                                   \
        const float _x = (x);              \
        const TY _h = (TY)_x;              \
        HI = _h;                           \
        LO = (TY)(_x - (float)_h);         \
    } while (0)

// (a_hi + a_lo) x b, a an fp32 operand split into bf16 halves, b a raw 16-bit input
// operand: bf16 b enters exactly (two products); fp16 b is split into an exact bf16
// pair b_hi + b_lo (11 mantissa bits in 8 + 8) and the a_lo x b_lo product, about
// 2^-16 of the whole, is dropped (three products).
template <bool F16>
__device__ __forceinline__ f32x4 mma_split(bf16x8 ah, bf16x8 al, bf16x8 b, f32x4 c) {
    if constexpr (F16) {
        const f16x8 bf = __builtin_bit_cast(f16x8, b);
        bf16x8 bh, bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) SPLIT2(bf16, (float)bf[e], bh[e], bl[e]);
        c = mma(ah, bh, c);
        c = mma(al, bh, c);
        return mma(ah, bl, c);
    } else {
        c = mma(ah, b, c);
        return mma(al, b, c);
    }
}

typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// (x0, x1) = hi + lo with bf16 halves: hi is the truncated upper half of each
// float (exact), lo = x - hi rounded to bf16, so |x - hi - lo| <= 2^-16 |x|.
__device__ __forceinline__ void split_bf16_pair(float x0, float x1, bf16x2& hi, bf16x2& lo) {
    const unsigned b0 = __builtin_bit_cast(unsigned, x0), b1 = __builtin_bit_cast(unsigned, x1);
    hi = __builtin_bit_cast(bf16x2, __builtin_amdgcn_perm(b1, b0, 0x07060302u));
    const float l0 = x0 - __builtin_bit_cast(float, b0 & 0xffff0000u);
    const float l1 = x1 - __builtin_bit_cast(float, b1 & 0xffff0000u);
    lo = __builtin_convertvector(f32x2{l0, l1}, bf16x2);
}
// four floats -> bf16x4 hi / lo
__device__ __forceinline__ void split_bf16x4(float x0, float x1, float x2, float x3, bf16x4& hi, bf16x4& lo) {
    bf16x2 h01, l01, h23, l23;
    split_bf16_pair(x0, x1, h01, l01);
    split_bf16_pair(x2, x3, h23, l23);
    hi = __builtin_shufflevector(h01, h23, 0, 1, 2, 3);
    lo = __builtin_shufflevector(l01, l23, 0, 1, 2, 3);
}
// (x0, x1) = hi + lo with fp16 halves (hi rounded to nearest)
__device__ __forceinline__ void split_f16_pair(float x0, float x1, f16x2& hi, f16x2& lo) {
    hi = __builtin_convertvector(f32x2{x0, x1}, f16x2);
    const f32x2 h = __builtin_convertvector(hi, f32x2);
    lo = __builtin_convertvector(f32x2{x0 - h[0], x1 - h[1]}, f16x2);
}

// q[0..3] = hi + lo with fp16 halves (hi rounded to nearest)
__device__ __forceinline__ void split_f16x4(const float q[4], f16x4& hi, f16x4& lo) {
    f16x2 h01, l01, h23, l23;
    split_f16_pair(q[0], q[1], h01, l01);
    split_f16_pair(q[2], q[3], h23, l23);
    hi = __builtin_shufflevector(h01, h23, 0, 1, 2, 3);
    lo = __builtin_shufflevector(l01, l23, 0, 1, 2, 3);
}

// DPP moves inside a 16-lane row.  Lanes whose source is outside the row read 0.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    // bound_ctrl: a lane whose source is out of its row reads 0 (every pattern used here
    // either has a source for every lane or wants 0 there), so no old value is needed
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
constexpr int kQuadXor1 = 0xB1;       // quad_perm(1,0,3,2)
constexpr int kQuadXor2 = 0x4E;       // quad_perm(2,3,0,1)
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;

// max of two floats as one v_max_f32, for operands that are never NaN (fmaxf would
// first canonicalise an operand that arrives through a bit cast, as DPP results do)
__device__ __forceinline__ float max_raw(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float row_max16(float x) {
    x = max_raw(x, dpp<kQuadXor1>(x));
    x = max_raw(x, dpp<kQuadXor2>(x));
    x = max_raw(x, dpp<kRowHalfMirror>(x));
    x = max_raw(x, dpp<kRowMirror>(x));
    return x;
}
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<kQuadXor1>(x);
    x += dpp<kQuadXor2>(x);
    x += dpp<kRowHalfMirror>(x);
    x += dpp<kRowMirror>(x);
    return x;
}
// Inclusive prefix sum over the 16 lanes of a row (Hillis-Steele).
__device__ __forceinline__ float row_scan16(float x) {
    x += dpp<kRowShr1>(x);
    x += dpp<kRowShr2>(x);
    x += dpp<kRowShr4>(x);
    x += dpp<kRowShr8>(x);
    return x;
}
// Lane 15 of each 16-lane row, broadcast over the row (DPP row_newbcast:15).
__device__ __forceinline__ float row_bcast15(float x) { return dpp<0x15F>(x); }
// max of three floats as one v_max3_f32, for operands that are never NaN (fmaxf would
// first canonicalise every operand that is not the result of an arithmetic op)
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// max / sum over the four 16-lane rows (lanes c, c+16, c+32, c+48)
__device__ __forceinline__ float rows_max4(float x) {
    x = max_raw(x, __shfl_xor(x, 16, 64));
    return max_raw(x, __shfl_xor(x, 32, 64));
}
__device__ __forceinline__ float rows_sum4(float x) {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
}

// max over the 64 lanes, as a wave-uniform value: DPP within rows, then the
// four row maxima read as scalars (no lane-index registers)
__device__ __forceinline__ float wave_max_dpp(float x) {
    const int b = __builtin_bit_cast(int, row_max16(x));
    auto lane_f = [b](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, l)); };
    return fmaxf(fmaxf(lane_f(0), lane_f(16)), fmaxf(lane_f(32), lane_f(48)));
}

template <typename V8, typename V4>
__device__ __forceinline__ V8 cat8(V4 lo, V4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
template <typename V8, typename E>
__device__ __forceinline__ V8 load8(const E* p) { return *reinterpret_cast<const V8*>(p); }
template <typename V4, typename E>
__device__ __forceinline__ V4 load4(const E* p) { return *reinterpret_cast<const V4*>(p); }
__device__ __forceinline__ bf16x8 zero8() {
    bf16x8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
    return z;
}

__device__ __forceinline__ void store4(void* Y, size_t idx, f32x4 v, int out_dtype) {
    if (out_dtype == FLARE_BF16) {
        bf16x4 o;
        o[0] = (bf16)v[0]; o[1] = (bf16)v[1]; o[2] = (bf16)v[2]; o[3] = (bf16)v[3];
        *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(Y) + idx) = o;
    } else if (out_dtype == FLARE_F16) {
        *reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(Y) + idx) = __builtin_convertvector(v, f16x4);
    } else {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(Y) + idx) = v;
    }
}

// Stage V^T[d][tau] for the value columns [d0, d0+nd) of one subtile into LDS
// as fp16 (row pitch P).  Threads [0, nthr) of the group take part.  Returns
// whether this thread saw a value outside the fp16 range.
template <int P>
__device__ __forceinline__ bool stage_vt_f16(f16* vt, const bf16* V, size_t row0, size_t stride, int t0,
                                             int t_end, int d0, int nd, int tid, int nthr) {
    bool big = false;
    for (int vi = tid; vi < T * nd / 8; vi += nthr) {
        const int tau = vi / (nd / 8), d8 = vi % (nd / 8);
        const int t = t0 + tau;
        const bf16x8 v = t < t_end ? load8<bf16x8>(V + row0 + (size_t)t * stride + d0 + 8 * d8) : zero8();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = (float)v[e];
            big |= fabsf(x) > kF16Max;
            vt[(d0 + 8 * d8 + e) * P + tau] = (f16)x;
        }
    }
    return big;
}
// Same, bf16 (used only when a subtile holds a value outside the fp16 range).
template <int P>
__device__ __forceinline__ void stage_vt_bf16(bf16* vt, const bf16* V, size_t row0, size_t stride, int t0,
                                              int t_end, int d0, int nd, int tid, int nthr) {
    for (int vi = tid; vi < T * nd / 8; vi += nthr) {
        const int tau = vi / (nd / 8), d8 = vi % (nd / 8);
        const int t = t0 + tau;
        const bf16x8 v = t < t_end ? load8<bf16x8>(V + row0 + (size_t)t * stride + d0 + 8 * d8) : zero8();
#pragma unroll
        for (int e = 0; e < 8; ++e) vt[(d0 + 8 * d8 + e) * P + tau] = v[e];
    }
}

// Rows of D bf16 values in LDS hold 16-byte chunk j at slot j ^ (row mod D/8):
// the 16 lanes that read one chunk of 16 consecutive rows hit distinct banks.
template <int D>
__device__ __forceinline__ int swz(int row, int j) { return j ^ (row & (D / 8 - 1)); }

// One 16-byte global_load_lds per lane: lane l's 16 bytes at `src` land at
// LDS byte offset 16 l from `wave_dst` (the wave's base).  A plain function so
// that templates instantiated more than once in a translation unit call one
// definition of the builtin (clang's host pass rejects the repeated inline
// builtin in template substitution).
__device__ __forceinline__ void global_to_lds16(const bf16* src, bf16* wave_dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)wave_dst, 16, 0, 0);
}

// T rows t0 .. t0+T of a [.., stride] bf16 tensor (one (b,h): row0) straight
// from HBM into swizzled LDS rows (global_load_lds: no registers), NTHR
// threads each moving 16-byte chunks into consecutive 1 KiB pieces per wave.
// Rows at or past `nrows` read row nrows-1 (their values are masked by the
// caller).  Completion is tracked by vmcnt like any other global load.
template <int D, int NTHR>
__device__ __forceinline__ void rows_to_lds(bf16* dst, const bf16* src, size_t row0, size_t stride, int t0,
                                            int nrows, int tid, int lane) {
    constexpr int KC = D / 8;
#pragma unroll
    for (int e0 = 0; e0 < T * KC; e0 += NTHR) {
        const int e = e0 + tid;
        if (T * KC % NTHR == 0 || e < T * KC) {
            const int row = e / KC, sl = e % KC;
            const int t = min(t0 + row, nrows - 1);
            global_to_lds16(src + row0 + (size_t)t * stride + 8 * swz<D>(row, sl), dst + (e - lane) * 8);
        }
    }
}
// The T rows t0 .. t0+T of a [.., stride] bf16 tensor (one (b,h): row0) held in
// registers by NTHR threads (16-byte chunks), then stored to LDS rows of D
// values with chunk j at slot j ^ (row mod D/8).  Rows at or past `nrows` read
// row nrows-1 (their values are masked by the caller).
template <int D, int NTHR>
struct KRows {
    static constexpr int KC = D / 8;
    static constexpr int NK = (T * KC + NTHR - 1) / NTHR;
    bf16x8 v[NK];
    __device__ __forceinline__ void load(const bf16* src, size_t row0, size_t stride, int t0, int nrows, int tid) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int e = tid + k * NTHR;
            if (T * KC % NTHR == 0 || e < T * KC) {
                const int row = e / KC, j = e % KC;
                const int t = min(t0 + row, nrows - 1);
                v[k] = load8<bf16x8>(src + row0 + (size_t)t * stride + 8 * j);
            }
        }
    }
    __device__ __forceinline__ void store(bf16* dst, int tid) const {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int e = tid + k * NTHR;
            if (T * KC % NTHR == 0 || e < T * KC) {
                const int row = e / KC, j = e % KC;
                *reinterpret_cast<bf16x8*>(dst + row * D + 8 * swz<D>(row, j)) = v[k];
            }
        }
    }
};

// Number of rows_to_lds loads each thread issues (for vmcnt bookkeeping).
template <int D, int NTHR>
constexpr int rows_to_lds_count() { return (T * (D / 8) + NTHR - 1) / NTHR; }

// Workgroup barrier that orders LDS only: this wave's LDS requests complete
// (lgkmcnt 0), then s_barrier.  Unlike __syncthreads() it does not wait for
// global loads still in flight (prefetches, or DMA into LDS, whose completion
// the caller waits for with vmcnt where needed); the asm statements keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);     // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) with the other counters left alone (n <= 15).
#define FLARE_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | (n))

// One subtile of V[t0 .. t0+T) x [d0, d0+ND) held in registers, NTHR threads
// of the group each holding NS 8-column slots, so that the next subtile can be
// fetched from HBM while the current one is being used.
template <int ND, int NTHR, bool F16 = false>
struct VTile {
    static constexpr int SLOTS = T * ND / 8;
    static constexpr int NS = (SLOTS + NTHR - 1) / NTHR;
    bf16x8 v[NS];

    // Slot vi -> (token tau, 8-column chunk d8).  Row-major for at most two
    // chunks per row; otherwise pairs of chunks x 32 tokens per 64 slots, so
    // that the transposed 2-byte LDS stores of one instruction fall in
    // distinct banks (row pitch 40 halves).
    __device__ __forceinline__ static void slot(int vi, int& tau, int& d8) {
        constexpr int NDC = ND / 8;
        if (NDC <= 2) {
            tau = vi / NDC;
            d8 = vi % NDC;
        } else {
            tau = (vi >> 1) & 31;
            d8 = (vi & 1) + 2 * ((vi >> 6) % (NDC / 2));
        }
    }
    __device__ __forceinline__ void load(const bf16* V, size_t row0, size_t stride, int t0, int t_end, int d0,
                                         int tid) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int vi = tid + k * NTHR;
            int tau, d8;
            slot(vi, tau, d8);
            const int t = t0 + tau;
            v[k] = (vi < SLOTS && t < t_end) ? load8<bf16x8>(V + row0 + (size_t)t * stride + d0 + 8 * d8) : zero8();
        }
    }
    // V^T[d][tau] (row pitch P) as fp16; returns whether a value exceeds the fp16 range.
    template <int P>
    __device__ __forceinline__ bool store_f16(f16* vt, int d0, int tid) const {
        float big = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int vi = tid + k * NTHR;
            if (SLOTS % NTHR == 0 || vi < SLOTS) {
                int tau, d8;
                slot(vi, tau, d8);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = in_f32<F16>(v[k][e]);
                    big = fmaxf(big, fabsf(x));
                    vt[(d0 + 8 * d8 + e) * P + tau] = (f16)x;
                }
            }
        }
        return big > kF16Max;
    }
    // Largest |v| this thread holds.
    __device__ __forceinline__ float absmax(int tid) const {
        float big = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; ++k)
            if (SLOTS % NTHR == 0 || tid + k * NTHR < SLOTS)
#pragma unroll
                for (int e = 0; e < 8; ++e) big = fmaxf(big, fabsf(in_f32<F16>(v[k][e])));
        return big;
    }
    // V^T[d][tau] (row pitch P) as fp16 of v * sc (sc a power of two).
    template <int P>
    __device__ __forceinline__ void store_f16_scaled(f16* vt, int d0, int tid, float sc) const {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int vi = tid + k * NTHR;
            if (SLOTS % NTHR == 0 || vi < SLOTS) {
                int tau, d8;
                slot(vi, tau, d8);
#pragma unroll
                for (int e = 0; e < 8; ++e) vt[(d0 + 8 * d8 + e) * P + tau] = (f16)(in_f32<F16>(v[k][e]) * sc);
            }
        }
    }
    // V^T[d][tau] (row pitch P), bf16 as loaded.
    template <int P>
    __device__ __forceinline__ void store_bf16(bf16* vt, int d0, int tid) const {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int vi = tid + k * NTHR;
            if (SLOTS % NTHR == 0 || vi < SLOTS) {
                int tau, d8;
                slot(vi, tau, d8);
#pragma unroll
                for (int e = 0; e < 8; ++e) vt[(d0 + 8 * d8 + e) * P + tau] = v[k][e];
            }
        }
    }
};

}  // namespace mfma
}  // namespace flare
