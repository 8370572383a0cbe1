// flare_ar_prep.hip -- phase 1 of the chunked causal FLARE forward on gfx950:
// the chunk summaries (max, den, num) of the reference's flare_chunk_prepare
// (training.py:914-1018) for bf16 or fp16 inputs, M in {128, 256}, D in {64, 128}.
//
// One workgroup per (chunk, b, h) with M/32 waves; wave w owns latents
// 32 w .. 32 w + 31 over every value column, so the waves never exchange data:
// per 64-token tile each wave forms S^T = K Q^T (tokens as rows), moves its lazy
// references when a score passes them by more than kLazy, takes
// E = 2^(S - R) straight from the score registers as the B operand of
// U^T += V^T E (the C layout of a 16x16 score tile is the B layout of the
// 32-deep contraction, with token slots tau(g, e) = 4 g + e and 16 + 4 g + e - 4),
// and reads V^T with transposed LDS reads.  K and V tiles reach LDS by DMA
// (global_load_lds into XOR-swizzled rows), three tiles in flight, one barrier
// per tile.
//
// Precision: S in fp32 from the bf16 / fp16 inputs; E (<= 2^kLazy) enters
// U^T += V^T E as fp16 against fp16 V -- the fp16 inputs, or bf16 V converted
// to fp16 in LDS one tile ahead (exact within the fp16 range).  A bf16 tile
// holding a value outside that range takes E as a bf16 hi + lo pair against
// bf16 V instead.  (A single bf16 rounding of E, as the reference's
// p.to(v.dtype) in training.py:985-990, leaves state errors near 2e-2 where
// sum E v cancels.)  den and the maxima in fp32.  The summary is returned
// relative to the true chunk max: (max, den 2^(R - max), U 2^(R - max)) in
// natural-log units, as chunk_prepare_pc writes it.
#include <type_traits>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"

namespace flare {
namespace mfma {

typedef short s16x4p __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4p lds_s16x4p;

namespace {

constexpr int TT = 64;   // tokens per tile

// Transposed 8-byte LDS read: with lane j of a 16-lane group pointing at row
// base + j / 4, columns c0 + 4 (j % 4) .. + 3, lane i receives column c0 + i of
// rows base .. base + 3.
template <bool F16>
__device__ __forceinline__ bf16x4 tr4(const bf16* p) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4p*)p));
}

// global_load_lds of 16 bytes per lane (lane l's bytes land at LDS byte offset 16 l
// from wave_dst) written as inline assembly: the compiler then does not track the
// LDS write, and inserts no wait for it before LDS reads of the other tiles (it
// cannot tell the three tile buffers apart there); the kernel orders the DMA with
// explicit vmcnt waits and barriers.
__device__ __forceinline__ void dma16(const bf16* src, bf16* wave_dst) {
    const unsigned lds = __builtin_amdgcn_readfirstlane(
        (unsigned)(uintptr_t)((__attribute__((address_space(3))) bf16*)wave_dst));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// The TT-row tiles of a [.., stride] 16-bit tensor (one (b,h)), one after another,
// into XOR-swizzled LDS rows by DMA (no registers): piece e = tid + k NTHR of a
// tile is row e / KC, LDS slot e % KC, and holds logical 16-byte column chunk
// swz(row, slot).  Each thread keeps the global addresses of its pieces and
// advances them by TT rows per tile.  Rows at or past `rows_end` repeat row
// rows_end - 1 (their scores are masked).
template <int D, int NTHR, int TT>
struct TileDma {
    static constexpr int KC = D / 8;
    static constexpr int NK = TT * KC / NTHR;
    static_assert(TT * KC % NTHR == 0, "the workgroup's threads must divide the pieces of a tile");
    const bf16* p[NK];
    __device__ __forceinline__ void init(const bf16* base, int t_first, size_t stride, int tid) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int e = tid + k * NTHR;
            p[k] = base + (size_t)(t_first + e / KC) * stride + 8 * swz<D>(e / KC, e % KC);
        }
    }
    // the next tile (rows t0 ..) into dst; wofs = 8 x (the wave's first thread index)
    __device__ __forceinline__ void issue(bf16* dst, int wofs, int t0, int rows_end, size_t stride, int tid) {
        if (t0 + TT <= rows_end) {
#pragma unroll
            for (int k = 0; k < NK; ++k) dma16(p[k], dst + wofs + k * NTHR * 8);
        } else {
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const int t = t0 + (tid + k * NTHR) / KC, tc = min(t, rows_end - 1);
                dma16(p[k] - (size_t)(t - tc) * stride, dst + wofs + k * NTHR * 8);
            }
        }
#pragma unroll
        for (int k = 0; k < NK; ++k) p[k] += (size_t)TT * stride;
    }
};

}  // namespace

template <int M, int D, bool F16, bool MASK, bool SMX = false, int TTK = TT, bool EMIT = false>
__global__ __launch_bounds__(2 * M) void chunk_prepare_tr(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                          const bf16* __restrict__ V, int N, int H, float scale2,
                                                          int chunk, float* __restrict__ cmax,
                                                          float* __restrict__ cden, float* __restrict__ cnum,
                                                          const int32_t* __restrict__ tmask, float power,
                                                          const float* __restrict__ s0max,
                                                          const float* __restrict__ s0den,
                                                          const float* __restrict__ s0num, int NC32) {
    // SMX: the stablemax encoder (smx_log2 on the scores; power > 0), else the softmax one.
    // TTK: tokens per tile (32 for 32-token chunks, whose 64-token tiles would be half masked)
    // EMIT: the running state instead of a summary.  The workgroup starts from its chunk's
    // exclusive prefix (s0max / s0den / s0num, [B*H, NC, M(, D)], from the scan) and writes
    // the state at the start of every 32-token chunk k that starts inside it to slot k of
    // cmax / cden / cnum ([B*H, NC32, M(, D)]): (R ln 2, den and U relative to 2^R) with R
    // the lazy reference.  These are the backward's chunk starting states.
    constexpr int TT = TTK;
    static_assert(!EMIT || TTK == 64, "the state is written at the two 32-token halves of a 64-token tile");
    constexpr int NT = 2 * M;           // M / 32 waves
    constexpr int KS = D / 32;          // k-steps of the scores
    constexpr int DT = D / 16;          // value-column tiles
    constexpr int TI = TT / 16;         // token tiles of a tile
    constexpr int KK = TT / 32;         // k-steps of U^T += V^T E
    // M = 256: the waves of the first half (threads 0 .. NT/2 - 1) issue every DMA and
    // convert every V tile, so that the second half, whose tile chain is the longer one
    // (it places its barrier after the scores), does neither
    constexpr bool SPLIT = M >= 256;
    constexpr int NTD = SPLIT ? NT / 2 : NT;   // threads that issue the DMA and convert V
    constexpr int NCV = TT * D / 8 / NTD;
    using Dma = TileDma<D, NTD, TT>;
    // K tiles j mod 3 and V tiles j mod 4 (DMA two tiles ahead; V of tile j is read
    // until iteration j + 1); bf16 inputs: V tiles j mod 2 converted to fp16
    __shared__ __attribute__((aligned(16))) bf16 ktl[3][TT * D];
    __shared__ __attribute__((aligned(16))) bf16 vtl[4][TT * D];
    __shared__ __attribute__((aligned(16))) f16 vhl[F16 ? 1 : 2][F16 ? 8 : TT * D];
    __shared__ int redo_bf16;

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int NC = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int m0 = 32 * w;
    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const int NS = (t_end - t_begin + TT - 1) / TT;
    const size_t stride = (size_t)H * D;
    const bf16* Kb = K + (size_t)b * N * stride + (size_t)h * D;
    const bf16* Vb = V + (size_t)b * N * stride + (size_t)h * D;

    // this wave's Q rows as MFMA B operands (n = m, k = d)
    bf16x8 qb[2][KS];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kq = 0; kq < KS; ++kq)
            qb[mt][kq] = load8<bf16x8>(Q + ((size_t)h * M + m0 + 16 * mt + c) * D + 32 * kq + 8 * g);
    // Q has arrived before the loop (the empty asm uses it), so that the compiler keeps
    // no wait for these loads inside the loop, where it would also wait for the DMA
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kq = 0; kq < KS; ++kq) asm volatile("" : "+v"(qb[mt][kq]));
    const int wofs = 8 * __builtin_amdgcn_readfirstlane(tid - lane);
    const bool dmaw = !SPLIT || tid < NTD;     // (wave-uniform)
    // per-lane LDS offsets (elements) of the swizzled operand reads: K rows 16 ti + c at
    // chunk 4 kq + g (row & (KC - 1) = c & (KC - 1)), and the transposed V reads of rows
    // 32 kk + 4 g + c / 4 (+ 16) at columns 16 di + 4 (c & 3) (row & (KC - 1) does not
    // depend on kk); the tile-dependent parts are compile-time offsets
    constexpr int KC = D / 8;
    int kofs[KS], vofs[DT];
#pragma unroll
    for (int kq = 0; kq < KS; ++kq) kofs[kq] = c * D + 8 * ((4 * kq + g) ^ (c & (KC - 1)));
#pragma unroll
    for (int di = 0; di < DT; ++di) {
        const int rl = 4 * g + (c >> 2);
        vofs[di] = rl * D + 8 * ((2 * di + ((c & 3) >> 1)) ^ (rl & (KC - 1))) + 4 * (c & 1);
    }
    // U^T[d = 16 di + 4 g + r][m = m0 + 16 mt + c]
    f32x4 U[DT][2];
    // per latent m0 + 16 mt + c (replicated over g): reference R, this lane's max rt and den dl
    float R[2], rt[2], dl[2];
    // EMIT: the reference and this lane's den in the middle of the last tile, and the
    // rescale of U between its two halves
    float Rmid[2] = {kNegInf, kNegInf}, dmid[2] = {0.0f, 0.0f}, g1[2] = {1.0f, 1.0f};

    // One pass over the chunk.  BF = false: fp16 E (<= 2^kLazy) against fp16 V (the fp16
    // inputs, or bf16 V converted in LDS); BF = true (bf16 inputs only, a rerun when the
    // first pass met a value outside the fp16 range): E as an exact bf16 hi + lo pair
    // against the bf16 V.
    auto pass = [&](auto bf_tag) __attribute__((always_inline)) {
        constexpr bool BF = decltype(bf_tag)::value;
        Dma kdma, vdma;
        kdma.init(Kb, t_begin, stride, tid);
        vdma.init(Vb, t_begin, stride, tid);
        if (dmaw) {
            kdma.issue(ktl[0], wofs, t_begin, t_end, stride, tid);
            vdma.issue(vtl[0], wofs, t_begin, t_end, stride, tid);
            kdma.issue(ktl[1], wofs, t_begin + TT, t_end, stride, tid);
            vdma.issue(vtl[1], wofs, t_begin + TT, t_end, stride, tid);
        }
#pragma unroll
        for (int di = 0; di < DT; ++di) U[di][0] = U[di][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            R[mt] = kNegInf;
            rt[mt] = kNegInf;
            dl[mt] = 0.0f;
        }
        // EMIT: the state at the start of 32-token chunk k: reference Rv, this lane's den dv
        auto emit = [&](int k, const float (&Rv)[2], const float (&dv)[2]) __attribute__((always_inline)) {
            if (k >= NC32 || 32 * k >= t_end) return;
            const size_t sb = ((size_t)bh * NC32 + k) * M;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float den = rows_sum4(dv[mt]);
                const int m = m0 + 16 * mt + c;
                if (g == 0) {
                    cmax[sb + m] = Rv[mt] == kNegInf ? kNegInf : Rv[mt] * kLn2;
                    cden[sb + m] = den;
                }
#pragma unroll
                for (int di = 0; di < DT; ++di)
                    *reinterpret_cast<f32x4*>(cnum + (sb + m) * D + 16 * di + 4 * g) = U[di][mt];
            }
        };
        if constexpr (EMIT) {
            // start from the chunk's exclusive prefix: reference R = its max (log2), den in
            // the g = 0 lanes (the den is summed over the four lane rows), U relative to 2^R
            const size_t pb = ((size_t)bh * NC + c_idx) * M;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int m = m0 + 16 * mt + c;
                const float pd = s0den[pb + m];
                R[mt] = pd > 0.0f ? s0max[pb + m] * kLog2e : kNegInf;
                dl[mt] = (g == 0 && pd > 0.0f) ? pd : 0.0f;
#pragma unroll
                for (int di = 0; di < DT; ++di)
                    U[di][mt] = pd > 0.0f ? *reinterpret_cast<const f32x4*>(s0num + (pb + m) * D + 16 * di + 4 * g)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
            }
            emit(t_begin / 32, R, dl);
        }
        // E of the previous tile in fp16, k-slot order tau(g, e): the B operand of U^T += V^T E
        f16x8 eh[KK][2];
        FLARE_WAIT_VMCNT((2 * Dma::NK));   // tile 0 has landed
        lds_barrier();
        // EMIT, after the k-step kk of tile jp's product: the state at the start of the next
        // 32-token chunk (the middle of tile jp, or its end), then U rescaled for the second
        // half's reference
        auto emit_half = [&](int jp, int kk) __attribute__((always_inline)) {
            if (kk == 0) {
                emit((t_begin + TT * jp) / 32 + 1, Rmid, dmid);
                if (__any(g1[0] != 1.0f || g1[1] != 1.0f)) {
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int di = 0; di < DT; ++di) U[di][mt] *= g1[mt];
                }
            } else {
                emit((t_begin + TT * jp) / 32 + 2, R, dl);
            }
        };
        auto value_product = [&](int jp) __attribute__((always_inline)) {
            auto vread = [&](const bf16* base, int kk, int di) __attribute__((always_inline)) {
                const bf16* p = base + vofs[di] + 32 * kk * D;
                return cat8<bf16x8>(tr4<F16>(p), tr4<F16>(p + 16 * D));
            };
            if constexpr (!BF) {
                const bf16* vf = F16 ? vtl[jp & 3] : reinterpret_cast<const bf16*>(vhl[jp & 1]);
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
                    for (int di = 0; di < DT; ++di) {
                        const f16x8 va = __builtin_bit_cast(f16x8, vread(vf, kk, di));
#pragma unroll
                        for (int mt = 0; mt < 2; ++mt) U[di][mt] = mma(va, eh[kk][mt], U[di][mt]);
                    }
                    if constexpr (EMIT) emit_half(jp, kk);
                }
            } else {
                bf16x8 hi[KK][2], lo[KK][2];
#pragma unroll
                for (int kk = 0; kk < KK; ++kk)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int i = 0; i < 8; ++i) SPLIT2(bf16, (float)eh[kk][mt][i], hi[kk][mt][i], lo[kk][mt][i]);
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
                    for (int di = 0; di < DT; ++di) {
                        const bf16x8 va = vread(vtl[jp & 3], kk, di);
#pragma unroll
                        for (int mt = 0; mt < 2; ++mt) {
                            U[di][mt] = mma(va, hi[kk][mt], U[di][mt]);
                            U[di][mt] = mma(va, lo[kk][mt], U[di][mt]);
                        }
                    }
                    if constexpr (EMIT) emit_half(jp, kk);
                }
            }
        };

        // S^T of tile j into acc (the ragged end and masked tokens score -inf)
        auto scores = [&](int j, f32x4 (&acc)[TI][2]) __attribute__((always_inline)) {
            const int t0 = t_begin + TT * j;
            // masked tokens of this lane (t = t0 + 16 ti + 4 g + r, bit 4 ti + r)
            unsigned drop = 0;
            if constexpr (MASK) {
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = t0 + 16 * ti + 4 * g + r;
                        if (t < t_end && tmask[(size_t)b * N + t] == 0) drop |= 1u << (4 * ti + r);
                    }
            }
            // ---- S^T = K Q^T: acc[ti][mt][r] = S[t = 16 ti + 4 g + r][m = 16 mt + c]
            const bf16* kt = ktl[j % 3];
#pragma unroll
            for (int ti = 0; ti < TI; ++ti) acc[ti][0] = acc[ti][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kq = 0; kq < KS; ++kq) {
                bf16x8 ka[TI];
#pragma unroll
                for (int ti = 0; ti < TI; ++ti) ka[ti] = load8<bf16x8>(kt + kofs[kq] + 16 * ti * D);
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) acc[ti][mt] = mma_in<F16>(ka[ti], qb[mt][kq], acc[ti][mt]);
            }
            // the ragged end of the chunk and masked tokens score -inf
            if (t0 + TT > t_end || MASK) {
                asm volatile("");   // a branch around this rare block, not selects on every tile
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (t0 + 16 * ti + 4 * g + r >= t_end || ((drop >> (4 * ti + r)) & 1))
                            acc[ti][0][r] = acc[ti][1][r] = kNegInf;
                    }
            }
            if constexpr (SMX) {
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[ti][mt][r] = smx_log2(acc[ti][mt][r], scale2, power);
            }
        };
        // the lazy references, then E = 2^(S - R) of the tile in acc into eh and its den
        auto exps = [&](f32x4 (&acc)[TI][2]) __attribute__((always_inline)) {
            // ---- lazy references: checked per lane, moved to the exact max over the latent rarely
            float mx[2];
            bool need = false;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                float x = max3_raw(acc[0][mt][0], acc[0][mt][1], acc[0][mt][2]);
                x = max3_raw(x, acc[0][mt][3], acc[1][mt][0]);
                x = max3_raw(x, acc[1][mt][1], acc[1][mt][2]);
                x = fmaxf(x, acc[1][mt][3]);
#pragma unroll
                for (int ti = 2; ti < TI; ++ti) {
                    x = max3_raw(x, acc[ti][mt][0], acc[ti][mt][1]);
                    x = max3_raw(x, acc[ti][mt][2], acc[ti][mt][3]);
                }
                mx[mt] = x * scale2;
                rt[mt] = fmaxf(rt[mt], mx[mt]);
                need |= mx[mt] > R[mt] + kLazy;
            }
            if (__any(need)) {
                asm volatile("");   // a branch: the rescale of U is rare
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const float m4 = rows_max4(mx[mt]);
                    const bool mv = m4 > R[mt] + kLazy;
                    const float Rn = mv ? m4 : R[mt];
                    const float gam = mv ? exp2f_fast(R[mt] - Rn) : 1.0f;   // 0 when R = -inf
                    R[mt] = Rn;
                    dl[mt] *= gam;
#pragma unroll
                    for (int di = 0; di < DT; ++di) U[di][mt] *= gam;
                }
            }
            // ---- E = 2^(S - R) (<= 2^kLazy, fp16) and its den.  A latent with no reference
            //      yet (every token so far masked) has E = 0.
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float nR = R[mt] == kNegInf ? kNegInf : -R[mt];
                float es = 0.0f;
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = exp2f_fast(fmaf(acc[ti][mt][r], scale2, nR));
                        es += e;
                        eh[ti >> 1][mt][4 * (ti & 1) + r] = (f16)e;
                    }
                dl[mt] += es;
            }
        };
        // EMIT: the same per 32-token half, so that the state in the middle of the tile has
        // a reference of its own: a move in the first half rescales U and den at once; a
        // move in the second half rescales den, and U only after the first half's product
        // (by g1, in emit_half), as E of that half is relative to the new reference.
        auto exps_emit = [&](f32x4 (&acc)[TI][2]) __attribute__((always_inline)) {
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                float mx[2];
                bool need = false;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    float x = max3_raw(acc[2 * hf][mt][0], acc[2 * hf][mt][1], acc[2 * hf][mt][2]);
                    x = max3_raw(x, acc[2 * hf][mt][3], acc[2 * hf + 1][mt][0]);
                    x = max3_raw(x, acc[2 * hf + 1][mt][1], acc[2 * hf + 1][mt][2]);
                    x = fmaxf(x, acc[2 * hf + 1][mt][3]);
                    mx[mt] = x * scale2;
                    need |= mx[mt] > R[mt] + kLazy;
                    if (hf == 1) g1[mt] = 1.0f;
                }
                if (__any(need)) {
                    asm volatile("");
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
                        const float m4 = rows_max4(mx[mt]);
                        const bool mv = m4 > R[mt] + kLazy;
                        const float Rn = mv ? m4 : R[mt];
                        const float gam = mv ? exp2f_fast(R[mt] - Rn) : 1.0f;   // 0 when R = -inf
                        R[mt] = Rn;
                        dl[mt] *= gam;
                        if (hf == 0) {
#pragma unroll
                            for (int di = 0; di < DT; ++di) U[di][mt] *= gam;
                        } else {
                            g1[mt] = gam;
                        }
                    }
                }
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const float nR = R[mt] == kNegInf ? kNegInf : -R[mt];
                    float es = 0.0f;
#pragma unroll
                    for (int ti = 2 * hf; ti < 2 * hf + 2; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float e = exp2f_fast(fmaf(acc[ti][mt][r], scale2, nR));
                            es += e;
                            eh[hf][mt][4 * (ti & 1) + r] = (f16)e;
                        }
                    dl[mt] += es;
                    if (hf == 0) {
                        dmid[mt] = dl[mt];
                        Rmid[mt] = R[mt];
                    }
                }
            }
        };
        // Iteration j issues the DMA of tile j + 2, converts V of tile j and runs, per wave,
        // ... S(j) E(j) | P(j) S(j+1) E(j+1) | ... (S scores, E exponentials, P the value
        // product).  The waves of the second half of a 256-latent workgroup place the
        // barrier one step later, after S(j) instead of after E(j): a SIMD then holds one
        // wave in its MFMA-heavy part (P, S) while the other is in its VALU-heavy part (E),
        // instead of both in the same part at once.  The first half, which does the DMA and
        // the V conversion for both, runs P(j - 1) before them, while the second half is in
        // E(j - 1).
        auto loop = [&](auto late_tag) __attribute__((always_inline)) {
            constexpr bool LATE = decltype(late_tag)::value;
            f32x4 acc[TI][2];
            for (int j = 0; j < NS; ++j) {
                const int t0 = t_begin + TT * j;
                if constexpr (!LATE) {
                    if (j > 0) value_product(j - 1);
                }
                // tile j + 2 (past the chunk's last tile: copies of its last row, never read), so
                // that every iteration issues the same number of DMA requests
                if (dmaw) {
                    kdma.issue(ktl[(j + 2) % 3], wofs, t0 + 2 * TT, t_end, stride, tid);
                    vdma.issue(vtl[(j + 2) & 3], wofs, t0 + 2 * TT, t_end, stride, tid);
                }
                // bf16 inputs, first pass: V of tile j (landed at the last barrier) to fp16 for
                // iteration j + 1 (a value outside the fp16 range becomes inf and shows in U)
                if (!F16 && !BF && dmaw) {
                    const bf16* src = vtl[j & 3];
                    f16* dst = vhl[j & 1];
#pragma unroll
                    for (int k = 0; k < NCV; ++k) {
                        const int idx = tid + k * NTD;
                        const bf16x8 x = load8<bf16x8>(src + 8 * idx);
                        f16x8 y;
#pragma unroll
                        for (int i = 0; i < 8; ++i) y[i] = (f16)(float)x[i];
                        *reinterpret_cast<f16x8*>(dst + 8 * idx) = y;
                    }
                }
                if constexpr (LATE) {
                    if (j > 0) {
                        if constexpr (EMIT) exps_emit(acc); else exps(acc);
                        value_product(j - 1);
                    }
                    scores(j, acc);
                } else {
                    scores(j, acc);
                    if constexpr (EMIT) exps_emit(acc); else exps(acc);
                }
                // tile j + 1 has landed (tile j + 2 may still be in flight); every wave is done
                // with the buffers that iteration j + 1 refills
                FLARE_WAIT_VMCNT((2 * Dma::NK));
                lds_barrier();   // no memory fence: it would wait for the DMA of tile j + 2
            }
            if constexpr (LATE) {
                if (NS > 0) {
                    if constexpr (EMIT) exps_emit(acc);
                    else exps(acc);
                }
            }
        };
        if (M >= 256 && w >= M / 64) loop(std::true_type{});
        else loop(std::false_type{});
        if (NS > 0) value_product(NS - 1);
        FLARE_WAIT_VMCNT(0);   // the DMA of the two tiles past the end has landed
    };

    if (tid == 0) redo_bf16 = 0;
    __syncthreads();
    if constexpr (EMIT && !F16) {
        // the running states of bf16 inputs: E as a bf16 hi + lo pair against bf16 V in one
        // pass (no fp16 copy of V whose range could overflow, so no second pass)
        pass(std::true_type{});
        return;
    }
    pass(std::false_type{});
    if constexpr (!F16) {
        // a bf16 value outside the fp16 range (or a non-finite input) left U non-finite:
        // the chunk is redone with bf16 V
        bool bad = false;
#pragma unroll
        for (int di = 0; di < DT; ++di)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(U[di][mt][r]);
        if (__any(bad) && lane == 0) redo_bf16 = 1;
        __syncthreads();
        if (redo_bf16) pass(std::true_type{});
    }
    if constexpr (EMIT) return;
    // ---- the summary relative to the true chunk max
    const size_t sbase = ((size_t)bh * NC + c_idx) * M;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const float Rt = rows_max4(rt[mt]);
        const float den = rows_sum4(dl[mt]);
        const float f = Rt == kNegInf ? 0.0f : exp2f_fast(R[mt] - Rt);   // <= 1
        const int m = m0 + 16 * mt + c;
        if (g == 0) {
            cmax[sbase + m] = Rt * kLn2;
            cden[sbase + m] = den * f;
        }
#pragma unroll
        for (int di = 0; di < DT; ++di)
            *reinterpret_cast<f32x4*>(cnum + (sbase + m) * D + 16 * di + 4 * g) = U[di][mt] * f;
    }
}

}  // namespace mfma
}  // namespace flare

namespace flare {
using namespace mfma;

int launch_prepare_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                      int64_t D, float scale, int64_t chunk, float* cmax, float* cden, float* cnum,
                      const int32_t* tmask, bool f16in, hipStream_t stream, float power) {
    FLARE_REQUIRE(chunk > 0, "chunk_prepare_tr: chunk must be positive");
    FLARE_REQUIRE(power <= 0.0f || tmask == nullptr, "chunk_prepare_tr: the stablemax encoder takes no token mask");
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "chunk_prepare_tr: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
    // 32-token chunks (the backward's): 32-token tiles, none of them half masked
    const bool t32 = chunk == 32 && tmask == nullptr;
#define FLARE_PREP_TR_T(MM, DD, F)                                                                           \
    do {                                                                                                     \
        if (t32 && power > 0.0f)                                                                             \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false, true, 32>), grid, dim3(2 * MM), 0, stream, \
                               (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                               cmax, cden, cnum, tmask, power, nullptr, nullptr, nullptr, 0);                                              \
        else if (t32)                                                                                        \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false, false, 32>), grid, dim3(2 * MM), 0, stream, \
                               (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                               cmax, cden, cnum, tmask, 0.0f, nullptr, nullptr, nullptr, 0);                                               \
        else if (power > 0.0f)                                                                               \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false, true>), grid, dim3(2 * MM), 0, stream,    \
                               (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                               cmax, cden, cnum, tmask, power, nullptr, nullptr, nullptr, 0);                                              \
        else if (tmask != nullptr)                                                                           \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, true>), grid, dim3(2 * MM), 0, stream,           \
                               (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                               cmax, cden, cnum, tmask, 0.0f, nullptr, nullptr, nullptr, 0);                                               \
        else                                                                                                 \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false>), grid, dim3(2 * MM), 0, stream,          \
                               (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, \
                               cmax, cden, cnum, tmask, 0.0f, nullptr, nullptr, nullptr, 0);                                               \
    } while (0)
#define FLARE_PREP_TR(MM, DD)                        \
    do {                                             \
        if (f16in) FLARE_PREP_TR_T(MM, DD, true);    \
        else FLARE_PREP_TR_T(MM, DD, false);         \
    } while (0)
    if (M == 128 && D == 64) FLARE_PREP_TR(128, 64);
    else if (M == 128 && D == 128) FLARE_PREP_TR(128, 128);
    else if (M == 256 && D == 64) FLARE_PREP_TR(256, 64);
    else FLARE_PREP_TR(256, 128);
#undef FLARE_PREP_TR
#undef FLARE_PREP_TR_T
    return check_launch("chunk_prepare_tr");
}

int launch_states_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* s0max, const float* s0den,
                     const float* s0num, float* smax, float* sden, float* snum, bool f16in, hipStream_t stream,
                     float power) {
    FLARE_REQUIRE(chunk > 0 && chunk % 64 == 0, "chunk_states: chunk must be a positive multiple of 64");
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "chunk_states: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    const int64_t NC = (N + chunk - 1) / chunk;
    const int NC32 = (int)((N + 31) / 32);
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
#define FLARE_STATES_T(MM, DD, F)                                                                            \
    do {                                                                                                     \
        if (power > 0.0f)                                                                                    \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false, true, TT, true>), grid, dim3(2 * MM), 0,  \
                               stream, (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2,    \
                               (int)chunk, smax, sden, snum, nullptr, power, s0max, s0den, s0num, NC32);      \
        else                                                                                                 \
            hipLaunchKernelGGL((chunk_prepare_tr<MM, DD, F, false, false, TT, true>), grid, dim3(2 * MM), 0, \
                               stream, (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2,    \
                               (int)chunk, smax, sden, snum, nullptr, 0.0f, s0max, s0den, s0num, NC32);       \
    } while (0)
#define FLARE_STATES(MM, DD)                         \
    do {                                             \
        if (f16in) FLARE_STATES_T(MM, DD, true);     \
        else FLARE_STATES_T(MM, DD, false);          \
    } while (0)
    if (M == 128 && D == 64) FLARE_STATES(128, 64);
    else if (M == 128 && D == 128) FLARE_STATES(128, 128);
    else if (M == 256 && D == 64) FLARE_STATES(256, 64);
    else FLARE_STATES(256, 128);
#undef FLARE_STATES
#undef FLARE_STATES_T
    return check_launch("chunk_prepare_tr (states)");
}

int prepare_tr_attributes(int64_t M, int64_t D, bool f16in, hipFuncAttributes* attr, int* threads) {
    const void* f = nullptr;
#define FLARE_PREP_TR_F(MM, DD)                                                                       \
    f = f16in ? (const void*)chunk_prepare_tr<MM, DD, true, false> : (const void*)chunk_prepare_tr<MM, DD, false, false>
    if (M == 128 && D == 64) FLARE_PREP_TR_F(128, 64);
    else if (M == 128 && D == 128) FLARE_PREP_TR_F(128, 128);
    else if (M == 256 && D == 64) FLARE_PREP_TR_F(256, 64);
    else if (M == 256 && D == 128) FLARE_PREP_TR_F(256, 128);
#undef FLARE_PREP_TR_F
    FLARE_REQUIRE(f != nullptr, "chunk_prepare_tr: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    *threads = (int)(2 * M);
    FLARE_REQUIRE(hipFuncGetAttributes(attr, f) == hipSuccess, "chunk_prepare_tr: hipFuncGetAttributes failed");
    return FLARE_OK;
}

}  // namespace flare
