// flare_ar_out.hip -- phase 3 of the chunked causal FLARE forward on gfx950
// (bf16 or fp16 inputs, M in {128, 256}, D in {64, 128}): the token replay of
// one chunk of one (b,h) in 32-token subtiles, with producer and consumer waves.
//
// Producers (M/64 waves, 64 latents each) turn subtile j into its softmax
// operands while consumers (D/32 waves, 32 value columns each, holding the
// numerator U[M][their columns] in registers) fold subtile j-1 into the output
// and the state.  Every operand that crosses waves goes through LDS in its
// natural row layout with 8- and 16-byte stores -- E[tau][m], W[t][m] and
// V[tau][d] -- and is read back transposed where an MFMA wants the token axis
// as its K dimension (ds_read_b64_tr_b16: lane j of a 16-lane group points at
// row base + j/4, columns 4 (j%4) .. +3, and lane i then holds column i of
// rows base .. base+3).  The K operand slots over a 32-token subtile are
// tau(g, e) = 4 g + e (e < 4) and 16 + 4 g + e - 4 (e >= 4) for lane row g,
// which is also the row order of a 16x16 MFMA result, so the intra-subtile
// weights G^T come out of one MFMA already in operand order.
//
// Notation (log2 domain, S = scale log2(e) k_t . q_m):
//   R[m]     lazy reference of latent m (moves when a score passes it by more
//            than kLazy, or its den passes kDenMax)
//   E[t,m]   = 2^(S - R)              d_t[m] = d0[m] + sum_{tau<=t} E[tau,m]
//   alpha    = softmax over all M latents of S[t,:]   (the decoder weights)
//   W[t,m]   = alpha / d_t            G[t,tau] = sum_m W[t,m] E[tau,m]  (tau <= t)
//   y_t      = sum_m W[t,m] U[m] + sum_tau G[t,tau] v_tau,   then U += E^T V
// This is the tokenwise recurrence of the reference (training.py:1282-1393,
// reference.py:446-496) regrouped into 16x16x32 contractions.
//
// Token softmax without a per-token maximum: producer w publishes, per token,
// a reference C_w (the largest R of its latents) and L_w(t) = sum_m E 2^(R - C_w);
// after the producers meet, each token's log-sum-exp is the merge of the NP
// pairs and alpha = E 2^(R - C_w) f_w(t) with f_w(t) = 2^(C_w - lse_t).  A
// producer whose partial would underflow (a token far below its references)
// publishes the exact pair (max_m S, sum 2^(S - max)) instead (general path).
//
// Precision: E <= 2^kLazy and W <= alpha enter the MFMAs as fp16 (11 bits);
// G = W E^T is accumulated in fp32 and enters G V as an fp16 hi + lo pair; U is
// rounded to fp16 for the readout only.  A subtile where a producer's reference moved (or
// its partial underflowed) takes the general path for that producer's latents:
// fp32 exponentials and DPP scans, W E^T from bf16 hi/lo splits in fp32 (its
// share of G then comes through LDS as fp32 instead of the consumers' fp16
// product), W1 = W d0 against z0 = U / d0 when a reference moved.
#include <type_traits>

#include "flare_common.h"
#include "flare_internal.h"
#include "flare_mfma.h"
#include "flare_replay.h"

namespace flare {
namespace mfma {

// Producer meetings of chunk_output_tr that gave up waiting (read by
// flare_device_faults; it should stay 0).
__device__ unsigned int g_meet_timeouts_tr = 0;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Transposed 8-byte LDS read (see the file comment): four 16-bit values.
__device__ __forceinline__ f16x4 lds_tr4(const f16* p) {
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}
// Raw buffer resource over [base, base + bytes): loads past the end return 0,
// stores past the end are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

template <int M, int D>
struct TrLayout {
    static constexpr int NP = M / 64;            // producer waves, 64 latents each
    static constexpr int NC = D / 32;            // consumer waves, 32 value columns each
    static constexpr int NT = 64 * (NP + NC);
    // Roles by wave index.  A workgroup's waves go to distinct SIMDs, and a second workgroup
    // on the same compute unit (the 128 x 64 bank fits two) places wave w on another SIMD
    // than the first's wave w, one step further round the SIMDs (measured on MI355X): with
    // producers and consumers interleaved (P, C, P, C) every SIMD then holds one producer
    // and one consumer, where P, P, C, C would put two producers on one SIMD and two
    // consumers on another.  One workgroup of 8 waves per CU gives waves w and w + 4 the
    // same SIMD, so P, P, P, P, C, C, C, C pairs them there.
    static constexpr bool IL = NP == 2 && NC == 2;
    static constexpr int MP = 64;
    static constexpr int MTP = 4;                // 16-latent tiles per producer
    static constexpr int MKP = 2;                // 32-latent k-steps per producer
    static constexpr int MTA = M / 16;
    static constexpr int MK = M / 32;
    static constexpr int DC = 32;
    static constexpr int DTC = 2;
    static constexpr int KS = D / 32;            // k-steps of the scores
    // Row pitch (halves) of E[tau][m] and W[t][m]: M + 40 keeps every access pattern used
    // below at the best rate measured on gfx950 -- the producers' 8-byte row stores, the
    // 16-byte reads down 16 rows and the transposed 8-byte reads of 4 consecutive rows with
    // either column pattern.  M + 48 (the same reads) costs 2x on the stores and 1.6x on
    // the den's transposed reads; pitches such as M + 24, M + 36 or M + 64 cost 1.5x to 10x
    // on one of them.
    static constexpr int RPW = M + 40;
    static constexpr int RPE = M + 40;
    static constexpr int VP = DC + 8;            // row pitch (halves) of a consumer's V[tau][d]
    static constexpr float kVCap = 2048.0f;      // bound on |V'| and |z'| (fp16 operands)
    static constexpr float kLazyE = 256.0f;      // 2^kLazy: an E above it moves the reference
    static constexpr float kTinyL = 0x1p-100f;   // smallest softmax partial of the common path
};

// Sum / max over the four 16-lane rows (lanes c, c+16, c+32, c+48) with the gfx950
// lane swaps (rows 0<->1, 2<->3, then halves 0-31 <-> 32-63): VALU only, no LDS.
// v_permlane16/32_swap exchange rows between their two operands; given x in two
// distinct registers, each lane then holds x from itself and from its partner.  The
// second operand is an opaque copy so that the two never share a register, and the
// two results pass through an empty asm before they are combined: this compiler
// otherwise folds the second result of the intrinsic into the first.
__device__ __forceinline__ void lane_pair(unsigned& r0, unsigned& r1, unsigned x, bool rows32) {
    unsigned xc = x;
    asm volatile("" : "+v"(xc));
    const auto p = rows32 ? __builtin_amdgcn_permlane32_swap(x, xc, false, false)
                          : __builtin_amdgcn_permlane16_swap(x, xc, false, false);
    r0 = p[0];
    r1 = p[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
}
template <bool MAX>
__device__ __forceinline__ float rows_reduce4(float x) {
    unsigned r0, r1;
    lane_pair(r0, r1, __builtin_bit_cast(unsigned, x), false);
    const float y = MAX ? fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1))
                        : __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
    lane_pair(r0, r1, __builtin_bit_cast(unsigned, y), true);
    return MAX ? fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1))
               : __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float rows_sum4_pl(float x) { return rows_reduce4<false>(x); }
__device__ __forceinline__ float rows_max4_pl(float x) { return rows_reduce4<true>(x); }

// (tau(g, e) <= t): the causal mask in operand slot order
__device__ __forceinline__ int tau_slot(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

// K rows of one subtile by DMA straight into swizzled LDS rows (global_load_lds, no
// registers).  Each thread's NK 16-byte pieces keep their row and column from one
// subtile to the next, so their global addresses are formed once and advanced by T rows.
template <int D, int NTHR>
struct KDma {
    static constexpr int KC = D / 8;
    static constexpr int NK = T * KC / NTHR;
    static_assert(T * KC % NTHR == 0, "the producers' threads must divide the K pieces of a subtile");
    const bf16* src[NK];
    __device__ __forceinline__ void init(const bf16* K, size_t row0, size_t stride, int t_begin, int tid) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int e = tid + k * NTHR;
            src[k] = K + row0 + (size_t)(t_begin + e / KC) * stride + 8 * swz<D>(e / KC, e % KC);
        }
    }
    // Rows t0 .. t0+T of subtile j (t0 = t_begin + T j) into dst; rows at or past nrows read
    // row nrows - 1 (the caller masks their scores).
    __device__ __forceinline__ void issue(bf16* dst, int j, int t0, int nrows, size_t stride, int tid,
                                          int lane) const {
        const size_t adv = (size_t)j * T * stride;
        if (t0 + T <= nrows) {
#pragma unroll
            for (int k = 0; k < NK; ++k) global_to_lds16(src[k] + adv, dst + (tid + k * NTHR - lane) * 8);
        } else {
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const int t = t0 + (tid + k * NTHR) / KC, tc = min(t, nrows - 1);
                global_to_lds16(src[k] + adv - (size_t)(t - tc) * stride, dst + (tid + k * NTHR - lane) * 8);
            }
        }
    }
};

// The tokenwise replay of an M x D chunk: value-column slices of DT columns, ROWS latents
// per thread, and the largest token tile (16 or less) whose LDS scratch fits `bytes`.
template <int M, int D>
struct ReplayShape {
    static constexpr int DT = replay_dt(M, D);
    static constexpr int ROWS = replay_rows(M, DT);
    static constexpr int NSL = DT > 0 ? D / DT : 0;
    template <size_t bytes>
    static constexpr int tt() {
        int t = 16;
        while (t > 1 && OutSmem{t, D, DT, M, kNT / DT, (kNT / DT) * ROWS, true}.floats() * sizeof(float) > bytes) t /= 2;
        return t;
    }
};

template <int M, int D, bool SEP, bool F16, bool SMX = false>
__global__ __launch_bounds__(64 * (M / 64 + D / 32), (512 / (64 * (M / 64 + D / 32))) > 0 ? 512 / (64 * (M / 64 + D / 32)) : 1)
void chunk_output_tr(const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ V, int N,
                     int H, float scale2, int chunk, const float* pmax, const float* pden,
                     const float* pnum, void* __restrict__ Y, int out_dtype,
                     const int32_t* __restrict__ tmask, const f16* __restrict__ alpha, int* __restrict__ redo,
                     int spin_limit, int record, float power, float scale, int replay) {
    // SMX (separate decoder weights only): the stablemax encoder, smx_log2 on the scores
    // record (shared decoder weights only): the prefix slot of this chunk (pmax, pden,
    // pnum, read once at the start) may be overwritten with the state at the start of
    // the first subtile whose reference jumped, so that the tokenwise fp32 replay only
    // covers the flagged subtiles (a narrow redo flag) instead of the whole chunk.
    // replay (shared decoder weights, with redo): the workgroup runs that replay itself
    // once its subtiles are done (the shapes whose threads make whole replay slices; the
    // host then launches no replay kernel).  scale: the natural-log score scale (scale2 =
    // scale log2(e)), for the replay.
    using L = TrLayout<M, D>;
    // K rows of the even / odd subtiles (swizzled, filled by DMA)
    __shared__ __attribute__((aligned(16))) bf16 ksl0[T * D];
    __shared__ __attribute__((aligned(16))) bf16 ksl1[T * D];
    __shared__ __attribute__((aligned(16))) f16 erl[2][T * L::RPE];            // E[tau][m] (fp16)
    __shared__ __attribute__((aligned(16))) f16 wl[2][T * L::RPW];             // W1[t][m] (fp16)
    __shared__ __attribute__((aligned(16))) f16 vrl[L::NC][T * L::VP];        // V'[tau][d], consumer-private
    __shared__ __attribute__((aligned(16))) f32x4 gpl[2][L::NP][3][64];       // general-path G^T tiles
    __shared__ __attribute__((aligned(16))) float2 lsep[2][L::NP][T];         // (reference, partial) per token
    __shared__ __attribute__((aligned(16))) float gaml[2][M];                 // rescale factor (moved latents)
    __shared__ __attribute__((aligned(16))) float d0l[2][M];                  // den at the subtile start
    __shared__ int movedl[2][L::NP];    // bit 0: a reference moved; bit 1: general path
    __shared__ int psync;               // producer arrivals (monotonic)
    __shared__ int redol;               // separate decoder: a reference jumped past kJumpMax;
                                        // shared weights: the chunk's redo flag (in-place replay)
    // shared weights: subtile j + 1 in jumpl[j & 1] when a reference jumped past kJumpMax
    // in subtile j (read by the other producers after their meeting); the references and
    // dens at the start of such a subtile (rare: written only then)
    __shared__ int jumpl[2];
    __shared__ float rsvl[SEP ? 1 : 2][SEP ? 1 : M];
    __shared__ float dsvl[SEP ? 1 : 2][SEP ? 1 : M];

    const int c_idx = blockIdx.x, bh = blockIdx.y;
    const int nchunks = gridDim.x;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const bool producer = L::IL ? (w & 1) == 0 : w < L::NP;
    const int pw = L::IL ? w >> 1 : w;            // producer index (producer waves)
    const int ptid = 64 * pw + lane;              // thread index among the producers
    const int g = lane >> 4, c = lane & 15;
    const int t_begin = c_idx * chunk;
    const int t_end = min(N, t_begin + chunk);
    const int NS = (t_end - t_begin + T - 1) / T;
    const size_t stride = (size_t)H * D;
    const size_t row0 = (size_t)b * N * stride + (size_t)h * D;
    const size_t pbase = ((size_t)bh * nchunks + c_idx) * M;
    if (tid == 0) {
        psync = 0;
        redol = 0;
        jumpl[0] = jumpl[1] = 0;
    }
    // the replay decision, taken by every consumer wave alike from the subtile flags
    // (movedl bit 2: a reference jumped, bit 3: a producer meeting gave up):
    // the whole chunk (a meeting gave up before any record), else subtiles rj1 .. rj2
    bool rwhole = false;
    int rj1 = -1, rj2 = -1;

    if (producer) {
        // =========================== producer ===========================
        const int mp0 = pw * L::MP;
        bf16x8 qa[L::MTP][L::KS];      // Q rows of this wave's latents (A operands: rows m, k = d)
#pragma unroll
        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
            for (int kq = 0; kq < L::KS; ++kq)
                qa[mi][kq] = load8<bf16x8>(Q + ((size_t)h * M + mp0 + 16 * mi + c) * D + 32 * kq + 8 * g);
        // B operand of the cumulative den over the subtile: 1 where tau(g, e) <= t = 16 ti + c
        f16x8 tri[2];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int e = 0; e < 8; ++e) tri[ti][e] = (f16)(tau_slot(g, e) <= 16 * ti + c ? 1.0f : 0.0f);
        // reference starts at the prefix's log-sum-exp: den = 1, U = z.  R is the same on the
        // 16 lanes of a row (latent m = mp0 + 16 mi + 4 g + r).
        float R[L::MTP][4], dn[L::MTP][4], A[L::MTP][4];
        float Cw = kNegInf;
        bool dnbig = false;
        bool rinf = false;   // some latent of this lane has no reference yet (R = -inf)
#pragma unroll
        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = mp0 + 16 * mi + 4 * g + r;
                const float pd = pden[pbase + m];
                R[mi][r] = pd > 0.0f ? pmax[pbase + m] * kLog2e + __log2f(pd) : kNegInf;
                dn[mi][r] = pd > 0.0f ? 1.0f : 0.0f;
                rinf |= R[mi][r] == kNegInf;
            }
        // C_w = max of this wave's references, A = 2^(R - C_w); refreshed when a reference moves
        auto refresh = [&]() {
            float mx = kNegInf;
#pragma unroll
            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, R[mi][r]);
            Cw = rows_max4_pl(mx);
#pragma unroll
            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) A[mi][r] = Cw == kNegInf ? 0.0f : exp2f_fast(R[mi][r] - Cw);
        };
        refresh();
        // The producers meet once per subtile at an LDS counter (consumers never take
        // part): each adds one arrival and waits for the count of meeting n.  Every
        // producer runs the same subtiles, so the count always arrives; past spin_limit
        // sleeps the wave gives up, counts a fault and flags the chunk for the tokenwise
        // replay, which rewrites its outputs.
        auto meet = [&](int n, bool& gave_up) {
            if (lane == 0) __hip_atomic_fetch_add(&psync, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            int spins = 0;
            while (__hip_atomic_load(&psync, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < L::NP * n) {
                if (spins++ >= spin_limit) {
                    gave_up = true;
                    if (lane == 0) atomicAdd(&g_meet_timeouts_tr, 1u);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        };
        // references and dens at a subtile's start to rsvl / dsvl (lanes c = 0..3 store rows r = c)
        // (one exec-masked store per latent: lane c = r of each row writes latent r; lane-derived
        // values from an opaque copy of the lane id, so that none becomes a loop invariant)
        auto stash = [&](int bf) {
            if constexpr (!SEP) {
                int ls = lane;
                asm volatile("" : "+v"(ls));
                const int cs = ls & 15;
                const int m0 = mp0 + 4 * (ls >> 4);
#pragma unroll
                for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (cs == r) {
                            rsvl[bf][m0 + 16 * mi + r] = R[mi][r];
                            dsvl[bf][m0 + 16 * mi + r] = dn[mi][r];
                        }
            }
        };
        KDma<D, 64 * L::NP> kdma;
        kdma.init(K, row0, stride, t_begin, ptid);
        kdma.issue(ksl0, 0, t_begin, N, stride, ptid, lane);
        FLARE_WAIT_VMCNT(0);
        __syncthreads();   // B0: K rows of subtile 0 visible
        auto subtile = [&](auto parity, int j) {
            constexpr int buf = decltype(parity)::value;
            const bf16* kj = buf ? ksl1 : ksl0;
            bf16* knext = buf ? ksl0 : ksl1;
            // lane-derived values are rebuilt from an opaque copy of the lane id each subtile
            int lq = lane;
            asm volatile("" : "+v"(lq));
            const int c = lq & 15, g = lq >> 4;
            if (j < NS) {
                const int t0 = t_begin + T * j;
                // token mask of this lane's tokens (a masked token has S = -inf everywhere)
                bool keep[2] = {true, true};
                if (tmask != nullptr) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int t = t0 + 16 * ti + c;
                        keep[ti] = t >= t_end || tmask[(size_t)b * N + t] != 0;
                    }
                }
                // decoder weights of this lane's tokens and latents (separate decoder only)
                f16x4 af[L::MTP][2];
                if constexpr (SEP) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int t = t0 + 16 * ti + c;
                        const bool ok = t < t_end;
                        const f16* arow = alpha + ((size_t)bh * N + (ok ? t : t0)) * M + mp0 + 4 * g;
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
                            af[mi][ti] = ok ? load4<f16x4>(arow + 16 * mi) : f16x4{0, 0, 0, 0};
                    }
                }
                if (j + 1 < NS) kdma.issue(knext, j + 1, t0 + T, N, stride, 64 * pw + lq, lq);
                // ---- raw scores A = Q K^T: acc[mi][ti][r] = A[t = 16 ti + c][m = 16 mi + 4 g + r]
                const bool ragged = t0 + T > t_end;
                f32x4 acc[L::MTP][2];
#pragma unroll
                for (int mi = 0; mi < L::MTP; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                bf16x8 kb[L::KS][2];
#pragma unroll
                for (int kq = 0; kq < L::KS; ++kq)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const int row = 16 * ti + c;
                        kb[kq][ti] = load8<bf16x8>(kj + row * D + 8 * swz<D>(row, 4 * kq + g));
                    }
#pragma unroll
                for (int kq = 0; kq < L::KS; ++kq)
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) acc[mi][ti] = mma_in<F16>(qa[mi][kq], kb[kq][ti], acc[mi][ti]);
                bool valid[2];
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) valid[ti] = t0 + 16 * ti + c < t_end && keep[ti];
                if (ragged || tmask != nullptr) {
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
                        if (!valid[ti])
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi) acc[mi][ti] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
                }
                if constexpr (SMX) {
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[mi][ti][r] = smx_log2(acc[mi][ti][r], scale2, power);
                }
                // one tile of the same scores again (general path only)
                auto scores = [&](int mi, int ti) {
                    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
                    const int row = 16 * ti + c;
#pragma unroll
                    for (int kq = 0; kq < L::KS; ++kq)
                        a = mma_in<F16>(qa[mi][kq], load8<bf16x8>(kj + row * D + 8 * swz<D>(row, 4 * kq + g)), a);
                    if (!valid[ti]) a = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
                    if constexpr (SMX) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) a[r] = smx_log2(a[r], scale2, power);
                    }
                    return a;
                };
                // ---- E = 2^(S - R) against the current references
                float e[L::MTP][2][4];
                float emax = 0.0f;
                f16x4 e16[L::MTP][2];     // E in fp16: the MFMA operand of the partials, den and numerator
                auto exps = [&]() __attribute__((always_inline)) {
                    emax = 0.0f;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            e[mi][0][r] = exp2f_fast(fmaf(acc[mi][0][r], scale2, -R[mi][r]));
                            e[mi][1][r] = exp2f_fast(fmaf(acc[mi][1][r], scale2, -R[mi][r]));
                            emax = fmaxf(emax, fmaxf(e[mi][0][r], e[mi][1][r]));
                        }
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti)
                            e16[mi][ti] = __builtin_convertvector(
                                (f32x4{e[mi][ti][0], e[mi][ti][1], e[mi][ti][2], e[mi][ti][3]}), f16x4);
                };
                if (__any(rinf)) {
                    // Some latent has no reference yet.  When no latent of the wave has one
                    // (nothing accumulated: a chunk with no earlier tokens) the references
                    // start at the subtile's log-sum-exp without a move, so there is nothing
                    // to rescale and the subtile takes the common path -- provided every
                    // E is at least 2^-12 (a token's den is then a sum of fp16 values with
                    // their full 11 bits) and every token of the subtile is valid (a masked
                    // token before the first valid one would have den 0).
                    bool seen = false;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) seen |= R[mi][r] != kNegInf;
                    if (!__any(seen)) {
                        bool tiny = false;
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                float x = row_max16(fmaxf(acc[mi][0][r], acc[mi][1][r])) * scale2;
                                tiny |= x == kNegInf;
                                if (x != kNegInf)
                                    x += __log2f(row_sum16(exp2f_fast(fmaf(acc[mi][0][r], scale2, -x)) +
                                                           exp2f_fast(fmaf(acc[mi][1][r], scale2, -x))));
#pragma unroll
                                for (int ti = 0; ti < 2; ++ti)
                                    tiny |= !valid[ti] | (fmaf(acc[mi][ti][r], scale2, -x) < -12.0f);
                                R[mi][r] = x;
                            }
                        if (__any(tiny)) {
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                                for (int r = 0; r < 4; ++r) R[mi][r] = kNegInf;
                        } else {
                            refresh();
                            rinf = false;
                        }
                    }
                }
                exps();
                dnbig |= rinf;   // some latent has no reference yet (fully masked so far): general path
                bool moved = __any((emax > L::kLazyE) | dnbig);
                bool jumped = false, gave_up = false;   // (flags of this subtile, wave-uniform)
                if (moved) {
                    stash(buf);     // the state before the move, for a replay record
                    // every latent of the wave had den 0 so far (a chunk with no earlier tokens)
                    float gam[L::MTP][4];
                    bool jump = false;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float mx = row_max16(fmaxf(acc[mi][0][r], acc[mi][1][r])) * scale2;
                            float Rn = mx > R[mi][r] + kLazy ? mx : R[mi][r];
                            // The running max of this latent at the subtile's first valid token:
                            // R, or (no reference yet) the smallest valid score.  Tokens whose
                            // running max lies more than kJumpMax below the new reference would
                            // see their den underflow against it: such a chunk is replayed
                            // tokenwise by the fp32 kernel afterwards.
                            const float s0 = acc[mi][0][r] * scale2, s1 = acc[mi][1][r] * scale2;
                            const float mn = -row_max16(fmaxf(s0 == kNegInf ? kNegInf : -s0, s1 == kNegInf ? kNegInf : -s1));
                            const float base = R[mi][r] == kNegInf ? mn : R[mi][r];
                            float g1 = exp2f_fast(R[mi][r] - Rn);                  // 0 when R = -inf
                            // den at the subtile's end against Rn: the old den plus this
                            // subtile's E.  Above 1 the reference rises to its log-sum-exp, so
                            // the den restarts at 1 and one move covers the subtile's own growth
                            // (a first subtile of flat scores would otherwise move again next).
                            float ss = 0.0f;
                            if (Rn != kNegInf)
                                ss = row_sum16(exp2f_fast(fmaf(acc[mi][0][r], scale2, -Rn)) +
                                               exp2f_fast(fmaf(acc[mi][1][r], scale2, -Rn)));
                            const float dd = dn[mi][r] * g1 + ss;
                            if (dd > 1.0f) {
                                Rn += __log2f(dd);
                                g1 = exp2f_fast(R[mi][r] - Rn);
                            }
                            jump |= Rn - base > kJumpMax;
                            gam[mi][r] = Rn == R[mi][r] ? 1.0f : g1;
                            R[mi][r] = Rn;
                            dn[mi][r] *= gam[mi][r];     // E is recomputed on the general path
                        }
                    if (jump) {
                        if constexpr (SEP) redol = 1;
                        else jumpl[buf] = j + 1;
                    }
                    jumped = __any(jump);
                    refresh();
                    rinf = false;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) rinf |= R[mi][r] == kNegInf;
                    // rescale factor and den at the subtile start: lanes c = 0..3 store rows r = c
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
                        float gsel = gam[mi][0], dsel = dn[mi][0];
#pragma unroll
                        for (int r = 1; r < 4; ++r) {
                            gsel = c == r ? gam[mi][r] : gsel;
                            dsel = c == r ? dn[mi][r] : dsel;
                        }
                        if (c < 4) {
                            gaml[buf][mp0 + 16 * mi + 4 * g + c] = gsel;
                            d0l[buf][mp0 + 16 * mi + 4 * g + c] = dsel;
                        }
                    }
                }
                // ---- the token softmax over all M latents: publish (reference, partial) per
                //      token, meet, merge; f[ti] = 2^(ref - lse_t) for this lane's tokens
                bool slow = moved;
                float ref[2] = {Cw, Cw}, f[2] = {0.0f, 0.0f};
                if constexpr (!SEP) {
                    float part[2] = {0.0f, 0.0f};
                    if (!moved) {
                        // sum_m E[t,m] A[m] over this wave's latents in fp32 (16 latents per lane,
                        // then the four lane rows): A spans the spread of the references, which
                        // can run past the fp16 range; the E rows then go to LDS at once
                        // (common path)
                        float pt[2] = {0.0f, 0.0f};
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                pt[0] = fmaf(e[mi][0][r], A[mi][r], pt[0]);
                                pt[1] = fmaf(e[mi][1][r], A[mi][r], pt[1]);
                            }
                        part[0] = rows_sum4_pl(pt[0]);
                        part[1] = rows_sum4_pl(pt[1]);
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti)
                                *reinterpret_cast<f16x4*>(erl[buf] + (16 * ti + c) * L::RPE + mp0 + 16 * mi + 4 * g) =
                                    e16[mi][ti];
                        slow = __any((valid[0] & (part[0] < L::kTinyL)) | (valid[1] & (part[1] < L::kTinyL)));
                    }
                    if (slow) {
                        // exact pair per token: (max_m S, sum_m 2^(S - max)) over this wave's latents
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) {
                            f32x4 sc[L::MTP];
                            float mx = kNegInf;
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi) {
                                sc[mi] = scores(mi, ti);
                                mx = max3_raw(mx, max3_raw(sc[mi][0], sc[mi][1], sc[mi][2]), sc[mi][3]);
                            }
                            const float lm = rows_max4_pl(mx) * scale2;
                            float ls = 0.0f;
#pragma unroll
                            for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    ls += lm == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[mi][r], scale2, -lm));
                            ref[ti] = lm;
                            part[ti] = rows_sum4_pl(ls);
                        }
                    }
                    if (g == 0) {
                        lsep[buf][pw][c] = float2{ref[0], part[0]};
                        lsep[buf][pw][16 + c] = float2{ref[1], part[1]};
                    }
                    meet(j + 1, gave_up);
                    // a jump in another producer's latents: this wave's (unmoved) state too
                    if (jumpl[buf] == j + 1 && !moved) stash(buf);
                    // merge: lane row g reads producer g's pair
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        const float2 pr = g < L::NP ? lsep[buf][g][16 * ti + c] : float2{kNegInf, 0.0f};
                        const float mm = rows_max4_pl(pr.x);
                        const float s = pr.y > 0.0f ? pr.y * exp2f_fast(pr.x - mm) : 0.0f;
                        const float ss = rows_sum4_pl(s);
                        f[ti] = (ss > 0.0f && ref[ti] != kNegInf) ? exp2f_fast(ref[ti] - mm) * __builtin_amdgcn_rcpf(ss)
                                                                 : 0.0f;
                    }
                }
                // the W path (the end of the producers' chain) outranks the consumers' readout
                __builtin_amdgcn_s_setprio(3);
                f16* er = erl[buf];
                f16* wq = wl[buf];
                // (separate decoder weights: no softmax partials, so slow == moved)
                auto light_path = [&](bool mv) {
                    if constexpr (SEP) return false;
                    else return !mv;
                };
                dnbig = false;
                if (!slow) {
                    // ---- common path: E rows to LDS (fp16), the cumulative den
                    //      d_t = d0 + sum_{tau<=t} E by MFMA against tri (E^T read transposed),
                    //      W = alpha / d_t (fp16) rows to LDS
                    if constexpr (SEP) {     // (shared weights: stored with the softmax partials)
#pragma unroll
                        for (int mi = 0; mi < L::MTP; ++mi)
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti)
                                *reinterpret_cast<f16x4*>(er + (16 * ti + c) * L::RPE + mp0 + 16 * mi + 4 * g) = e16[mi][ti];
                    }
                    f32x4 dcum[L::MTP][2];
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
                        const f16* col = er + mp0 + 16 * mi + 4 * (c & 3);
                        const f16x8 ea = cat8<f16x8>(lds_tr4(col + (4 * g + (c >> 2)) * L::RPE),
                                                     lds_tr4(col + (16 + 4 * g + (c >> 2)) * L::RPE));
                        const f32x4 d0 = f32x4{dn[mi][0], dn[mi][1], dn[mi][2], dn[mi][3]};
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) dcum[mi][ti] = mma(ea, tri[ti], d0);
                    }
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) {
                            f32x4 q;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float p = SEP ? (float)af[mi][ti][r] : e[mi][ti][r] * (A[mi][r] * f[ti]);
                                q[r] = p * __builtin_amdgcn_rcpf(dcum[mi][ti][r]);
                            }
                            *reinterpret_cast<f16x4*>(wq + (16 * ti + c) * L::RPW + mp0 + 16 * mi + 4 * g) =
                                __builtin_convertvector(q, f16x4);
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) dn[mi][r] = row_bcast15(dcum[mi][1][r]);   // den at t = 31
                    }
                    float dmx = 0.0f;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) dmx = fmaxf(dmx, fmaxf(fmaxf(dn[mi][0], dn[mi][1]), fmaxf(dn[mi][2], dn[mi][3])));
                    dnbig = dmx > kDenMax;
                } else if (light_path(moved)) {
                    // ---- a token's softmax partial would underflow against C_w, and no reference
                    //      moved (e.g. latents whose reference jumped far above every later score:
                    //      their E underflows while their alpha does not).  As the common path,
                    //      with alpha = 2^(S - ref) f from the scores again instead of E A f.
                    f32x4 dcum[L::MTP][2];
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
                        const f16* col = er + mp0 + 16 * mi + 4 * (c & 3);
                        const f16x8 ea = cat8<f16x8>(lds_tr4(col + (4 * g + (c >> 2)) * L::RPE),
                                                     lds_tr4(col + (16 + 4 * g + (c >> 2)) * L::RPE));
                        const f32x4 d0 = f32x4{dn[mi][0], dn[mi][1], dn[mi][2], dn[mi][3]};
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) dcum[mi][ti] = mma(ea, tri[ti], d0);
                    }
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) {
#pragma unroll
                        for (int ti = 0; ti < 2; ++ti) {
                            const f32x4 sc = scores(mi, ti);
                            f32x4 q;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float p = ref[ti] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[r], scale2, -ref[ti])) * f[ti];
                                q[r] = p * __builtin_amdgcn_rcpf(dcum[mi][ti][r]);
                            }
                            *reinterpret_cast<f16x4*>(wq + (16 * ti + c) * L::RPW + mp0 + 16 * mi + 4 * g) =
                                __builtin_convertvector(q, f16x4);
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) dn[mi][r] = row_bcast15(dcum[mi][1][r]);   // den at t = 31
                    }
                    float dmx = 0.0f;
#pragma unroll
                    for (int mi = 0; mi < L::MTP; ++mi) dmx = fmaxf(dmx, fmaxf(fmaxf(dn[mi][0], dn[mi][1]), fmaxf(dn[mi][2], dn[mi][3])));
                    dnbig = dmx > kDenMax;
                    slow = false;     // the consumers form this wave's share of G as on the common path
                } else {
                    // ---- general path: alpha = 2^(S - ref) f, guarded 1 / d_t, W1 = W d0 when a reference
                    //      moved (the consumers then read out z0 = U / d0), this wave's share of G^T in fp32
                    //      from bf16 hi/lo splits
                    f32x4 gacc[3];    // G^T tiles (tau tile, t tile) = (0,0), (0,1), (1,1)
#pragma unroll
                    for (int q3 = 0; q3 < 3; ++q3) gacc[q3] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < L::MKP; ++kk) {
                        bf16x4 ehi[2][2], elo[2][2], whi[2][2], wlo[2][2];
#pragma unroll
                        for (int jb = 0; jb < 2; ++jb) {
                            const int mi = 2 * kk + jb;
                            const f32x4 sc[2] = {scores(mi, 0), scores(mi, 1)};
                            float em[2][4];
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    em[ti][r] = R[mi][r] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[ti][r], scale2, -R[mi][r]));
                            // E rows (fp16) to LDS; the cumulative den in fp32 (DPP scans over the token
                            // lanes): here E may lie far below the fp16 range
                            f32x4 dcum[2];
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti)
                                *reinterpret_cast<f16x4*>(er + (16 * ti + c) * L::RPE + mp0 + 16 * mi + 4 * g) =
                                    __builtin_convertvector((f32x4{em[ti][0], em[ti][1], em[ti][2], em[ti][3]}), f16x4);
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float c0 = row_scan16(em[0][r]);
                                dcum[0][r] = c0;
                                dcum[1][r] = row_bcast15(c0) + row_scan16(em[1][r]);
                            }
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti) {
                                float q[4];
                                f16x4 w1;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    const float dt = dn[mi][r] + dcum[ti][r];
                                    const float p = SEP ? (float)af[mi][ti][r]
                                                        : ref[ti] == kNegInf ? 0.0f : exp2f_fast(fmaf(sc[ti][r], scale2, -ref[ti])) * f[ti];
                                    q[r] = dt > 0.0f ? p * __builtin_amdgcn_rcpf(dt) : 0.0f;
                                    w1[r] = (f16)(moved ? q[r] * dn[mi][r] : q[r]);
                                }
                                split_bf16x4(em[ti][0], em[ti][1], em[ti][2], em[ti][3], ehi[jb][ti], elo[jb][ti]);
                                split_bf16x4(q[0], q[1], q[2], q[3], whi[jb][ti], wlo[jb][ti]);
                                *reinterpret_cast<f16x4*>(wq + (16 * ti + c) * L::RPW + mp0 + 16 * mi + 4 * g) = w1;
                            }
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                dn[mi][r] += row_bcast15(dcum[1][r]);
                                dnbig |= dn[mi][r] > kDenMax;
                            }
                        }
#pragma unroll
                        for (int q3 = 0; q3 < 3; ++q3) {
                            const int ui = q3 == 2 ? 1 : 0, ti = q3 == 0 ? 0 : 1;
                            const bf16x8 e_h = cat8<bf16x8>(ehi[0][ui], ehi[1][ui]);
                            const bf16x8 e_o = cat8<bf16x8>(elo[0][ui], elo[1][ui]);
                            const bf16x8 wh = cat8<bf16x8>(whi[0][ti], whi[1][ti]);
                            const bf16x8 wo = cat8<bf16x8>(wlo[0][ti], wlo[1][ti]);
                            gacc[q3] = mma(e_h, wh, gacc[q3]);
                            gacc[q3] = mma(e_o, wh, gacc[q3]);
                            gacc[q3] = mma(e_h, wo, gacc[q3]);
                        }
                    }
#pragma unroll
                    for (int q3 = 0; q3 < 3; ++q3) gpl[buf][pw][q3][lq] = gacc[q3];
                }
                __builtin_amdgcn_s_setprio(0);
                if (lq == 0) movedl[buf][pw] = (moved ? 1 : 0) | (slow ? 2 : 0) | (jumped ? 4 : 0) | (gave_up ? 8 : 0);
                FLARE_WAIT_VMCNT(0);     // this wave's K rows of the next subtile have landed
            }
            __syncthreads();   // hand-off: subtile j's operands visible, subtile j-1's consumed
        };
        for (int j = 0; j <= NS; j += 2) {
            subtile(std::integral_constant<int, 0>{}, j);
            if (j + 1 <= NS) subtile(std::integral_constant<int, 1>{}, j + 1);
        }
    } else {
        // =========================== consumer ===========================
        const int cw = L::IL ? w >> 1 : w - L::NP;
        const int dc0 = cw * L::DC;
        // U[mi][di][r] = U[m][d = dc0 + 16 di + c] for latent m = lat(mi, g) + r: lane row g holds
        // the 8 consecutive latents 32 k + 8 g .. + 7 of each 32-latent k-step k in tiles 2 k and
        // 2 k + 1, so that one 16-byte LDS read gives the matching W or E operand of the readout
        auto lat = [](int mi, int gg) { return 32 * (mi >> 1) + 8 * gg + 4 * (mi & 1); };
        f32x4 U[L::MTA][L::DTC];
#pragma unroll
        for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pd = pden[pbase + lat(mi, g) + r];
                const float ip = pd > 0.0f ? 1.0f / pd : 0.0f;
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
                    U[mi][di][r] = pnum[(pbase + lat(mi, g) + r) * D + dc0 + 16 * di + c] * ip;
            }
        // The wave keeps V' = V vs and U' = U vs with vs a power of two <= 1 chosen so
        // that |V'| and the prefix's |z'| stay below kVCap: every fp16 operand below is
        // then in range (|U'| <= kDenMax kVCap, |z0'| <= kVCap); y is scaled back at the store.
        float vs = 1.0f;
        {
            float zmax = 0.0f;
#pragma unroll
            for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
#pragma unroll
                    for (int r = 0; r < 4; ++r) zmax = fmaxf(zmax, fabsf(U[mi][di][r]));
            zmax = wave_max_dpp(zmax);
            if (zmax > L::kVCap && __builtin_isfinite(zmax)) {
                int ex;
                frexpf(zmax / L::kVCap, &ex);
                vs = ldexpf(1.0f, -ex);
#pragma unroll
                for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) U[mi][di] *= vs;
            }
        }
        // V and Y rows of this chunk through buffer resources: rows past the chunk's end
        // load 0 and drop their stores, so every subtile issues the same memory instructions
        const int esize = out_dtype == FLARE_F32 ? 4 : 2;
        const size_t vbase = row0 + (size_t)t_begin * stride;
        const unsigned rbytes = (unsigned)((size_t)(t_end - t_begin - 1) * stride + D);
        const __amdgpu_buffer_rsrc_t vres = buffer_rsrc(V + vbase, rbytes * 2);
        const __amdgpu_buffer_rsrc_t yres = buffer_rsrc((char*)Y + vbase * esize, rbytes * esize);
        // slot k of this lane: token tau = s / 4, columns 8 (s % 4) .. +7 of the wave's 32, s = lane + 64 k
        u32x4 vr[2];
        auto vload = [&](int tl) {     // tl: subtile start relative to t_begin
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int s = lane + 64 * k;
                vr[k] = __builtin_amdgcn_raw_buffer_load_b128(
                    vres, (unsigned)(((size_t)(tl + (s >> 2)) * stride + dc0 + 8 * (s & 3)) * 2), 0, 0);
            }
        };
        f16* vw = vrl[cw];
        vload(0);
        FLARE_WAIT_VMCNT(0);
        __syncthreads();   // B0
        for (int it = 0; it <= NS; ++it) {
            if (it > 0) {
                const int j = it - 1;
                const int buf = j & 1;
                const int tl = T * j;
                int mv[L::NP];
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2) mv[w2] = movedl[buf][w2];
                if constexpr (!SEP) {
                    // A reference jumped in subtile j (or a meeting gave up): the first such
                    // subtile's starting state -- U here, before this subtile's rescales, and
                    // the producers' stashed references and dens -- goes to the chunk's prefix
                    // slot, and the replay covers subtiles rj1 .. rj2.  A meeting that gave up
                    // before any record leaves the prefix intact for a whole-chunk replay.
                    int fl = 0;
#pragma unroll
                    for (int w2 = 0; w2 < L::NP; ++w2) fl |= mv[w2];
                    const bool tj = (fl & 8) != 0, jj = (fl & 4) != 0;
                    if (fl & 12) {
                        if (tj) {
                            if (rj1 < 0) rwhole = true;
                            else rj2 = NS - 1;
                        }
                        if (jj && !rwhole) {
                            if (!record) {
                                rwhole = true;
                            } else {
                                if (rj1 < 0) {
                                    rj1 = j;
                                    // buffer stores: one per-lane offset, the per-entry offsets
                                    // are constants (plain addresses would be loop invariants that
                                    // the compiler keeps live across the subtile loop)
                                    const __amdgpu_buffer_rsrc_t nres =
                                        buffer_rsrc(pnum + pbase * D, (unsigned)(M * D * 4));
                                    const unsigned voff = (unsigned)((8 * g * D + dc0 + c) * 4);
                                    const float iv = 1.0f / vs;
#pragma unroll
                                    for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                                        for (int di = 0; di < L::DTC; ++di)
#pragma unroll
                                            for (int r = 0; r < 4; ++r)
                                                __builtin_amdgcn_raw_buffer_store_b32(
                                                    __builtin_bit_cast(unsigned, U[mi][di][r] * iv), nres, voff,
                                                    ((32 * (mi >> 1) + 4 * (mi & 1) + r) * D + 16 * di) * 4, 0);
                                    if (cw == 0) {
                                        float* rmax = const_cast<float*>(pmax);
                                        float* rden = const_cast<float*>(pden);
                                        for (int m = lane; m < M; m += 64) {
                                            const float rr = rsvl[buf][m];
                                            rmax[pbase + m] = rr == kNegInf ? kNegInf : rr * kLn2;
                                            rden[pbase + m] = dsvl[buf][m];
                                        }
                                    }
                                }
                                rj2 = max(rj2, j);
                            }
                        }
                    }
                }
                // ---- V' rows of subtile j (fp16) to this wave's LDS region
                float vv[2][8];
                float vlane = 0.0f;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const bf16x8 x = __builtin_bit_cast(bf16x8, vr[k]);
#pragma unroll
                    for (int e2 = 0; e2 < 8; ++e2) {
                        vv[k][e2] = in_f32<F16>(x[e2]);
                        vlane = fmaxf(vlane, fabsf(vv[k][e2]));
                    }
                }
                vlane *= vs;
                vlane = __builtin_isfinite(vlane) ? vlane : 0.0f;   // inf / nan propagate unscaled
                if (__any(vlane > L::kVCap)) {      // rare: rescale the wave's columns
                    const float vmax = wave_max_dpp(vlane);
                    int ex;
                    frexpf(vmax / L::kVCap, &ex);
                    const float fsc = ldexpf(1.0f, -ex);
                    vs *= fsc;
#pragma unroll
                    for (int mi = 0; mi < L::MTA; ++mi)
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) U[mi][di] *= fsc;
                }
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int s = lane + 64 * k;
                    f16x8 o;
#pragma unroll
                    for (int e2 = 0; e2 < 8; ++e2) o[e2] = (f16)(vv[k][e2] * vs);
                    *reinterpret_cast<f16x8*>(vw + (s >> 2) * L::VP + 8 * (s & 3)) = o;
                }
                vload(tl + T);    // the next subtile's V (past the chunk's end: zeros, unused)
                // The readout runs at a raised wave priority: its fp16 conversions of U
                // otherwise queue behind the producer's exponentials on the shared SIMD
                // and hold up the MFMAs behind them (measured: config 3's readout 3870 ->
                // 2140 cycles per subtile).
                __builtin_amdgcn_s_setprio(2);
                // ---- readout at the subtile start, y = sum_m W1[t,m] U[m], fused with
                //      G^T[tau][t] = sum_m E[tau,m] W[t,m] over the producers on the common path;
                //      for the latents of a producer that moved a reference, z0 = U / d0
                auto normalise = [&](int w2, bool back) {
#pragma unroll
                    for (int mt = 0; mt < L::MTP; ++mt) {
                        const int mi = w2 * L::MTP + mt;
                        const f32x4 da = *reinterpret_cast<const f32x4*>(d0l[buf] + lat(mi, g));
                        f32x4 gm;
                        if (back) {
                            gm = da;
                        } else {
                            const f32x4 ga = *reinterpret_cast<const f32x4*>(gaml[buf] + lat(mi, g));
#pragma unroll
                            for (int r = 0; r < 4; ++r) gm[r] = da[r] > 0.0f ? ga[r] / da[r] : 0.0f;
                        }
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) U[mi][di] *= gm;
                    }
                };
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2)
                    if (mv[w2] & 1) normalise(w2, false);
                const f16* wq = wl[buf];
                const f16* er = erl[buf];
                f32x4 yt[L::DTC][2], gt[3];
#pragma unroll
                for (int di = 0; di < L::DTC; ++di) yt[di][0] = yt[di][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q3 = 0; q3 < 3; ++q3) gt[q3] = f32x4{0.f, 0.f, 0.f, 0.f};
                // W rows (B operands: t = 16 ti + c, the k-step's latent slots) and E rows
                // (A operands of G^T: tau = 16 ui + c) of k-step kk, fetched one step ahead.  The
                // loop comes in two copies: without a general-path producer (the common case) it
                // has no branch, so the loads of one step overlap the MFMAs of the previous one.
                auto fused = [&](auto any_general) {
                    constexpr bool AG = decltype(any_general)::value;
                    f16x8 wbn[2], ean[2];
                    auto fetch = [&](int kk) {
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            wbn[q] = load8<f16x8>(wq + (16 * q + c) * L::RPW + 32 * kk + 8 * g);
                            ean[q] = load8<f16x8>(er + (16 * q + c) * L::RPE + 32 * kk + 8 * g);
                        }
                    };
                    fetch(0);
#pragma unroll
                    for (int kk = 0; kk < L::MK; ++kk) {
                        const f16x8 wb[2] = {wbn[0], wbn[1]};
                        const f16x8 ea[2] = {ean[0], ean[1]};
                        if (kk + 1 < L::MK) fetch(kk + 1);
#pragma unroll
                        for (int di = 0; di < L::DTC; ++di) {
                            f16x8 za;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                za[r] = (f16)U[2 * kk][di][r];
                                za[4 + r] = (f16)U[2 * kk + 1][di][r];
                            }
#pragma unroll
                            for (int ti = 0; ti < 2; ++ti) yt[di][ti] = mma(za, wb[ti], yt[di][ti]);
                        }
                        if (!AG || !(mv[kk / L::MKP] & 2)) {
                            gt[0] = mma(ea[0], wb[0], gt[0]);
                            gt[1] = mma(ea[0], wb[1], gt[1]);
                            gt[2] = mma(ea[1], wb[1], gt[2]);
                        }
                    }
                };
                int anyg = 0;
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2) anyg |= mv[w2];
                if (anyg & 2) fused(std::true_type{});
                else fused(std::false_type{});
#pragma unroll
                for (int w2 = 0; w2 < L::NP; ++w2) {
                    if (mv[w2] & 1) normalise(w2, true);    // back from z0 to the (rescaled) numerator
                    if (mv[w2] & 2)
#pragma unroll
                        for (int q3 = 0; q3 < 3; ++q3) gt[q3] += gpl[buf][w2][q3][lane];
                }
                __builtin_amdgcn_s_setprio(0);
                // ---- V' operands in slot order (rows tau(g, e), column d = 16 di + c)
                f16x8 va[L::DTC];
#pragma unroll
                for (int di = 0; di < L::DTC; ++di) {
                    const f16* col = vw + 16 * di + 4 * (c & 3);
                    va[di] = cat8<f16x8>(lds_tr4(col + (4 * g + (c >> 2)) * L::VP),
                                         lds_tr4(col + (16 + 4 * g + (c >> 2)) * L::VP));
                }
                // ---- + V'^T G^T (causal: tau <= t) with G = hi + lo in fp16: early in a sequence
                //      G is O(1) and y a cancelling sum, where one fp16 rounding of G is too coarse
                f16x8 gh[2], gl[2];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool on = 4 * g + r <= c;     // diagonal tiles
                    const float x[4] = {on ? gt[0][r] : 0.0f, 0.0f, gt[1][r], on ? gt[2][r] : 0.0f};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f16 hq = (f16)x[q];
                        gh[q >> 1][4 * (q & 1) + r] = hq;
                        gl[q >> 1][4 * (q & 1) + r] = (f16)(x[q] - (float)hq);
                    }
                }
#pragma unroll
                for (int di = 0; di < L::DTC; ++di)
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        yt[di][ti] = mma(va[di], gh[ti], yt[di][ti]);
                        yt[di][ti] = mma(va[di], gl[ti], yt[di][ti]);
                    }
                // ---- U' += E^T V' (E^T read transposed from the E rows)
#pragma unroll
                for (int mi = 0; mi < L::MTA; ++mi) {
                    const f16* col = er + 32 * (mi >> 1) + 4 * (mi & 1) + 8 * (c & 3);   // latents lat(mi, .)
                    const f16x8 et = cat8<f16x8>(lds_tr4(col + (4 * g + (c >> 2)) * L::RPE),
                                                 lds_tr4(col + (16 + 4 * g + (c >> 2)) * L::RPE));
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) U[mi][di] = mma(et, va[di], U[mi][di]);
                }
                // ---- Y[b, t, h, d]: token t = 16 ti + c, columns dc0 + 16 di + 4 g .. + 3
                const float ys = vs == 1.0f ? 1.0f : 1.0f / vs;
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                    for (int di = 0; di < L::DTC; ++di) {
                        const f32x4 v = yt[di][ti] * ys;
                        const unsigned off = (unsigned)((size_t)(tl + 16 * ti + c) * stride + dc0 + 16 * di + 4 * g);
                        if (out_dtype == FLARE_F32) {
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yres, off * 4, 0, 0);
                        } else if (out_dtype == FLARE_F16) {
                            __builtin_amdgcn_raw_buffer_store_b64(
                                __builtin_bit_cast(u32x2, __builtin_convertvector(v, f16x4)), yres, off * 2, 0, 0);
                        } else {
                            bf16x4 o;
                            o[0] = (bf16)v[0]; o[1] = (bf16)v[1]; o[2] = (bf16)v[2]; o[3] = (bf16)v[3];
                            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), yres, off * 2, 0, 0);
                        }
                    }
            }
            __syncthreads();   // hand-off
        }
    }
    if (redo != nullptr) {
        __syncthreads();
        if constexpr (SEP) {
            if (tid == 0) redo[(size_t)bh * nchunks + c_idx] = redol;
        } else {
            if (!producer && w == (L::IL ? 1 : L::NP) && lane == 0) {   // the first consumer
                const int fl = rwhole ? kRedoWhole : rj1 >= 0 ? redo_narrow(rj1, rj2) : 0;
                redo[(size_t)bh * nchunks + c_idx] = fl;
                redol = fl;
            }
            // In-place replay of a flagged chunk: slice s of the value columns by threads
            // 256 s .. 256 s + 255, over the E / W rows (free once the subtiles are done).
            using RS = ReplayShape<M, D>;
            if constexpr (RS::NSL * kNT == L::NT) {
                static_assert(RS::NSL <= 2 && sizeof(erl) == sizeof(wl), "one LDS region per replay slice");
                static_assert(OutSmem{RS::template tt<sizeof(erl)>(), D, RS::DT, M, kNT / RS::DT, (kNT / RS::DT) * RS::ROWS,
                                      true}.floats() * sizeof(float) <= sizeof(erl),
                              "the replay's LDS scratch fits one region");
                if (replay) {
                    __syncthreads();
                    const int fl = redol;
                    if (fl != 0) {
                        using TI = std::conditional_t<F16, __half, __hip_bfloat16>;
                        const int sl = tid / kNT;
                        float* sm = reinterpret_cast<float*>(sl == 0 ? erl[0] : wl[0]);
                        output_chunk_replay<TI, RS::ROWS>(
                            (const TI*)Q, (const TI*)K, (const TI*)V, (const TI*)K, (const TI*)Q, N, H, M, D, D, RS::DT,
                            RS::template tt<sizeof(erl)>(), scale, chunk, true, pmax, pden, pnum, Y, out_dtype, nullptr,
                            tmask, 0.0f, sm, c_idx, bh, sl * RS::DT, nchunks, tid % kNT, fl);
                    }
                }
            }
        }
    }
}

}  // namespace mfma

using namespace mfma;

int launch_output_tr(const void* Q, const void* K, const void* V, int64_t B, int64_t N, int64_t H, int64_t M,
                     int64_t D, float scale, int64_t chunk, const float* pmax, const float* pden,
                     const float* pnum, void* Y, int out_dtype, const int32_t* tmask, const void* alpha,
                     bool f16in, int* redo, int spin_limit, hipStream_t stream, bool record, float power) {
    FLARE_REQUIRE(chunk % T == 0, "chunk_output_tr: chunk must be a multiple of %d", T);
    FLARE_REQUIRE(power <= 0.0f || alpha != nullptr, "chunk_output_tr: the stablemax encoder needs decoder weights");
    // a narrow redo flag holds subtile indices below kRedoMaxSubtiles
    const int rec = record && alpha == nullptr && chunk / T < kRedoMaxSubtiles ? 1 : 0;
    FLARE_REQUIRE((M == 128 || M == 256) && (D == 64 || D == 128),
                  "chunk_output_tr: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    FLARE_REQUIRE((uint64_t)chunk * H * D * 4 < (1ull << 31), "chunk_output_tr: chunk too long for 32-bit offsets");
    const int64_t NC = (N + chunk - 1) / chunk;
    dim3 grid((unsigned)NC, (unsigned)(B * H));
    const float s2 = scale * kLog2e;
    const int inl = redo != nullptr && alpha == nullptr && output_tr_replays_inline(M, D, false) ? 1 : 0;
#define FLARE_OUT_TR_T(MM, DD, SP, F, SX)                                                                      \
    hipLaunchKernelGGL((chunk_output_tr<MM, DD, SP, F, SX>), grid, dim3(64 * (MM / 64 + DD / 32)), 0, stream,  \
                       (const bf16*)Q, (const bf16*)K, (const bf16*)V, (int)N, (int)H, s2, (int)chunk, pmax, pden, \
                       pnum, Y, out_dtype, tmask, (const f16*)alpha, redo, spin_limit, rec, power, scale,      \
                       inl)
#define FLARE_OUT_TR(MM, DD)                                            \
    do {                                                                \
        if (f16in) {                                                    \
            if (alpha && power > 0.0f) FLARE_OUT_TR_T(MM, DD, true, true, true); \
            else if (alpha) FLARE_OUT_TR_T(MM, DD, true, true, false);  \
            else FLARE_OUT_TR_T(MM, DD, false, true, false);            \
        } else {                                                        \
            if (alpha && power > 0.0f) FLARE_OUT_TR_T(MM, DD, true, false, true); \
            else if (alpha) FLARE_OUT_TR_T(MM, DD, true, false, false); \
            else FLARE_OUT_TR_T(MM, DD, false, false, false);           \
        }                                                               \
    } while (0)
    if (M == 128 && D == 64) FLARE_OUT_TR(128, 64);
    else if (M == 128 && D == 128) FLARE_OUT_TR(128, 128);
    else if (M == 256 && D == 64) FLARE_OUT_TR(256, 64);
    else FLARE_OUT_TR(256, 128);
#undef FLARE_OUT_TR
#undef FLARE_OUT_TR_T
    return check_launch("chunk_output_tr");
}

bool output_tr_replays_inline(int64_t M, int64_t D, bool sep) {
    if (sep || !output_pc_enabled() || !output_tr_enabled()) return false;
#define FLARE_INL(MM, DD) (ReplayShape<MM, DD>::NSL * kNT == TrLayout<MM, DD>::NT)
    if (M == 128 && D == 64) return FLARE_INL(128, 64);
    if (M == 128 && D == 128) return FLARE_INL(128, 128);
    if (M == 256 && D == 64) return FLARE_INL(256, 64);
    if (M == 256 && D == 128) return FLARE_INL(256, 128);
#undef FLARE_INL
    return false;
}

int meet_timeouts_tr(hipStream_t stream, unsigned int* count, bool reset) {
    if (hipMemcpyFromSymbolAsync(count, HIP_SYMBOL(g_meet_timeouts_tr), sizeof(unsigned int), 0,
                                 hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return FLARE_ERR_LAUNCH;
    if (reset) {
        const unsigned int z = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(g_meet_timeouts_tr), &z, sizeof(z), 0, hipMemcpyHostToDevice,
                                   stream) != hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess)
            return FLARE_ERR_LAUNCH;
    }
    return FLARE_OK;
}

int output_tr_attributes(int64_t M, int64_t D, bool sep, bool f16in, hipFuncAttributes* attr, int* threads) {
    const void* f = nullptr;
#define FLARE_OUT_TR_F(MM, DD)                                                                          \
    f = sep ? (f16in ? (const void*)chunk_output_tr<MM, DD, true, true> : (const void*)chunk_output_tr<MM, DD, true, false>) \
            : (f16in ? (const void*)chunk_output_tr<MM, DD, false, true> : (const void*)chunk_output_tr<MM, DD, false, false>)
    if (M == 128 && D == 64) FLARE_OUT_TR_F(128, 64);
    else if (M == 128 && D == 128) FLARE_OUT_TR_F(128, 128);
    else if (M == 256 && D == 64) FLARE_OUT_TR_F(256, 64);
    else if (M == 256 && D == 128) FLARE_OUT_TR_F(256, 128);
#undef FLARE_OUT_TR_F
    FLARE_REQUIRE(f != nullptr, "chunk_output_tr: unsupported M=%lld D=%lld", (long long)M, (long long)D);
    *threads = (int)(64 * (M / 64 + D / 32));
    FLARE_REQUIRE(hipFuncGetAttributes(attr, f) == hipSuccess, "chunk_output_tr: hipFuncGetAttributes failed");
    return FLARE_OK;
}

}  // namespace flare
