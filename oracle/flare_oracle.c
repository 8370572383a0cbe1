/*
 * flare_oracle.c -- CPU fp32 restatement of the causal FLARE forward paths.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this file: it is the checker that the HIP kernels are compared with
 * (tests/, __graft_entry__.smoke()) and the CPU baseline that bench.py times.
 *
 * Three functions, each a restatement of one reference algorithm (citations
 * are path:line in vpuri3/causal-flare):
 *
 *   oracle_ar_chunked     causal_flare/autoregressive/reference.py:203-512
 *                         (flare_autoregressive_pytorch: per-chunk summaries,
 *                         exclusive prefix scan over chunks, tokenwise replay)
 *   oracle_ar_recurrent   causal_flare/autoregressive/inference.py:231-315
 *                         (flare_prefill_pytorch; decode = one-token prefill,
 *                         inference.py:318-351)
 *   oracle_semi_ar        causal_flare/semi_autoregressive/reference.py:308-536
 *                         (_block_causal_forward_pytorch)
 *
 * All arithmetic is fp32, as in the reference paths (FLARE_REFERENCE_FP32 and
 * compute_dtype=float32).  Reductions run in plain index order; the reference
 * uses torch einsum/bmm, so the two agree to fp32 rounding, not bitwise.
 *
 * Layouts (all contiguous, row-major):
 *   Q [H,M,Dk]  K [B,N,H,Dk]  V [B,N,H,Dv]  Qdec [B,N,H,Dk]  Kdec [H,M,Dk]
 *   mask [B,N] (uint8, nonzero = valid)   Y [B,N,H,Dv]
 *   state m,d [B,H,M]  u [B,H,M,Dv]       (fp32)
 *   semi-AR: LSE_dec [B,H,N]  LSE_enc [B,H,NB,M]
 * Parallelism: OpenMP over the independent (b,h) pairs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NEG_INF (-INFINITY)

static inline int neg_inf(float x) { return isinf(x) && x < 0.0f; }

static inline float dotf(const float* a, const float* b, int n) {
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

/* inf-safe merge of one latent's stats b into a (reference.py:160-187,
 * inference.py:194-228). */
static inline void merge_one(float* ma, float* da, float* ua, float mb, float db,
                             const float* ub, int Dv) {
    float m_new = fmaxf(*ma, mb);
    int a_inf = neg_inf(*ma), b_inf = neg_inf(mb), n_inf = neg_inf(m_new);
    float m_safe = n_inf ? 0.0f : m_new;
    float sa = (a_inf && n_inf) ? 1.0f : (a_inf ? 0.0f : expf(*ma - m_safe));
    float sb = (b_inf && n_inf) ? 1.0f : (b_inf ? 0.0f : expf(mb - m_safe));
    *da = *da * sa + db * sb;
    for (int j = 0; j < Dv; ++j) ua[j] = ua[j] * sa + ub[j] * sb;
    *ma = m_new;
}

/* inf-safe tokenwise update of one latent (reference.py:461-473,
 * inference.py:273-285). */
static inline void token_update(float* m, float* d, float* u, float s, const float* v, int Dv) {
    float m_new = fmaxf(*m, s);
    int m_inf = neg_inf(*m), n_inf = neg_inf(m_new);
    float m_safe = n_inf ? 0.0f : m_new;
    float gamma = (m_inf && n_inf) ? 1.0f : (m_inf ? 0.0f : expf(*m - m_safe));
    float eta = n_inf ? 0.0f : expf(s - m_safe);
    *d = *d * gamma + eta;
    for (int j = 0; j < Dv; ++j) u[j] = u[j] * gamma + eta * v[j];
    *m = m_new;
}

/* y = sum_m alpha_m * z_m with alpha = softmax(a) * valid and z = u / d_safe
 * (reference.py:484-496, inference.py:287-301). */
static void latent_readout(const float* a_in, int valid, const float* d, const float* u,
                           int M, int Dv, float* y, float* a_tmp) {
    for (int j = 0; j < Dv; ++j) y[j] = 0.0f;
    if (!valid) return; /* alpha * valid == 0 */
    float amax = NEG_INF;
    for (int m = 0; m < M; ++m) { a_tmp[m] = a_in[m]; amax = fmaxf(amax, a_tmp[m]); }
    float asum = 0.0f;
    for (int m = 0; m < M; ++m) { a_tmp[m] = expf(a_tmp[m] - amax); asum += a_tmp[m]; }
    for (int m = 0; m < M; ++m) {
        float alpha = a_tmp[m] / asum;
        float dsafe = d[m] > 0.0f ? d[m] : 1.0f;
        const float* um = u + (size_t)m * Dv;
        for (int j = 0; j < Dv; ++j) y[j] += alpha * (um[j] / dsafe);
    }
}

/* decoder score a[m] for token t of (b,h): shared weights give a = s
 * (reference.py:479-483). */
static void decoder_scores(const float* s, const float* Qdec, const float* Kdec, const float* Q,
                           const float* K, int shared, int sep_q, int sep_k, int b, int t, int h,
                           int N, int H, int M, int Dk, float scale, float* a) {
    if (shared) { memcpy(a, s, sizeof(float) * M); return; }
    const float* qd = sep_q ? Qdec + (((size_t)b * N + t) * H + h) * Dk
                            : K + (((size_t)b * N + t) * H + h) * Dk;
    const float* kd = sep_k ? Kdec + (size_t)h * M * Dk : Q + (size_t)h * M * Dk;
    for (int m = 0; m < M; ++m) a[m] = dotf(qd, kd + (size_t)m * Dk, Dk) * scale;
}

/*
 * Chunked forward, reference.py:203-512.  Qdec/Kdec may be NULL (defaults:
 * Q_dec = K, K_dec = Q, _reference_utils.py:24-57).  shared != 0 means both
 * defaults apply (weight_sharing_enc_dec).  mask/state_in/state_out may be NULL.
 */
int oracle_ar_chunked(const float* Q, const float* K, const float* V, const float* Qdec,
                      const float* Kdec, const uint8_t* mask, const float* m_in,
                      const float* d_in, const float* u_in, int B, int N, int H, int M, int Dk,
                      int Dv, float scale, int C, int shared, float* Y, float* m_out,
                      float* d_out, float* u_out, int nthreads) {
    if (C <= 0) return -1;
    const int NC = (N + C - 1) / C;
    const int sep_q = Qdec != NULL, sep_k = Kdec != NULL;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const float* q = Q + (size_t)h * M * Dk;
        float* s_all = malloc(sizeof(float) * (size_t)NC * C * M);     /* score_chunk */
        float* cmax = malloc(sizeof(float) * (size_t)NC * M);
        float* cden = malloc(sizeof(float) * (size_t)NC * M);
        float* cnum = calloc((size_t)NC * M * Dv, sizeof(float));
        float* pmax = malloc(sizeof(float) * (size_t)NC * M);            /* score_prev_* */
        float* pden = malloc(sizeof(float) * (size_t)NC * M);
        float* pnum = malloc(sizeof(float) * (size_t)NC * M * Dv);
        float* mc = malloc(sizeof(float) * M);
        float* dc = malloc(sizeof(float) * M);
        float* uc = malloc(sizeof(float) * (size_t)M * Dv);
        float* a = malloc(sizeof(float) * M);
        float* atmp = malloc(sizeof(float) * M);
        float* y = malloc(sizeof(float) * Dv);
        float* vzero = calloc(Dv, sizeof(float));

        /* Phase 1: per-chunk summaries (reference.py:326-347). */
        for (int c = 0; c < NC; ++c) {
            for (int i = 0; i < C; ++i) {
                int t = c * C + i;
                float* st = s_all + ((size_t)c * C + i) * M;
                int valid = t < N && (mask == NULL || mask[(size_t)b * N + t]);
                for (int m = 0; m < M; ++m) {
                    if (!valid) { st[m] = NEG_INF; continue; }
                    const float* kt = K + (((size_t)b * N + t) * H + h) * Dk;
                    st[m] = scale * dotf(kt, q + (size_t)m * Dk, Dk);
                }
            }
            for (int m = 0; m < M; ++m) {
                float mx = NEG_INF;
                for (int i = 0; i < C; ++i) mx = fmaxf(mx, s_all[((size_t)c * C + i) * M + m]);
                float safe = neg_inf(mx) ? 0.0f : mx;
                float den = 0.0f;
                float* num = cnum + ((size_t)c * M + m) * Dv;
                for (int i = 0; i < C; ++i) {
                    int t = c * C + i;
                    float e = expf(s_all[((size_t)c * C + i) * M + m] - safe);
                    den += e;
                    if (t < N && e != 0.0f) {
                        const float* vt = V + (((size_t)b * N + t) * H + h) * Dv;
                        for (int j = 0; j < Dv; ++j) num[j] += e * vt[j];
                    }
                }
                cmax[(size_t)c * M + m] = mx;
                cden[(size_t)c * M + m] = den;
            }
        }

        /* Phase 2: exclusive prefix over chunks (reference.py:378-412). */
        for (int m = 0; m < M; ++m) {
            size_t sidx = (size_t)bh * M + m;
            mc[m] = m_in ? m_in[sidx] : NEG_INF;
            dc[m] = d_in ? d_in[sidx] : 0.0f;
            for (int j = 0; j < Dv; ++j) uc[(size_t)m * Dv + j] = u_in ? u_in[sidx * Dv + j] : 0.0f;
        }
        for (int c = 0; c < NC; ++c) {
            memcpy(pmax + (size_t)c * M, mc, sizeof(float) * M);
            memcpy(pden + (size_t)c * M, dc, sizeof(float) * M);
            memcpy(pnum + (size_t)c * M * Dv, uc, sizeof(float) * M * Dv);
            for (int m = 0; m < M; ++m)
                merge_one(&mc[m], &dc[m], uc + (size_t)m * Dv, cmax[(size_t)c * M + m],
                          cden[(size_t)c * M + m], cnum + ((size_t)c * M + m) * Dv, Dv);
        }
        if (m_out) {
            for (int m = 0; m < M; ++m) {
                size_t sidx = (size_t)bh * M + m;
                m_out[sidx] = mc[m];
                d_out[sidx] = dc[m];
                memcpy(u_out + sidx * Dv, uc + (size_t)m * Dv, sizeof(float) * Dv);
            }
        }

        /* Phase 3: tokenwise replay from each chunk's prefix (reference.py:445-496). */
        for (int c = 0; c < NC; ++c) {
            memcpy(mc, pmax + (size_t)c * M, sizeof(float) * M);
            memcpy(dc, pden + (size_t)c * M, sizeof(float) * M);
            memcpy(uc, pnum + (size_t)c * M * Dv, sizeof(float) * M * Dv);
            for (int i = 0; i < C; ++i) {
                int t = c * C + i;
                const float* st = s_all + ((size_t)c * C + i) * M;
                const float* vt = t < N ? V + (((size_t)b * N + t) * H + h) * Dv : vzero;
                for (int m = 0; m < M; ++m)
                    token_update(&mc[m], &dc[m], uc + (size_t)m * Dv, st[m], vt, Dv);
                if (t >= N) continue;
                int valid = mask == NULL || mask[(size_t)b * N + t];
                decoder_scores(st, Qdec, Kdec, Q, K, shared, sep_q, sep_k, b, t, h, N, H, M, Dk,
                               scale, a);
                latent_readout(a, valid, dc, uc, M, Dv, y, atmp);
                memcpy(Y + (((size_t)b * N + t) * H + h) * Dv, y, sizeof(float) * Dv);
            }
        }
        free(s_all); free(cmax); free(cden); free(cnum); free(pmax); free(pden); free(pnum);
        free(mc); free(dc); free(uc); free(a); free(atmp); free(y); free(vzero);
    }
    return 0;
}

/*
 * Tokenwise recurrent prefill, inference.py:231-315.  A decode step is the
 * one-token case (inference.py:318-351).  state_in may be NULL (fresh state,
 * inference.py:66-84); state_out must be given.
 */
int oracle_ar_recurrent(const float* Q, const float* K, const float* V, const float* Qdec,
                        const float* Kdec, const uint8_t* mask, const float* m_in,
                        const float* d_in, const float* u_in, int B, int T, int H, int M,
                        int Dk, int Dv, float scale, int shared, float* Y, float* m_out,
                        float* d_out, float* u_out, int nthreads) {
    const int sep_q = Qdec != NULL, sep_k = Kdec != NULL;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const float* q = Q + (size_t)h * M * Dk;
        float* s = malloc(sizeof(float) * M);
        float* a = malloc(sizeof(float) * M);
        float* atmp = malloc(sizeof(float) * M);
        float* y = malloc(sizeof(float) * Dv);
        float* mc = m_out + (size_t)bh * M;
        float* dc = d_out + (size_t)bh * M;
        float* uc = u_out + (size_t)bh * M * Dv;
        for (int m = 0; m < M; ++m) {
            size_t sidx = (size_t)bh * M + m;
            mc[m] = m_in ? m_in[sidx] : NEG_INF;
            dc[m] = d_in ? d_in[sidx] : 0.0f;
            for (int j = 0; j < Dv; ++j) uc[(size_t)m * Dv + j] = u_in ? u_in[sidx * Dv + j] : 0.0f;
        }
        for (int t = 0; t < T; ++t) {
            const float* kt = K + (((size_t)b * T + t) * H + h) * Dk;
            const float* vt = V + (((size_t)b * T + t) * H + h) * Dv;
            int valid = mask == NULL || mask[(size_t)b * T + t];
            for (int m = 0; m < M; ++m) s[m] = valid ? dotf(q + (size_t)m * Dk, kt, Dk) * scale : NEG_INF;
            for (int m = 0; m < M; ++m) token_update(&mc[m], &dc[m], uc + (size_t)m * Dv, s[m], vt, Dv);
            decoder_scores(s, Qdec, Kdec, Q, K, shared, sep_q, sep_k, b, t, h, T, H, M, Dk, scale, a);
            latent_readout(a, valid, dc, uc, M, Dv, y, atmp);
            memcpy(Y + (((size_t)b * T + t) * H + h) * Dv, y, sizeof(float) * Dv);
        }
        free(s); free(a); free(atmp); free(y);
    }
    return 0;
}

/*
 * Block-causal (semi-autoregressive) forward, semi_autoregressive/reference.py:308-536.
 * Requires N % block == 0 and block % C == 0 (validated by the caller,
 * reference.py:17-51).  LSE_dec [B,H,N] and LSE_enc [B,H,NB,M] may be NULL.
 */
int oracle_semi_ar(const float* Q, const float* K, const float* V, const float* Qdec,
                   const float* Kdec, int B, int N, int H, int M, int Dk, int Dv, float scale,
                   int block, int C, float* Y, float* lse_dec, float* lse_enc, int nthreads) {
    if (block <= 0 || C <= 0 || N % block || block % C) return -1;
    const int NB = N / block, CPB = block / C;
    const int sep_q = Qdec != NULL, sep_k = Kdec != NULL;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const float* q = Q + (size_t)h * M * Dk;
        float* z = malloc(sizeof(float) * (size_t)NB * M * Dv);    /* z_block */
        float* bmax = malloc(sizeof(float) * M);
        float* bden = malloc(sizeof(float) * M);
        float* bnum = malloc(sizeof(float) * (size_t)M * Dv);
        float* mc = malloc(sizeof(float) * M);
        float* dc = malloc(sizeof(float) * M);
        float* uc = calloc((size_t)M * Dv, sizeof(float));
        float* sc = malloc(sizeof(float) * (size_t)C * M);
        float* cnum = malloc(sizeof(float) * Dv);
        float* a = malloc(sizeof(float) * M);
        for (int m = 0; m < M; ++m) { mc[m] = NEG_INF; dc[m] = 0.0f; }

        for (int g = 0; g < NB; ++g) {
            /* Phase 1: block-local summary, merged chunk by chunk (reference.py:413-450). */
            for (int m = 0; m < M; ++m) { bmax[m] = NEG_INF; bden[m] = 0.0f; }
            memset(bnum, 0, sizeof(float) * (size_t)M * Dv);
            for (int lc = 0; lc < CPB; ++lc) {
                int t0 = g * block + lc * C;
                for (int i = 0; i < C; ++i) {
                    const float* kt = K + (((size_t)b * N + t0 + i) * H + h) * Dk;
                    for (int m = 0; m < M; ++m) sc[(size_t)i * M + m] = scale * dotf(kt, q + (size_t)m * Dk, Dk);
                }
                for (int m = 0; m < M; ++m) {
                    float cm = NEG_INF;
                    for (int i = 0; i < C; ++i) cm = fmaxf(cm, sc[(size_t)i * M + m]);
                    float cden = 0.0f;
                    for (int j = 0; j < Dv; ++j) cnum[j] = 0.0f;
                    for (int i = 0; i < C; ++i) {
                        float e = expf(sc[(size_t)i * M + m] - cm);
                        cden += e;
                        const float* vt = V + (((size_t)b * N + t0 + i) * H + h) * Dv;
                        for (int j = 0; j < Dv; ++j) cnum[j] += e * vt[j];
                    }
                    float mn = fmaxf(bmax[m], cm);
                    float rp = expf(bmax[m] - mn), rc = expf(cm - mn);
                    bden[m] = bden[m] * rp + cden * rc;
                    for (int j = 0; j < Dv; ++j)
                        bnum[(size_t)m * Dv + j] = bnum[(size_t)m * Dv + j] * rp + cnum[j] * rc;
                    bmax[m] = mn;
                }
            }
            /* Phase 2: inclusive scan, LSE_enc and normalised z_block (reference.py:452-492). */
            for (int m = 0; m < M; ++m) {
                float mn = fmaxf(mc[m], bmax[m]);
                float rp = expf(mc[m] - mn), rb = expf(bmax[m] - mn);
                dc[m] = dc[m] * rp + bden[m] * rb;
                for (int j = 0; j < Dv; ++j)
                    uc[(size_t)m * Dv + j] = uc[(size_t)m * Dv + j] * rp + bnum[(size_t)m * Dv + j] * rb;
                mc[m] = mn;
                float lse = logf(fmaxf(dc[m], 1e-20f)) + mc[m];
                if (lse_enc) lse_enc[((size_t)bh * NB + g) * M + m] = lse;
                float w = expf(mc[m] - lse);
                for (int j = 0; j < Dv; ++j)
                    z[((size_t)g * M + m) * Dv + j] = uc[(size_t)m * Dv + j] * w;
            }
        }
        /* Phase 3: per-token latent softmax readout of z_block (reference.py:494-503). */
        for (int t = 0; t < N; ++t) {
            int g = t / block;
            const float* qd = sep_q ? Qdec + (((size_t)b * N + t) * H + h) * Dk
                                    : K + (((size_t)b * N + t) * H + h) * Dk;
            const float* kd = sep_k ? Kdec + (size_t)h * M * Dk : q;
            float amax = NEG_INF;
            for (int m = 0; m < M; ++m) { a[m] = scale * dotf(qd, kd + (size_t)m * Dk, Dk); amax = fmaxf(amax, a[m]); }
            float asum = 0.0f;
            for (int m = 0; m < M; ++m) asum += expf(a[m] - amax);
            float lse = logf(asum) + amax;
            if (lse_dec) lse_dec[(size_t)bh * N + t] = lse;
            float* yt = Y + (((size_t)b * N + t) * H + h) * Dv;
            for (int j = 0; j < Dv; ++j) yt[j] = 0.0f;
            for (int m = 0; m < M; ++m) {
                float alpha = expf(a[m] - lse);
                const float* zm = z + ((size_t)g * M + m) * Dv;
                for (int j = 0; j < Dv; ++j) yt[j] += alpha * zm[j];
            }
        }
        free(z); free(bmax); free(bden); free(bnum); free(mc); free(dc); free(uc); free(sc);
        free(cnum); free(a);
    }
    return 0;
}
