/*
 * Chunked DGDA prefill on the CPU -- TEST INFRASTRUCTURE ONLY.
 *
 * C/OpenMP restatement of the reference CPU backend's chunked WY/UT algorithm
 * (maba_sparse/kernels/cpu_dgda.py:33-197), in float32 like the reference after
 * its bf16/fp16 upcast (cpu_dgda.py:49-61).  It streams one chunk at a time per
 * (batch, head) instead of materialising [B,H,nC,C,C,dk] temporaries
 * (cpu_dgda.py:101-107), and solves (I+L)u = v_e exactly by forward
 * substitution (the reference's "exact" inversion_method, cpu_dgda.py:130-131).
 *
 * Used by tests/ as a second oracle and by bench.py as the timed CPU baseline
 * ("port").  Never linked by the product library.
 *
 * Per chunk of n tokens with inclusive cumulative log-decay Lam (clamped
 * log-decay in [-46, 0], cpu_dgda.py:63-68):
 *   L_ij = sum_d bk_id exp(Lam_id - Lam_jd) k_jd            (i > j)
 *   A_ij = sum_d q_id  exp(Lam_id - Lam_jd) k_jd            (i >= j)
 *   v_e  = w*v - (bk * e^Lam) S0
 *   u    = (I + L)^-1 v_e
 *   o    = (q * e^Lam) S0 + A u
 *   S    = e^{Lam_last} S0 + (k * e^{Lam_last - Lam})^T u
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Gate arrays are [B,H,L,d] when *_pc != 0 and [B,H,L] (one value per token,
 * broadcast over channels) when *_pc == 0. */
static inline float gate_at(const float* g, int pc, int64_t bh, int64_t L, int64_t d,
                            int64_t t, int64_t c) {
    return pc ? g[(bh * L + t) * d + c] : g[bh * L + t];
}

int oracle_dgda_prefill_f32(int B, int H, int L, int dk, int dv, int chunk,
                            const float* q, const float* k, const float* v,
                            const float* log_alpha, int la_pc,
                            const float* bg, int b_pc,
                            const float* wg, int w_pc,
                            const float* s0, float* out, float* s_final,
                            int nthreads) {
    if (B < 0 || H < 0 || L < 0 || dk <= 0 || dv <= 0 || chunk <= 0) return 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    const int64_t BH = (int64_t)B * H;
    int err = 0;
#pragma omp parallel
    {
        const int C = chunk;
        float* S = (float*)malloc(sizeof(float) * dk * dv);
        float* cla = (float*)malloc(sizeof(float) * C * dk);
        float* lam = (float*)malloc(sizeof(float) * C * dk);
        float* bk = (float*)malloc(sizeof(float) * C * dk);
        float* Lm = (float*)malloc(sizeof(float) * C * C);
        float* Am = (float*)malloc(sizeof(float) * C * C);
        float* u = (float*)malloc(sizeof(float) * C * dv);
        float* tmp = (float*)malloc(sizeof(float) * dv);
        if (!S || !cla || !lam || !bk || !Lm || !Am || !u || !tmp) {
#pragma omp atomic write
            err = 2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t bh = 0; bh < BH; ++bh) {
                if (s0) memcpy(S, s0 + bh * dk * dv, sizeof(float) * dk * dv);
                else memset(S, 0, sizeof(float) * dk * dv);
                const float* qb = q + bh * (int64_t)L * dk;
                const float* kb = k + bh * (int64_t)L * dk;
                const float* vb = v + bh * (int64_t)L * dv;
                float* ob = out + bh * (int64_t)L * dv;
                for (int s = 0; s < L; s += C) {
                    const int n = (L - s < C) ? (L - s) : C;
                    /* cumulative clamped log decay (cpu_dgda.py:63-68,101) */
                    for (int c = 0; c < dk; ++c) {
                        float acc = 0.f;
                        for (int i = 0; i < n; ++i) {
                            float la = gate_at(log_alpha, la_pc, bh, L, dk, s + i, c);
                            la = la < -46.f ? -46.f : (la > 0.f ? 0.f : la);
                            acc += la;
                            cla[i * dk + c] = acc;
                            lam[i * dk + c] = expf(acc);
                            bk[i * dk + c] = gate_at(bg, b_pc, bh, L, dk, s + i, c) * kb[(int64_t)(s + i) * dk + c];
                        }
                    }
                    /* L (strict lower) and A (lower incl. diagonal) (cpu_dgda.py:102-107,125-126) */
                    for (int i = 0; i < n; ++i) {
                        for (int j = 0; j <= i; ++j) {
                            float l = 0.f, a = 0.f;
                            const float* kj = kb + (int64_t)(s + j) * dk;
                            const float* qi = qb + (int64_t)(s + i) * dk;
                            if (la_pc) {
                                for (int c = 0; c < dk; ++c) {
                                    float dec = expf(cla[i * dk + c] - cla[j * dk + c]);
                                    l += bk[i * dk + c] * dec * kj[c];
                                    a += qi[c] * dec * kj[c];
                                }
                            } else {
                                float dec = expf(cla[i * dk] - cla[j * dk]);
                                for (int c = 0; c < dk; ++c) {
                                    l += bk[i * dk + c] * kj[c];
                                    a += qi[c] * kj[c];
                                }
                                l *= dec;
                                a *= dec;
                            }
                            Lm[i * C + j] = (j < i) ? l : 0.f;
                            Am[i * C + j] = a;
                        }
                    }
                    /* v_e, then forward substitution (I+L)u = v_e (cpu_dgda.py:129-131) */
                    for (int i = 0; i < n; ++i) {
                        for (int e = 0; e < dv; ++e)
                            tmp[e] = gate_at(wg, w_pc, bh, L, dv, s + i, e) * vb[(int64_t)(s + i) * dv + e];
                        for (int c = 0; c < dk; ++c) {
                            const float f = bk[i * dk + c] * lam[i * dk + c];
                            const float* Sr = S + (int64_t)c * dv;
                            for (int e = 0; e < dv; ++e) tmp[e] -= f * Sr[e];
                        }
                        for (int j = 0; j < i; ++j) {
                            const float l = Lm[i * C + j];
                            const float* uj = u + j * dv;
                            for (int e = 0; e < dv; ++e) tmp[e] -= l * uj[e];
                        }
                        memcpy(u + i * dv, tmp, sizeof(float) * dv);
                    }
                    /* o = (q*e^Lam) S0 + A u (cpu_dgda.py:143-145) */
                    for (int i = 0; i < n; ++i) {
                        float* oi = ob + (int64_t)(s + i) * dv;
                        for (int e = 0; e < dv; ++e) tmp[e] = 0.f;
                        const float* qi = qb + (int64_t)(s + i) * dk;
                        for (int c = 0; c < dk; ++c) {
                            const float f = qi[c] * lam[i * dk + c];
                            const float* Sr = S + (int64_t)c * dv;
                            for (int e = 0; e < dv; ++e) tmp[e] += f * Sr[e];
                        }
                        for (int j = 0; j <= i; ++j) {
                            const float a = Am[i * C + j];
                            const float* uj = u + j * dv;
                            for (int e = 0; e < dv; ++e) tmp[e] += a * uj[e];
                        }
                        memcpy(oi, tmp, sizeof(float) * dv);
                    }
                    /* S = e^{Lam_last} S0 + (k * e^{Lam_last - Lam})^T u (cpu_dgda.py:120-123,146) */
                    for (int c = 0; c < dk; ++c) {
                        const float last = cla[(n - 1) * dk + c];
                        float* Sr = S + (int64_t)c * dv;
                        const float g = lam[(n - 1) * dk + c];
                        for (int e = 0; e < dv; ++e) Sr[e] *= g;
                        for (int i = 0; i < n; ++i) {
                            const float f = kb[(int64_t)(s + i) * dk + c] * expf(last - cla[i * dk + c]);
                            const float* ui = u + i * dv;
                            for (int e = 0; e < dv; ++e) Sr[e] += f * ui[e];
                        }
                    }
                }
                memcpy(s_final + bh * dk * dv, S, sizeof(float) * dk * dv);
            }
        }
        free(S); free(cla); free(lam); free(bk); free(Lm); free(Am); free(u); free(tmp);
    }
    return err;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
