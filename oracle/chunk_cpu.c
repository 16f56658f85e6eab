/*
 * f32 chunked CPU scan: a C restatement of the reference's CPU tensor solver
 * `chunk::scan` for the GDN-2 kind (crates/mixers/src/chunk.rs:129-250).
 *
 * TEST / BASELINE INFRASTRUCTURE ONLY.  It is the "f32 chunked CPU scan" leg of
 * bench.py's cpu_baseline (timed on the GPU box's host cores) and is checked
 * against the f64 oracle by tests/test_chunk_cpu.py.  Nothing in the product
 * path (the HIP library and its Python mirror) uses it.
 *
 * Per chunk of `chunk` tokens, in f32, with the reference's steps:
 *   masking  q, k, v, erase, write *= valid; alpha' = alpha (1 - reset) valid
 *            + (1 - valid)                                      (chunk.rs:155-169)
 *   prefix   cumulative product of alpha' over the chunk        (:170)
 *   decay    decay[r][s] = prod_{u = s+1..r} alpha'_u, 1 at r = s (:171-182)
 *   lower    L[r][s] = sum_i (erase k)_r[i] decay[r][s][i] k_s[i]   (:183-189)
 *   rhs      write v - (erase k prefix) S                        (:190-194)
 *   edits    (I + strict_lower(L))^-1 rhs                         (:211-221)
 *   out      (q prefix) S + lower(Q overlap) edits                (:226-227)
 *   score    |k| |edits|, zero at a zero edit                     (:228-234)
 *   state    prefix_last S + (decay_last k)^T edits               (:235-241)
 * The reference inverts by the nilpotent doubling series and allows chunks of
 * 1..16 (:137-140, :211-220); here the unit lower-triangular system is solved
 * by forward substitution, which is exact in exact arithmetic for any chunk
 * (the reference's chunk cap exists for its doubling series) and is stable at
 * the 64-token chunk of the benchmark configurations.
 * Layouts: sequences [B,T,H,C], masks [B,T], states [B,H,K,V], all dense.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int gdn2_chunk_cpu_threads(void) { return omp_get_max_threads(); }

int gdn2_chunk_cpu_f32(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int chunk,
                       const float *q, const float *k, const float *v, const float *alpha,
                       const float *erase, const float *write, const float *valid,
                       const float *reset, const float *initial, float *out,
                       float *final_state, float *scores) {
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || chunk < 1) return 1;
    const int64_t C = chunk;
    int err = 0;
#pragma omp parallel
    {
        float *S = malloc(sizeof(float) * K * V);
        float *qa = malloc(sizeof(float) * C * K), *ka = malloc(sizeof(float) * C * K);
        float *ea = malloc(sizeof(float) * C * K), *aa = malloc(sizeof(float) * C * K);
        float *pre = malloc(sizeof(float) * C * K), *dec = malloc(sizeof(float) * C * C * K);
        float *L = malloc(sizeof(float) * C * C), *Qo = malloc(sizeof(float) * C * C);
        float *X = malloc(sizeof(float) * C * V), *wv = malloc(sizeof(float) * C * V);
        if (!S || !qa || !ka || !ea || !aa || !pre || !dec || !L || !Qo || !X || !wv) {
#pragma omp atomic write
            err = 2;
        } else {
#pragma omp for schedule(dynamic)
            for (int64_t bh = 0; bh < B * H; ++bh) {
                const int64_t b = bh / H, h = bh % H;
                if (initial)
                    memcpy(S, initial + bh * K * V, sizeof(float) * K * V);
                else
                    memset(S, 0, sizeof(float) * K * V);
                for (int64_t first = 0; first < T; first += C) {
                    const int64_t n = (T - first) < C ? (T - first) : C;
                    for (int64_t r = 0; r < n; ++r) {  /* masking */
                        const int64_t t = first + r, row = (b * T + t) * H + h;
                        const float act = valid[b * T + t], rs = reset[b * T + t];
                        for (int64_t i = 0; i < K; ++i) {
                            const float kk = k[row * K + i] * act;
                            qa[r * K + i] = q[row * K + i] * act;
                            ka[r * K + i] = kk;
                            ea[r * K + i] = erase[row * K + i] * act * kk;  /* erase k */
                            aa[r * K + i] = alpha[row * K + i] * (1.0f - rs) * act + (1.0f - act);
                        }
                        for (int64_t j = 0; j < V; ++j)
                            wv[r * V + j] = write[row * V + j] * act * (v[row * V + j] * act);
                    }
                    for (int64_t i = 0; i < K; ++i) {  /* prefix and decay */
                        float p = 1.0f;
                        for (int64_t r = 0; r < n; ++r) {
                            p *= aa[r * K + i];
                            pre[r * K + i] = p;
                        }
                        for (int64_t r = 0; r < n; ++r) {
                            float d = 1.0f;
                            dec[(r * C + r) * K + i] = 1.0f;
                            for (int64_t s = r - 1; s >= 0; --s) {
                                d *= aa[(s + 1) * K + i];
                                dec[(r * C + s) * K + i] = d;
                            }
                        }
                    }
                    for (int64_t r = 0; r < n; ++r)  /* key overlaps */
                        for (int64_t s = 0; s <= r; ++s) {
                            float l = 0.f, o = 0.f;
                            const float *dd = dec + (r * C + s) * K;
                            for (int64_t i = 0; i < K; ++i) {
                                const float f = dd[i] * ka[s * K + i];
                                l += ea[r * K + i] * f;
                                o += qa[r * K + i] * f;
                            }
                            L[r * C + s] = l;
                            Qo[r * C + s] = o;
                        }
                    for (int64_t r = 0; r < n; ++r) {  /* rhs, then forward substitution */
                        float *x = X + r * V;
                        for (int64_t j = 0; j < V; ++j) x[j] = wv[r * V + j];
                        for (int64_t i = 0; i < K; ++i) {
                            const float c = ea[r * K + i] * pre[r * K + i];
                            if (c == 0.f) continue;
                            const float *Si = S + i * V;
                            for (int64_t j = 0; j < V; ++j) x[j] -= c * Si[j];
                        }
                        for (int64_t s = 0; s < r; ++s) {
                            const float c = L[r * C + s];
                            const float *xs = X + s * V;
                            for (int64_t j = 0; j < V; ++j) x[j] -= c * xs[j];
                        }
                    }
                    for (int64_t r = 0; r < n; ++r) {  /* outputs and scores */
                        const int64_t t = first + r, row = (b * T + t) * H + h;
                        float *o = out + row * V;
                        for (int64_t j = 0; j < V; ++j) o[j] = 0.f;
                        for (int64_t i = 0; i < K; ++i) {
                            const float c = qa[r * K + i] * pre[r * K + i];
                            if (c == 0.f) continue;
                            const float *Si = S + i * V;
                            for (int64_t j = 0; j < V; ++j) o[j] += c * Si[j];
                        }
                        for (int64_t s = 0; s <= r; ++s) {
                            const float c = Qo[r * C + s];
                            const float *xs = X + s * V;
                            for (int64_t j = 0; j < V; ++j) o[j] += c * xs[j];
                        }
                        float kk2 = 0.f, ee2 = 0.f;
                        for (int64_t i = 0; i < K; ++i) kk2 += ka[r * K + i] * ka[r * K + i];
                        for (int64_t j = 0; j < V; ++j) ee2 += X[r * V + j] * X[r * V + j];
                        const float m = kk2 * ee2;
                        scores[row] = m == 0.f ? 0.f : sqrtf(m);
                    }
                    for (int64_t i = 0; i < K; ++i) {  /* state update */
                        float *Si = S + i * V;
                        const float f = pre[(n - 1) * K + i];
                        for (int64_t j = 0; j < V; ++j) Si[j] *= f;
                        for (int64_t s = 0; s < n; ++s) {
                            const float c = dec[((n - 1) * C + s) * K + i] * ka[s * K + i];
                            if (c == 0.f) continue;
                            const float *xs = X + s * V;
                            for (int64_t j = 0; j < V; ++j) Si[j] += c * xs[j];
                        }
                    }
                }
                memcpy(final_state + bh * K * V, S, sizeof(float) * K * V);
            }
        }
        free(S), free(qa), free(ka), free(ea), free(aa), free(pre), free(dec), free(L), free(Qo),
            free(X), free(wv);
    }
    return err;
}
