/*
 * gdn2_oracle.c -- CPU restatement of delta-block-lm's GDN-2 recurrence.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * Python host mirror) links, loads or calls this file.  It is the checker:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * What it restates (read as text from the reference, never executed):
 *   - gdn2_oracle_scan      crates/mixers/src/reference.rs:41-119 (GDN-2 arm)
 *   - gdn2_oracle_backward  crates/mixers/src/reference.rs:127-257 (GDN-2 arm)
 *   - SplitMix64            crates/experiment/src/data.rs:13-21
 *                           (identical to reuse/crates/dre-gdn2/src/tests.rs:7-16)
 *   - uniform / normal      reuse/crates/dre-gdn2/src/tests.rs:18-32
 *
 * Arithmetic is f64 and follows the reference loop order.  The backward keeps
 * bounded memory: the reference stores every per-token state (reference.rs:55);
 * here forward states are checkpointed every `GDN2_ORACLE_REPLAY` tokens and a
 * chunk is replayed from its checkpoint.  Replay runs the same step function in
 * the same order, so the replayed states are bit-identical to a full store.
 *
 * Pinning (tests/test_oracle.py): closed forms at T=1 and for the aligned
 * fixture (reference checks.rs:181-198), f64 central differences along random
 * directions for every input group and the initial state, the reference's own
 * fixture assertions (chunk_tests.rs:148-170), the unit-lower-triangular solve
 * special case against numpy.linalg.solve, and brute-force chunk invariance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GDN2_ORACLE_REPLAY 64

/* ------------------------------------------------------------------------- */
/* Deterministic generator                                                    */
/* ------------------------------------------------------------------------- */

/* SplitMix64 step (data.rs:15-21). */
uint64_t gdn2_oracle_splitmix_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Uniform in [0,1): top 53 bits (tests.rs:18-21). */
static double uniform01(uint64_t *state) {
    return (double)(gdn2_oracle_splitmix_next(state) >> 11) / 9007199254740992.0;
}

/* Fill `out` with n standard normals, Box-Muller cosine branch (tests.rs:28-32).
 * Each normal consumes two draws: the radius draw first, then the angle draw. */
void gdn2_oracle_normals(uint64_t *state, int64_t n, double *out) {
    const double tau = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; ++i) {
        double radius = sqrt(-2.0 * log(1.0 - uniform01(state)));
        out[i] = radius * cos(tau * uniform01(state));
    }
}

/* Raw SplitMix64 outputs, for checking other implementations of the stream. */
void gdn2_oracle_splitmix_fill(uint64_t *state, int64_t n, uint64_t *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = gdn2_oracle_splitmix_next(state);
}

/* ------------------------------------------------------------------------- */
/* One sequence (one (batch, head) pair)                                       */
/* ------------------------------------------------------------------------- */

/* Token-major sequence layout used by the per-sequence routines:
 *   q, k, alpha, erase : [T][K]     v, write : [T][V]
 *   valid, reset       : [T] (0/1)  state    : [K][V] (key-major, chunk.rs:126) */

static int all_finite(const double *x, int n) {
    for (int i = 0; i < n; ++i)
        if (!isfinite(x[i])) return 0;
    return 1;
}

/* Advance `state` over token t.  Writes out[V] and *score.  Returns 0, or -1
 * on a nonfinite input (reference.rs:58-61 asserts).  `edit` is V scratch. */
static int step(int K, int V, double *state, const double *q, const double *k,
                const double *v, const double *alpha, const double *erase,
                const double *write, int valid, int reset, double *out,
                double *score, double *edit) {
    if (!all_finite(q, K) || !all_finite(k, K) || !all_finite(v, V) ||
        !all_finite(alpha, K) || !all_finite(erase, K) || !all_finite(write, V))
        return -1;
    if (!valid) { /* reference.rs:62-67: zero output and score, keep the state */
        for (int j = 0; j < V; ++j) out[j] = 0.0;
        *score = 0.0;
        return 0;
    }
    if (reset) /* reference.rs:68-70 */
        for (int x = 0; x < K * V; ++x) state[x] = 0.0;
    for (int i = 0; i < K; ++i) /* decay, reference.rs:71-75 */
        for (int j = 0; j < V; ++j) state[i * V + j] *= alpha[i];
    for (int j = 0; j < V; ++j) { /* GDN-2 edit, reference.rs:79-84 */
        edit[j] = write[j] * v[j];
        for (int i = 0; i < K; ++i) edit[j] -= erase[i] * k[i] * state[i * V + j];
    }
    double kk = 0.0, ee = 0.0; /* score, reference.rs:99-101 */
    for (int i = 0; i < K; ++i) kk += k[i] * k[i];
    for (int j = 0; j < V; ++j) ee += edit[j] * edit[j];
    *score = sqrt(kk * ee);
    for (int j = 0; j < V; ++j) out[j] = 0.0;
    for (int i = 0; i < K; ++i) /* update and read, reference.rs:102-108 */
        for (int j = 0; j < V; ++j) {
            state[i * V + j] += k[i] * edit[j];
            out[j] += q[i] * state[i * V + j];
        }
    return 0;
}

/* Forward scan of one sequence (reference.rs:41-119).
 * initial may be NULL (zero state).  states may be NULL; otherwise it receives
 * the state after every token, [T][K][V].  Returns 0 or -1 (nonfinite input). */
int gdn2_oracle_scan(int T, int K, int V, const double *q, const double *k,
                     const double *v, const double *alpha, const double *erase,
                     const double *write, const uint8_t *valid,
                     const uint8_t *reset, const double *initial, double *output,
                     double *final_state, double *scores, double *states) {
    double *state = final_state;
    double *edit = (double *)malloc(sizeof(double) * (size_t)V);
    if (!edit) return -2;
    if (initial) memcpy(state, initial, sizeof(double) * (size_t)K * V);
    else memset(state, 0, sizeof(double) * (size_t)K * V);
    int rc = 0;
    for (int t = 0; t < T && rc == 0; ++t) {
        rc = step(K, V, state, q + (size_t)t * K, k + (size_t)t * K,
                  v + (size_t)t * V, alpha + (size_t)t * K, erase + (size_t)t * K,
                  write + (size_t)t * V, valid[t], reset[t], output + (size_t)t * V,
                  scores + t, edit);
        if (states) memcpy(states + (size_t)t * K * V, state, sizeof(double) * (size_t)K * V);
    }
    free(edit);
    return rc;
}

/* Analytic VJP of (output, final state, scores) for one sequence, including
 * the initial-state adjoint (reference.rs:127-257, GDN-2 arm).
 * upstream [T][V], final_adjoint [K][V], score_adjoint [T]; any may be NULL
 * (zero).  Gradients are written (not accumulated) to dq..dwrite and
 * d_initial [K][V]. */
int gdn2_oracle_backward(int T, int K, int V, const double *q, const double *k,
                         const double *v, const double *alpha, const double *erase,
                         const double *write, const uint8_t *valid,
                         const uint8_t *reset, const double *initial,
                         const double *upstream, const double *final_adjoint,
                         const double *score_adjoint, double *dq, double *dk,
                         double *dv, double *dalpha, double *derase,
                         double *dwrite, double *d_initial) {
    const size_t S = (size_t)K * V;
    const int R = GDN2_ORACLE_REPLAY;
    const int nck = (T + R - 1) / R;
    double *ck = (double *)malloc(sizeof(double) * S * (size_t)(nck + 1));
    double *chunk = (double *)malloc(sizeof(double) * S * (size_t)R);
    double *zero = (double *)calloc(S, sizeof(double));
    double *init = (double *)calloc(S, sizeof(double));
    double *adj = (double *)malloc(sizeof(double) * S);
    double *bar = (double *)malloc(sizeof(double) * S);
    double *dbar = (double *)malloc(sizeof(double) * S);
    double *delta = (double *)malloc(sizeof(double) * (size_t)V);
    double *dz = (double *)malloc(sizeof(double) * (size_t)V);
    double *outbuf = (double *)malloc(sizeof(double) * (size_t)V);
    int rc = 0;
    if (!ck || !chunk || !zero || !init || !adj || !bar || !dbar || !delta || !dz || !outbuf) {
        rc = -2;
        goto done;
    }
    if (initial) memcpy(init, initial, sizeof(double) * S);
    /* Forward pass recording chunk-start checkpoints. */
    memcpy(ck, init, sizeof(double) * S);
    {
        double *state = (double *)malloc(sizeof(double) * S);
        if (!state) { rc = -2; goto done; }
        memcpy(state, init, sizeof(double) * S);
        for (int t = 0; t < T && rc == 0; ++t) {
            double sc;
            rc = step(K, V, state, q + (size_t)t * K, k + (size_t)t * K, v + (size_t)t * V,
                      alpha + (size_t)t * K, erase + (size_t)t * K, write + (size_t)t * V,
                      valid[t], reset[t], outbuf, &sc, delta);
            if ((t + 1) % R == 0) memcpy(ck + (size_t)((t + 1) / R) * S, state, sizeof(double) * S);
        }
        free(state);
        if (rc) goto done;
    }
    memset(dq, 0, sizeof(double) * (size_t)T * K);
    memset(dk, 0, sizeof(double) * (size_t)T * K);
    memset(dv, 0, sizeof(double) * (size_t)T * V);
    memset(dalpha, 0, sizeof(double) * (size_t)T * K);
    memset(derase, 0, sizeof(double) * (size_t)T * K);
    memset(dwrite, 0, sizeof(double) * (size_t)T * V);
    if (final_adjoint) memcpy(adj, final_adjoint, sizeof(double) * S);
    else memset(adj, 0, sizeof(double) * S);

    for (int c = nck - 1; c >= 0; --c) {
        const int first = c * R;
        const int n = (T - first < R) ? T - first : R;
        /* Replay: chunk[r] = state after token first+r. */
        {
            double sc;
            double *state = chunk; /* walk in place, copying forward */
            memcpy(state, ck + (size_t)c * S, sizeof(double) * S);
            for (int r = 0; r < n; ++r) {
                if (r > 0) memcpy(chunk + (size_t)r * S, chunk + (size_t)(r - 1) * S, sizeof(double) * S);
                int t = first + r;
                step(K, V, chunk + (size_t)r * S, q + (size_t)t * K, k + (size_t)t * K,
                     v + (size_t)t * V, alpha + (size_t)t * K, erase + (size_t)t * K,
                     write + (size_t)t * V, valid[t], reset[t], outbuf, &sc, delta);
            }
            (void)state;
        }
        for (int r = n - 1; r >= 0; --r) {
            const int t = first + r;
            if (!valid[t]) continue; /* reference.rs:146-148 */
            const double *xq = q + (size_t)t * K, *xk = k + (size_t)t * K;
            const double *xv = v + (size_t)t * V, *xa = alpha + (size_t)t * K;
            const double *xe = erase + (size_t)t * K, *xw = write + (size_t)t * V;
            const double *up = upstream ? upstream + (size_t)t * V : NULL;
            double *gq = dq + (size_t)t * K, *gk = dk + (size_t)t * K;
            double *gv = dv + (size_t)t * V, *ga = dalpha + (size_t)t * K;
            double *ge = derase + (size_t)t * K, *gw = dwrite + (size_t)t * V;
            const double *after = chunk + (size_t)r * S;
            const double *previous; /* reference.rs:152-158 */
            if (reset[t]) previous = zero;
            else if (t == 0) previous = init;
            else if (r == 0) previous = ck + (size_t)c * S;
            else previous = chunk + (size_t)(r - 1) * S;
            for (int i = 0; i < K; ++i) /* reference.rs:160-166 */
                for (int j = 0; j < V; ++j) {
                    double u = up ? up[j] : 0.0;
                    gq[i] += after[i * V + j] * u;
                    adj[i * V + j] += xq[i] * u;
                    bar[i * V + j] = xa[i] * previous[i * V + j];
                }
            memcpy(dbar, adj, sizeof(double) * S);
            for (int j = 0; j < V; ++j) { /* reference.rs:170-178 */
                delta[j] = xw[j] * xv[j];
                dz[j] = 0.0;
                for (int i = 0; i < K; ++i) {
                    delta[j] -= xe[i] * xk[i] * bar[i * V + j];
                    dz[j] += adj[i * V + j] * xk[i];
                }
            }
            double nk = 0.0, nd = 0.0; /* reference.rs:179-188 */
            for (int i = 0; i < K; ++i) nk += xk[i] * xk[i];
            for (int j = 0; j < V; ++j) nd += delta[j] * delta[j];
            nk = sqrt(nk);
            nd = sqrt(nd);
            const double sa = score_adjoint ? score_adjoint[t] : 0.0;
            if (nk > 0.0 && nd > 0.0) {
                for (int i = 0; i < K; ++i) gk[i] += sa * nd / nk * xk[i];
                for (int j = 0; j < V; ++j) dz[j] += sa * nk / nd * delta[j];
            }
            for (int i = 0; i < K; ++i) /* reference.rs:189-195 */
                for (int j = 0; j < V; ++j) {
                    gk[i] += adj[i * V + j] * delta[j] - bar[i * V + j] * xe[i] * dz[j];
                    ge[i] -= bar[i * V + j] * xk[i] * dz[j];
                    dbar[i * V + j] -= xe[i] * xk[i] * dz[j];
                }
            for (int j = 0; j < V; ++j) { /* reference.rs:196-199 */
                gv[j] = xw[j] * dz[j];
                gw[j] = xv[j] * dz[j];
            }
            for (int i = 0; i < K; ++i) /* reference.rs:242-251 */
                for (int j = 0; j < V; ++j) {
                    ga[i] += dbar[i * V + j] * previous[i * V + j];
                    adj[i * V + j] = reset[t] ? 0.0 : xa[i] * dbar[i * V + j];
                }
        }
    }
    memcpy(d_initial, adj, sizeof(double) * S); /* reference.rs:253-256 */
done:
    free(ck); free(chunk); free(zero); free(init); free(adj); free(bar);
    free(dbar); free(delta); free(dz); free(outbuf);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* Batched [batch, time, head, channel] wrappers                               */
/* ------------------------------------------------------------------------- */

/* Gather field (b,h) of a [B,T,H,W] array into [T][W]. */
static void gather(const double *src, double *dst, int T, int H, int W, int b, int h) {
    for (int t = 0; t < T; ++t)
        memcpy(dst + (size_t)t * W, src + (((size_t)b * T + t) * H + h) * W, sizeof(double) * W);
}
static void scatter(const double *src, double *dst, int T, int H, int W, int b, int h) {
    for (int t = 0; t < T; ++t)
        memcpy(dst + (((size_t)b * T + t) * H + h) * W, src + (size_t)t * W, sizeof(double) * W);
}

/* Batched forward over all (b,h), OpenMP-parallel over sequences.
 * Inputs [B,T,H,K|V] contiguous f64; valid/reset [B,T] u8; initial [B,H,K,V]
 * or NULL.  Outputs: output [B,T,H,V], final_state [B,H,K,V], scores [B,T,H].
 * Returns the number of sequences that failed (nonfinite input). */
int gdn2_oracle_scan_bthw(int B, int T, int H, int K, int V, const double *q,
                          const double *k, const double *v, const double *alpha,
                          const double *erase, const double *write,
                          const uint8_t *valid, const uint8_t *reset,
                          const double *initial, double *output,
                          double *final_state, double *scores) {
    int failed = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : failed)
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const size_t S = (size_t)K * V;
        double *buf = (double *)malloc(sizeof(double) * ((size_t)T * (4 * K + 3 * V + 1)));
        double *sq = buf, *sk = sq + (size_t)T * K, *sa = sk + (size_t)T * K,
               *se = sa + (size_t)T * K, *sv = se + (size_t)T * K, *sw = sv + (size_t)T * V,
               *so = sw + (size_t)T * V, *ss = so + (size_t)T * V;
        gather(q, sq, T, H, K, b, h);
        gather(k, sk, T, H, K, b, h);
        gather(alpha, sa, T, H, K, b, h);
        gather(erase, se, T, H, K, b, h);
        gather(v, sv, T, H, V, b, h);
        gather(write, sw, T, H, V, b, h);
        int rc = gdn2_oracle_scan(T, K, V, sq, sk, sv, sa, se, sw, valid + (size_t)b * T,
                                  reset + (size_t)b * T, initial ? initial + (size_t)bh * S : NULL,
                                  so, final_state + (size_t)bh * S, ss, NULL);
        failed += rc != 0;
        scatter(so, output, T, H, V, b, h);
        for (int t = 0; t < T; ++t) scores[((size_t)b * T + t) * H + h] = ss[t];
        free(buf);
    }
    return failed;
}

/* Batched backward over all (b,h).  upstream [B,T,H,V], final_adjoint
 * [B,H,K,V], score_adjoint [B,T,H]; each may be NULL (zero).  Gradients in
 * the input layouts; d_initial [B,H,K,V]. */
int gdn2_oracle_backward_bthw(int B, int T, int H, int K, int V, const double *q,
                              const double *k, const double *v, const double *alpha,
                              const double *erase, const double *write,
                              const uint8_t *valid, const uint8_t *reset,
                              const double *initial, const double *upstream,
                              const double *final_adjoint, const double *score_adjoint,
                              double *dq, double *dk, double *dv, double *dalpha,
                              double *derase, double *dwrite, double *d_initial) {
    int failed = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : failed)
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const size_t S = (size_t)K * V;
        size_t per = (size_t)T * (4 * K + 3 * V + 1);
        double *buf = (double *)malloc(sizeof(double) * 2 * per);
        double *sq = buf, *sk = sq + (size_t)T * K, *sa = sk + (size_t)T * K,
               *se = sa + (size_t)T * K, *sv = se + (size_t)T * K, *sw = sv + (size_t)T * V,
               *su = sw + (size_t)T * V, *ssa = su + (size_t)T * V;
        double *g = buf + per;
        double *gq = g, *gk = gq + (size_t)T * K, *ga = gk + (size_t)T * K,
               *ge = ga + (size_t)T * K, *gv = ge + (size_t)T * K, *gw = gv + (size_t)T * V;
        gather(q, sq, T, H, K, b, h);
        gather(k, sk, T, H, K, b, h);
        gather(alpha, sa, T, H, K, b, h);
        gather(erase, se, T, H, K, b, h);
        gather(v, sv, T, H, V, b, h);
        gather(write, sw, T, H, V, b, h);
        if (upstream) gather(upstream, su, T, H, V, b, h);
        if (score_adjoint)
            for (int t = 0; t < T; ++t) ssa[t] = score_adjoint[((size_t)b * T + t) * H + h];
        int rc = gdn2_oracle_backward(
            T, K, V, sq, sk, sv, sa, se, sw, valid + (size_t)b * T, reset + (size_t)b * T,
            initial ? initial + (size_t)bh * S : NULL, upstream ? su : NULL,
            final_adjoint ? final_adjoint + (size_t)bh * S : NULL, score_adjoint ? ssa : NULL,
            gq, gk, gv, ga, ge, gw, d_initial + (size_t)bh * S);
        failed += rc != 0;
        scatter(gq, dq, T, H, K, b, h);
        scatter(gk, dk, T, H, K, b, h);
        scatter(ga, dalpha, T, H, K, b, h);
        scatter(ge, derase, T, H, K, b, h);
        scatter(gv, dv, T, H, V, b, h);
        scatter(gw, dwrite, T, H, V, b, h);
        free(buf);
    }
    return failed;
}

/* Number of OpenMP threads the batched wrappers use. */
int gdn2_oracle_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}
