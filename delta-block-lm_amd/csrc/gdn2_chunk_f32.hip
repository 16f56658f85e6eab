// Chunked channel-wise GDN-2 in f32 on gfx950: the reference's own op
// configuration (f32 q/k/v, d_k = 32, d_v = 64, 16-token chunks;
// crates/kernels/src/gdn2.rs:10-12, crates/kernels/src/gdn_training.rs:8-9), and
// every d_k, d_v <= 64.
//
// Recurrence per valid token t (crates/mixers/src/reference.rs:68-111):
//   bar = diag(alpha_t) S;  delta_t = w_t.v_t - bar^T (e_t.k_t);
//   S_t = bar + k_t delta_t^T;  o_t = S_t^T q_t;  score_t = |k_t| |delta_t|.
// Per chunk of C = 16 tokens with start state S0 and, per key channel i, the
// decays as direct products of the gates, as the reference's chunked kernels
// form them (gdn2.rs:23-64), so zero and negative gates need no special case:
//   D_ts = prod_{s < u <= t} alpha_u   (s <= t, same segment; resets cut segments)
//   b_t = prod_{u <= t} alpha_u [segment 0],  lam_s = prod_{s < u <= 15} alpha_u [last segment]
//   ehat = e.k,  Ahat = b.ehat,  Qhat = b.q,  Ktil = lam.k,  wv = w.v
//   A_ts = sum_i ehat_t D_ts k_s (s < t),  T = (I + A)^-1,  P_ts = sum_i q_t D_ts k_s (s <= t)
//   R = wv - Ahat S0,  delta = T R,  O = Qhat S0 + P delta
//   S_16 = diag(b_15) S0 + Ktil^T (U - W' S0),  W' = T Ahat,  U = T wv.
// Padding tokens have alpha 1 and zero k, q, e, w (state kept, zero output).
//
// Five kernels: prep (A, T, the map's factors), a scan over the chunks of each
// (batch, head) (states forward, state adjoints in reverse), out (delta, O,
// scores), bprep (the adjoint map's additive term N) and bgrad (every
// gradient).  Work per chunk is small at these widths (a chunk's products are
// 16 x 64 x 64 at most), so the kernels run in f32 on the VALU with LDS tiles:
// one 256-thread workgroup per chunk, thread (token t = tid / 16, channels
// 4 (tid % 16) .. + 3) for the [token][channel] tiles.
#include "gdn2_chunk_f32.h"
#include "gdn2_mfma.h"

#include <algorithm>

namespace gdn2 {

namespace {

constexpr int C = FC_C;
constexpr int FK = FC_MAX;
constexpr int NT = 256;
constexpr int LQ = FK + 4;  // f32 row stride of [token][channel] tiles
constexpr int LS = FK + 1;  // f32 row stride of [key][value] tiles
constexpr int LT = C + 1;   // f32 row stride of 16 x 16 tiles

struct Masks {
    float val[C];
    int rs[C];   // a valid reset
    int seg[C];  // valid resets at or before the token
};

// Token masks (valid / reset, or the document limits) and segments.  Ends with
// a barrier.
__device__ void fc_masks(const SeqArgs &s, int b, int c, Masks &m, int tid) {
    if (tid < C) {
        const int tg = c * C + tid;
        float vld = 0.f, rst = 0.f;
        if (tg < s.T) {
            if (s.doc) {
                const int st = reinterpret_cast<const int *>(s.doc_start.data)[b * s.doc_start.s0 + tg * s.doc_start.s1];
                const int en = reinterpret_cast<const int *>(s.doc_end.data)[b * s.doc_end.s0 + tg * s.doc_end.s1];
                vld = en >= st ? 1.f : 0.f;
                rst = st == tg ? 1.f : 0.f;
            } else {
                vld = ld4<float>(s.valid, b, tg, 0, 0);
                rst = ld4<float>(s.reset, b, tg, 0, 0);
            }
        }
        m.val[tid] = vld != 0.f ? 1.f : 0.f;
        m.rs[tid] = (vld != 0.f && rst != 0.f) ? 1 : 0;
    }
    __syncthreads();
    if (tid == 0) {
        int sg = 0;
        for (int t = 0; t < C; ++t) {
            sg += m.rs[t];
            m.seg[t] = sg;
        }
    }
    __syncthreads();
}

// A [token][channel] input at (b, tg, h, ch): zero past the sequence, past the
// width or on a padding token.
__device__ __forceinline__ float fc_in(const View &v, int b, int tg, int h, int ch, int T, int W, bool on) {
    return (on && tg < T && ch < W) ? ld4<float>(v, b, tg, h, ch) : 0.f;
}

// b_t and lam_t of channel i (threads i < K): running products of the gates.
__device__ void fc_decay_rows(const float *al, const Masks &m, float *bt, float *lam, int K, int tid) {
    if (tid < K) {
        const int i = tid, sg15 = m.seg[C - 1];
        float p = 1.f;
        for (int t = 0; t < C; ++t) {
            p *= al[t * LQ + i];
            bt[t * LQ + i] = m.seg[t] == 0 ? p : 0.f;
        }
        float q = 1.f;
        for (int s = C - 1; s >= 0; --s) {
            lam[s * LQ + i] = m.seg[s] == sg15 ? q : 0.f;
            q *= al[s * LQ + i];
        }
    }
}

// b_t alone (threads i < K).
__device__ void fc_b_row(const float *al, const Masks &m, float *bt, int K, int tid) {
    if (tid < K) {
        float p = 1.f;
        for (int t = 0; t < C; ++t) {
            p *= al[t * LQ + tid];
            bt[t * LQ + tid] = m.seg[t] == 0 ? p : 0.f;
        }
    }
}

// out[t][s] = sum_i x[t][i] D_ts[i] y[s][i] for s < t (STRICT) or s <= t in the
// same segment, zero elsewhere (the diagonal too when STRICT).  Thread
// (t = tid / 16, g = tid % 16) takes channels 4 g .. 4 g + 3 of row t, forming
// D_ts for s = t, t - 1, .. by a running product; the 16 partial rows of one t
// (16 adjacent lanes) are summed by lane shuffles.  All 256 threads call it.
template <bool STRICT>
__device__ __forceinline__ void fc_tri(const float *x, const float *y, const float *al, const Masks &m,
                                       float *out, int K, int tid) {
    const int t = tid >> 4, g = tid & 15;
    float acc[C];
#pragma unroll
    for (int s = 0; s < C; ++s) acc[s] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        if (i < K) {
            const float xt = x[t * LQ + i];
            float d = 1.f;
#pragma unroll
            for (int s = C - 1; s >= 0; --s)
                if (s <= t) {
                    acc[s] += xt * d * y[s * LQ + i];
                    d *= al[s * LQ + i];
                }
        }
    }
    float r = 0.f;
#pragma unroll
    for (int s = 0; s < C; ++s) {
        float a = acc[s];
        a += __shfl_xor(a, 1);
        a += __shfl_xor(a, 2);
        a += __shfl_xor(a, 4);
        a += __shfl_xor(a, 8);
        if (s == g) r = a;
    }
    const bool keep = (STRICT ? g < t : g <= t) && m.seg[g] == m.seg[t];
    out[t * LT + g] = keep ? r : 0.f;
}

struct FcPrepSmem {
    Masks m;
    float k[C * LQ], al[C * LQ], eh[C * LQ], wv[C * LQ], bt[C * LQ], lam[C * LQ];
    float A[C * LT], T[C * LT];
};

struct FcOutSmem {
    Masks m;
    float q[C * LQ], k[C * LQ], al[C * LQ], eh[C * LQ], wv[C * LQ], bt[C * LQ], r[C * LQ], dl[C * LQ];
    float s0[FK * LS];
    float T[C * LT], P[C * LT];
    float kk[C], dd[C];
};

struct FcBPrepSmem {
    Masks m;
    float q[C * LQ], k[C * LQ], al[C * LQ], bt[C * LQ], dO[C * LQ], dl[C * LQ], x[C * LQ], w[C * LQ];
    float P[C * LT];
    float cs[C];
};

struct FcBGradSmem {
    Masks m;
    float q[C * LQ], k[C * LQ], v[C * LQ], al[C * LQ], e[C * LQ], w[C * LQ], eh[C * LQ], dO[C * LQ];
    float dl[C * LQ], dd[C * LQ], dr[C * LQ], bt[C * LQ], lam[C * LQ];
    float ga[C * LQ], gq[C * LQ], gk[C * LQ];  // dAhat, dQhat, dKtil [token][key]
    float s0[FK * LS], ds[FK * LS];
    float T[C * LT], P[C * LT], dA[C * LT], dP[C * LT];
    float cs[C], ck[C], fs[FK];
};

}  // namespace

// ---- prep: gates, A, T and the factored map of every chunk ---------------------
__global__ void __launch_bounds__(NT) fc_prep_kernel(FcArgs a) {
    __shared__ FcPrepSmem sm;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid >> 4, g = tid & 15, tg = c * C + t;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_in(s.k, b, tg, h, i, s.T, K, on);
        const float al = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = al;
        sm.eh[t * LQ + i] = fc_in(s.erase, b, tg, h, i, s.T, K, on) * kv;
        sm.wv[t * LQ + i] = fc_in(s.write, b, tg, h, i, s.T, V, on) * fc_in(s.v, b, tg, h, i, s.T, V, on);
    }
    __syncthreads();
    fc_decay_rows(sm.al, sm.m, sm.bt, sm.lam, K, tid);
    fc_tri<true>(sm.eh, sm.k, sm.al, sm.m, sm.A, K, tid);  // A, strictly lower
    __syncthreads();
    if (tid < C) {
        // T = (I + A)^-1 by forward substitution, column j = tid: x_r = [r == j] -
        // sum_{q < r} A_rq x_q, whose entries above row j come out zero.
        const int j = tid;
        float tc[C];
#pragma unroll
        for (int r = 0; r < C; ++r) {
            float x = r == j ? 1.f : 0.f;
#pragma unroll
            for (int q = 0; q < r; ++q) x -= sm.A[r * LT + q] * tc[q];
            tc[r] = x;
        }
#pragma unroll
        for (int r = 0; r < C; ++r) sm.T[r * LT + j] = tc[r];
    }
    __syncthreads();
    // W' = T (b . ehat), U = T wv, Ktil = lam . k: token t, channels 4g .. 4g + 3;
    // W', Ktil and gv zero on the key padding up to KP.
    const int KP = fc_kp(K);
    const int64_t fo = (int64_t)ci * C;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        if (i < KP) {
            float wsum = 0.f;
            if (i < K)
                for (int q = 0; q <= t; ++q) wsum += sm.T[t * LT + q] * sm.bt[q * LQ + i] * sm.eh[q * LQ + i];
            a.fw[(fo + t) * KP + i] = wsum;
            a.fk[(fo + t) * KP + i] = i < K ? sm.lam[t * LQ + i] * sm.k[t * LQ + i] : 0.f;
        }
        if (i < V) {
            float usum = 0.f;
            for (int q = 0; q <= t; ++q) usum += sm.T[t * LT + q] * sm.wv[q * LQ + i];
            a.fu[(fo + t) * V + i] = usum;
        }
    }
    if (tid < KP) a.gv[(int64_t)ci * KP + tid] = tid < K ? sm.bt[(C - 1) * LQ + tid] : 0.f;
    a.tm[(int64_t)ci * C * C + tid] = sm.T[(tid >> 4) * LT + (tid & 15)];
}

// ---- the scan over the chunks of one (batch, head) -----------------------------
// One wave per (batch, head, 16 value columns j = 16 cg + l % 16), on
// v_mfma_f32_16x16x4f32 (exact f32 products).  The state's key axis is cut
// into KT tiles of 16 rows; tile tau lives in the accumulator layout: lane l
// (g = l / 16, n = l % 16) holds S[16 tau + 4 g + r][16 cg + n] in register r.
// Per chunk, forward:  v = U - W' S,          S <- diag(gv) S + Ktil^T v
//            reverse:  v = Ktil X,            X <- diag(gv) X + N - W'^T v
// Each product's 16-long reduction runs as four k = 4 MFMA steps s whose
// k-slice is {4 g + s}: the B operand of step s is then register s of the
// lane's own accumulator tile (rows 4 g + s of S or X, rows 4 g + s of v), so
// no value changes lanes; the A operand is the matching element of W' or Ktil,
// read from global memory into registers one chunk ahead.
template <int KT>
struct FcScanOps {
    float w[KT][4], k[KT][4], g[KT][4], a[KT][4];  // A operands, gv rows, U or N
};

template <int KT, bool REV>
__device__ __forceinline__ void fc_scan_load(const FcArgs &a, int64_t ci, int cg, FcScanOps<KT> &o) {
    const int K = a.s.K, V = a.s.V, KP = 16 * KT, l = lane_id(), g = l >> 4, n = l & 15, j = 16 * cg + n;
    const float *fw = a.fw + ci * C * KP, *fk = a.fk + ci * C * KP;
#pragma unroll
    for (int tau = 0; tau < KT; ++tau)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // the operand (token l % 16, key 16 tau + 4 g + s) and (token 4 g + s, key 16 tau + l % 16)
            const float rowk = (REV ? fk : fw)[n * KP + 16 * tau + 4 * g + s];
            const float colk = (REV ? fw : fk)[(4 * g + s) * KP + 16 * tau + n];
            o.w[tau][s] = REV ? rowk : -rowk;
            o.k[tau][s] = REV ? -colk : colk;
            o.g[tau][s] = a.gv[ci * KP + 16 * tau + 4 * g + s];
            if (REV) {
                const int i = 16 * tau + 4 * g + s;
                o.a[tau][s] = (i < K && j < V) ? a.n[(ci * K + i) * V + j] : 0.f;
            } else {
                o.a[tau][s] = (tau == 0 && j < V) ? a.fu[(ci * C + 4 * g + s) * V + j] : 0.f;
            }
        }
}

template <int KT, bool REV>
__global__ void __launch_bounds__(64) fc_scan_kernel(FcArgs a) {
    const SeqArgs &s = a.s;
    const int K = s.K, V = s.V, ng = (V + 15) / 16;
    const int wg = blockIdx.x, bh = wg / ng, cg = wg % ng, b = bh / s.H, h = bh % s.H;
    const int l = lane_id(), g = l >> 4, n = l & 15, j = 16 * cg + n;
    const bool jv = j < V;
    f32x4 X[KT];
#pragma unroll
    for (int tau = 0; tau < KT; ++tau)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * tau + 4 * g + r;
            float x = 0.f;
            if (i < K && jv) {
                if (!REV) x = s.initial.data ? ld4<float>(s.initial, b, h, i, j) : 0.f;
                else x = s.dfinal ? s.dfinal[((int64_t)bh * K + i) * V + j] : 0.f;
            }
            X[tau][r] = x;
        }
    FcScanOps<KT> cur, nxt;
    fc_scan_load<KT, REV>(a, (int64_t)bh * a.nc + (REV ? a.nc - 1 : 0), cg, cur);
    float *keep = REV ? a.ds : a.st;
    for (int step = 0; step < a.nc; ++step) {
        const int c = REV ? a.nc - 1 - step : step;
        const int64_t ci = (int64_t)bh * a.nc + c;
        if (step + 1 < a.nc) fc_scan_load<KT, REV>(a, ci + (REV ? -1 : 1), cg, nxt);
        // the state before (forward) / the adjoint after (reverse) this chunk
#pragma unroll
        for (int tau = 0; tau < KT; ++tau)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * tau + 4 * g + r;
                if (i < K && jv) keep[(ci * K + i) * V + j] = X[tau][r];
            }
        // v[t][j], t = 4 g + r: U - W' S (forward) or Ktil X (reverse)
        f32x4 v = REV ? zero4() : f32x4{cur.a[0][0], cur.a[0][1], cur.a[0][2], cur.a[0][3]};
#pragma unroll
        for (int tau = 0; tau < KT; ++tau)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.w[tau][q], X[tau][q], v, 0, 0, 0);
        // S <- diag(gv) S (+ N) + Ktil^T v, or X <- diag(gv) X + N - W'^T v
#pragma unroll
        for (int tau = 0; tau < KT; ++tau) {
            f32x4 x;
#pragma unroll
            for (int r = 0; r < 4; ++r) x[r] = cur.g[tau][r] * X[tau][r] + (REV ? cur.a[tau][r] : 0.f);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                x = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[tau][q], v[q], x, 0, 0, 0);
            X[tau] = x;
        }
        cur = nxt;
    }
    float *fin = REV ? s.dinitial : s.final_state;
    if (fin)
#pragma unroll
        for (int tau = 0; tau < KT; ++tau)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * tau + 4 * g + r;
                if (i < K && jv) fin[((int64_t)bh * K + i) * V + j] = X[tau][r];
            }
}

template <bool REV>
static void launch_fc_scan(const FcArgs &a, hipStream_t stream) {
    const dim3 grid(a.s.B * a.s.H * ((a.s.V + 15) / 16)), block(64);
    switch (fc_kp(a.s.K) / 16) {
        case 1: hipLaunchKernelGGL((fc_scan_kernel<1, REV>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((fc_scan_kernel<2, REV>), grid, block, 0, stream, a); break;
        case 3: hipLaunchKernelGGL((fc_scan_kernel<3, REV>), grid, block, 0, stream, a); break;
        default: hipLaunchKernelGGL((fc_scan_kernel<4, REV>), grid, block, 0, stream, a); break;
    }
}

// ---- out: edits, outputs, scores ----------------------------------------------
__global__ void __launch_bounds__(NT) fc_out_kernel(FcArgs a) {
    __shared__ FcOutSmem sm;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid >> 4, g = tid & 15, tg = c * C + t;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    float ksq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_in(s.k, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_in(s.q, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.eh[t * LQ + i] = fc_in(s.erase, b, tg, h, i, s.T, K, on) * kv;
        sm.wv[t * LQ + i] = fc_in(s.write, b, tg, h, i, s.T, V, on) * fc_in(s.v, b, tg, h, i, s.T, V, on);
        ksq += kv * kv;
    }
    ksq += __shfl_xor(ksq, 1);
    ksq += __shfl_xor(ksq, 2);
    ksq += __shfl_xor(ksq, 4);
    ksq += __shfl_xor(ksq, 8);
    if (g == 0) sm.kk[t] = ksq;
    const float *st = a.st + (int64_t)ci * K * V;
    for (int e = tid; e < K * V; e += NT) sm.s0[(e / V) * LS + e % V] = st[e];
    sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    __syncthreads();
    fc_b_row(sm.al, sm.m, sm.bt, K, tid);
    fc_tri<false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);  // P, lower with the diagonal
    __syncthreads();
    // R = wv - Ahat S0 (token t, columns 4g ..)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        if (j < V) {
            float x = 0.f;
            for (int i = 0; i < K; ++i) x += sm.bt[t * LQ + i] * sm.eh[t * LQ + i] * sm.s0[i * LS + j];
            sm.r[t * LQ + j] = sm.wv[t * LQ + j] - x;
        }
    }
    __syncthreads();
    // delta = T R and |delta_t|^2
    float dsq = 0.f, dlt[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        float x = 0.f;
        if (j < V)
            for (int q = 0; q <= t; ++q) x += sm.T[t * LT + q] * sm.r[q * LQ + j];
        dlt[e] = x;
        if (j < V) sm.dl[t * LQ + j] = x;
        dsq += x * x;
    }
    dsq += __shfl_xor(dsq, 1);
    dsq += __shfl_xor(dsq, 2);
    dsq += __shfl_xor(dsq, 4);
    dsq += __shfl_xor(dsq, 8);
    if (g == 0) sm.dd[t] = dsq;
    __syncthreads();
    // O = Qhat S0 + P delta; delta to the checkpoint
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        if (j < V) {
            float x = 0.f;
            for (int i = 0; i < K; ++i) x += sm.bt[t * LQ + i] * sm.q[t * LQ + i] * sm.s0[i * LS + j];
            for (int q = 0; q <= t; ++q) x += sm.P[t * LT + q] * sm.dl[q * LQ + j];
            if (tg < s.T) store_out(s.out, s.out_bf16, (((int64_t)b * s.T + tg) * s.H + h) * V + j, x);
            a.dl[((int64_t)ci * C + t) * V + j] = dlt[e];
        }
    }
    if (s.scores && tid < C && c * C + tid < s.T)
        s.scores[((int64_t)b * s.T + c * C + tid) * s.H + h] =
            sm.m.val[tid] != 0.f ? sqrtf(sm.kk[tid] * sm.dd[tid]) : 0.f;
}

// ---- bprep: N = Qhat^T dO - W'^T X, X = P^T dO + c delta ------------------------
__global__ void __launch_bounds__(NT) fc_bprep_kernel(FcArgs a) {
    __shared__ FcBPrepSmem sm;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid >> 4, g = tid & 15, tg = c * C + t;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    const bool score_adj = s.dscores != nullptr;
    float ksq = 0.f, dsq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_in(s.k, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_in(s.q, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.dO[t * LQ + i] = (s.dout.data && on && tg < s.T && i < V) ? ld4<float>(s.dout, b, tg, h, i) : 0.f;
        const float d = i < V ? a.dl[((int64_t)ci * C + t) * V + i] : 0.f;
        sm.dl[t * LQ + i] = d;
        ksq += kv * kv;
        dsq += d * d;
    }
    ksq += __shfl_xor(ksq, 1), ksq += __shfl_xor(ksq, 2), ksq += __shfl_xor(ksq, 4), ksq += __shfl_xor(ksq, 8);
    dsq += __shfl_xor(dsq, 1), dsq += __shfl_xor(dsq, 2), dsq += __shfl_xor(dsq, 4), dsq += __shfl_xor(dsq, 8);
    if (g == 0) {
        const float nk = sqrtf(ksq), nd = sqrtf(dsq);
        const float dsc = (score_adj && tg < s.T) ? s.dscores[((int64_t)b * s.T + tg) * s.H + h] : 0.f;
        sm.cs[t] = (on && nk > 0.f && nd > 0.f) ? dsc * nk / nd : 0.f;
    }
    __syncthreads();
    fc_b_row(sm.al, sm.m, sm.bt, K, tid);
    fc_tri<false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);  // P, lower with the diagonal
    // W' rows of this chunk
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        sm.w[t * LQ + i] = i < K ? a.fw[((int64_t)ci * C + t) * fc_kp(K) + i] : 0.f;
    }
    __syncthreads();
    // X = P^T dO + c delta (token t, columns 4g ..)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        float x = sm.cs[t] * sm.dl[t * LQ + j];
        for (int q = t; q < C; ++q) x += sm.P[q * LT + t] * sm.dO[q * LQ + j];
        sm.x[t * LQ + j] = x;
    }
    __syncthreads();
    // N[i][j] = sum_t Qhat[t][i] dO[t][j] - W'[t][i] X[t][j]: thread (i = tid / 4,
    // columns 16 (tid % 4) ..)
    {
        const int i = tid >> 2, j0 = 16 * (tid & 3);
        if (i < K) {
            float nacc[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) nacc[q] = 0.f;
            for (int tt = 0; tt < C; ++tt) {
                const float qh = sm.bt[tt * LQ + i] * sm.q[tt * LQ + i], wq = sm.w[tt * LQ + i];
#pragma unroll
                for (int q = 0; q < 16; ++q) nacc[q] += qh * sm.dO[tt * LQ + j0 + q] - wq * sm.x[tt * LQ + j0 + q];
            }
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (j0 + q < V) a.n[((int64_t)ci * K + i) * V + j0 + q] = nacc[q];
        }
    }
}

// ---- bgrad: every gradient of one chunk -----------------------------------------
// With S0 (forward scan), delta (out) and dS at the chunk end (adjoint scan):
//   ddelta = P^T dO + Ktil dS + c delta,  dR = T^T ddelta,  dw = dR.v,  dv = dR.w
//   dAhat = -dR S0^T,  dQhat = dO S0^T,  dKtil = delta dS^T
//   dA = -strict_lower(dR delta^T),  dP = lower(dO delta^T)   (same segment)
//   eA_t = sum_s dA_ts D_ts k_s,  qP_t = sum_s dP_ts D_ts k_s,
//   kAP_s = sum_t (dA_ts ehat_t + dP_ts q_t) D_ts
//   dq = b dQhat + qP;  dehat = b dAhat + eA;  de = k dehat;
//   dk = lam dKtil + kAP + e dehat + c' k
// and dalpha_u = sum over the pairs (hi, lo) with lo < u <= hi of the pair's
// coefficient times the product of the gates over (lo, hi] without u (interior
// pairs (dA_ts ehat_t + dP_ts q_t) k_s; start pairs ehat_t dAhat_t + q_t dQhat_t
// through b_t; end pairs k_s dKtil_s through lam_s; rowsum(S0 . dS) through
// b_15): exact for zero and negative gates.
__global__ void __launch_bounds__(NT) fc_bgrad_kernel(FcArgs a) {
    __shared__ FcBGradSmem sm;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid >> 4, g = tid & 15, tg = c * C + t;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    const bool score_adj = s.dscores != nullptr;
    float ksq = 0.f, dsq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_in(s.k, b, tg, h, i, s.T, K, on);
        const float ev = fc_in(s.erase, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_in(s.q, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.e[t * LQ + i] = ev;
        sm.eh[t * LQ + i] = ev * kv;
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.v[t * LQ + i] = fc_in(s.v, b, tg, h, i, s.T, V, on);
        sm.w[t * LQ + i] = fc_in(s.write, b, tg, h, i, s.T, V, on);
        sm.dO[t * LQ + i] = (s.dout.data && on && tg < s.T && i < V) ? ld4<float>(s.dout, b, tg, h, i) : 0.f;
        const float d = i < V ? a.dl[((int64_t)ci * C + t) * V + i] : 0.f;
        sm.dl[t * LQ + i] = d;
        ksq += kv * kv;
        dsq += d * d;
    }
    ksq += __shfl_xor(ksq, 1), ksq += __shfl_xor(ksq, 2), ksq += __shfl_xor(ksq, 4), ksq += __shfl_xor(ksq, 8);
    dsq += __shfl_xor(dsq, 1), dsq += __shfl_xor(dsq, 2), dsq += __shfl_xor(dsq, 4), dsq += __shfl_xor(dsq, 8);
    if (g == 0) {
        const float nk = sqrtf(ksq), nd = sqrtf(dsq);
        const float dsc = (score_adj && tg < s.T) ? s.dscores[((int64_t)b * s.T + tg) * s.H + h] : 0.f;
        const bool ok = on && nk > 0.f && nd > 0.f;
        sm.cs[t] = ok ? dsc * nk / nd : 0.f;
        sm.ck[t] = ok ? dsc * nd / nk : 0.f;
    }
    {
        const float *st = a.st + (int64_t)ci * K * V, *ds = a.ds + (int64_t)ci * K * V;
        for (int e = tid; e < K * V; e += NT) {
            sm.s0[(e / V) * LS + e % V] = st[e];
            sm.ds[(e / V) * LS + e % V] = ds[e];
        }
    }
    sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    __syncthreads();
    fc_decay_rows(sm.al, sm.m, sm.bt, sm.lam, K, tid);
    fc_tri<false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);
    if (tid < K) {  // rowsum(S0 . dS) of key channel i
        float f = 0.f;
        for (int j = 0; j < V; ++j) f += sm.s0[tid * LS + j] * sm.ds[tid * LS + j];
        sm.fs[tid] = f;
    }
    __syncthreads();
    // ddelta = P^T dO + Ktil dS + c delta
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        float x = sm.cs[t] * sm.dl[t * LQ + j];
        if (j < V) {
            for (int q = t; q < C; ++q) x += sm.P[q * LT + t] * sm.dO[q * LQ + j];
            for (int i = 0; i < K; ++i) x += sm.lam[t * LQ + i] * sm.k[t * LQ + i] * sm.ds[i * LS + j];
        }
        sm.dd[t * LQ + j] = x;
    }
    __syncthreads();
    // dR = T^T ddelta; dw, dv
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * g + e;
        float x = 0.f;
        for (int q = t; q < C; ++q) x += sm.T[q * LT + t] * sm.dd[q * LQ + j];
        sm.dr[t * LQ + j] = x;
        if (j < V && tg < s.T) {
            const int64_t o = (((int64_t)b * s.T + tg) * s.H + h) * V + j;
            if (s.dwrite) s.dwrite[o] = on ? x * sm.v[t * LQ + j] : 0.f;
            if (s.dv) store_out(s.dv, 0, o, on ? x * sm.w[t * LQ + j] : 0.f);
        }
    }
    __syncthreads();
    // dAhat = -dR S0^T, dQhat = dO S0^T, dKtil = delta dS^T (token t, keys 4g ..)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        float xa = 0.f, xq = 0.f, xk = 0.f;
        if (i < K)
            for (int j = 0; j < V; ++j) {
                xa -= sm.dr[t * LQ + j] * sm.s0[i * LS + j];
                xq += sm.dO[t * LQ + j] * sm.s0[i * LS + j];
                xk += sm.dl[t * LQ + j] * sm.ds[i * LS + j];
            }
        sm.ga[t * LQ + i] = xa;
        sm.gq[t * LQ + i] = xq;
        sm.gk[t * LQ + i] = xk;
    }
    {  // dA (strict, same segment) and dP (with the diagonal): pair (t, s) = (tid / 16, tid % 16)
        const int tt = tid >> 4, ss = tid & 15;
        float xa = 0.f, xp = 0.f;
        if (ss <= tt && sm.m.seg[tt] == sm.m.seg[ss])
            for (int j = 0; j < V; ++j) {
                xa -= sm.dr[tt * LQ + j] * sm.dl[ss * LQ + j];
                xp += sm.dO[tt * LQ + j] * sm.dl[ss * LQ + j];
            }
        sm.dA[tt * LT + ss] = ss < tt ? xa : 0.f;
        sm.dP[tt * LT + ss] = xp;
    }
    __syncthreads();
    // Per key channel i (threads i < K): the decay-weighted sums through running
    // products, then dq, dk, de and dalpha for every token of the channel.
    if (tid < K) {
        const int i = tid, sg15 = sm.m.seg[C - 1];
        float eA[C], qP[C], kAP[C], al[C];
#pragma unroll
        for (int u = 0; u < C; ++u) {
            eA[u] = qP[u] = kAP[u] = 0.f;
            al[u] = sm.al[u * LQ + i];
        }
#pragma unroll
        for (int tt = 0; tt < C; ++tt) {
            const float et = sm.eh[tt * LQ + i], qt = sm.q[tt * LQ + i];
            float d = 1.f;  // D_{tt, ss}
#pragma unroll
            for (int ss = tt; ss >= 0; --ss) {
                if (sm.m.seg[ss] != sm.m.seg[tt]) break;
                const float dA = sm.dA[tt * LT + ss], dP = sm.dP[tt * LT + ss];
                const float ks = sm.k[ss * LQ + i];
                eA[tt] += dA * d * ks;
                qP[tt] += dP * d * ks;
                kAP[ss] += (dA * et + dP * qt) * d;
                d *= al[ss];
            }
        }
        // dalpha by the pair products (see the kernel comment): lo = -1 is the
        // chunk start, hi = 15 also stands for the chunk end.
        float dal[C];
#pragma unroll
        for (int u = 0; u < C; ++u) dal[u] = 0.f;
        for (int lo = -1; lo < C - 1; ++lo) {
            float Y[C], y = 0.f;
#pragma unroll
            for (int u = C - 1; u >= 0; --u) {
                float cf = 0.f;
                if (u > lo) {
                    if (lo < 0) {
                        cf = sm.m.seg[u] == 0 ? sm.eh[u * LQ + i] * sm.ga[u * LQ + i] + sm.q[u * LQ + i] * sm.gq[u * LQ + i] : 0.f;
                        if (u == C - 1 && sg15 == 0) cf += sm.fs[i];
                    } else {
                        cf = (sm.dA[u * LT + lo] * sm.eh[u * LQ + i] + sm.dP[u * LT + lo] * sm.q[u * LQ + i]) *
                             sm.k[lo * LQ + i];
                        if (u == C - 1 && sm.m.seg[lo] == sg15) cf += sm.k[lo * LQ + i] * sm.gk[lo * LQ + i];
                    }
                }
                y = u == C - 1 ? cf : cf + al[u + 1] * y;
                Y[u] = y;
            }
            float L = 1.f;
#pragma unroll
            for (int u = 0; u < C; ++u)
                if (u > lo) {
                    dal[u] += L * Y[u];
                    L *= al[u];
                }
        }
        const int K_ = K;
#pragma unroll
        for (int u = 0; u < C; ++u) {
            const int tq = c * C + u;
            if (tq >= s.T) continue;
            const bool von = sm.m.val[u] != 0.f;
            const float bt = sm.bt[u * LQ + i], lt = sm.lam[u * LQ + i];
            const float q = sm.q[u * LQ + i], k = sm.k[u * LQ + i], ev = sm.e[u * LQ + i];
            const float dq = bt * sm.gq[u * LQ + i] + qP[u];
            const float deh = bt * sm.ga[u * LQ + i] + eA[u];
            const float dk = lt * sm.gk[u * LQ + i] + kAP[u] + ev * deh + sm.ck[u] * k;
            const int64_t o = (((int64_t)b * s.T + tq) * s.H + h) * K_ + i;
            if (s.dq) store_out(s.dq, 0, o, von ? dq : 0.f);
            if (s.dk) store_out(s.dk, 0, o, von ? dk : 0.f);
            if (s.derase) s.derase[o] = von ? k * deh : 0.f;
            if (s.dalpha) s.dalpha[o] = (von && !sm.m.rs[u]) ? dal[u] : 0.f;
            (void)q;
        }
    }
}

static inline void fmark(const hipEvent_t *ev, int i, hipStream_t stream) {
    if (ev) (void)hipEventRecord(ev[i], stream);
}

hipError_t launch_fc_fwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int n = a.s.B * a.s.H * a.nc;
    fmark(ev, 0, stream);
    hipLaunchKernelGGL(fc_prep_kernel, dim3(n), dim3(NT), 0, stream, a);
    fmark(ev, 1, stream);
    fmark(ev, 2, stream);
    launch_fc_scan<false>(a, stream);
    fmark(ev, 3, stream);
    fmark(ev, 4, stream);
    hipLaunchKernelGGL(fc_out_kernel, dim3(n), dim3(NT), 0, stream, a);
    fmark(ev, 5, stream);
    return hipGetLastError();
}

hipError_t launch_fc_bwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int n = a.s.B * a.s.H * a.nc;
    fmark(ev, 0, stream);
    hipLaunchKernelGGL(fc_bprep_kernel, dim3(n), dim3(NT), 0, stream, a);
    fmark(ev, 1, stream);
    fmark(ev, 2, stream);
    launch_fc_scan<true>(a, stream);
    fmark(ev, 3, stream);
    fmark(ev, 4, stream);
    hipLaunchKernelGGL(fc_bgrad_kernel, dim3(n), dim3(NT), 0, stream, a);
    fmark(ev, 5, stream);
    return hipGetLastError();
}

}  // namespace gdn2
