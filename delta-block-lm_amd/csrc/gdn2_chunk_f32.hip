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

// q, k, v and dO elements as the caller holds them: f32, or bf16 when bf (the
// products then run on the exact f32 values of the bf16 inputs).
__device__ __forceinline__ float fc_ld(const View &v, bool bf, int b, int tg, int h, int ch) {
    return bf ? ld4<bf16_t>(v, b, tg, h, ch) : ld4<float>(v, b, tg, h, ch);
}
__device__ __forceinline__ float fc_x(const View &v, bool bf, int b, int tg, int h, int ch, int T, int W, bool on) {
    return (on && tg < T && ch < W) ? fc_ld(v, bf, b, tg, h, ch) : 0.f;
}

// b_t and lam_t of channel i (threads i < K): running products of the gates;
// zero on the channels K .. 63, which the MFMA products read as padding.
__device__ void fc_decay_rows(const float *al, const Masks &m, float *bt, float *lam, int K, int tid) {
    if (tid >= K && tid < FK)
        for (int t = 0; t < C; ++t) bt[t * LQ + tid] = lam[t * LQ + tid] = 0.f;
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

// b_t alone (threads i < K; zero on the channels K .. 63).
__device__ void fc_b_row(const float *al, const Masks &m, float *bt, int K, int tid) {
    if (tid >= K && tid < FK)
        for (int t = 0; t < C; ++t) bt[t * LQ + tid] = 0.f;
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
    float q[C * LQ], k[C * LQ], al[C * LQ], eh[C * LQ], wv[C * LQ], bt[C * LQ];
    float s0[FK * LS];  // S0, zero-padded to whole 16 x 16 tiles
    float T[C * LT], P[C * LT];
    float kk[C], ddp[4][C];
};

struct FcBPrepSmem {
    Masks m;
    float q[C * LQ], k[C * LQ], al[C * LQ], bt[C * LQ], dO[C * LQ], dl[C * LQ], w[C * LQ];
    float P[C * LT];
    float cs[C];
};

struct FcBGradSmem {
    Masks m;
    float q[C * LQ], k[C * LQ], e[C * LQ], al[C * LQ], dO[C * LQ], dl[C * LQ], dr[C * LQ];
    float bt[C * LQ], lam[C * LQ];
    union {
        struct {
            float s0[FK * LS], ds[FK * LS];  // S0 and dS, zero-padded to whole 16 x 16 tiles
        } st;
        struct {
            float ga[C * LQ], gq[C * LQ], gk[C * LQ];  // dAhat, dQhat, dKtil [token][key]
            float part[4 * C * 64];  // dalpha partials: 4 rpw groups x C rows x 64 / rpw channels
        } gr;
    } u;
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
        const float kv = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, on);
        const float al = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = al;
        sm.eh[t * LQ + i] = fc_in(s.erase, b, tg, h, i, s.T, K, on) * kv;
        sm.wv[t * LQ + i] = fc_in(s.write, b, tg, h, i, s.T, V, on) * fc_x(s.v, a.in_bf16, b, tg, h, i, s.T, V, on);
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
    // Ktil = lam . k (token t, channels 4g .. 4g + 3) and gv = b_15; zero on the
    // key padding up to KP.
    const int KP = fc_kp(K), KT = KP >> 4, VT = (V + 15) >> 4;
    const int64_t fo = (int64_t)ci * C;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        if (i < KP) a.fk[(fo + t) * KP + i] = i < K ? sm.lam[t * LQ + i] * sm.k[t * LQ + i] : 0.f;
    }
    if (tid < KP) a.gv[(int64_t)ci * KP + tid] = tid < K ? sm.bt[(C - 1) * LQ + tid] : 0.f;
    a.tm[(int64_t)ci * C * C + tid] = sm.T[(tid >> 4) * LT + (tid & 15)];
    // W' = T (b . ehat) and U = T wv on v_mfma_f32_16x16x4f32: tiles 0 .. KT - 1
    // of W' (key tiles), then VT tiles of U, taken by the waves in turn (lane
    // (lg, ln): tokens 4 lg + r, column 16 tile + ln).
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    for (int n = w; n < KT + VT; n += 4) {
        const bool isw = n < KT;
        const int col = 16 * (isw ? n : n - KT) + ln;
        f32x4 x = zero4();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ss = 4 * lg + q;
            const float bv = isw ? sm.bt[ss * LQ + col] * sm.eh[ss * LQ + col] : sm.wv[ss * LQ + col];
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[ln * LT + ss], bv, x, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tt = 4 * lg + r;
            if (isw) a.fw[(fo + tt) * KP + col] = x[r];
            else if (col < V) a.fu[(fo + tt) * V + col] = x[r];
        }
    }
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
    // Every load is issued (indices past the widths are clamped and their values
    // dropped by a select), so no load sits behind a branch and the compiler's
    // memory-counter waits stay exact across the prefetch ring.
    const int K = a.s.K, V = a.s.V, KP = 16 * KT, l = lane_id(), g = l >> 4, n = l & 15, j = 16 * cg + n;
    const bool jv = j < V;
    const int jc = jv ? j : 0;
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
                const bool in = i < K && jv;
                const float x = a.n[(ci * K + (i < K ? i : 0)) * V + jc];
                o.a[tau][s] = in ? x : 0.f;
            } else if (tau == 0) {
                const float x = a.fu[(ci * C + 4 * g + s) * V + jc];
                o.a[tau][s] = jv ? x : 0.f;
            } else {
                o.a[tau][s] = 0.f;
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
    // A ring of D chunks' operands in registers: chunk step + D is loaded (the
    // last chunk again past the end) as soon as step's operands are used.
    constexpr int D = KT <= 2 ? 3 : 2;
    FcScanOps<KT> ring[D];
    auto chunk_at = [&](int step) {
        const int sc = step < a.nc ? step : a.nc - 1;
        return (int64_t)bh * a.nc + (REV ? a.nc - 1 - sc : sc);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) fc_scan_load<KT, REV>(a, chunk_at(d), cg, ring[d]);
    float *keep = REV ? a.ds : a.st;
    for (int s0 = 0; s0 < a.nc; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int step = s0 + d;
            if (step >= a.nc) break;
            const int64_t ci = chunk_at(step);
            const FcScanOps<KT> &cur = ring[d];
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
            // S <- diag(gv) S + Ktil^T v, or X <- diag(gv) X + N - W'^T v
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
            fc_scan_load<KT, REV>(a, chunk_at(step + D), cg, ring[d]);
        }
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
    const int KP = fc_kp(K), VT = (V + 15) >> 4, VP = 16 * VT;
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    float ksq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.eh[t * LQ + i] = fc_in(s.erase, b, tg, h, i, s.T, K, on) * kv;
        sm.wv[t * LQ + i] = fc_in(s.write, b, tg, h, i, s.T, V, on) * fc_x(s.v, a.in_bf16, b, tg, h, i, s.T, V, on);
        ksq += kv * kv;
    }
    ksq += __shfl_xor(ksq, 1);
    ksq += __shfl_xor(ksq, 2);
    ksq += __shfl_xor(ksq, 4);
    ksq += __shfl_xor(ksq, 8);
    if (g == 0) sm.kk[t] = ksq;
    {
        const float *st = a.st + (int64_t)ci * K * V;
        for (int e = tid; e < KP * VP; e += NT) {
            const int i = e / VP, j = e - i * VP;
            sm.s0[i * LS + j] = (i < K && j < V) ? st[i * V + j] : 0.f;
        }
    }
    sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    __syncthreads();
    fc_b_row(sm.al, sm.m, sm.bt, K, tid);
    fc_tri<false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);  // P, lower with the diagonal
    __syncthreads();
    // Wave w: value tile w on v_mfma_f32_16x16x4f32 (lane (lg, ln): rows 4 lg + r,
    // column 16 w + ln).  R = wv - Ahat S0, O = Qhat S0 over the key axis; then
    // delta = T R and O += P delta with the accumulator rows as the B operand
    // (step q reduces over the tokens 4 lg + q).
    if (w < VT) {
        const int j = 16 * w + ln;
        f32x4 x = zero4(), o = zero4();
        for (int kk = 0; kk < KP; kk += 4) {
            const int i = kk + lg;
            const float sv = sm.s0[i * LS + j], bti = sm.bt[ln * LQ + i];
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(bti * sm.eh[ln * LQ + i], sv, x, 0, 0, 0);
            o = __builtin_amdgcn_mfma_f32_16x16x4f32(bti * sm.q[ln * LQ + i], sv, o, 0, 0, 0);
        }
        f32x4 r, d = zero4();
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = sm.wv[(4 * lg + q) * LQ + j] - x[q];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[ln * LT + 4 * lg + q], r[q], d, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.P[ln * LT + 4 * lg + q], d[q], o, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float p = d[q] * d[q];
            p += __shfl_xor(p, 1);
            p += __shfl_xor(p, 2);
            p += __shfl_xor(p, 4);
            p += __shfl_xor(p, 8);
            const int tt = 4 * lg + q, tq = c * C + tt;
            if (ln == 0) sm.ddp[w][tt] = p;
            if (j < V) {
                a.dl[((int64_t)ci * C + tt) * V + j] = d[q];
                if (tq < s.T) store_out(s.out, s.out_bf16, (((int64_t)b * s.T + tq) * s.H + h) * V + j, o[q]);
            }
        }
    }
    __syncthreads();
    if (s.scores && tid < C && c * C + tid < s.T) {
        float dd = 0.f;
        for (int x = 0; x < VT; ++x) dd += sm.ddp[x][tid];
        s.scores[((int64_t)b * s.T + c * C + tid) * s.H + h] = sm.m.val[tid] != 0.f ? sqrtf(sm.kk[tid] * dd) : 0.f;
    }
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
        const float kv = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.dO[t * LQ + i] = (s.dout.data && on && tg < s.T && i < V) ? fc_ld(s.dout, a.in_bf16, b, tg, h, i) : 0.f;
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
    // Wave w: value tile w on v_mfma_f32_16x16x4f32 (lane (lg, ln): rows 4 lg + r,
    // column 16 w + ln).  X = P^T dO + c delta, then per key tile tau
    // N = Qhat^T dO - W'^T X, X's accumulator rows as the B operand.
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15, VT = (V + 15) >> 4, KT = fc_kp(K) >> 4;
    if (w < VT) {
        const int j = 16 * w + ln;
        f32x4 x;
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = sm.cs[4 * lg + q] * sm.dl[(4 * lg + q) * LQ + j];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.P[(4 * lg + q) * LT + ln], sm.dO[(4 * lg + q) * LQ + j], x,
                                                     0, 0, 0);
        for (int tau = 0; tau < KT; ++tau) {
            const int i = 16 * tau + ln;
            f32x4 n = zero4();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tt = 4 * lg + q;
                n = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.bt[tt * LQ + i] * sm.q[tt * LQ + i], sm.dO[tt * LQ + j], n,
                                                         0, 0, 0);
                n = __builtin_amdgcn_mfma_f32_16x16x4f32(-sm.w[tt * LQ + i], x[q], n, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ii = 16 * tau + 4 * lg + r;
                if (ii < K && j < V) a.n[((int64_t)ci * K + ii) * V + j] = n[r];
            }
        }
    }
}

// ---- bgrad: every gradient of one chunk -----------------------------------------
// With S0 (forward scan), delta (out) and dS at the chunk end (adjoint scan):
//   ddelta = P^T dO + Ktil dS + c delta,  dR = T^T ddelta,  dw = dR.v,  dv = dR.w
//   dAhat = -dR S0^T,  dQhat = dO S0^T,  dKtil = delta dS^T
//   dA = -strict_lower(dR delta^T),  dP = lower(dO delta^T)   (same segment)
// on v_mfma_f32_16x16x4f32 (wave w takes value tile w in the first group, the
// 16 x 16 output tiles in turn in the second); then per key channel on the VALU
//   eA_t = sum_s dA_ts D_ts k_s,  qP_t = sum_s dP_ts D_ts k_s,
//   kAP_s = sum_t (dA_ts ehat_t + dP_ts q_t) D_ts
//   dq = b dQhat + qP;  dehat = b dAhat + eA;  de = k dehat;
//   dk = lam dKtil + kAP + e dehat + c' k
// and dalpha_u = sum over the pairs (hi, lo) with lo < u <= hi of the pair's
// coefficient times the product of the gates over (lo, hi] without u (interior
// pairs (dA_ts ehat_t + dP_ts q_t) k_s; start pairs ehat_t dAhat_t + q_t dQhat_t
// through b_t; end pairs k_s dKtil_s through lam_s; rowsum(S0 . dS) through
// b_15): sum_{lo < u} L(lo, u) Y(u, lo) with L the gates over (lo, u) and Y by
// Horner over hi, exact for zero and negative gates.
__global__ void __launch_bounds__(NT) fc_bgrad_kernel(FcArgs a) {
    __shared__ FcBGradSmem sm;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid >> 4, g = tid & 15, tg = c * C + t;
    const int KT = (K + 15) >> 4, VT = (V + 15) >> 4, VP = 16 * VT;
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    const bool score_adj = s.dscores != nullptr;
    float ksq = 0.f, dsq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float kv = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.q[t * LQ + i] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, on);
        sm.k[t * LQ + i] = kv;
        sm.e[t * LQ + i] = fc_in(s.erase, b, tg, h, i, s.T, K, on);
        sm.al[t * LQ + i] = (on && i < K) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        sm.dO[t * LQ + i] = (s.dout.data && on && tg < s.T && i < V) ? fc_ld(s.dout, a.in_bf16, b, tg, h, i) : 0.f;
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
        const int KP = 16 * KT;
        for (int e = tid; e < KP * VP; e += NT) {
            const int i = e / VP, j = e - i * VP;
            const bool in = i < K && j < V;
            sm.u.st.s0[i * LS + j] = in ? st[i * V + j] : 0.f;
            sm.u.st.ds[i * LS + j] = in ? ds[i * V + j] : 0.f;
        }
    }
    sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    __syncthreads();
    fc_decay_rows(sm.al, sm.m, sm.bt, sm.lam, K, tid);
    fc_tri<false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);
    {  // rowsum(S0 . dS) of key channel i = tid / 4, in four column quarters
        const int i = tid >> 2, j0 = 16 * (tid & 3);
        float f = 0.f;
        if (i < 16 * KT && j0 < VP)  // inside the zero-padded tiles
#pragma unroll
            for (int j = 0; j < 16; ++j) f += sm.u.st.s0[i * LS + j0 + j] * sm.u.st.ds[i * LS + j0 + j];
        f += __shfl_xor(f, 1);
        f += __shfl_xor(f, 2);
        if ((tid & 3) == 0) sm.fs[i] = f;
    }
    __syncthreads();
    // ddelta and dR of value tile w (lane (lg, ln): rows 4 lg + r, column 16 w + ln)
    if (w < VT) {
        const int j = 16 * w + ln;
        f32x4 dd;
#pragma unroll
        for (int r = 0; r < 4; ++r) dd[r] = sm.cs[4 * lg + r] * sm.dl[(4 * lg + r) * LQ + j];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dd = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.P[(4 * lg + q) * LT + ln], sm.dO[(4 * lg + q) * LQ + j], dd,
                                                      0, 0, 0);
        for (int tau = 0; tau < KT; ++tau)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = 16 * tau + 4 * lg + q;
                dd = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.lam[ln * LQ + i] * sm.k[ln * LQ + i],
                                                          sm.u.st.ds[i * LS + j], dd, 0, 0, 0);
            }
        f32x4 dr = zero4();
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dr = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[(4 * lg + q) * LT + ln], dd[q], dr, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tt = 4 * lg + r, tq = c * C + tt;
            sm.dr[tt * LQ + j] = dr[r];
            if (j < V && tq < s.T) {
                const bool von = sm.m.val[tt] != 0.f;
                const int64_t o = (((int64_t)b * s.T + tq) * s.H + h) * V + j;
                if (s.dwrite) s.dwrite[o] = von ? dr[r] * fc_ld(s.v, a.in_bf16, b, tq, h, j) : 0.f;
                if (s.dv) store_out(s.dv, a.in_bf16, o, von ? dr[r] * ld4<float>(s.write, b, tq, h, j) : 0.f);
            }
        }
    }
    __syncthreads();
    // The 16 x 16 products over the value axis: tiles 0 .. 3 KT - 1 are dAhat,
    // dQhat, dKtil of key tile tau = n / 3; tile 3 KT is dA, 3 KT + 1 is dP.
    const int ntile = 3 * KT + 2;
    f32x4 res[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int n = w + 4 * m;
        res[m] = zero4();
        if (n >= ntile) continue;
        const int kind = n < 3 * KT ? n % 3 : 3 + (n - 3 * KT), tau = n < 3 * KT ? n / 3 : 0;
        const float *xa = kind == 0 || kind == 3 ? sm.dr : (kind == 2 ? sm.dl : sm.dO);
        const float *yb = kind == 2 ? sm.u.st.ds : sm.u.st.s0;
        const int yo = kind >= 3 ? 0 : (16 * tau + ln) * LS, ys = kind >= 3 ? LQ : LS;
        const float *yy = kind >= 3 ? sm.dl + ln * LQ : yb + yo;
        (void)ys;
        f32x4 acc = zero4();
        for (int kk = 0; kk < VP; kk += 4)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[ln * LQ + kk + lg], yy[kk + lg], acc, 0, 0, 0);
        res[m] = acc;
    }
    __syncthreads();  // S0 and dS are no longer read: their space takes dAhat, dQhat, dKtil
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int n = w + 4 * m;
        if (n >= ntile) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tt = 4 * lg + r;
            if (n < 3 * KT) {
                const int kind = n % 3, i = 16 * (n / 3) + ln;
                float *dst = kind == 0 ? sm.u.gr.ga : (kind == 1 ? sm.u.gr.gq : sm.u.gr.gk);
                dst[tt * LQ + i] = kind == 0 ? -res[m][r] : res[m][r];
            } else {
                const bool same = sm.m.seg[tt] == sm.m.seg[ln];
                if (n == 3 * KT) sm.dA[tt * LT + ln] = (ln < tt && same) ? -res[m][r] : 0.f;
                else sm.dP[tt * LT + ln] = (ln <= tt && same) ? res[m][r] : 0.f;
            }
        }
    }
    __syncthreads();
    // Per key channel: lane i of a group of cpl lanes, rpw groups per wave; the
    // lane keeps its channel's gates, k, q and ehat of the whole chunk in
    // registers.  Group (w, sub) takes the rows u = 4 rpw p + rpw w + sub
    // (p < 4 / rpw): the token rows of eA, qP, kAP and the outputs, then the
    // start rows lo = u - 1 of the alpha gradient's pairs, whose partial sums
    // over lo meet in LDS.
    const int cpl = K <= 16 ? 16 : (K <= 32 ? 32 : 64), rpw = 64 / cpl;
    const int i = l % cpl, sub = l / cpl, sg15 = sm.m.seg[C - 1], np = 4 / rpw;
    const bool iv = i < K;
    float ra[C], rk[C], rq[C], re[C];
    int sg[C];
#pragma unroll
    for (int x = 0; x < C; ++x) {
        ra[x] = sm.al[x * LQ + i];
        rk[x] = sm.k[x * LQ + i];
        rq[x] = sm.q[x * LQ + i];
        re[x] = sm.e[x * LQ + i] * rk[x];
        sg[x] = sm.m.seg[x];
    }
    for (int p = 0; p < np; ++p) {
        const int u = 4 * rpw * p + rpw * w + sub, su = sm.m.seg[u];
        // eA, qP of row u (s <= u) and kAP of row u (t >= u); the running
        // decays stop at u's segment, where dA and dP end as well
        float eA = 0.f, qP = 0.f, kAP = 0.f, d = 1.f, d2 = 1.f;
#pragma unroll
        for (int x = C - 1; x >= 0; --x) {
            if (x <= u) {
                eA += sm.dA[u * LT + x] * d * rk[x];
                qP += sm.dP[u * LT + x] * d * rk[x];
                d = (x > 0 && sg[x - 1] == su) ? d * ra[x] : 0.f;
            }
        }
#pragma unroll
        for (int x = 0; x < C; ++x) {
            if (x >= u) {
                d2 = x == u ? 1.f : (sg[x] == su ? d2 * ra[x] : 0.f);
                kAP += (sm.dA[x * LT + u] * re[x] + sm.dP[x * LT + u] * rq[x]) * d2;
            }
        }
        const int tq = c * C + u;
        if (iv && tq < s.T) {
            const bool von = sm.m.val[u] != 0.f;
            const float bt = sm.bt[u * LQ + i], lt = sm.lam[u * LQ + i];
            const float k = sm.k[u * LQ + i], ev = sm.e[u * LQ + i];
            const float dq = bt * sm.u.gr.gq[u * LQ + i] + qP;
            const float deh = bt * sm.u.gr.ga[u * LQ + i] + eA;
            const float dk = lt * sm.u.gr.gk[u * LQ + i] + kAP + ev * deh + sm.ck[u] * k;
            const int64_t o = (((int64_t)b * s.T + tq) * s.H + h) * K + i;
            if (s.dq) store_out(s.dq, a.in_bf16, o, von ? dq : 0.f);
            if (s.dk) store_out(s.dk, a.in_bf16, o, von ? dk : 0.f);
            if (s.derase) s.derase[o] = von ? k * deh : 0.f;
        }
    }
    // dalpha partials: for each start row lo of this group, Y(u, lo) for u > lo
    // by Horner over u descending, then dal[u] += L(lo, u) Y(u, lo) ascending.
    float dal[C];
#pragma unroll
    for (int x = 0; x < C; ++x) dal[x] = 0.f;
    for (int p = 0; p < np; ++p) {
        const int lo = 4 * rpw * p + rpw * w + sub - 1;  // -1 .. 14
        const float kl = lo >= 0 ? sm.k[lo * LQ + i] : 0.f;
        const float endc = (lo >= 0 && sm.m.seg[lo] == sg15) ? kl * sm.u.gr.gk[lo * LQ + i] : 0.f;
        float Y[C], y = 0.f;
#pragma unroll
        for (int x = C - 1; x >= 0; --x) {
            float cf = 0.f;
            if (x > lo) {
                if (lo >= 0) {
                    cf = (sm.dA[x * LT + lo] * re[x] + sm.dP[x * LT + lo] * rq[x]) * kl;
                    if (x == C - 1) cf += endc;
                } else {
                    cf = sg[x] == 0 ? re[x] * sm.u.gr.ga[x * LQ + i] + rq[x] * sm.u.gr.gq[x * LQ + i] : 0.f;
                    if (x == C - 1 && sg15 == 0) cf += sm.fs[i];
                }
            }
            y = x == C - 1 ? cf : cf + ra[x + 1] * y;
            Y[x] = y;
        }
        float L = 1.f;
#pragma unroll
        for (int x = 0; x < C; ++x)
            if (x > lo) {
                dal[x] += L * Y[x];
                L *= ra[x];
            }
    }
    // partials [group][u][channel] (4 rpw groups of C x cpl), then one sum per (u, channel)
    float *part = sm.u.gr.part + (w * rpw + sub) * (C * cpl);
#pragma unroll
    for (int x = 0; x < C; ++x) part[x * cpl + i] = dal[x];
    __syncthreads();
    for (int e = tid; e < C * cpl; e += NT) {
        const int u = e / cpl, ch = e - u * cpl;
        if (ch >= K) continue;
        float x = 0.f;
        for (int gq = 0; gq < 4 * rpw; ++gq) x += sm.u.gr.part[gq * (C * cpl) + e];
        const int tq = c * C + u;
        if (tq < s.T && s.dalpha)
            s.dalpha[(((int64_t)b * s.T + tq) * s.H + h) * K + ch] =
                (sm.m.val[u] != 0.f && !sm.m.rs[u]) ? x : 0.f;
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
