// Chunked channel-wise GDN-2 in f32 on gfx950: the reference's own op
// configuration (f32 q/k/v, d_k = 32, d_v = 64, 16-token chunks;
// crates/kernels/src/gdn2.rs:10-12, crates/kernels/src/gdn_training.rs:8-9), and
// every d_k, d_v <= 128.
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
// 16 x 128 x 128 at most), so the kernels run in f32 with LDS tiles: one
// 256-thread workgroup per chunk.  Each kernel is built for two tile widths FK:
// 64 (d_k, d_v <= 64) and 128 (either above 64).  Thread (token t = tid / 16,
// g = tid % 16) holds FK / 16 channels of the [token][channel] tiles: 4 g .. 4 g
// + 3 at FK = 64, g + 16 e at FK = 128 (adjacent lanes on adjacent banks).
#include "gdn2_chunk_f32.h"
#include "gdn2_mfma.h"

#include <algorithm>

namespace gdn2 {

namespace {

constexpr int C = FC_C;
constexpr int LT = C + 1;  // f32 row stride of 16 x 16 tiles
constexpr int VB = 64;     // value columns per S0 / dS block in bgrad
constexpr int LB = VB + 4; // f32 row stride of [key][value block] tiles

// Geometry of the FK-wide kernels: 4 FK threads per workgroup (256 or 512),
// LPT lanes per token row of the [token][channel] tiles, four channels each.
template <int FK>
struct Fc {
    static constexpr int NT = 4 * FK;
    static constexpr int NW = NT / 64;    // waves
    static constexpr int LPT = NT / C;    // lanes per token row: 16 or 32
    static constexpr int EPT = FK / LPT;  // channels per lane: 4
    static constexpr int LQ = FK + 4;     // f32 row stride of [token][channel] tiles
    static constexpr int LS = FK + 16;    // f32 row stride of [key][value] tiles: rows 16 banks apart
    // channel e of lane column g (adjacent lanes on adjacent banks at FK = 128)
    static __device__ __forceinline__ int ch(int g, int e) { return FK == 64 ? 4 * g + e : g + LPT * e; }
    // sum over the LPT lanes of a token row
    static __device__ __forceinline__ float row_sum(float x) {
#pragma unroll
        for (int m = 1; m < LPT; m <<= 1) x += __shfl_xor(x, m);
        return x;
    }
};

struct Masks {
    float val[C];
    int rs[C];   // a valid reset
    int seg[C];  // valid resets at or before the token
};

// Token masks (valid / reset, or the document limits) and segments (an
// inclusive prefix sum of the valid resets over the chunk's 16 tokens, by lane
// shuffles in wave 0).  Ends with a barrier.
__device__ void fc_masks(const SeqArgs &s, int b, int c, Masks &m, int tid) {
    if (tid < 64) {
        const int tg = c * C + tid;
        float vld = 0.f, rst = 0.f;
        if (tid < C && tg < s.T) {
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
        const int r = (vld != 0.f && rst != 0.f) ? 1 : 0;
        int sg = r;
#pragma unroll
        for (int d = 1; d < C; d <<= 1) {
            const int y = __shfl_up(sg, d);
            if (tid >= d) sg += y;
        }
        if (tid < C) {
            m.val[tid] = vld != 0.f ? 1.f : 0.f;
            m.rs[tid] = r;
            m.seg[tid] = sg;
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
// zero on the channels K .. FK - 1, which the MFMA products read as padding.
// The channel's 16 gates are read first, so that the reads issue together
// instead of one LDS round trip per step.
template <int FK, int LQ = Fc<FK>::LQ, int FW = FK>
__device__ void fc_decay_rows(const float *al, const Masks &m, float *bt, float *lam, int K, int tid) {
    if (tid >= K && tid < FW)
#pragma unroll
        for (int t = 0; t < C; ++t) bt[t * LQ + tid] = lam[t * LQ + tid] = 0.f;
    if (tid < K) {
        const int i = tid, sg15 = m.seg[C - 1];
        float a[C];
#pragma unroll
        for (int t = 0; t < C; ++t) a[t] = al[t * LQ + i];
        float p = 1.f;
#pragma unroll
        for (int t = 0; t < C; ++t) {
            p *= a[t];
            bt[t * LQ + i] = m.seg[t] == 0 ? p : 0.f;
        }
        float q = 1.f;
#pragma unroll
        for (int s = C - 1; s >= 0; --s) {
            lam[s * LQ + i] = m.seg[s] == sg15 ? q : 0.f;
            q *= a[s];
        }
    }
}

// b_t alone (threads i < K; zero on the channels K .. FK - 1).
template <int FK, int LQ = Fc<FK>::LQ, int FW = FK>
__device__ void fc_b_row(const float *al, const Masks &m, float *bt, int K, int tid) {
    if (tid >= K && tid < FW)
#pragma unroll
        for (int t = 0; t < C; ++t) bt[t * LQ + tid] = 0.f;
    if (tid < K) {
        float a[C];
#pragma unroll
        for (int t = 0; t < C; ++t) a[t] = al[t * LQ + tid];
        float p = 1.f;
#pragma unroll
        for (int t = 0; t < C; ++t) {
            p *= a[t];
            bt[t * LQ + tid] = m.seg[t] == 0 ? p : 0.f;
        }
    }
}

// out[t][s] = sum_i x[t][i] D_ts[i] y[s][i] for s < t (STRICT) or s <= t in the
// same segment, zero elsewhere (the diagonal too when STRICT).  Thread
// (t = tid / LPT, g = tid % LPT) takes its four channels of row t, forming
// D_ts for s = t, t - 1, .. by a running product; the LPT partial rows of one
// t (adjacent lanes) are summed by lane shuffles.  All threads call it.
template <int FK, bool STRICT, int LQ = Fc<FK>::LQ>
__device__ __forceinline__ void fc_tri(const float *x, const float *y, const float *al, const Masks &m,
                                       float *out, int K, int tid) {
    const int t = tid / Fc<FK>::LPT, g = tid % Fc<FK>::LPT;
    float acc[C];
#pragma unroll
    for (int s = 0; s < C; ++s) acc[s] = 0.f;
    // Per channel, its y and gate columns are read whole before the running
    // product (the reads issue together instead of one LDS round trip per
    // step; the terms past t are selected away, t differing between the lane
    // groups of a wave).  One channel at a time keeps the registers down.
#pragma unroll 1
    for (int e = 0; e < Fc<FK>::EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        const bool iv = i < K;
        const int ic = iv ? i : 0;  // channels past K read channel 0, unused
        const float xt = x[t * LQ + ic];
        float yv[C], av[C];
#pragma unroll
        for (int s = 0; s < C; ++s) {
            yv[s] = y[s * LQ + ic];
            av[s] = al[s * LQ + ic];
        }
        float d = 1.f;
#pragma unroll
        for (int s = C - 1; s >= 0; --s) {
            const bool in = iv && s <= t;
            acc[s] += in ? xt * d * yv[s] : 0.f;
            d = in ? d * av[s] : d;
        }
    }
    float r = 0.f;
#pragma unroll
    for (int s = 0; s < C; ++s) {
        const float a = Fc<FK>::row_sum(acc[s]);
        if (s == g) r = a;
    }
    if (g < C) {
        const bool keep = (STRICT ? g < t : g <= t) && m.seg[g] == m.seg[t];
        out[t * LT + g] = keep ? r : 0.f;
    }
}

// Stage value tiles vt0 .. vt0 + NVT - 1 of the tile-packed arrays src0 (and
// src1) (element (((vt * KT + tau) * 4 + g) * 16 + n) * 4 + r at row
// 16 tau + 4 g + r, column 16 vt + n) into rows 0 .. 16 KT - 1 and columns
// 0 .. 16 NVT - 1 of dst0 (dst1), row stride dld; zero where row >= rv, column
// >= cv or vt >= VT.  One 16-byte load per lane and tile; each thread issues U
// loads per source before it stores any.
template <int NT, int NVT, int U>
__device__ __forceinline__ void fc_stage_tiles(float *dst0, float *dst1, int dld, const float *src0,
                                               const float *src1, int KT, int VT, int vt0, int rv, int cv,
                                               int tid) {
    const int n = NVT * KT * 64;
    for (int e0 = tid; e0 < n; e0 += U * NT) {
        float4 x0[U], x1[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * NT, vt = vt0 + e / (KT * 64), o = e % (KT * 64);
            const bool in = e < n && vt < VT;
            const int64_t off = ((int64_t)vt * KT * 64 + o) * 4;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            x0[u] = in ? *reinterpret_cast<const float4 *>(src0 + off) : z;
            x1[u] = (in && src1) ? *reinterpret_cast<const float4 *>(src1 + off) : z;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * NT, vl = e / (KT * 64), o = e % (KT * 64);
            const int l = o & 63, i = 16 * (o >> 6) + 4 * (l >> 4), jl = 16 * vl + (l & 15);
            if (e < n) {
                const bool cj = 16 * vt0 + jl < cv;
                const float a0[4] = {x0[u].x, x0[u].y, x0[u].z, x0[u].w};
                const float a1[4] = {x1[u].x, x1[u].y, x1[u].z, x1[u].w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool ok = cj && i + r < rv;
                    dst0[(i + r) * dld + jl] = ok ? a0[r] : 0.f;
                    if (dst1) dst1[(i + r) * dld + jl] = ok ? a1[r] : 0.f;
                }
            }
        }
    }
}

template <int FK>
struct FcPrepSmem {
    static constexpr int LQ = Fc<FK>::LQ;
    Masks m;
    float k[C * LQ], al[C * LQ], eh[C * LQ], wv[C * LQ], bt[C * LQ], lam[C * LQ];
    float A[C * LT], T[C * LT];
};

// FKK: the key tiles' width (FK, or 32 when d_k <= 32, so that the tiles of
// the reference's K32/V64 shape fit four workgroups per CU).
template <int FK, int FKK>
struct FcOutSmem {
    static constexpr int LQ = Fc<FK>::LQ, LQK = FKK + 4;
    Masks m;
    float q[C * LQK], k[C * LQK], al[C * LQK], eh[C * LQK], bt[C * LQK];  // key side
    float wv[C * LQ];
    float s0[FKK * Fc<FK>::LS];  // S0, zero-padded to whole 16 x 16 tiles
    float T[C * LT], P[C * LT];
    float kk[C], ddp[FK / 16][C];
};

template <int FK>
struct FcBPrepSmem {
    static constexpr int LQ = Fc<FK>::LQ;
    Masks m;
    float q[C * LQ], k[C * LQ], al[C * LQ], bt[C * LQ], dO[C * LQ], dl[C * LQ], w[C * LQ];
    float P[C * LT];
    float cs[C];
};

// FKK: the key tiles' width (FK, or 32 when d_k <= 32: the reference's K32/V64
// shape then fits three workgroups per CU).
template <int FK, int FKK>
struct FcBGradSmem {
    static constexpr int LQ = Fc<FK>::LQ, LQK = FKK + 4;
    Masks m;
    float q[C * LQK], k[C * LQK], e[C * LQK], al[C * LQK], bt[C * LQK], lam[C * LQK];  // key side
    union {
        struct {
            float dO[C * LQ], dl[C * LQ], dr[C * LQ];  // value side, read until the products end
        } v;
        struct {
            float ga[C * LQK], gq[C * LQK], gk[C * LQK];  // then dAhat, dQhat, dKtil [token][key]
        } g;
    } w;
    union {
        struct {
            // one block of VB value columns of S0 and dS, zero outside K x V
            float s0[FKK * LB], ds[FKK * LB];
        } st;
        float part[Fc<FK>::NT * C];  // then dalpha partials: NT / cpl groups x C rows x cpl channels
    } u;
    float T[C * LT], P[C * LT], dA[C * LT], dP[C * LT];
    float cs[C], ck[C], fs[FK];
    static_assert(sizeof(u.st) >= sizeof(u.part), "the partials fit the S0 / dS block");
};

}  // namespace

// ---- prep: gates, A, T and the factored map of every chunk ---------------------
template <int FK>
__global__ void __launch_bounds__(Fc<FK>::NT) fc_prep_kernel(FcArgs a) {
    __shared__ FcPrepSmem<FK> sm;
    constexpr int LQ = Fc<FK>::LQ, NW = Fc<FK>::NW;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid / Fc<FK>::LPT, g = tid % Fc<FK>::LPT, tg = c * C + t;
    // The token rows are loaded before the masks arrive and masked after.
    constexpr int EPT = Fc<FK>::EPT;
    float rk[EPT], ral[EPT], re[EPT], rw[EPT], rv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        rk[e] = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, true);
        ral[e] = (i < K && tg < s.T) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        re[e] = fc_in(s.erase, b, tg, h, i, s.T, K, true);
        rw[e] = fc_in(s.write, b, tg, h, i, s.T, V, true);
        rv[e] = fc_x(s.v, a.in_bf16, b, tg, h, i, s.T, V, true);
    }
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        const float kv = on ? rk[e] : 0.f;
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = on ? ral[e] : 1.f;
        sm.eh[t * LQ + i] = (on ? re[e] : 0.f) * kv;
        sm.wv[t * LQ + i] = on ? rw[e] * rv[e] : 0.f;
    }
    __syncthreads();
    fc_decay_rows<FK>(sm.al, sm.m, sm.bt, sm.lam, K, tid);
    fc_tri<FK, true>(sm.eh, sm.k, sm.al, sm.m, sm.A, K, tid);  // A, strictly lower
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
    // Ktil = lam . k (token t, the thread's channels) and gv = b_15; zero on the
    // key padding up to KP.
    const int KP = fc_kp(K), KT = KP >> 4, VT = (V + 15) >> 4;
    const int64_t fo = (int64_t)ci * C;
#pragma unroll
    for (int e = 0; e < Fc<FK>::EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        if (i < KP) a.fk[(fo + t) * KP + i] = i < K ? sm.lam[t * LQ + i] * sm.k[t * LQ + i] : 0.f;
    }
    if (tid < KP) a.gv[(int64_t)ci * KP + tid] = tid < K ? sm.bt[(C - 1) * LQ + tid] : 0.f;
    if (tid < C * C) a.tm[(int64_t)ci * C * C + tid] = sm.T[(tid >> 4) * LT + (tid & 15)];
    // W' = T (b . ehat) and U = T wv on v_mfma_f32_16x16x4f32: tiles 0 .. KT - 1
    // of W' (key tiles), then VT tiles of U, taken by the waves in turn (lane
    // (lg, ln): tokens 4 lg + r, column 16 tile + ln).
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    for (int n = w; n < KT + VT; n += NW) {
        const bool isw = n < KT;
        const int col = 16 * (isw ? n : n - KT) + ln;
        f32x4 x = zero4();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ss = 4 * lg + q;
            const float bv = isw ? sm.bt[ss * LQ + col] * sm.eh[ss * LQ + col] : sm.wv[ss * LQ + col];
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[ln * LT + ss], bv, x, 0, 0, 0);
        }
        if (isw) {
#pragma unroll
            for (int r = 0; r < 4; ++r) a.fw[(fo + 4 * lg + r) * KP + col] = x[r];
        } else {  // lane-packed for the scan (zero past V: wv is)
            *reinterpret_cast<float4 *>(&a.fu[(((int64_t)ci * VT + n - KT) * 64 + l) * 4]) =
                make_float4(x[0], x[1], x[2], x[3]);
        }
    }
}

// ---- the scan over the chunks of one (batch, head) -----------------------------
// One workgroup per (batch, head, 16 value columns j = 16 cg + l % 16), one wave
// per 16-row key tile tau = w, on v_mfma_f32_16x16x4f32 (exact f32 products).
// Wave tau holds its tile of the state in the accumulator layout: lane l
// (g = l / 16, n = l % 16) holds S[16 tau + 4 g + r][j] in register r.
// Per chunk, forward:  v = U - W' S,          S <- diag(gv) S + Ktil^T v
//            reverse:  v = Ktil X,            X <- diag(gv) X + N - W'^T v
// v sums over the key axis: each wave forms its tile's part (four k = 4 MFMA
// steps whose k-slice {4 g + s} makes register s of the lane's own accumulator
// the B operand), the parts meet in LDS (double-buffered by step parity, one
// barrier per step) and every wave adds them in tile order, so all waves hold
// the same v; each then updates its own tile, v's accumulator rows as the B
// operand.  The A operands (W' or Ktil rows, gv, the lane-packed U or N) are
// read from global memory into registers D chunks ahead.
template <int KT>
struct FcScanOps {
    float4 w, g, a;  // A operands (token n, keys 16 tau + 4 g ..), gv rows, U or N rows
    float k[4];      // A operands (tokens 4 g + s, key 16 tau + n)
};

template <int KT, bool REV>
__device__ __forceinline__ void fc_scan_load(const FcArgs &a, int64_t ci, int cg, int VT, int tau,
                                             FcScanOps<KT> &o) {
    // Every load is issued (past the value tiles the lanes read tile 0, their
    // values unused), so no load sits behind a branch and the compiler's
    // memory-counter waits stay exact across the prefetch ring.
    constexpr int KP = 16 * KT;
    const int l = lane_id(), g = l >> 4, n = l & 15, cc = cg < VT ? cg : 0;
    const float *fw = a.fw + ci * C * KP, *fk = a.fk + ci * C * KP;
    const float *rw = REV ? fk : fw, *ck = REV ? fw : fk;
    o.w = *reinterpret_cast<const float4 *>(&rw[n * KP + 16 * tau + 4 * g]);
    o.g = *reinterpret_cast<const float4 *>(&a.gv[ci * KP + 16 * tau + 4 * g]);
#pragma unroll
    for (int s = 0; s < 4; ++s) o.k[s] = ck[(4 * g + s) * KP + 16 * tau + n];
    o.a = REV ? *reinterpret_cast<const float4 *>(&a.n[(((ci * VT + cc) * KT + tau) * 64 + l) * 4])
              : *reinterpret_cast<const float4 *>(&a.fu[((ci * VT + cc) * 64 + l) * 4]);
}

template <int KT, bool REV>
__global__ void __launch_bounds__(64 * KT) fc_scan_kernel(FcArgs a) {
    __shared__ float4 vpart[2][KT][64];  // each wave's part of v, by step parity
    const SeqArgs &s = a.s;
    const int K = s.K, V = s.V, VT = (V + 15) / 16;
    const int tau = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg = blockIdx.x, bh = wg / VT, cg = wg % VT, b = bh / s.H, h = bh % s.H;
    const int l = lane_id(), g = l >> 4, n = l & 15, j = 16 * cg + n;
    const bool jv = j < V;
    f32x4 X;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = 16 * tau + 4 * g + r;
        float x = 0.f;
        if (i < K && jv) {
            if (!REV) x = s.initial.data ? ld4<float>(s.initial, b, h, i, j) : 0.f;
            else x = s.dfinal ? s.dfinal[((int64_t)bh * K + i) * V + j] : 0.f;
        }
        X[r] = x;
    }
    // A ring of D chunks' operands in registers: chunk step + D is loaded (the
    // last chunk again past the end) as soon as step's operands are used.
    constexpr int D = 4;
    FcScanOps<KT> ring[D];
    auto chunk_at = [&](int step) {
        const int sc = step < a.nc ? step : a.nc - 1;
        return (int64_t)bh * a.nc + (REV ? a.nc - 1 - sc : sc);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) fc_scan_load<KT, REV>(a, chunk_at(d), cg, VT, tau, ring[d]);
    float *keep = REV ? a.ds : a.st;
    for (int s0 = 0; s0 < a.nc; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int step = s0 + d;
            if (step >= a.nc) break;
            const int64_t ci = chunk_at(step);
            const FcScanOps<KT> &cur = ring[d];
            // the state before (forward) / the adjoint after (reverse) this chunk
            {
                float kx[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) kx[r] = (16 * tau + 4 * g + r < K && jv) ? X[r] : 0.f;
                *reinterpret_cast<float4 *>(&keep[(((ci * VT + cg) * KT + tau) * 64 + l) * 4]) =
                    make_float4(kx[0], kx[1], kx[2], kx[3]);
            }
            // this tile's part of v[t][j], t = 4 g + r: -W' S (+ U in tile 0) or Ktil X
            f32x4 vp = (!REV && tau == 0) ? f32x4{cur.a.x, cur.a.y, cur.a.z, cur.a.w} : zero4();
            const float wq[4] = {cur.w.x, cur.w.y, cur.w.z, cur.w.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                vp = __builtin_amdgcn_mfma_f32_16x16x4f32(REV ? wq[q] : -wq[q], X[q], vp, 0, 0, 0);
            f32x4 v = vp;
            if (KT > 1) {
                const int par = step & 1;
                vpart[par][tau][l] = make_float4(vp[0], vp[1], vp[2], vp[3]);
                __syncthreads();
                float4 t0 = vpart[par][0][l];
                v = f32x4{t0.x, t0.y, t0.z, t0.w};
#pragma unroll
                for (int u = 1; u < KT; ++u) {
                    const float4 t = vpart[par][u][l];
                    v += f32x4{t.x, t.y, t.z, t.w};
                }
            }
            // S <- diag(gv) S + Ktil^T v, or X <- diag(gv) X + N - W'^T v
            const float gq[4] = {cur.g.x, cur.g.y, cur.g.z, cur.g.w};
            const float an[4] = {cur.a.x, cur.a.y, cur.a.z, cur.a.w};
            f32x4 x;
#pragma unroll
            for (int r = 0; r < 4; ++r) x[r] = gq[r] * X[r] + (REV ? an[r] : 0.f);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                x = __builtin_amdgcn_mfma_f32_16x16x4f32(REV ? -cur.k[q] : cur.k[q], v[q], x, 0, 0, 0);
            X = x;
            fc_scan_load<KT, REV>(a, chunk_at(step + D), cg, VT, tau, ring[d]);
        }
    }
    float *fin = REV ? s.dinitial : s.final_state;
    if (fin)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * tau + 4 * g + r;
            if (i < K && jv) fin[((int64_t)bh * K + i) * V + j] = X[r];
        }
}

template <bool REV>
static void launch_fc_scan(const FcArgs &a, hipStream_t stream) {
    const int KT = fc_kp(a.s.K) / 16;
    const dim3 grid(a.s.B * a.s.H * ((a.s.V + 15) / 16)), block(64 * KT);
    switch (KT) {
        case 1: hipLaunchKernelGGL((fc_scan_kernel<1, REV>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((fc_scan_kernel<2, REV>), grid, block, 0, stream, a); break;
        case 3: hipLaunchKernelGGL((fc_scan_kernel<3, REV>), grid, block, 0, stream, a); break;
        case 4: hipLaunchKernelGGL((fc_scan_kernel<4, REV>), grid, block, 0, stream, a); break;
        case 5: hipLaunchKernelGGL((fc_scan_kernel<5, REV>), grid, block, 0, stream, a); break;
        case 6: hipLaunchKernelGGL((fc_scan_kernel<6, REV>), grid, block, 0, stream, a); break;
        case 7: hipLaunchKernelGGL((fc_scan_kernel<7, REV>), grid, block, 0, stream, a); break;
        default: hipLaunchKernelGGL((fc_scan_kernel<8, REV>), grid, block, 0, stream, a); break;
    }
}

// ---- out: edits, outputs, scores ----------------------------------------------
template <int FK, int FKK>
__global__ void __launch_bounds__(Fc<FK>::NT) fc_out_kernel(FcArgs a) {
    __shared__ FcOutSmem<FK, FKK> sm;
    constexpr int LQ = Fc<FK>::LQ, LQK = FcOutSmem<FK, FKK>::LQK, LS = Fc<FK>::LS, NT = Fc<FK>::NT,
                  NW = Fc<FK>::NW;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid / Fc<FK>::LPT, g = tid % Fc<FK>::LPT, tg = c * C + t;
    const int KP = fc_kp(K), VT = (V + 15) >> 4, VP = 16 * VT;
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    // The token rows, S0 and T are loaded before the masks arrive; the rows are
    // masked after.
    constexpr int EPT = Fc<FK>::EPT;
    float rk[EPT], rq[EPT], ral[EPT], re[EPT], rw[EPT], rv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        rk[e] = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, true);
        rq[e] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, true);
        ral[e] = (i < K && tg < s.T) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        re[e] = fc_in(s.erase, b, tg, h, i, s.T, K, true);
        rw[e] = fc_in(s.write, b, tg, h, i, s.T, V, true);
        rv[e] = fc_x(s.v, a.in_bf16, b, tg, h, i, s.T, V, true);
    }
    // S0 rows 0 .. KP - 1, all FK columns (zero outside K x V)
    fc_stage_tiles<NT, FK / 16, FK / 32>(sm.s0, nullptr, LS, a.st + (int64_t)ci * KP * VP, nullptr, KP / 16, VT, 0,
                                         K, V, tid);
    if (tid < C * C) sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    float ksq = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        const float kv = on ? rk[e] : 0.f;
        if (i < FKK) {
            sm.q[t * LQK + i] = on ? rq[e] : 0.f;
            sm.k[t * LQK + i] = kv;
            sm.al[t * LQK + i] = on ? ral[e] : 1.f;
            sm.eh[t * LQK + i] = (on ? re[e] : 0.f) * kv;
        }
        sm.wv[t * LQ + i] = on ? rw[e] * rv[e] : 0.f;
        ksq += kv * kv;
    }
    ksq = Fc<FK>::row_sum(ksq);
    if (g == 0) sm.kk[t] = ksq;
    __syncthreads();
    fc_b_row<FK, LQK, FKK>(sm.al, sm.m, sm.bt, K, tid);
    fc_tri<FK, false, LQK>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);  // P, lower with the diagonal
    __syncthreads();
    // Wave w: value tiles w, w + NW, .. on v_mfma_f32_16x16x4f32 (lane (lg, ln):
    // rows 4 lg + r, column 16 vt + ln).  R = wv - Ahat S0, O = Qhat S0 over the
    // key axis; then delta = T R and O += P delta with the accumulator rows as the
    // B operand (step q reduces over the tokens 4 lg + q).
    for (int vt = w; vt < VT; vt += NW) {
        const int j = 16 * vt + ln;
        f32x4 x = zero4(), o = zero4();
        for (int kk = 0; kk < KP; kk += 4) {
            const int i = kk + lg;
            const float sv = sm.s0[i * LS + j], bti = sm.bt[ln * LQK + i];
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(bti * sm.eh[ln * LQK + i], sv, x, 0, 0, 0);
            o = __builtin_amdgcn_mfma_f32_16x16x4f32(bti * sm.q[ln * LQK + i], sv, o, 0, 0, 0);
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
            if (ln == 0) sm.ddp[vt][tt] = p;
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
template <int FK>
__global__ void __launch_bounds__(Fc<FK>::NT) fc_bprep_kernel(FcArgs a) {
    __shared__ FcBPrepSmem<FK> sm;
    constexpr int LQ = Fc<FK>::LQ, NW = Fc<FK>::NW;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid / Fc<FK>::LPT, g = tid % Fc<FK>::LPT, tg = c * C + t;
    // The token rows are loaded before the masks arrive and masked after.
    constexpr int EPT = Fc<FK>::EPT;
    float rk[EPT], rq[EPT], ral[EPT], rdo[EPT], rdl[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        rk[e] = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, true);
        rq[e] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, true);
        ral[e] = (i < K && tg < s.T) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        rdo[e] = (s.dout.data && tg < s.T && i < V) ? fc_ld(s.dout, a.in_bf16, b, tg, h, i) : 0.f;
        rdl[e] = i < V ? a.dl[((int64_t)ci * C + t) * V + i] : 0.f;
    }
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    const bool score_adj = s.dscores != nullptr;
    float ksq = 0.f, dsq = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        const float kv = on ? rk[e] : 0.f;
        sm.q[t * LQ + i] = on ? rq[e] : 0.f;
        sm.k[t * LQ + i] = kv;
        sm.al[t * LQ + i] = on ? ral[e] : 1.f;
        sm.dO[t * LQ + i] = on ? rdo[e] : 0.f;
        const float d = rdl[e];
        sm.dl[t * LQ + i] = d;
        ksq += kv * kv;
        dsq += d * d;
    }
    ksq = Fc<FK>::row_sum(ksq);
    dsq = Fc<FK>::row_sum(dsq);
    if (g == 0) {
        const float nk = sqrtf(ksq), nd = sqrtf(dsq);
        const float dsc = (score_adj && tg < s.T) ? s.dscores[((int64_t)b * s.T + tg) * s.H + h] : 0.f;
        sm.cs[t] = (on && nk > 0.f && nd > 0.f) ? dsc * nk / nd : 0.f;
    }
    __syncthreads();
    fc_b_row<FK>(sm.al, sm.m, sm.bt, K, tid);
    fc_tri<FK, false>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);  // P, lower with the diagonal
    // W' rows of this chunk
#pragma unroll
    for (int e = 0; e < Fc<FK>::EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        sm.w[t * LQ + i] = i < K ? a.fw[((int64_t)ci * C + t) * fc_kp(K) + i] : 0.f;
    }
    __syncthreads();
    // Wave w: value tiles w, w + NW, .. on v_mfma_f32_16x16x4f32 (lane (lg, ln):
    // rows 4 lg + r, column 16 vt + ln).  X = P^T dO + c delta, then per key tile
    // tau N = Qhat^T dO - W'^T X, X's accumulator rows as the B operand.
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15, VT = (V + 15) >> 4, KT = fc_kp(K) >> 4;
    for (int vt = w; vt < VT; vt += NW) {
        const int j = 16 * vt + ln;
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
            // lane-packed for the scan; zero outside K x V, where the tiles are
            *reinterpret_cast<float4 *>(&a.n[((((int64_t)ci * VT + vt) * KT + tau) * 64 + l) * 4]) =
                make_float4(n[0], n[1], n[2], n[3]);
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
template <int FK, int FKK>
__global__ void __launch_bounds__(Fc<FK>::NT) fc_bgrad_kernel(FcArgs a) {
    __shared__ FcBGradSmem<FK, FKK> sm;
    constexpr int LQ = Fc<FK>::LQ, LQK = FcBGradSmem<FK, FKK>::LQK, NT = Fc<FK>::NT, NW = Fc<FK>::NW;
    const SeqArgs &s = a.s;
    const int tid = threadIdx.x, ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / s.H, h = bh % s.H;
    const int K = s.K, V = s.V, t = tid / Fc<FK>::LPT, g = tid % Fc<FK>::LPT, tg = c * C + t;
    const int KT = (K + 15) >> 4, VT = (V + 15) >> 4, VP = 16 * VT, KP = 16 * KT;
    const int w = tid >> 6, l = tid & 63, lg = l >> 4, ln = l & 15;
    // The token rows and T are loaded before the masks arrive; the rows are
    // masked after.
    constexpr int EPT = Fc<FK>::EPT;
    float xk[EPT], xq[EPT], xe[EPT], xal[EPT], xdo[EPT], xdl[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        xk[e] = fc_x(s.k, a.in_bf16, b, tg, h, i, s.T, K, true);
        xq[e] = fc_x(s.q, a.in_bf16, b, tg, h, i, s.T, K, true);
        xe[e] = fc_in(s.erase, b, tg, h, i, s.T, K, true);
        xal[e] = (i < K && tg < s.T) ? ld4<float>(s.alpha, b, tg, h, i) : 1.f;
        xdo[e] = (s.dout.data && tg < s.T && i < V) ? fc_ld(s.dout, a.in_bf16, b, tg, h, i) : 0.f;
        xdl[e] = i < V ? a.dl[((int64_t)ci * C + t) * V + i] : 0.f;
    }
    if (tid < C * C) sm.T[(tid >> 4) * LT + (tid & 15)] = a.tm[(int64_t)ci * C * C + tid];
    fc_masks(s, b, c, sm.m, tid);
    const bool on = sm.m.val[t] != 0.f;
    const bool score_adj = s.dscores != nullptr;
    float ksq = 0.f, dsq = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = Fc<FK>::ch(g, e);
        const float kv = on ? xk[e] : 0.f;
        if (i < FKK) {
            sm.q[t * LQK + i] = on ? xq[e] : 0.f;
            sm.k[t * LQK + i] = kv;
            sm.e[t * LQK + i] = on ? xe[e] : 0.f;
            sm.al[t * LQK + i] = on ? xal[e] : 1.f;
        }
        sm.w.v.dO[t * LQ + i] = on ? xdo[e] : 0.f;
        const float d = xdl[e];
        sm.w.v.dl[t * LQ + i] = d;
        ksq += kv * kv;
        dsq += d * d;
    }
    ksq = Fc<FK>::row_sum(ksq);
    dsq = Fc<FK>::row_sum(dsq);
    if (g == 0) {
        const float nk = sqrtf(ksq), nd = sqrtf(dsq);
        const float dsc = (score_adj && tg < s.T) ? s.dscores[((int64_t)b * s.T + tg) * s.H + h] : 0.f;
        const bool ok = on && nk > 0.f && nd > 0.f;
        sm.cs[t] = ok ? dsc * nk / nd : 0.f;
        sm.ck[t] = ok ? dsc * nd / nk : 0.f;
    }
    __syncthreads();
    fc_decay_rows<FK, LQK, FKK>(sm.al, sm.m, sm.bt, sm.lam, K, tid);
    fc_tri<FK, false, LQK>(sm.q, sm.k, sm.al, sm.m, sm.P, K, tid);
    // The value axis in blocks of VB columns (one block at FK = 64, two at FK =
    // 128), each with its columns of S0 and dS in LDS.  Per block: ddelta and dR
    // of its value tiles, then the 16 x 16 products that reduce over the value
    // axis take the block's part: tiles 0 .. 3 KT - 1 are dAhat, dQhat, dKtil of
    // key tile tau = n / 3; tile 3 KT is dA, 3 KT + 1 is dP (wave w takes tiles
    // w, w + NW, ..).
    constexpr int MT = (3 * (FK / 16) + 2 + NW - 1) / NW;
    const int ntile = 3 * KT + 2;
    f32x4 res[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) res[m] = zero4();
    const float *st = a.st + (int64_t)ci * KP * VP, *dst = a.ds + (int64_t)ci * KP * VP;
    for (int j0 = 0; j0 < VP; j0 += VB) {
        if (j0 > 0) __syncthreads();  // the previous block's products have read S0 and dS
        fc_stage_tiles<NT, VB / 16, 2>(sm.u.st.s0, sm.u.st.ds, LB, st, dst, KT, VT, j0 / 16, K, V, tid);
        __syncthreads();
        {  // rowsum(S0 . dS) of key channel i over the block: TPC threads per channel
            constexpr int TPC = NT / FK, CW = VB / TPC;
            const int i = tid / TPC, jq = CW * (tid % TPC);
            float f = 0.f;
            if (i < KP)  // rows past KP are not loaded
#pragma unroll
                for (int j = 0; j < CW; ++j) f += sm.u.st.s0[i * LB + jq + j] * sm.u.st.ds[i * LB + jq + j];
            f += __shfl_xor(f, 1);
            f += __shfl_xor(f, 2);
            static_assert(TPC == 4, "four threads per key channel");
            if (tid % TPC == 0) sm.fs[i] = (j0 > 0 ? sm.fs[i] : 0.f) + f;
        }
        // ddelta and dR of value tile vt = j0 / 16 + w, waves 0 .. 3 (lane (lg, ln):
        // rows 4 lg + r, column 16 vt + ln)
        const int vt = j0 / 16 + w;
        if (w < VB / 16 && vt < VT) {
            const int j = 16 * vt + ln, jl = j - j0;
            f32x4 dd;
#pragma unroll
            for (int r = 0; r < 4; ++r) dd[r] = sm.cs[4 * lg + r] * sm.w.v.dl[(4 * lg + r) * LQ + j];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dd = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.P[(4 * lg + q) * LT + ln], sm.w.v.dO[(4 * lg + q) * LQ + j],
                                                          dd, 0, 0, 0);
            for (int tau = 0; tau < KT; ++tau)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = 16 * tau + 4 * lg + q;
                    dd = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.lam[ln * LQK + i] * sm.k[ln * LQK + i],
                                                              sm.u.st.ds[i * LB + jl], dd, 0, 0, 0);
                }
            f32x4 dr = zero4();
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dr = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.T[(4 * lg + q) * LT + ln], dd[q], dr, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tt = 4 * lg + r, tq = c * C + tt;
                sm.w.v.dr[tt * LQ + j] = dr[r];
                if (j < V && tq < s.T) {
                    const bool von = sm.m.val[tt] != 0.f;
                    const int64_t o = (((int64_t)b * s.T + tq) * s.H + h) * V + j;
                    if (s.dwrite) s.dwrite[o] = von ? dr[r] * fc_ld(s.v, a.in_bf16, b, tq, h, j) : 0.f;
                    if (s.dv) store_out(s.dv, a.in_bf16, o, von ? dr[r] * ld4<float>(s.write, b, tq, h, j) : 0.f);
                }
            }
        }
        __syncthreads();  // the block's dR columns are in LDS
        const int je = VP - j0 < VB ? VP - j0 : VB;  // the block's columns inside the value tiles
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int n = w + NW * m;
            if (n >= ntile) continue;
            const int kind = n < 3 * KT ? n % 3 : 3 + (n - 3 * KT), tau = n < 3 * KT ? n / 3 : 0;
            // A: [token][value] rows; B: S0 or dS rows of key 16 tau + ln (block
            // columns), or delta rows (value columns) for dA and dP
            const float *xa = (kind == 0 || kind == 3 ? sm.w.v.dr : (kind == 2 ? sm.w.v.dl : sm.w.v.dO)) + ln * LQ + j0;
            const float *yy = kind >= 3 ? sm.w.v.dl + ln * LQ + j0
                                        : (kind == 2 ? sm.u.st.ds : sm.u.st.s0) + (16 * tau + ln) * LB;
            f32x4 acc = res[m];
            for (int kk = 0; kk < je; kk += 4)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kk + lg], yy[kk + lg], acc, 0, 0, 0);
            res[m] = acc;
        }
    }
    __syncthreads();  // dO, delta and dR are no longer read: their space takes dAhat, dQhat, dKtil
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int n = w + NW * m;
        if (n >= ntile) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tt = 4 * lg + r;
            if (n < 3 * KT) {
                const int kind = n % 3, i = 16 * (n / 3) + ln;
                float *dst = kind == 0 ? sm.w.g.ga : (kind == 1 ? sm.w.g.gq : sm.w.g.gk);
                dst[tt * LQK + i] = kind == 0 ? -res[m][r] : res[m][r];
            } else {
                const bool same = sm.m.seg[tt] == sm.m.seg[ln];
                if (n == 3 * KT) sm.dA[tt * LT + ln] = (ln < tt && same) ? -res[m][r] : 0.f;
                else sm.dP[tt * LT + ln] = (ln <= tt && same) ? res[m][r] : 0.f;
            }
        }
    }
    __syncthreads();
    // Per key channel: thread i of a group of cpl threads, ngr = NT / cpl groups
    // (at most C; threads of further groups idle here);
    // the thread keeps its channel's gates, k, q and ehat of the whole chunk in
    // registers.  Group gi takes the rows u = ngr p + gi (p < C / ngr): the token
    // rows of eA, qP, kAP and the outputs, then the start rows lo = u - 1 of the
    // alpha gradient's pairs, whose partial sums over lo meet in LDS.
    const int cpl = K <= 16 ? 16 : (K <= 32 ? 32 : (K <= 64 ? 64 : 128)), ngr = min(NT / cpl, C);
    const int i = tid % cpl, gi = tid / cpl, sg15 = sm.m.seg[C - 1], np = gi < ngr ? C / ngr : 0;
    const bool iv = i < K;
    float ra[C], rk[C], rq[C], re[C];
    int sg[C];
#pragma unroll
    for (int x = 0; x < C; ++x) {
        ra[x] = sm.al[x * LQK + i];
        rk[x] = sm.k[x * LQK + i];
        rq[x] = sm.q[x * LQK + i];
        re[x] = sm.e[x * LQK + i] * rk[x];
        sg[x] = sm.m.seg[x];
    }
    for (int p = 0; p < np; ++p) {
        const int u = ngr * p + gi, su = sm.m.seg[u];
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
            const float bt = sm.bt[u * LQK + i], lt = sm.lam[u * LQK + i];
            const float k = sm.k[u * LQK + i], ev = sm.e[u * LQK + i];
            const float dq = bt * sm.w.g.gq[u * LQK + i] + qP;
            const float deh = bt * sm.w.g.ga[u * LQK + i] + eA;
            const float dk = lt * sm.w.g.gk[u * LQK + i] + kAP + ev * deh + sm.ck[u] * k;
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
        const int lo = ngr * p + gi - 1;  // -1 .. 14
        const float kl = lo >= 0 ? sm.k[lo * LQK + i] : 0.f;
        const float endc = (lo >= 0 && sm.m.seg[lo] == sg15) ? kl * sm.w.g.gk[lo * LQK + i] : 0.f;
        float Y[C], y = 0.f;
#pragma unroll
        for (int x = C - 1; x >= 0; --x) {
            float cf = 0.f;
            if (x > lo) {
                if (lo >= 0) {
                    cf = (sm.dA[x * LT + lo] * re[x] + sm.dP[x * LT + lo] * rq[x]) * kl;
                    if (x == C - 1) cf += endc;
                } else {
                    cf = sg[x] == 0 ? re[x] * sm.w.g.ga[x * LQK + i] + rq[x] * sm.w.g.gq[x * LQK + i] : 0.f;
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
    // partials [group][u][channel] (ngr groups of C x cpl), then one sum per (u, channel)
    float *part = sm.u.part + gi * (C * cpl);
#pragma unroll
    for (int x = 0; x < C; ++x) part[x * cpl + i] = dal[x];
    __syncthreads();
    for (int e = tid; e < C * cpl; e += NT) {
        const int u = e / cpl, ch = e - u * cpl;
        if (ch >= K) continue;
        float x = 0.f;
        for (int gq = 0; gq < ngr; ++gq) x += sm.u.part[gq * (C * cpl) + e];
        const int tq = c * C + u;
        if (tq < s.T && s.dalpha)
            s.dalpha[(((int64_t)b * s.T + tq) * s.H + h) * K + ch] =
                (sm.m.val[u] != 0.f && !sm.m.rs[u]) ? x : 0.f;
    }
}

static inline void fmark(const hipEvent_t *ev, int i, hipStream_t stream) {
    if (ev) (void)hipEventRecord(ev[i], stream);
}

// FK = 128 when either width is above 64.
static bool fc_wide(const FcArgs &a) { return a.s.K > 64 || a.s.V > 64; }

template <int FK>
static void fc_fwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int n = a.s.B * a.s.H * a.nc;
    fmark(ev, 0, stream);
    hipLaunchKernelGGL(fc_prep_kernel<FK>, dim3(n), dim3(Fc<FK>::NT), 0, stream, a);
    fmark(ev, 1, stream);
    fmark(ev, 2, stream);
    launch_fc_scan<false>(a, stream);
    fmark(ev, 3, stream);
    fmark(ev, 4, stream);
    bool narrow = false;
    if constexpr (FK == 64) {
        narrow = a.s.K <= 32;
        if (narrow) hipLaunchKernelGGL((fc_out_kernel<64, 32>), dim3(n), dim3(Fc<64>::NT), 0, stream, a);
    }
    if (!narrow) hipLaunchKernelGGL((fc_out_kernel<FK, FK>), dim3(n), dim3(Fc<FK>::NT), 0, stream, a);
    fmark(ev, 5, stream);
}

template <int FK>
static void fc_bwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int n = a.s.B * a.s.H * a.nc;
    fmark(ev, 0, stream);
    hipLaunchKernelGGL(fc_bprep_kernel<FK>, dim3(n), dim3(Fc<FK>::NT), 0, stream, a);
    fmark(ev, 1, stream);
    fmark(ev, 2, stream);
    launch_fc_scan<true>(a, stream);
    fmark(ev, 3, stream);
    fmark(ev, 4, stream);
    bool narrow = false;
    if constexpr (FK == 64) {
        narrow = a.s.K <= 32;
        if (narrow) hipLaunchKernelGGL((fc_bgrad_kernel<64, 32>), dim3(n), dim3(Fc<64>::NT), 0, stream, a);
    }
    if (!narrow) hipLaunchKernelGGL((fc_bgrad_kernel<FK, FK>), dim3(n), dim3(Fc<FK>::NT), 0, stream, a);
    fmark(ev, 5, stream);
}

hipError_t launch_fc_fwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    if (fc_wide(a)) fc_fwd<128>(a, stream, ev);
    else fc_fwd<64>(a, stream, ev);
    return hipGetLastError();
}

hipError_t launch_fc_bwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    if (fc_wide(a)) fc_bwd<128>(a, stream, ev);
    else fc_bwd<64>(a, stream, ev);
    return hipGetLastError();
}

}  // namespace gdn2
