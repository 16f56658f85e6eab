// Chunk-WY channel-wise GDN-2 (the reference's GdnTrainingOps recurrence) on
// gfx950 MFMA, d_k = d_v = 64, bf16 q/k/v, f32 gates.
//
// Recurrence per valid token t (crates/mixers/src/reference.rs:68-111):
//   bar = diag(alpha_t) S;  delta_t = w_t.v_t - bar^T (e_t.k_t);
//   S_t = bar + k_t delta_t^T;  o_t = S_t^T q_t;  score_t = |k_t| |delta_t|.
// Per chunk of CC = 16 tokens (the reference's own chunk for this op,
// crates/kernels/src/gdn2.rs) with start state S0, per key channel i:
//   Lambda_t = sum_{u <= t} log alpha_u           (chunk-local, padding: 0)
//   D_ts     = exp(Lambda_t - Lambda_s), s <= t   (decay over tokens s+1..t, <= 1)
//   b_t = exp(Lambda_t) [segment 0],  lam_s = exp(Lambda_15 - Lambda_s) [last segment]
//   ehat = e.k,  Ahat = b.ehat,  Qhat = b.q,  Ktil = lam.k,  wv = w.v
//   A_ts = sum_i ehat_t D_ts k_s   (s < t, same segment),  T = (I + A)^-1
//   P_ts = sum_i q_t D_ts k_s      (s <= t, same segment)
//   R = wv - Ahat S0,  delta = T R,  O = Qhat S0 + P delta
//   S_16 = A_c S0 + B_c,  A_c = diag(b_15) - Ktil^T W',  W' = T Ahat,
//                          B_c = Ktil^T U,  U = T wv.
// Segments split the chunk at valid resets, as in gdn2_chunk.hip.  The decay
// factors are elementwise per channel, so A and P (16 x 16, one exponential
// per channel and token pair) are formed on the VALU; every product with the
// state (R, delta, O, W', U and, in the backward, every state-sized adjoint)
// runs on v_mfma_f32_16x16x32_bf16 with the 16-token reduction padded to 32 by
// zero rows or columns.  The chunk map is rank 16 beside its diagonal, so it
// leaves prep as its factors (-W'^T, Ktil, U^T, b_15: 8.25 KiB per chunk
// against 24 KiB for A_c and B_c) for the factored scan of gdn2_chunk_lr.hip
// over the T / 16 chunks.
//
// With document limits (the doc-limit op) a token is live when end >= start and
// resets the state when start == t; the backward is the exact VJP of that
// forward, whose adjoint never crosses a reset, as the reference's chunked
// kernels compute it (crates/kernels/src/gdn2.rs:24-65, :288-490).
//
// log alpha is floored at -80 (exp(-80) ~ 2e-35) in the decays: below that a
// decay is taken as exp(-80).  These kernels need alpha >= 0 on valid tokens:
// a negative alpha turns its chunk's log decay into NaN, which then reaches the
// outputs, the state and every gradient of the sequence (the token-sequential
// kernels take any alpha).  The alpha gradient does not go through the log:
// it sums each gradient pair's coefficient times the product of the other
// alphas of the pair's span (cw_bgrad phase 7), so alpha = 0 and small alphas
// get their exact gradient.
#include "gdn2_chunk_tile.h"

#include <algorithm>

namespace gdn2 {

namespace {

constexpr int CC = CW_C;           // tokens per chunk
constexpr int NW4 = 4, NT4 = 256;  // four waves per workgroup
constexpr float LOG_FLOOR = -80.f;
constexpr int LDL = 64;            // f32 row stride of [token][channel] tiles (a multiple of the bank count)
constexpr int LDW = 40;            // bf16 row stride of [channel][token] tiles (32 used)
constexpr int LDI = 17;            // f32 row stride of 16 x 16 tiles
constexpr int RT32 = 32 * LDB;     // [token][channel] bf16 tile with rows 16..31 zero
constexpr int RT16 = CC * LDB;     // [token][channel] bf16 tile, 16 rows
constexpr int CT64 = 64 * LDW;     // [channel][token] bf16 tile, columns 16..31 zero

__device__ __forceinline__ void zero_lds(uint16_t *p, int n, int tid) {
    for (int i = tid; i < n; i += NT4) p[i] = 0;
}

// Token t's channels [c0, c0 + 4) of a bf16 sequence (unit channel stride).
__device__ __forceinline__ void load4_bf16(const uint16_t *base, const int64_t *s, int b, int tg,
                                           int h, int c0, bool inb, float (&o)[4]) {
    uint2 r = make_uint2(0, 0);
    if (inb) r = *reinterpret_cast<const uint2 *>(base + (int64_t)b * s[0] + (int64_t)tg * s[1] +
                                                  (int64_t)h * s[2] + c0);
    o[0] = bf16_val((uint16_t)(r.x & 0xffff));
    o[1] = bf16_val((uint16_t)(r.x >> 16));
    o[2] = bf16_val((uint16_t)(r.y & 0xffff));
    o[3] = bf16_val((uint16_t)(r.y >> 16));
}

__device__ __forceinline__ void load4_f32(const View &v, int b, int tg, int h, int c0, bool inb,
                                          float fill, float (&o)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = inb ? ld4<float>(v, b, tg, h, c0 + e) : fill;
}

// Padding tokens read as fill (the loads themselves are unconditional, so
// they need not wait for the token's flags).
__device__ __forceinline__ void mask4(float (&x)[4], bool on, float fill) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = on ? x[e] : fill;
}

__device__ __forceinline__ void put4_bf16(uint16_t *p, const float (&x)[4]) {
    *reinterpret_cast<uint2 *>(p) = make_uint2(bf16_pack2(x[0], x[1]), bf16_pack2(x[2], x[3]));
}

// Four values as bf16 hi/lo pairs (x ~= hi + lo, ~16 mantissa bits over both).
__device__ __forceinline__ void put4_split(uint16_t *hi, uint16_t *lo, const float (&x)[4]) {
    uint16_t h[4], o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split_bf16(x[e], h[e], o[e]);
    *reinterpret_cast<uint2 *>(hi) =
        make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    *reinterpret_cast<uint2 *>(lo) =
        make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
}

// P^T (from the f32 P checkpoint, 16 x 16) into hi/lo LDS rows [s][t];
// thread (s = tid/16, t = tid%16).
__device__ __forceinline__ void load_pt_split(const float *ckp, uint16_t *ph, uint16_t *pl, int tid) {
    const int s = tid >> 4, t = tid & 15;
    uint16_t hi, lo;
    split_bf16(ckp[t * CC + s], hi, lo);
    ph[s * LDB + t] = hi;
    pl[s * LDB + t] = lo;
}

__device__ __forceinline__ void put4_f32(float *p, const float (&x)[4]) {
    *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
}

__device__ __forceinline__ void get4_f32(const float *p, float (&x)[4]) {
    const float4 v = *reinterpret_cast<const float4 *>(p);
    x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
}

// (I + A)^-1 of a strictly lower 16 x 16 A (f32, row stride lda) into T (row
// stride ldt) by forward substitution; one wave.  Lane (col = l/4, part = l%4)
// holds rows part, part + 4, part + 8, part + 12 of column col, and the four
// parts of a column (one DPP quad) split each row's dot product.
__device__ __forceinline__ void inv16(const float *A, int lda, float *T, int ldt) {
    const int l = lane_id(), col = l >> 2, part = l & 3;
    float Tq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < CC; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int s = part + 4 * m;
            if (s < r) acc += A[r * lda + s] * Tq[m];
        }
        acc += dpp<0xB1>(acc);  // lane ^ 1
        acc += dpp<0x4E>(acc);  // lane ^ 2
        if ((r & 3) == part) Tq[r >> 2] = (r == col ? 1.f : 0.f) - acc;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) T[(part + 4 * m) * ldt + col] = Tq[m];
}

// Token pair p (0 <= p < n) of a 16-token chunk: strictly lower pairs
// (t, s), s < t (n = 120) or lower pairs s <= t (n = 136).
__device__ __forceinline__ void pair_of(int p, bool strict, int &t, int &s) {
    // the largest r with r (r + 1) / 2 <= p, by the inverse triangular number
    const int q = p;
    int r = (int)((sqrtf(8.f * (float)q + 1.f) - 1.f) * 0.5f);
    // row r covers [r (r + 1) / 2, (r + 1)(r + 2) / 2): fix float rounding
    while ((r + 1) * (r + 2) / 2 <= q) ++r;
    while (r * (r + 1) / 2 > q) --r;
    const int off = q - r * (r + 1) / 2;
    if (strict) {  // pairs (r + 1, off), off <= r
        t = r + 1;
        s = off;
    } else {  // pairs (r, off), off <= r
        t = r;
        s = off;
    }
}

// Elementwise decay product of a token pair over 32 channels [32 half, +32):
// sum_i x_t[i] exp(L_t[i] - L_s[i]) y_s[i] (f32 tiles, row stride LDL).  Each
// lane walks its 32 channels from its own starting offset (lane mod 32).  With
// the row stride a multiple of the bank count, a word's bank is its channel
// alone, so the 32 lanes of a half-wave, whatever rows t and s their pairs
// have, read 32 distinct banks at every step (a stride of 68 put rows 4 banks
// apart and made lanes of different rows meet: 2.0 against 0.6-1.0 conflict
// cycles per LDS instruction in prep and out).
__device__ __forceinline__ float pair_dot32(const float *x, const float *y, const float *L, int t,
                                            int s, int half) {
    const int rot = lane_id() & 31;
    const float *xt = x + t * LDL + 32 * half, *lt = L + t * LDL + 32 * half;
    const float *ys = y + s * LDL + 32 * half, *ls = L + s * LDL + 32 * half;
    float acc = 0.f;
#pragma unroll 8
    for (int j = 0; j < 32; ++j) {
        const int i = (j + rot) & 31;
        acc += xt[i] * __expf(lt[i] - ls[i]) * ys[i];
    }
    return acc;
}

struct CwPrepSmem {
    float lam[CC * LDL];   // log alpha, then Lambda
    float eh[CC * LDL];    // e.k (f32)
    float kf[CC * LDL];    // k (bf16 values)
    uint16_t ah[RT32];     // Ahat rows hi (rows 16..31 zero)
    uint16_t wv[RT32];     // w.v rows hi (rows 16..31 zero)
    uint16_t ahl[RT32], wvl[RT32];  // lo parts
    uint16_t tb[RT16], tbl[RT16];   // T rows hi/lo (columns 16..31 zero)
    float af[CC * LDI], tf[CC * LDI];
    float val[CC];
    int rs[CC], seg[CC];
};

}  // namespace

// ---- prep: gates, A, T and the factored state map of every 16-token chunk ------
// The map S_16 = diag(b_15) S0 + Ktil^T (U - W' S0) leaves as its factors:
// -W'^T and Ktil (bf16), U^T and b_15 (f32), for the scan of gdn2_chunk_lr.hip.
// One chunk's inputs to prep, held in registers: the mask words (valid and reset,
// or the document limits: both are [B,T] views of 4-byte elements, so one pair
// of loads serves either) and k, v, alpha, erase, write.  Rows past the
// sequence end read the last row and are masked at the staging, so the loads
// take no branch.
struct CwPrepIn {
    uint32_t m1, m2;
    uint2 k, v;
    float al[4], er[4], wr[4];
};
__device__ __forceinline__ void cwprep_load(const ChunkArgs &a, int ci, int tid, CwPrepIn &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid >> 4, c0 = 4 * (tid & 15), tg = c * CC + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    const View &v1 = a.doc ? a.doc_start : a.valid, &v2 = a.doc ? a.doc_end : a.reset;
    x.m1 = reinterpret_cast<const uint32_t *>(v1.data)[b * v1.s0 + tr * v1.s1];
    x.m2 = reinterpret_cast<const uint32_t *>(v2.data)[b * v2.s0 + tr * v2.s1];
    x.k = *reinterpret_cast<const uint2 *>(row_ptr(a.k, a.ks, b, tr, h) + c0);
    x.v = *reinterpret_cast<const uint2 *>(row_ptr(a.v, a.vs, b, tr, h) + c0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x.al[e] = ld4<float>(a.alpha, b, tr, h, c0 + e);
        x.er[e] = ld4<float>(a.erase, b, tr, h, c0 + e);
        x.wr[e] = ld4<float>(a.write, b, tr, h, c0 + e);
    }
}

// What prep stores once the inverse is done, held until the next chunk's
// staging: T (f32, this thread's element), the gate block (threads < 16),
// Lambda (this thread's four), -W'^T (bf16) and U^T (f32) from the accumulators.
struct CwPrepOut {
    float tx, val, lam[4];
    int seg;
    f32x4 x, y;
};
__device__ __forceinline__ void cwprep_store(const ChunkArgs &a, int ci, int tid, int w, const CwPrepOut &o) {
    const int t = tid >> 4, c0 = 4 * (tid & 15);
    a.ck_tf[(int64_t)ci * CC * CC + tid] = o.tx;  // (r, s) = (tid / 16, tid % 16)
    if (tid < CC) {
        a.ck_cwg[ci].val[tid] = o.val;
        a.ck_cwg[ci].seg[tid] = o.seg;
    }
    put4_f32(a.ck_lam + (int64_t)ci * CC * 64 + t * 64 + c0, o.lam);
    const int64_t row = (int64_t)(16 * w + acc_col()) * CC + acc_row(0);
    const float nw[4] = {-o.x[0], -o.x[1], -o.x[2], -o.x[3]};
    uint16_t *wt = a.lr_wt + (int64_t)ci * 2 * 64 * CC + row;  // -W'^T hi, then lo
    put4_split(wt, wt + 64 * CC, nw);
    *reinterpret_cast<float4 *>(a.lr_u + (int64_t)ci * 64 * CC + row) = make_float4(o.y[0], o.y[1], o.y[2], o.y[3]);
}

// Workgroups walk chunks blockIdx.x, blockIdx.x + gridDim.x, ... (as many
// workgroups as fit the GPU at once): the next chunk's inputs are loaded into
// registers while the current one computes, and the stores after the inverse
// are issued after the next chunk's staging.
__global__ void __launch_bounds__(NT4) cw_prep_kernel(ChunkArgs a, int nchunks) {
    __shared__ CwPrepSmem sm;
    {  // zero padding (rows 16..31 of the token-row tiles, columns 16..31 of T), once
        const int tid = threadIdx.x;
        zero_lds(sm.ah + RT16, RT32 - RT16, tid);
        zero_lds(sm.wv + RT16, RT32 - RT16, tid);
        zero_lds(sm.ahl + RT16, RT32 - RT16, tid);
        zero_lds(sm.wvl + RT16, RT32 - RT16, tid);
        for (int i = tid; i < CC * 16; i += NT4) {
            sm.tb[(i >> 4) * LDB + 16 + (i & 15)] = 0;
            sm.tbl[(i >> 4) * LDB + 16 + (i & 15)] = 0;
        }
    }
    CwPrepIn in;
    cwprep_load(a, blockIdx.x, threadIdx.x, in);
    CwPrepOut po;
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the lane- and wave-dependent address arithmetic inside
    // the loop (hoisted, it would stay live across it).
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = ci % a.nc;
    const int t = tid >> 4, c0 = 4 * (tid & 15), tg = c * CC + t;
    const bool inb = tg < a.T;
    // The next chunk.  Past the end the loads need no branch either: every lane
    // addresses this chunk as thread 0 would, so each load instruction touches
    // a line or two that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    float vld, rst;
    if (a.doc) {
        const int st = (int)in.m1, en = (int)in.m2;
        vld = (inb && en >= st) ? 1.f : 0.f;
        rst = (inb && st == tg) ? 1.f : 0.f;
    } else {
        vld = inb ? __uint_as_float(in.m1) : 0.f;
        rst = inb ? __uint_as_float(in.m2) : 0.f;
    }
    const bool on = vld != 0.f;
    float kv[4], vv[4], al[4], er[4], wr[4];
    kv[0] = bf16_val((uint16_t)(in.k.x & 0xffff)), kv[1] = bf16_val((uint16_t)(in.k.x >> 16));
    kv[2] = bf16_val((uint16_t)(in.k.y & 0xffff)), kv[3] = bf16_val((uint16_t)(in.k.y >> 16));
    vv[0] = bf16_val((uint16_t)(in.v.x & 0xffff)), vv[1] = bf16_val((uint16_t)(in.v.x >> 16));
    vv[2] = bf16_val((uint16_t)(in.v.y & 0xffff)), vv[3] = bf16_val((uint16_t)(in.v.y >> 16));
#pragma unroll
    for (int e = 0; e < 4; ++e) al[e] = in.al[e], er[e] = in.er[e], wr[e] = in.wr[e];
    mask4(kv, on, 0.f), mask4(vv, on, 0.f), mask4(al, on, 1.f), mask4(er, on, 0.f), mask4(wr, on, 0.f);
    {
        float la[4], eh[4], wv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // a negative alpha is outside these kernels' log-domain decays: it
            // poisons the chunk (NaN), so the caller sees it instead of a wrong value
            la[e] = on ? (al[e] < 0.f ? __builtin_nanf("") : fmaxf(__logf(al[e]), LOG_FLOOR)) : 0.f;
            eh[e] = er[e] * kv[e];
            wv[e] = wr[e] * vv[e];
        }
        put4_f32(&sm.lam[t * LDL + c0], la);
        put4_f32(&sm.eh[t * LDL + c0], eh);
        put4_f32(&sm.kf[t * LDL + c0], kv);
        put4_split(&sm.wv[t * LDB + c0], &sm.wvl[t * LDB + c0], wv);
        if (c0 == 0) {
            sm.val[t] = on ? 1.f : 0.f;
            sm.rs[t] = (on && rst != 0.f) ? 1 : 0;
        }
    }
    if (ci != (int)blockIdx.x) cwprep_store(a, ci - gridDim.x, tid, w, po);  // the previous chunk's
    cwprep_load(a, cn, tn, in);
    __syncthreads();
    // Lambda: running sums over the chunk's tokens, one channel per thread;
    // segment index of every token.
    if (tid < 64) {
        float acc = 0.f;
#pragma unroll
        for (int tt = 0; tt < CC; ++tt) {
            acc += sm.lam[tt * LDL + tid];
            sm.lam[tt * LDL + tid] = acc;
        }
    } else if (tid == 64) {
        int s2 = 0;
#pragma unroll
        for (int tt = 0; tt < CC; ++tt) {
            s2 += sm.rs[tt];
            sm.seg[tt] = s2;
        }
    }
    __syncthreads();
    {  // Ahat rows; Ktil rows and b at the chunk end (the map's diagonal) out
        const int sgt = sm.seg[t], sg15 = sm.seg[CC - 1];
        float ah[4], kl[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float L = sm.lam[t * LDL + c0 + e], L15 = sm.lam[(CC - 1) * LDL + c0 + e];
            ah[e] = (sgt == 0 ? __expf(L) : 0.f) * sm.eh[t * LDL + c0 + e];
            kl[e] = (sgt == sg15 ? __expf(L15 - L) : 0.f) * kv[e];
        }
        put4_split(&sm.ah[t * LDB + c0], &sm.ahl[t * LDB + c0], ah);
        uint16_t *kt = a.lr_kt + ((int64_t)ci * 2 * CC + t) * 64 + c0;  // Ktil hi, then lo
        put4_split(kt, kt + CC * 64, kl);
        if (t == CC - 1) {
            float bc[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) bc[e] = sg15 == 0 ? __expf(sm.lam[(CC - 1) * LDL + c0 + e]) : 0.f;
            put4_f32(a.lr_gv + (int64_t)ci * 64 + c0, bc);
        }
    }
    {  // A (strictly lower, same segment): pair p on lanes 2p, 2p + 1 (channel halves)
        const int p = tid >> 1, half = tid & 1;
        int tt = 0, ss = 0;
        if (p < 120) pair_of(p, true, tt, ss);
        float acc = p < 120 ? pair_dot32(sm.eh, sm.kf, sm.lam, tt, ss, half) : 0.f;
        acc += dpp<0xB1>(acc);
        if (p < 120 && half == 0) sm.af[tt * LDI + ss] = sm.seg[tt] == sm.seg[ss] ? acc : 0.f;
    }
    __syncthreads();
    if (w == 0) inv16(sm.af, LDI, sm.tf, LDI);
    __syncthreads();
    {  // T (unit lower): hi/lo LDS operands; T, the gate block and Lambda kept for the stores
        const int r = tid >> 4, s2 = tid & 15;
        const float x = s2 <= r ? sm.tf[r * LDI + s2] : 0.f;
        uint16_t hi, lo;
        split_bf16(x, hi, lo);
        sm.tb[r * LDB + s2] = hi;
        sm.tbl[r * LDB + s2] = lo;
        po.tx = x;
        if (tid < CC) {
            po.val = sm.val[tid];
            po.seg = sm.seg[tid];
        }
        get4_f32(&sm.lam[t * LDL + c0], po.lam);
    }
    __syncthreads();
    // W' = T Ahat, U = T wv (wave w: channel tile w); products of hi/lo pairs keep
    // three terms (hi hi, hi lo, lo hi); -W'^T and U^T leave from the accumulators
    // after the next chunk's staging.
    {
        const bf16x8_t ta = frag(sm.tb, LDB, 0), tal = frag(sm.tbl, LDB, 0);
        const bf16x8_t ab = frag_tr(sm.ah, 0, 16 * w), abl = frag_tr(sm.ahl, 0, 16 * w);
        const bf16x8_t vb = frag_tr(sm.wv, 0, 16 * w), vbl = frag_tr(sm.wvl, 0, 16 * w);
        f32x4 x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, ab, zero4(), 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, abl, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tal, ab, x, 0, 0, 0);
        f32x4 y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, vb, zero4(), 0, 0, 0);
        y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, vbl, y, 0, 0, 0);
        y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tal, vb, y, 0, 0, 0);
        po.x = x;
        po.y = y;
    }
    __syncthreads();  // the next chunk's staging overwrites the tiles read above
    }
    {
        const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        cwprep_store(a, last, tid, w, po);
    }
}

// ---- out: outputs, edits and scores of every chunk ------------------------------
namespace {
struct CwOutSmem {
    float lam[CC * LDL];   // Lambda
    float qf[CC * LDL];    // q (bf16 values)
    float kf[CC * LDL];    // k
    float wvf[CC * LDL];   // w.v (f32)
    uint16_t qh[RT16], qhl[RT16];  // Qhat rows hi/lo;  O rows (bf16) over qh at the end
    uint16_t ah[RT16], ahl[RT16];  // Ahat rows hi/lo
    uint16_t st[64 * LDB], stl[64 * LDB];  // S0^T rows [v][k] hi/lo
    uint16_t tb[RT16], tbl[RT16];  // T rows hi/lo (columns 16..31 zero)
    uint16_t pr[RT16], prl[RT16];  // P rows hi/lo (columns 16..31 zero)
    uint16_t rt[CT64], rtl[CT64];  // R^T hi/lo
    uint16_t dt[CT64], dtl[CT64];  // delta^T hi/lo
    float dd[NW4][CC];
    float kk[CC];
    float val[CC];
    int seg[CC];
};
}  // namespace

// One chunk's inputs to out, held in registers.  Rows past the sequence end read
// the last row (the gate block marks those tokens invalid and the staging
// zeroes them), so the loads take no branch.  Part 0: the gate block, q, k, v,
// erase, write, Lambda; part 1: S0 (hi/lo) and T.
struct CwOutIn {
    float va;
    int sg;
    uint2 q, k, v;
    float er[4], wr[4], L[4];
    uint4 s0[2], s0l[2];
    float tf;
};
template <int P>
__device__ __forceinline__ void cwout_load(const ChunkArgs &a, int ci, int tid, CwOutIn &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid >> 4, c0 = 4 * (tid & 15), tg = c * CC + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    if constexpr (P == 0) {
        const CwGate *gb = a.ck_cwg + ci;
        x.va = gb->val[t];
        x.sg = gb->seg[t];
        x.q = *reinterpret_cast<const uint2 *>(row_ptr(a.q, a.qs, b, tr, h) + c0);
        x.k = *reinterpret_cast<const uint2 *>(row_ptr(a.k, a.ks, b, tr, h) + c0);
        x.v = *reinterpret_cast<const uint2 *>(row_ptr(a.v, a.vs, b, tr, h) + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x.er[e] = ld4<float>(a.erase, b, tr, h, c0 + e);
            x.wr[e] = ld4<float>(a.write, b, tr, h, c0 + e);
        }
        get4_f32(a.ck_lam + (int64_t)ci * CC * 64 + t * 64 + c0, x.L);
    } else {
        const uint16_t *S0 = a.ck_state + (int64_t)ci * 64 * 64;
        const uint16_t *S0l = a.ck_state_lo + (int64_t)ci * 64 * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int p = tid + NT4 * i, r = p >> 3, cb = 8 * (p & 7);
            x.s0[i] = *reinterpret_cast<const uint4 *>(S0 + r * 64 + cb);
            x.s0l[i] = *reinterpret_cast<const uint4 *>(S0l + r * 64 + cb);
        }
        x.tf = a.ck_tf[(int64_t)ci * CC * CC + tid];
    }
}

// The last stores of an out chunk, held until the next chunk's staging: the O
// row piece of threads < 128 (bf16 output) and the score of threads < 16.
struct CwOutOut {
    uint4 o;
    float score;
};
__device__ __forceinline__ void cwout_store(const ChunkArgs &a, int ci, int tid, const CwOutOut &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H, t0 = c * CC;
    if (a.out_bf16 && tid < CC * 8) {
        const int r = tid >> 3, cb = 8 * (tid & 7), tq = t0 + r;
        if (tq < a.T)
            *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.out) + (((int64_t)b * a.T + tq) * a.H + h) * 64 + cb) =
                x.o;
    }
    if (a.scores && tid < CC && t0 + tid < a.T) a.scores[((int64_t)b * a.T + t0 + tid) * a.H + h] = x.score;
}

// Workgroups walk chunks blockIdx.x, blockIdx.x + gridDim.x, ... (as many
// workgroups as fit the GPU at once): the next chunk's inputs are loaded into
// registers while the current one computes, and a chunk's O rows and scores
// are stored after the next chunk's staging.
__global__ void __launch_bounds__(NT4) cw_out_kernel(ChunkArgs a, int nchunks) {
    __shared__ CwOutSmem sm;
    {  // zero padding (columns 16..31 of T, P, R^T and delta^T), once
        const int tid = threadIdx.x;
        for (int i = tid; i < CC * 16; i += NT4) {
            const int r = i >> 4, cc = 16 + (i & 15);
            sm.tb[r * LDB + cc] = 0;
            sm.tbl[r * LDB + cc] = 0;
            sm.pr[r * LDB + cc] = 0;
            sm.prl[r * LDB + cc] = 0;
        }
        for (int i = tid; i < 4 * 64 * 16; i += NT4) {
            uint16_t *tl = (i >> 10) == 0 ? sm.rt : (i >> 10) == 1 ? sm.rtl : (i >> 10) == 2 ? sm.dt : sm.dtl;
            tl[((i >> 4) & 63) * LDW + 16 + (i & 15)] = 0;
        }
    }
    CwOutIn in;
    cwout_load<0>(a, blockIdx.x, threadIdx.x, in);
    cwout_load<1>(a, blockIdx.x, threadIdx.x, in);
    CwOutOut po;
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the lane- and wave-dependent address arithmetic inside
    // the loop (hoisted, it would stay live across it).
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid >> 4, c0 = 4 * (tid & 15), t0 = c * CC;
    // The next chunk.  Past the end the loads need no branch either: every lane
    // addresses this chunk as thread 0 would, so each load instruction touches
    // a line or two that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    {
        const float va = in.va;
        const int sg = in.sg;
        const bool on = va != 0.f;
        float qv[4], kv[4], vv[4], er[4], wr[4], L[4];
        qv[0] = bf16_val((uint16_t)(in.q.x & 0xffff)), qv[1] = bf16_val((uint16_t)(in.q.x >> 16));
        qv[2] = bf16_val((uint16_t)(in.q.y & 0xffff)), qv[3] = bf16_val((uint16_t)(in.q.y >> 16));
        kv[0] = bf16_val((uint16_t)(in.k.x & 0xffff)), kv[1] = bf16_val((uint16_t)(in.k.x >> 16));
        kv[2] = bf16_val((uint16_t)(in.k.y & 0xffff)), kv[3] = bf16_val((uint16_t)(in.k.y >> 16));
        vv[0] = bf16_val((uint16_t)(in.v.x & 0xffff)), vv[1] = bf16_val((uint16_t)(in.v.x >> 16));
        vv[2] = bf16_val((uint16_t)(in.v.y & 0xffff)), vv[3] = bf16_val((uint16_t)(in.v.y >> 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) er[e] = in.er[e], wr[e] = in.wr[e], L[e] = in.L[e];
        mask4(qv, on, 0.f), mask4(kv, on, 0.f), mask4(vv, on, 0.f), mask4(er, on, 0.f), mask4(wr, on, 0.f);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int p = tid + NT4 * i, r = p >> 3, cb = 8 * (p & 7);
            *reinterpret_cast<uint4 *>(&sm.st[r * LDB + cb]) = in.s0[i];
            *reinterpret_cast<uint4 *>(&sm.stl[r * LDB + cb]) = in.s0l[i];
        }
        {
            uint16_t hi, lo;
            split_bf16(in.tf, hi, lo);
            sm.tb[(tid >> 4) * LDB + (tid & 15)] = hi;
            sm.tbl[(tid >> 4) * LDB + (tid & 15)] = lo;
        }
        float b4[4], qh[4], ah[4], wv[4];
        float ksq = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            b4[e] = sg == 0 ? __expf(L[e]) : 0.f;
            qh[e] = b4[e] * qv[e];
            ah[e] = b4[e] * er[e] * kv[e];
            wv[e] = wr[e] * vv[e];
            ksq += kv[e] * kv[e];
        }
        put4_f32(&sm.lam[t * LDL + c0], L);
        put4_f32(&sm.qf[t * LDL + c0], qv);
        put4_f32(&sm.kf[t * LDL + c0], kv);
        put4_f32(&sm.wvf[t * LDL + c0], wv);
        put4_split(&sm.qh[t * LDB + c0], &sm.qhl[t * LDB + c0], qh);
        put4_split(&sm.ah[t * LDB + c0], &sm.ahl[t * LDB + c0], ah);
        // |k_t|^2: sum over the 16 threads of token t (lanes 16 r .. 16 r + 15)
        ksq = row16_sum(ksq);
        if ((tid & 15) == 0) {
            sm.kk[t] = ksq;
            sm.val[t] = va;
            sm.seg[t] = sg;
        }
    }
    if (ci != (int)blockIdx.x) cwout_store(a, ci - gridDim.x, tid, po);  // the previous chunk's
    cwout_load<0>(a, cn, tn, in);
    __syncthreads();
    cwout_load<1>(a, cn, tn, in);
    // P (lower, same segment), elementwise; pair p on lanes 2p, 2p + 1.
    for (int base = 0; base < 2 * 136; base += NT4) {
        const int task = base + tid, p = task >> 1, half = task & 1;
        int tt = 0, ss = 0;
        if (p < 136) pair_of(p, false, tt, ss);
        float acc = p < 136 ? pair_dot32(sm.qf, sm.kf, sm.lam, tt, ss, half) : 0.f;
        acc += dpp<0xB1>(acc);
        if (p < 136 && half == 0) {
            const float pv = sm.seg[tt] == sm.seg[ss] ? acc : 0.f;
            uint16_t hi, lo;
            split_bf16(pv, hi, lo);
            sm.pr[tt * LDB + ss] = hi;
            sm.prl[tt * LDB + ss] = lo;
            a.ck_p[(int64_t)ci * CC * CC + tt * CC + ss] = pv;  // for the backward
        }
    }
    for (int i = tid; i < 120; i += NT4) {  // zero the strict upper triangle of P
        int tt, ss;
        pair_of(i, true, tt, ss);
        sm.pr[ss * LDB + tt] = 0;
        sm.prl[ss * LDB + tt] = 0;
        a.ck_p[(int64_t)ci * CC * CC + ss * CC + tt] = 0.f;
    }
    // R = w.v - Ahat S0 and Qhat S0 for value tile w.
    f32x4 qs = zero4();
    {
        f32x4 x = zero4();
#pragma unroll
        for (int r = 0; r < 64; r += 32) {
            const bf16x8_t sb = frag(&sm.st[(16 * w) * LDB], LDB, r);
            const bf16x8_t sbl = frag(&sm.stl[(16 * w) * LDB], LDB, r);
            const bf16x8_t ab = frag(sm.ah, LDB, r), qb = frag(sm.qh, LDB, r);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, sb, x, 0, 0, 0);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.ahl, LDB, r), sb, x, 0, 0, 0);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, sbl, x, 0, 0, 0);
            qs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qb, sb, qs, 0, 0, 0);
            qs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.qhl, LDB, r), sb, qs, 0, 0, 0);
            qs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qb, sbl, qs, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = sm.wvf[acc_row(i) * LDL + 16 * w + acc_col()] - x[i];
        store_tile_t_split(&sm.rt[(16 * w) * LDW], &sm.rtl[(16 * w) * LDW], LDW, x);
    }
    __syncthreads();
    // delta = T R; |delta_t|^2 partials; delta^T hi/lo; delta to the checkpoint.
    f32x4 dl = zero4();
    {
        const bf16x8_t ta = frag(sm.tb, LDB, 0), tal = frag(sm.tbl, LDB, 0);
        const bf16x8_t rb = frag(&sm.rt[(16 * w) * LDW], LDW, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, rb, dl, 0, 0, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, frag(&sm.rtl[(16 * w) * LDW], LDW, 0), dl, 0, 0, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tal, rb, dl, 0, 0, 0);
        float p4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p4[i] = dl[i] * dl[i];
        row_reduce_store(p4, sm.dd[w], 0);
        store_tile_t_split(&sm.dt[(16 * w) * LDW], &sm.dtl[(16 * w) * LDW], LDW, dl);
        float *dck = a.ck_delta + (int64_t)ci * CC * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) dck[acc_row(i) * 64 + 16 * w + acc_col()] = dl[i];
    }
    __syncthreads();
    // O = Qhat S0 + P delta (P hi/lo x delta hi/lo, three terms).
    {
        f32x4 x = qs;
        const bf16x8_t ph = frag(sm.pr, LDB, 0), pl = frag(sm.prl, LDB, 0);
        const bf16x8_t dh = frag(&sm.dt[(16 * w) * LDW], LDW, 0), dlo = frag(&sm.dtl[(16 * w) * LDW], LDW, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, dh, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, dlo, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, dh, x, 0, 0, 0);
        if (a.out_bf16) {
            store_tile_rm(&sm.qh[16 * w], LDB, x);  // O rows over Qhat (read in phase 1)
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tq = t0 + acc_row(i);
                if (tq < a.T)
                    reinterpret_cast<float *>(a.out)[(((int64_t)b * a.T + tq) * a.H + h) * 64 + 16 * w +
                                                     acc_col()] = x[i];
            }
        }
    }
    __syncthreads();
    // O row pieces and scores into registers (stored after the next staging).
    po.o = *reinterpret_cast<const uint4 *>(&sm.qh[(tid >> 3 & 15) * LDB + 8 * (tid & 7)]);
    {
        const int tk = tid & 15;
        const float dd = sm.dd[0][tk] + sm.dd[1][tk] + sm.dd[2][tk] + sm.dd[3][tk];
        po.score = sm.val[tk] != 0.f ? sqrtf(sm.kk[tk] * dd) : 0.f;
    }
    __syncthreads();  // the next chunk's staging overwrites the tiles read above
    }
    {
        const int tid = threadIdx.x;
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        cwout_store(a, last, tid, po);
    }
}

// ---- backward prep: N of the adjoint map dS0 = A_c^T dS_16 + N -----------------
// N = Y - W'^T X with Y = Qhat^T dO, X = P^T dO + diag(c) delta, W' = T Ahat
// (formed again with prep's operands, P from the forward's checkpoint),
// c_s = dscore_s |k_s| / |delta_s|.
namespace {
struct CwBPrepSmem {
    uint16_t qh[RT32], qhl[RT32];  // Qhat rows hi/lo (rows 16..31 zero)
    uint16_t ah[RT32], ahl[RT32];  // Ahat rows hi/lo (rows 16..31 zero)
    uint16_t dor[RT32];   // dO rows (rows 16..31 zero)
    uint16_t tb[RT16], tbl[RT16];  // T rows hi/lo (columns 16..31 zero)
    uint16_t ptr[RT16], ptrl[RT16];  // P^T rows hi/lo ([s][t], columns 16..31 zero)
    uint16_t wt[CT64], wtl[CT64];    // W'^T hi/lo
    uint16_t xt[CT64], xtl[CT64];    // X^T hi/lo
    float cs[CC];
};
}  // namespace

// One chunk's inputs to bprep, held in registers.  Rows past the sequence end
// read the last row (the gate block marks those tokens invalid and the staging
// zeroes them), a missing dO reads q (zeroed at the staging) and a missing
// score adjoint reads the delta checkpoint, so the loads take no branch.
// Part 0: q, k, dO and the gate block; part 1: erase, Lambda, delta, T, P and
// the score terms.
struct CwBpIn {
    uint2 q, k, dO;
    float er[4], L[4], dl[4], dacc[4];
    float tf, pf, va, dsc;
    int sg;
};
template <int P>
__device__ __forceinline__ void cwbp_load(const ChunkArgs &a, int ci, int tid, int w, CwBpIn &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid >> 4, c0 = 4 * (tid & 15), tg = c * CC + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    if constexpr (P == 0) {
        x.q = *reinterpret_cast<const uint2 *>(row_ptr(a.q, a.qs, b, tr, h) + c0);
        x.k = *reinterpret_cast<const uint2 *>(row_ptr(a.k, a.ks, b, tr, h) + c0);
        x.dO = *reinterpret_cast<const uint2 *>(row_ptr(a.dout ? a.dout : a.q, a.dout ? a.ds : a.qs, b, tr, h) + c0);
        const CwGate *gb = a.ck_cwg + ci;
        x.va = gb->val[t];
        x.sg = gb->seg[t];
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) x.er[e] = ld4<float>(a.erase, b, tr, h, c0 + e);
        get4_f32(a.ck_lam + (int64_t)ci * CC * 64 + t * 64 + c0, x.L);
        const float *dck = a.ck_delta + (int64_t)ci * CC * 64;
        get4_f32(dck + t * 64 + c0, x.dl);
#pragma unroll
        for (int i = 0; i < 4; ++i) x.dacc[i] = dck[acc_row(i) * 64 + 16 * w + acc_col()];
        x.tf = a.ck_tf[(int64_t)ci * CC * CC + (tid >> 4) * CC + (tid & 15)];
        x.pf = a.ck_p[(int64_t)ci * CC * CC + (tid & 15) * CC + (tid >> 4)];
        x.dsc = (a.dscores ? a.dscores : a.ck_delta)[((int64_t)b * a.T + tr) * a.H + h];
    }
}

// N of chunk ci (transposed, f32) from the registers it was formed in.
__device__ __forceinline__ void cwbp_store(const ChunkArgs &a, int ci, int w, const f32x4 (&n)[4]) {
    float *Nt = a.ws_n + (int64_t)ci * 64 * 64;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
        *reinterpret_cast<float4 *>(&Nt[(16 * tn + acc_col()) * 64 + 16 * w + acc_row(0)]) =
            make_float4(n[tn][0], n[tn][1], n[tn][2], n[tn][3]);
}

// Workgroups walk chunks blockIdx.x, blockIdx.x + gridDim.x, ... (as many
// workgroups as fit the GPU at once): the next chunk's inputs are loaded into
// registers while the current one computes, and a chunk's N is stored after
// the next chunk's staging, so that no chunk but a workgroup's first waits on
// its loads or on the previous chunk's stores.
__global__ void __launch_bounds__(NT4) cw_bprep_kernel(ChunkArgs a, int nchunks) {
    __shared__ CwBPrepSmem sm;
    {  // zero padding (rows 16..31 of the token-row tiles, columns 16..31 of the others), once
        const int tid = threadIdx.x;
        zero_lds(sm.qh + RT16, RT32 - RT16, tid);
        zero_lds(sm.qhl + RT16, RT32 - RT16, tid);
        zero_lds(sm.ah + RT16, RT32 - RT16, tid);
        zero_lds(sm.ahl + RT16, RT32 - RT16, tid);
        zero_lds(sm.dor + RT16, RT32 - RT16, tid);
        for (int i = tid; i < CC * 16; i += NT4) {
            const int r = i >> 4, cc = 16 + (i & 15);
            sm.tb[r * LDB + cc] = 0;
            sm.tbl[r * LDB + cc] = 0;
            sm.ptr[r * LDB + cc] = 0;
            sm.ptrl[r * LDB + cc] = 0;
        }
        for (int i = tid; i < 4 * 64 * 16; i += NT4) {
            uint16_t *tl = (i >> 10) == 0 ? sm.wt : (i >> 10) == 1 ? sm.wtl : (i >> 10) == 2 ? sm.xt : sm.xtl;
            tl[((i >> 4) & 63) * LDW + 16 + (i & 15)] = 0;
        }
    }
    CwBpIn in;
    {
        const int w0 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        cwbp_load<0>(a, blockIdx.x, threadIdx.x, w0, in);
        cwbp_load<1>(a, blockIdx.x, threadIdx.x, w0, in);
    }
    f32x4 nacc[4];  // N = Y - W'^T X, held until the next chunk's staging is done
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the lane- and wave-dependent address arithmetic inside
    // the loop (hoisted, it would stay live across it).
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = tid >> 4, c0 = 4 * (tid & 15);
    // The next chunk.  Past the end the loads need no branch either: every lane
    // addresses this chunk as thread 0 would, so each load instruction touches
    // a line or two that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    {
        const bool on = in.va != 0.f;
        float qv[4], kv[4], dov[4], er[4];
        const uint2 q2 = in.q, k2 = in.k, d2 = in.dO;
        qv[0] = bf16_val((uint16_t)(q2.x & 0xffff)), qv[1] = bf16_val((uint16_t)(q2.x >> 16));
        qv[2] = bf16_val((uint16_t)(q2.y & 0xffff)), qv[3] = bf16_val((uint16_t)(q2.y >> 16));
        kv[0] = bf16_val((uint16_t)(k2.x & 0xffff)), kv[1] = bf16_val((uint16_t)(k2.x >> 16));
        kv[2] = bf16_val((uint16_t)(k2.y & 0xffff)), kv[3] = bf16_val((uint16_t)(k2.y >> 16));
        dov[0] = bf16_val((uint16_t)(d2.x & 0xffff)), dov[1] = bf16_val((uint16_t)(d2.x >> 16));
        dov[2] = bf16_val((uint16_t)(d2.y & 0xffff)), dov[3] = bf16_val((uint16_t)(d2.y >> 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) er[e] = in.er[e];
        mask4(qv, on, 0.f), mask4(kv, on, 0.f), mask4(dov, on && a.dout, 0.f), mask4(er, on, 0.f);
        {
            uint16_t hi, lo;
            split_bf16(in.tf, hi, lo);
            sm.tb[(tid >> 4) * LDB + (tid & 15)] = hi;
            sm.tbl[(tid >> 4) * LDB + (tid & 15)] = lo;
            split_bf16(in.pf, hi, lo);
            sm.ptr[(tid >> 4) * LDB + (tid & 15)] = hi;
            sm.ptrl[(tid >> 4) * LDB + (tid & 15)] = lo;
        }
        float qh[4], ah[4], ksq = 0.f, dsq = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float bt = in.sg == 0 ? __expf(in.L[e]) : 0.f;
            qh[e] = bt * qv[e];
            ah[e] = bt * er[e] * kv[e];
            ksq += kv[e] * kv[e];
            dsq += in.dl[e] * in.dl[e];
        }
        put4_split(&sm.qh[t * LDB + c0], &sm.qhl[t * LDB + c0], qh);
        put4_split(&sm.ah[t * LDB + c0], &sm.ahl[t * LDB + c0], ah);
        put4_bf16(&sm.dor[t * LDB + c0], dov);
        ksq = row16_sum(ksq);
        dsq = row16_sum(dsq);
        if ((tid & 15) == 0) {
            const float nk = sqrtf(ksq), nd = sqrtf(dsq);
            sm.cs[t] = (a.dscores && nk > 0.f && nd > 0.f) ? in.dsc * nk / nd : 0.f;
        }
    }
    float dacc[4];  // delta at this lane's accumulator positions (value tile w)
#pragma unroll
    for (int i = 0; i < 4; ++i) dacc[i] = in.dacc[i];
    if (ci != (int)blockIdx.x) cwbp_store(a, ci - gridDim.x, w, nacc);  // the previous chunk's N
    cwbp_load<0>(a, cn, tn, w, in);
    __syncthreads();
    cwbp_load<1>(a, cn, tn, w, in);
    // Y = Qhat^T dO (row tile w of keys, all value tiles) and W' = T Ahat (tile w).
    f32x4 y[4];
    {
        const bf16x8_t qa = frag_tr(sm.qh, 0, 16 * w);  // A[k][t] = Qhat[t][16 w + k]
        const bf16x8_t qal = frag_tr(sm.qhl, 0, 16 * w);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            const bf16x8_t db = frag_tr(sm.dor, 0, 16 * tn);
            y[tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, db, zero4(), 0, 0, 0);
            y[tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qal, db, y[tn], 0, 0, 0);
        }
        const bf16x8_t ta = frag(sm.tb, LDB, 0), tal = frag(sm.tbl, LDB, 0);
        const bf16x8_t ab = frag_tr(sm.ah, 0, 16 * w);
        f32x4 x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, ab, zero4(), 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, frag_tr(sm.ahl, 0, 16 * w), x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tal, ab, x, 0, 0, 0);
        store_tile_t_split(&sm.wt[(16 * w) * LDW], &sm.wtl[(16 * w) * LDW], LDW, x);
    }
    __syncthreads();
    // X = P^T dO + c delta (value tile w), stored transposed hi/lo.
    {
        const bf16x8_t db = frag_tr(sm.dor, 0, 16 * w);  // B[t][v] = dO[t][16 w + v]
        f32x4 x = zero4();
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.ptr, LDB, 0), db, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.ptrl, LDB, 0), db, x, 0, 0, 0);
        if (a.dscores) {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] += sm.cs[acc_row(i)] * dacc[i];
        }
        store_tile_t_split(&sm.xt[(16 * w) * LDW], &sm.xtl[(16 * w) * LDW], LDW, x);
    }
    __syncthreads();
    // N = Y - W'^T X: key row tile w, value tiles 0..3, in registers.
    {
        const bf16x8_t wa = frag(&sm.wt[(16 * w) * LDW], LDW, 0), wal = frag(&sm.wtl[(16 * w) * LDW], LDW, 0);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            const bf16x8_t xb = frag(&sm.xt[(16 * tn) * LDW], LDW, 0), xbl = frag(&sm.xtl[(16 * tn) * LDW], LDW, 0);
            f32x4 x = zero4();
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xb, x, 0, 0, 0);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xbl, x, 0, 0, 0);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wal, xb, x, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) nacc[tn][e] = y[tn][e] - x[e];
        }
    }
    __syncthreads();  // the next chunk's staging overwrites the tiles read above
    }
    {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        cwbp_store(a, last, w, nacc);
    }
}

// ---- bgrad: every gradient of one chunk -----------------------------------------
// Given S0, delta and P (forward checkpoint) and dS at the chunk end (adjoint
// scan):
//   ddelta = P^T dO + Ktil dS + diag(c) delta;   dR = T^T ddelta
//   dw = dR.v,  dv = dR.w;   dAhat = -dR S0^T;  dQhat = dO S0^T;  dKtil = delta dS^T
//   dA = -strict_lower(dR delta^T),  dP = lower(dO delta^T)   (same segment)
//   through the decays D_ts (elementwise, per channel i):
//     eA_t = sum_s dA_ts D_ts k_s,  qP_t = sum_s dP_ts D_ts k_s,
//     kAP_s = sum_t (dA_ts D_ts ehat_t + dP_ts D_ts q_t)
//   dq = b dQhat + qP;  dehat = b dAhat + eA;  de = k dehat
//   dk = lam dKtil + kAP + e dehat + c' k
//   dalpha_u = sum over the pairs (hi, lo) with lo < u <= hi of the pair's
//              coefficient times the product of alpha over (lo, hi] without u:
//              interior pairs (dA_ts ehat_t + dP_ts q_t) k_s, start pairs
//              ehat_t dAhat_t + q_t dQhat_t (through b_t), end pairs k_s dKtil_s
//              (through lam_s) and rowsum(S0 . dS) (through b_15)
// (zero on padding and on valid reset tokens, where the reference's alpha' is
// alpha (1 - reset) and carries no gradient).
namespace {
constexpr int BG_STATE = 64 * LDB;  // bf16 elements of a staged 64 x 64 tile

// Two LDS regions change hands at barriers, so that two workgroups fit a CU:
// region A holds dS^T (hi/lo) through phase 1, then ddelta^T, dR and dA/dP;
// region B holds S0^T (hi/lo) through phase 4, then the sums of phase 5.
struct CwBGradSmem {
    float lam[CC * LDL], ehf[CC * LDL];
    float dRf[CC * LDL];   // dR (f32) for dw, dv; dLambda afterwards
    uint16_t qb[RT16], kb[RT16];     // q, k rows (bf16)
    uint16_t dor[RT32];    // dO rows (rows 16..31 zero)
    uint16_t kl[RT16], kll[RT16];    // Ktil rows hi/lo
    uint16_t ttr[RT16], ttrl[RT16];  // T^T rows hi/lo ([s][t], columns 16..31 zero)
    uint16_t dh[RT16], dlo[RT16];    // delta rows hi/lo
    uint16_t ptr[RT16], ptrl[RT16];  // P^T rows hi/lo; dq, dk rows (bf16) at the end
    union {
        uint16_t ds[2][BG_STATE];  // dS^T rows [v][k], hi and lo
        struct {
            uint16_t ddt[CT64], ddtl[CT64];    // ddelta^T hi/lo
            uint16_t drr[RT16], drrl[RT16];    // dR rows hi/lo
            float dA[CC * LDI], dP[CC * LDI];  // 16 x 16, same segment
        } g;
    } ra;
    union {
        uint16_t st[2][BG_STATE];  // S0^T rows [v][k], hi and lo
        float sums[3][CC * LDL];   // eA, qP, kAP [token][channel]
    } rb;
    float cs[CC], ck[CC], val[CC];
    int seg[CC];
    float fr[NW4][64];
};

// T^T (from the f32 T checkpoint) into hi/lo LDS rows [s][t]; thread
// (t = tid/16, s = tid%16).
__device__ __forceinline__ void load_tt_split(const float *ckt, uint16_t *th, uint16_t *tl, int tid) {
    const int t = tid >> 4, s = tid & 15;
    uint16_t hi, lo;
    split_bf16(ckt[t * CC + s], hi, lo);
    th[s * LDB + t] = hi;
    tl[s * LDB + t] = lo;
}
}  // namespace

// SCORE: a score adjoint is given (its terms are compiled in only then).
template <bool SCORE>
__global__ void __launch_bounds__(NT4) cw_bgrad_kernel(ChunkArgs a) {
    __shared__ CwBGradSmem sm;
    static_assert(sizeof(CwBGradSmem) <= 80 * 1024, "two workgroups per CU");
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid >> 4, c0 = 4 * (tid & 15), t0 = c * CC, tg = t0 + t;
    const bool inb = tg < a.T;
    zero_lds(sm.dor + RT16, RT32 - RT16, tid);
    for (int i = tid; i < CC * 16; i += NT4) {
        const int r = i >> 4, cc = 16 + (i & 15);
        sm.ttr[r * LDB + cc] = 0;
        sm.ttrl[r * LDB + cc] = 0;
        sm.ptr[r * LDB + cc] = 0;
        sm.ptrl[r * LDB + cc] = 0;
    }
    const CwGate *gb = a.ck_cwg + ci;
    const float va = gb->val[t];
    const int sg = gb->seg[t], sg15 = gb->seg[CC - 1];
    const bool on = va != 0.f;
    float qv[4], kv[4], vv[4], dov[4], er[4], wr[4], L[4], dl4[4];
    load4_bf16(a.q, a.qs, b, tg, h, c0, inb, qv);
    load4_bf16(a.k, a.ks, b, tg, h, c0, inb, kv);
    load4_bf16(a.v, a.vs, b, tg, h, c0, inb, vv);
    if (a.dout) load4_bf16(a.dout, a.ds, b, tg, h, c0, inb, dov);
    else dov[0] = dov[1] = dov[2] = dov[3] = 0.f;
    load4_f32(a.erase, b, tg, h, c0, inb, 0.f, er);
    load4_f32(a.write, b, tg, h, c0, inb, 0.f, wr);
    mask4(qv, on, 0.f), mask4(kv, on, 0.f), mask4(vv, on, 0.f), mask4(dov, on, 0.f);
    mask4(er, on, 0.f), mask4(wr, on, 0.f);
    const float *lck = a.ck_lam + (int64_t)ci * CC * 64;
    get4_f32(lck + t * 64 + c0, L);
    const float *dck = a.ck_delta + (int64_t)ci * CC * 64;
    get4_f32(dck + t * 64 + c0, dl4);
    // Loads of phases 6 and 7, issued with the rest so that their latency is
    // not exposed after a barrier: erase at this lane's accumulator positions
    // (key tile w), and alpha at this thread's token and channels.
    float eacc[4], dacc[4], alv4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int tq = t0 + acc_row(e);
        eacc[e] = tq < a.T ? ld4<float>(a.erase, b, tq, h, 16 * w + acc_col()) : 0.f;
        dacc[e] = SCORE ? dck[acc_row(e) * 64 + 16 * w + acc_col()] : 0.f;
    }
    if (a.dalpha) load4_f32(a.alpha, b, tg, h, c0, inb, 1.f, alv4);
    {
        const int64_t so = (int64_t)ci * 64 * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int p = tid + NT4 * i, r = p >> 3, cb = 8 * (p & 7), o = r * 64 + cb;
            *reinterpret_cast<uint4 *>(&sm.rb.st[0][r * LDB + cb]) = *reinterpret_cast<const uint4 *>(a.ck_state + so + o);
            *reinterpret_cast<uint4 *>(&sm.rb.st[1][r * LDB + cb]) = *reinterpret_cast<const uint4 *>(a.ck_state_lo + so + o);
            *reinterpret_cast<uint4 *>(&sm.ra.ds[0][r * LDB + cb]) = *reinterpret_cast<const uint4 *>(a.ws_dstate + so + o);
            *reinterpret_cast<uint4 *>(&sm.ra.ds[1][r * LDB + cb]) = *reinterpret_cast<const uint4 *>(a.ws_dstate_lo + so + o);
        }
        load_tt_split(a.ck_tf + (int64_t)ci * CC * CC, sm.ttr, sm.ttrl, tid);
        load_pt_split(a.ck_p + (int64_t)ci * CC * CC, sm.ptr, sm.ptrl, tid);
    }
    {
        float eh[4], klv[4], ksq = 0.f, dsq = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float L15 = lck[(CC - 1) * 64 + c0 + e];
            eh[e] = er[e] * kv[e];
            klv[e] = (sg == sg15 ? __expf(L15 - L[e]) : 0.f) * kv[e];
            ksq += kv[e] * kv[e];
            dsq += dl4[e] * dl4[e];
        }
        put4_f32(&sm.lam[t * LDL + c0], L);
        put4_f32(&sm.ehf[t * LDL + c0], eh);
        put4_bf16(&sm.qb[t * LDB + c0], qv);  // exact: q, k are bf16 values
        put4_bf16(&sm.kb[t * LDB + c0], kv);
        put4_bf16(&sm.dor[t * LDB + c0], dov);
        put4_split(&sm.kl[t * LDB + c0], &sm.kll[t * LDB + c0], klv);
        put4_split(&sm.dh[t * LDB + c0], &sm.dlo[t * LDB + c0], dl4);
        ksq = row16_sum(ksq);
        dsq = row16_sum(dsq);
        if ((tid & 15) == 0) {
            const float dsc = (SCORE && inb) ? a.dscores[((int64_t)b * a.T + tg) * a.H + h] : 0.f;
            const float nk = sqrtf(ksq), nd = sqrtf(dsq);
            const bool ok = nk > 0.f && nd > 0.f;
            sm.cs[t] = ok ? dsc * nk / nd : 0.f;
            sm.ck[t] = ok ? dsc * nd / nk : 0.f;
            sm.val[t] = va;
            sm.seg[t] = sg;
        }
    }
    __syncthreads();
    // Phase 1: dQhat (key tile w), Ktil dS (value tile w), dKtil = delta dS^T (key
    // tile w); rowsum(S0 . dS) per key channel.
    const uint16_t *st = sm.rb.st[0], *stl = sm.rb.st[1];
    f32x4 gqh = zero4(), kds = zero4(), gkt = zero4();
    {
        const uint16_t *dst = sm.ra.ds[0], *dstl = sm.ra.ds[1];
#pragma unroll
        for (int r = 0; r < 64; r += 32) {
            const bf16x8_t sb = frag_tr(st, r, 16 * w), db = frag_tr(dst, r, 16 * w);
            const bf16x8_t sbl = frag_tr(stl, r, 16 * w), dbl = frag_tr(dstl, r, 16 * w);
            const bf16x8_t ob = frag(sm.dor, LDB, r);
            gqh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ob, sb, gqh, 0, 0, 0);
            gqh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ob, sbl, gqh, 0, 0, 0);
            const bf16x8_t dsb = frag(&dst[(16 * w) * LDB], LDB, r), kb = frag(sm.kl, LDB, r);
            kds = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, dsb, kds, 0, 0, 0);
            kds = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.kll, LDB, r), dsb, kds, 0, 0, 0);
            kds = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, frag(&dstl[(16 * w) * LDB], LDB, r), kds, 0, 0, 0);
            const bf16x8_t hb = frag(sm.dh, LDB, r);
            gkt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hb, db, gkt, 0, 0, 0);
            gkt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.dlo, LDB, r), db, gkt, 0, 0, 0);
            gkt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hb, dbl, gkt, 0, 0, 0);
        }
        {  // rowsum_v S0[i][v] dS[i][v], key channel i = tid % 64, rows v of quarter w
            const int i = tid & 63;
            float f = 0.f;
#pragma unroll 8
            for (int v = 16 * w; v < 16 * w + 16; ++v)
                f += (bf16_val(st[v * LDB + i]) + bf16_val(stl[v * LDB + i])) *
                     (bf16_val(dst[v * LDB + i]) + bf16_val(dstl[v * LDB + i]));
            sm.fr[w][i] = f;
        }
    }
    __syncthreads();  // dS is dead: region A takes ddelta^T, dR, dA, dP
    auto &g = sm.ra.g;
    for (int i = tid; i < 2 * 64 * 16; i += NT4)
        ((i >> 10) == 0 ? g.ddt : g.ddtl)[((i >> 4) & 63) * LDW + 16 + (i & 15)] = 0;
    // Phase 2: ddelta = P^T dO + Ktil dS + c delta (value tile w) -> ddelta^T hi/lo.
    {
        const bf16x8_t db = frag_tr(sm.dor, 0, 16 * w);
        f32x4 x = kds;
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.ptr, LDB, 0), db, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(sm.ptrl, LDB, 0), db, x, 0, 0, 0);
        if (SCORE) {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] += sm.cs[acc_row(e)] * dacc[e];
        }
        store_tile_t_split(&g.ddt[(16 * w) * LDW], &g.ddtl[(16 * w) * LDW], LDW, x);
    }
    __syncthreads();
    // Phase 3: dR = T^T ddelta (value tile w) -> dR rows (hi/lo) and f32.
    {
        const bf16x8_t ta = frag(sm.ttr, LDB, 0), tal = frag(sm.ttrl, LDB, 0);  // A[s][t] = T[t][s]
        const bf16x8_t db = frag(&g.ddt[(16 * w) * LDW], LDW, 0);
        f32x4 x = zero4();
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, db, x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, frag(&g.ddtl[(16 * w) * LDW], LDW, 0), x, 0, 0, 0);
        x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tal, db, x, 0, 0, 0);
        store_tile_rm_split(&g.drr[16 * w], &g.drrl[16 * w], LDB, x);
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.dRf[acc_row(e) * LDL + 16 * w + acc_col()] = x[e];
    }
    __syncthreads();
    // Phase 4: dAhat = -dR S0^T (key tile w); dA (wave 0) and dP (wave 1); dw, dv.
    f32x4 gah = zero4();
#pragma unroll
    for (int r = 0; r < 64; r += 32) {
        const bf16x8_t sb = frag_tr(st, r, 16 * w), rb = frag(g.drr, LDB, r);
        gah = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rb, sb, gah, 0, 0, 0);
        gah = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(g.drrl, LDB, r), sb, gah, 0, 0, 0);
        gah = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rb, frag_tr(stl, r, 16 * w), gah, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) gah[e] = -gah[e];
    if (w < 2) {
        f32x4 x = zero4();
        const uint16_t *lhs = w == 0 ? g.drr : sm.dor;
#pragma unroll
        for (int r = 0; r < 64; r += 32) {
            const bf16x8_t la = frag(lhs, LDB, r), dhb = frag(sm.dh, LDB, r);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(la, dhb, x, 0, 0, 0);
            x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(la, frag(sm.dlo, LDB, r), x, 0, 0, 0);
            if (w == 0) x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(g.drrl, LDB, r), dhb, x, 0, 0, 0);
        }
        const int ss = acc_col();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tt = acc_row(e);
            const bool same = sm.seg[tt] == sm.seg[ss];
            if (w == 0) g.dA[tt * LDI + ss] = (ss < tt && same) ? -x[e] : 0.f;
            else g.dP[tt * LDI + ss] = (ss <= tt && same) ? x[e] : 0.f;
        }
    }
    if (inb) {  // dw = dR.v, dv = dR.w (token t, channels c0 .. c0 + 3)
        float dr[4], dw4[4], dv4[4];
        get4_f32(&sm.dRf[t * LDL + c0], dr);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dw4[e] = on ? dr[e] * vv[e] : 0.f;
            dv4[e] = on ? dr[e] * wr[e] : 0.f;
        }
        const int64_t row = ((int64_t)b * a.T + tg) * a.H + h;
        if (a.dwrite) put4_f32(a.dwrite + row * 64 + c0, dw4);
        if (a.dv) put4_bf16(reinterpret_cast<uint16_t *>(a.dv) + row * 64 + c0, dv4);
    }
    __syncthreads();  // S0 is dead: region B takes the sums of phase 5
    // Phase 5: the decay-weighted sums, elementwise.  Thread (channel i = tid/4,
    // part = tid%4) takes the rows t = part, part + 4, part + 8, part + 12 and every
    // s <= t: eA_t, qP_t are its own; kAP_s is summed over the four parts (a DPP
    // quad).
    float *seA = sm.rb.sums[0], *sqP = sm.rb.sums[1], *skAP = sm.rb.sums[2];
    {
        const int i = tid >> 2, part = tid & 3;
        float eA[4] = {0.f, 0.f, 0.f, 0.f}, qP[4] = {0.f, 0.f, 0.f, 0.f};
        float kAP[CC], Ls[CC], ks[CC];
#pragma unroll
        for (int s = 0; s < CC; ++s) {
            kAP[s] = 0.f;
            Ls[s] = sm.lam[s * LDL + i];
            ks[s] = bf16_val(sm.kb[s * LDB + i]);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int tt = part + 4 * m;
            const float Lt = sm.lam[tt * LDL + i], et = sm.ehf[tt * LDL + i];
            const float qt = bf16_val(sm.qb[tt * LDB + i]);
#pragma unroll
            for (int s = 0; s < CC; ++s) {
                if (s > tt) continue;
                const float D = s == tt ? 1.f : __expf(Lt - Ls[s]);
                const float dA = g.dA[tt * LDI + s], dP = g.dP[tt * LDI + s];
                const float kd = ks[s] * D;
                eA[m] += dA * kd;
                qP[m] += dP * kd;
                kAP[s] += (dA * et + dP * qt) * D;
            }
        }
#pragma unroll
        for (int s = 0; s < CC; ++s) {
            float x = kAP[s];
            x += dpp<0xB1>(x);
            x += dpp<0x4E>(x);
            kAP[s] = x;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            seA[(part + 4 * m) * LDL + i] = eA[m];
            sqP[(part + 4 * m) * LDL + i] = qP[m];
        }
        if (part == 0) {
#pragma unroll
            for (int s = 0; s < CC; ++s) skAP[s * LDL + i] = kAP[s];
        }
    }
    __syncthreads();
    // Phase 6: assemble dq, dk, de at key tile w (accumulator layout), and the
    // alpha gradient's start- and end-pair coefficients (phase 7) over the dead
    // ddelta^T, alpha (1 on padding) over the dead dR rows.
    float *stc = reinterpret_cast<float *>(g.ddt), *enc = stc + CC * LDL;
    float *alf = reinterpret_cast<float *>(g.drr);
    static_assert(2 * CC * LDL * sizeof(float) <= 2 * sizeof(g.ddt), "pair coefficients over ddelta^T");
    static_assert(CC * LDL * sizeof(float) <= 2 * sizeof(g.drr), "alpha over the dR rows");
    if (a.dalpha) {
        float ae[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ae[e] = on ? alv4[e] : 1.f;
        put4_f32(&alf[t * LDL + c0], ae);
    }
    {
        const int i = 16 * w + acc_col();
        const float L15 = sm.lam[(CC - 1) * LDL + i];
        f32x4 gq, gk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tt = acc_row(e), tq = t0 + tt;
            const bool von = sm.val[tt] != 0.f;
            const float Lt = sm.lam[tt * LDL + i];
            const float bt = sm.seg[tt] == 0 ? __expf(Lt) : 0.f;
            const float lt = sm.seg[tt] == sm.seg[CC - 1] ? __expf(L15 - Lt) : 0.f;
            const float q = bf16_val(sm.qb[tt * LDB + i]), k = bf16_val(sm.kb[tt * LDB + i]);
            const float eh = sm.ehf[tt * LDL + i];
            const float ee = von ? eacc[e] : 0.f;
            const float eA = seA[tt * LDL + i], qP = sqP[tt * LDL + i], kAP = skAP[tt * LDL + i];
            const float dq = bt * gqh[e] + qP;
            const float deh = bt * gah[e] + eA;
            const float dk = lt * gkt[e] + kAP + ee * deh + sm.ck[tt] * k;
            gq[e] = von ? dq : 0.f;
            gk[e] = von ? dk : 0.f;
            stc[tt * LDL + i] = sm.seg[tt] == 0 ? eh * gah[e] + q * gqh[e] : 0.f;
            enc[tt * LDL + i] = sm.seg[tt] == sm.seg[CC - 1] ? k * gkt[e] : 0.f;
            if (a.derase && tq < a.T)
                a.derase[(((int64_t)b * a.T + tq) * a.H + h) * 64 + i] = von ? k * deh : 0.f;
        }
        store_tile_rm(&sm.ptr[16 * w], LDB, gq);   // dq rows over P^T (dead)
        store_tile_rm(&sm.ptrl[16 * w], LDB, gk);  // dk rows
    }
    __syncthreads();
    if (tid < CC * 8) {  // dq, dk rows: 16-byte pieces
        const int r = tid >> 3, cb = 8 * (tid & 7), tq = t0 + r;
        if (tq < a.T) {
            const int64_t o = (((int64_t)b * a.T + tq) * a.H + h) * 64 + cb;
            if (a.dq) *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.dq) + o) =
                *reinterpret_cast<const uint4 *>(&sm.ptr[r * LDB + cb]);
            if (a.dk) *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.dk) + o) =
                *reinterpret_cast<const uint4 *>(&sm.ptrl[r * LDB + cb]);
        }
    }
    if (a.dalpha) {
        // Phase 7: dalpha without dividing by alpha.  Every gradient term that
        // alpha_u enters is a pair (hi, lo) of the chunk with lo < u <= hi whose
        // decay is the product of alpha over (lo, hi]: interior pairs of tokens
        // (s < t), start pairs (t, start) through b_t, end pairs (end, s) through
        // lam_s and the pair (end, start) through b_15 (end acts as token 15,
        // start as token -1).  With C the pair coefficients,
        //   dalpha_u = sum_{lo < u <= hi} C[hi][lo] prod_{lo < u' <= hi, u' != u} alpha_u'
        //            = sum_{lo < u} L(lo, u) Y(u, lo),
        //   L(lo, u) = prod_{lo < u' < u} alpha_u',
        //   Y(u, lo) = C[u][lo] + alpha_{u+1} Y(u + 1, lo),
        // so alpha = 0 gets its exact gradient and a small alpha loses no
        // precision.  Pairs never cross a reset (their coefficients are zero), and
        // padding has alpha 1.  Thread (channel i = tid / 4, part p = tid % 4)
        // takes lo = p - 1, p + 3, p + 7, p + 11; the four parts are summed by a
        // DPP quad.
        const int i = tid >> 2, p = tid & 3;
        const int sg15 = sm.seg[CC - 1];
        const float fs = sg15 == 0 ? sm.fr[0][i] + sm.fr[1][i] + sm.fr[2][i] + sm.fr[3][i] : 0.f;
        float alv[CC], ehv[CC], qv16[CC], acc[CC];
#pragma unroll
        for (int u = 0; u < CC; ++u) {
            alv[u] = alf[u * LDL + i];
            ehv[u] = sm.ehf[u * LDL + i];
            qv16[u] = bf16_val(sm.qb[u * LDB + i]);
            acc[u] = 0.f;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int lo = p - 1 + 4 * m;  // -1 .. 14
            const float klo = lo >= 0 ? bf16_val(sm.kb[lo * LDB + i]) : 0.f;
            const float elo = lo >= 0 ? enc[lo * LDL + i] : fs;  // end pair with lo
            float Yr[CC], Y = 0.f;
#pragma unroll
            for (int u = CC - 1; u >= 0; --u) {
                const int lc = lo >= 0 ? lo : 0;
                const float inner = (g.dA[u * LDI + lc] * ehv[u] + g.dP[u * LDI + lc] * qv16[u]) * klo;
                float cf = lo < 0 ? stc[u * LDL + i] : (u > lo ? inner : 0.f);
                if (u == CC - 1) cf += elo;
                Y = u == CC - 1 ? cf : cf + alv[u + 1] * Y;
                Yr[u] = Y;
            }
            float L = 1.f;
#pragma unroll
            for (int u = 0; u < CC; ++u)
                if (u > lo) {
                    acc[u] += L * Yr[u];
                    L *= alv[u];
                }
        }
#pragma unroll
        for (int u = 0; u < CC; ++u) {
            float x = acc[u];
            x += dpp<0xB1>(x);
            x += dpp<0x4E>(x);
            acc[u] = x;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int u = p + 4 * m, tq = t0 + u;
            const float da = p == 0 ? acc[4 * m] : p == 1 ? acc[4 * m + 1] : p == 2 ? acc[4 * m + 2] : acc[4 * m + 3];
            const bool von = sm.val[u] != 0.f;
            // the reset token's own alpha (applied to a zeroed state) carries no gradient
            const bool rs = von && (u == 0 ? sm.seg[0] == 1 : sm.seg[u] != sm.seg[u - 1]);
            if (tq < a.T) a.dalpha[(((int64_t)b * a.T + tq) * a.H + h) * 64 + i] = von && !rs ? da : 0.f;
        }
    }
}

static inline void cmark(const hipEvent_t *ev, int i, hipStream_t stream) {
    if (ev) (void)hipEventRecord(ev[i], stream);
}

// The factored scan over a head's 16-token chunks: forward (states and their
// lo parts, U of prep) or reverse (state adjoints and their lo parts, N of
// bprep).
static hipError_t cw_scan(const ChunkArgs &a, bool reverse, hipStream_t stream) {
    LrScanArgs p{};
    p.nc = a.nc;
    p.B = a.B;
    p.H = a.H;
    p.vd = 64;
    p.wt = a.lr_wt;
    p.kt = a.lr_kt;
    p.gv = a.lr_gv;
    p.reverse = reverse ? 1 : 0;
    if (!reverse) {
        p.u = a.lr_u;
        p.ckpt = a.ck_state;
        p.ckpt_lo = a.ck_state_lo;
        p.x0 = a.initial;
        p.xout = a.final_state;
    } else {
        p.n = a.ws_n;
        p.ckpt = a.ws_dstate;
        p.ckpt_lo = a.ws_dstate_lo;
        p.x0.data = a.dfinal;
        p.x0.s0 = (int64_t)a.H * 64 * 64;
        p.x0.s1 = 64 * 64;
        p.x0.s2 = 64;
        p.x0.s3 = 1;
        p.xout = a.dinitial;
    }
    return launch_lr_scan(p, 64, CC, stream);
}

hipError_t launch_cw_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nch = a.B * a.H * a.nc;
    cmark(ev, 0, stream);
    hipLaunchKernelGGL(cw_prep_kernel, dim3(std::min(nch, 4 * device_cus())), dim3(NT4), 0, stream, a, nch);
    cmark(ev, 1, stream);
    cmark(ev, 2, stream);
    const hipError_t e = cw_scan(a, false, stream);
    if (e != hipSuccess) return e;
    cmark(ev, 3, stream);
    cmark(ev, 4, stream);
    hipLaunchKernelGGL(cw_out_kernel, dim3(std::min(nch, 2 * device_cus())), dim3(NT4), 0, stream, a, nch);
    cmark(ev, 5, stream);
    return hipGetLastError();
}

hipError_t launch_cw_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nch = a.B * a.H * a.nc;
    cmark(ev, 0, stream);
    hipLaunchKernelGGL(cw_bprep_kernel, dim3(std::min(nch, 3 * device_cus())), dim3(NT4), 0, stream, a, nch);
    cmark(ev, 1, stream);
    cmark(ev, 2, stream);
    const hipError_t e = cw_scan(a, true, stream);
    if (e != hipSuccess) return e;
    cmark(ev, 3, stream);
    cmark(ev, 4, stream);
    if (a.dscores)
        hipLaunchKernelGGL(cw_bgrad_kernel<true>, dim3(nch), dim3(NT4), 0, stream, a);
    else
        hipLaunchKernelGGL(cw_bgrad_kernel<false>, dim3(nch), dim3(NT4), 0, stream, a);
    cmark(ev, 5, stream);
    return hipGetLastError();
}

}  // namespace gdn2
