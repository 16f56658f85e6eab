// Chunk-WY scalar-gate gated delta rule for d_k = d_v = 128 on gfx950 MFMA.
//
// The chunk form is that of gdn2_chunk.hip (per chunk of C = 64 tokens with
// start state S0: A = strict_lower(beta_t Gam_ts k_t.k_s), T = (I + A)^-1,
// R = diag(beta)(V - diag(gam) K S0), delta = T R, O = diag(gam) Q S0 +
// (Gam .* Q K^T) delta, S_C = gam_63 S0 + Ktil^T (U - W S0) with Ktil = lam K,
// W = T diag(beta gam) K, U = T diag(beta) V).  Key-side products reduce over
// all D = 128 key channels; value columns evolve independently, so every
// value-side product is cut into two value blocks of 64 columns, which one
// workgroup per chunk walks in turn after forming the block-independent
// products (gates, A, T, P = Gam . QK^T, W) once:
//   prep   gates, A, T, and the chunk map's factors -W^T, Ktil, U^T, gam_63
//   scan   the factored scan of gdn2_chunk_lr.hip (the map is rank 64 beside
//          its diagonal, so its factors are 64 KiB per chunk against 96 KiB
//          for A_c and B_c)
//   out    per block: delta, O and |delta|^2; then the scores
//   bprep  per block: N of the adjoint map
//   bgrad  per block: the block's contributions to dq, dk, dbeta and dG,
//          summed in registers and LDS; then the masked products, dg and the
//          stores
// Precision follows gdn2_chunk.hip: R, delta, P, dd, dP, W, U and the scan's X
// and V enter their products as bf16 hi + lo pairs; S0, T, Q, K, V, dS and the
// scan's -W and Ktil as bf16, U as f32.
#include "gdn2_chunk_tile.h"

#include <algorithm>

namespace gdn2 {

namespace {

constexpr int KD = WIDE_D;      // key width (= value width)
constexpr int NVB = WIDE_NVB;   // value blocks of 64
constexpr int NKB = KD / 64;    // key blocks of 64
constexpr int LDK = KD + 8;     // bf16 row stride of a 64 x KD tile
constexpr int KTILE = 64 * LDK;
static_assert(NVB == 2 && NKB == 2, "the wide kernels cut D into two blocks of 64");

// Token t's channel pieces [8 cb, 8 cb + 8) and [64 + 8 cb, 72 + 8 cb).
struct Row2 {
    uint4 p[NKB];
};
__device__ __forceinline__ Row2 load_row2(const uint16_t *base, const int64_t *s, int b, int tg,
                                          int h, int cb, bool inb) {
    Row2 r;
#pragma unroll
    for (int i = 0; i < NKB; ++i) r.p[i] = load8(base, s, b, tg, h, cb + 8 * i, inb);
    return r;
}
__device__ __forceinline__ void put_row2(uint16_t *tile, int t, int cb, const Row2 &r) {
#pragma unroll
    for (int i = 0; i < NKB; ++i) put_row8(tile, t, cb + 8 * i, r.p[i], LDK);
}
__device__ __forceinline__ Row2 mask_row2(Row2 r, bool on) {
#pragma unroll
    for (int i = 0; i < NKB; ++i) r.p[i] = mask8(r.p[i], on);
    return r;
}
__device__ __forceinline__ uint4 scale8(uint4 v, float f) {
    Pack8 p;
    p.u = v;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) o[e / 2] = bf16_pack2(f * bf16_val(p.h[e]), f * bf16_val(p.h[e + 1]));
    return make_uint4(o[0], o[1], o[2], o[3]);
}
// f * v as a bf16 hi/lo pair (f * v ~= hi + lo).
__device__ __forceinline__ void scale8_split(uint4 v, float f, uint4 &hi, uint4 &lo) {
    Pack8 p, h, l;
    p.u = v;
#pragma unroll
    for (int e = 0; e < 8; ++e) split_bf16(f * bf16_val(p.h[e]), h.h[e], l.h[e]);
    hi = h.u;
    lo = l.u;
}
__device__ __forceinline__ float sq8(uint4 v) {
    Pack8 p;
    p.u = v;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = bf16_val(p.h[e]);
        s += x * x;
    }
    return s;
}

struct Mat2 {
    uint4 p[NKB];
};
// T at byte offset off (per lane, 32 bits) of a workgroup-uniform base: the
// load takes the scalar-base + 32-bit vector-offset form, one VGPR of address
// per load instead of two.
template <typename Tv>
__device__ __forceinline__ Tv ld_off(const void *base, uint32_t off) {
    return *reinterpret_cast<const Tv *>(static_cast<const char *>(base) + off);
}
__device__ __forceinline__ Mat2 load_mat2(const uint16_t *src, int tid) {
    Mat2 m;
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
        const int p = tid + NT * i, r = p / (KD / 8), c0 = 8 * (p % (KD / 8));
        m.p[i] = ld_off<uint4>(src, 2u * (uint32_t)(r * KD + c0));
    }
    return m;
}
__device__ __forceinline__ void put_mat2(uint16_t *tile, const Mat2 &m, int tid) {
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
        const int p = tid + NT * i, r = p / (KD / 8), c0 = 8 * (p % (KD / 8));
        *reinterpret_cast<uint4 *>(&tile[r * LDK + c0]) = m.p[i];
    }
}

struct WPrepSmem {
    uint16_t ks[KTILE];  // K rows; T (bf16, row stride LDB) once A is formed
    union {
        struct {
            float Af[C * LDF];
            float Tf[C * LDF];
        } inv;
        struct {
            uint16_t kbg[NKB][TILE];   // beta gam K rows (hi), key block kb
            uint16_t kbgl[NKB][TILE];  // their lo parts
            uint16_t vbt[NVB][TILE];  // beta V rows, value block vb
        } wu;                          // once the inverse is done
    } u;
    GateLds gl;
};

}  // namespace

// ---- prep: gates, the UT inverse and the chunk's factored map ------------------
// The chunk map S_C = gam_63 S0 + Ktil^T (U - W S0) (Ktil = lam K, W = T diag(beta
// gam) K, U = T diag(beta) V) leaves as its factors: -W^T and Ktil (bf16), U^T
// (f32) and the diagonal gam_63, with the gate block and T.  One workgroup per
// chunk forms A and T once and W, U for both key and value blocks.
__global__ void __launch_bounds__(NT) wide_prep_kernel(ChunkArgs a) {
    __shared__ WPrepSmem sm;
    uint16_t *Ks = sm.ks, *Tb = sm.ks;  // T over K once A is formed
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tg = c * C + t;
    const int tm = w >> 1, tn0 = 2 * (w & 1);
    const bool inb = tg < a.T;
    const Row2 kraw = load_row2(a.k, a.ks, b, tg, h, cb, inb);
    const Row2 vraw = load_row2(a.v, a.vs, b, tg, h, cb, inb);
    const float vld = inb ? ld4<float>(a.valid, b, tg, 0, 0) : 0.f;
    float rst = 0.f, gt = 0.f, bt = 0.f;
    if (w == 0 && inb) {
        rst = ld4<float>(a.reset, b, tg, 0, 0);
        gt = ld4<float>(a.g, b, tg, h, 0);
        bt = ld4<float>(a.beta, b, tg, h, 0);
    }
    const bool on = vld != 0.f;
    const Row2 k8 = mask_row2(kraw, on), v8 = mask_row2(vraw, on);
    put_row2(Ks, t, cb, k8);
    if (w == 0) {
        const float G = wave_scan_add(on ? gt : 0.f);
        const int seg = wave_scan_add((on && rst != 0.f) ? 1 : 0);
        const float bm = on ? bt : 0.f;
        gates_derive(sm.gl, G, bm, on ? 1.f : 0.f, seg);
        GateBlock *gb = a.ck_gate + ci;
        gb->G[t] = G;
        gb->beta[t] = bm;
        gb->val[t] = on ? 1.f : 0.f;
        gb->seg[t] = seg;
    }
    __syncthreads();
    {  // the map's Ktil = lam K as the K rows (masked, bf16) and lam (after the diagonal)
#pragma unroll
        for (int i = 0; i < NKB; ++i)
            *reinterpret_cast<uint4 *>(a.lr_kt + ((int64_t)ci * C + t) * KD + 64 * i + 8 * cb) = k8.p[i];
        float *gv = a.lr_gv + (int64_t)ci * (KD + C);
        if (tid < KD) gv[tid] = sm.gl.gamC;
        else if (tid < KD + C) gv[tid] = sm.gl.lam[tid - KD];
    }
    // A = strict_lower(beta_t Gam_ts k_t.k_s) in f32 (tiles with tn <= tm only).
    if (tn0 <= tm) {
        f32x4 kk[2] = {zero4(), zero4()};
        gemm2<KD, LDK, LDK>(kk, &Ks[(16 * tm) * LDK], Ks, tn0);
        const RowGates rg = row_gates(sm.gl, tm);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                sm.u.inv.Af[tt * LDF + ss] = (ss < tt && rg.seg[i] == sgs)
                                                 ? rg.beta[i] * __expf(rg.G[i] - Gs) * kk[j][i]
                                                 : 0.f;
            }
        }
    }
    __syncthreads();
    ut_inverse(sm.u.inv.Af, sm.u.inv.Tf, w);
    {  // T (bf16, row-major, zero above the diagonal): LDS operand and checkpoint
        const int r = tid >> 3, c0 = 8 * (tid & 7);
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s0 = c0 + 2 * e;
            pk[e] = bf16_pack2(s0 <= r ? sm.u.inv.Tf[r * LDF + s0] : 0.f,
                               s0 + 1 <= r ? sm.u.inv.Tf[r * LDF + s0 + 1] : 0.f);
        }
        const uint4 v = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *reinterpret_cast<uint4 *>(a.ck_t + (int64_t)ci * C * C + r * C + c0) = v;
        *reinterpret_cast<uint4 *>(&Tb[r * LDB + c0]) = v;
    }
    __syncthreads();  // T read out of the inverse's scratch: beta gam K and beta V take it
    {
        const float bg = sm.gl.beta[t] * sm.gl.gam[t], be = sm.gl.beta[t];
#pragma unroll
        for (int i = 0; i < NKB; ++i) {
            uint4 kh, kl;
            scale8_split(k8.p[i], bg, kh, kl);
            put_row8(sm.u.wu.kbg[i], t, cb, kh);
            put_row8(sm.u.wu.kbgl[i], t, cb, kl);
            put_row8(sm.u.wu.vbt[i], t, cb, scale8(v8.p[i], be));
        }
    }
    __syncthreads();
    // W = T (beta gam K), U = T (beta V), block by block, straight from the
    // accumulators: -W^T (bf16) and U^T (f32), [column][token].
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
        f32x4 x[2] = {zero4(), zero4()}, y[2] = {zero4(), zero4()};
        gemm2_tr(x, &Tb[(16 * tm) * LDB], sm.u.wu.kbg[i], tn0);
        gemm2_tr(x, &Tb[(16 * tm) * LDB], sm.u.wu.kbgl[i], tn0);
        gemm2_tr(y, &Tb[(16 * tm) * LDB], sm.u.wu.vbt[i], tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t o = ((int64_t)ci * KD + 64 * i + 16 * (tn0 + j) + acc_col()) * C + 16 * tm + acc_row(0);
            *reinterpret_cast<uint2 *>(a.lr_wt + o) =
                make_uint2(bf16_pack2(-x[j][0], -x[j][1]), bf16_pack2(-x[j][2], -x[j][3]));
            *reinterpret_cast<float4 *>(a.lr_u + o) = make_float4(y[j][0], y[j][1], y[j][2], y[j][3]);
        }
    }
}

// ---- out: outputs, edits, their norms and the scores -----------------------------
// Q, K, T and P = Gam . QK^T once per chunk; R, delta and O for each value block
// in turn; the scores from both blocks' |delta|^2.  One workgroup per CU walks
// chunks blockIdx.x, blockIdx.x + gridDim.x, ...: the next chunk's inputs are
// loaded into registers while the current one computes, and the last block's
// stores are issued after the next chunk's staging, so that no chunk waits on
// its loads (or the previous chunk's stores) but a workgroup's first.
namespace {
struct WOutSmem {
    uint16_t q[KTILE];   // Q rows
    uint16_t k[KTILE];   // K rows
    uint16_t st[KTILE];  // S0^T rows of block vb ([v][k])
    uint16_t vt[TILE];   // V_vb^T, then R^T lo
    uint16_t rt[TILE];   // R^T hi
    uint16_t tb[TILE];   // T rows
    uint16_t pt[TILE], ptl[TILE];  // P^T hi/lo
    uint16_t dt[TILE], dl[TILE];   // delta^T hi/lo of block vb; S0^T lo rows of block vb before phase 2
    float df[C * LDF];             // delta rows (f32) of block vb, for the checkpoint
    uint16_t os[TILE];             // O rows of block vb (bf16 output)
    GateLds gl;
    float kk[NW][C];
    float dd[NVB][2][C];
};

// One chunk's inputs: rows past the sequence end read the last row (the gate
// block marks those tokens invalid and the staging zeroes them), so the loads
// take no branch and the compiler's memory-counter waits stay exact.
struct WOutIn {
    Row2 q, k;
    uint4 v[NVB];
    Mat2 s0[NVB], s0l[NVB];  // S0^T rows, bf16 hi and lo
    uint4 t;
    float G, be, va;
    int sg;
};
// Part P: 0 q, k; 1 V and S0 of block 0; 2 T and the gates; 3 V and S0 of block 1.
template <int P>
__device__ __forceinline__ void wout_load(const ChunkArgs &a, int ci, int tid, WOutIn &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tg = c * C + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    if constexpr (P == 0) {
        x.q = load_row2(a.q, a.qs, b, tr, h, cb, true);
        x.k = load_row2(a.k, a.ks, b, tr, h, cb, true);
    } else if constexpr (P == 1 || P == 3) {
        constexpr int vb = P == 1 ? 0 : 1;
        x.v[vb] = load8(a.v + 64 * vb, a.vs, b, tr, h, cb, true);
        x.s0[vb] = load_mat2(a.ck_state + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
        x.s0l[vb] = load_mat2(a.ck_state_lo + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
    } else {
        x.t = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
        const GateBlock *gb = a.ck_gate + ci;
        x.G = gb->G[t], x.be = gb->beta[t], x.va = gb->val[t];
        x.sg = gb->seg[t];
    }
}

// Value block vb's delta rows (checkpoint) and, for bf16 output, O rows.
__device__ __forceinline__ void wout_store(const ChunkArgs &a, int ci, int vb, int tid, const WOutSmem &sm) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int r = tid >> 3, c0 = 8 * (tid & 7), tq = c * C + r;
    float *dck = a.ck_delta + (int64_t)ci * C * KD + r * KD + 64 * vb + c0;
    *reinterpret_cast<float4 *>(dck) = *reinterpret_cast<const float4 *>(&sm.df[r * LDF + c0]);
    *reinterpret_cast<float4 *>(dck + 4) = *reinterpret_cast<const float4 *>(&sm.df[r * LDF + c0 + 4]);
    if (a.out_bf16 && tq < a.T)
        *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.out) + (((int64_t)b * a.T + tq) * a.H + h) * KD +
                                   64 * vb + c0) = *reinterpret_cast<const uint4 *>(&sm.os[r * LDB + c0]);
}

// Wave 0's per-token terms of a chunk (lane == token): |k_t|^2, each block's
// |delta_t|^2 and the score |k_t| |delta_t| (0 on padding).
struct WOutTok {
    float kk, dd[NVB], score;
};
__device__ __forceinline__ void wout_store_tok(const ChunkArgs &a, int ci, const WOutTok &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = lane_id(), tg = c * C + t;
    a.ck_kk[(int64_t)ci * C + t] = x.kk;
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) a.ck_ddp[((int64_t)ci * NVB + vb) * C + t] = x.dd[vb];
    if (tg < a.T) a.scores[((int64_t)b * a.T + tg) * a.H + h] = x.score;
}
}  // namespace

__global__ void __launch_bounds__(NT) wide_out_kernel(ChunkArgs a, int nchunks) {
    __shared__ WOutSmem sm;
    uint16_t *Qs = sm.q, *Ks = sm.k, *Vt = sm.vt, *Tb = sm.tb, *St = sm.st, *Rt = sm.rt;
    uint16_t *Pt = sm.pt, *Ptl = sm.ptl, *Dt = sm.dt, *Dl = sm.dl;
    // S0^T lo rows of the current block over delta^T's tiles, which phase 1 does not use.
    uint16_t *Sl = sm.dt;
    static_assert(sizeof(sm.dt) + sizeof(sm.dl) >= sizeof(sm.st), "S0^T lo over dt, dl");
    WOutIn in;
    wout_load<0>(a, blockIdx.x, threadIdx.x, in);
    wout_load<1>(a, blockIdx.x, threadIdx.x, in);
    wout_load<2>(a, blockIdx.x, threadIdx.x, in);
    wout_load<3>(a, blockIdx.x, threadIdx.x, in);
    WOutTok tok{};  // wave 0: the previous chunk's per-token terms
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the lane- and wave-dependent address arithmetic inside
    // the loop (hoisted, it would stay live across it and exhaust the registers).
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, t0 = c * C;
    const int tm = w >> 1, tn0 = 2 * (w & 1);
    // The next chunk.  Past the end the loads need no branch either: every lane
    // addresses this chunk as thread 0 would, so each load instruction touches
    // a line or two that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    const bool on = in.va != 0.f;
    {
        const Row2 k8 = mask_row2(in.k, on);
        put_row2(Qs, t, cb, mask_row2(in.q, on));
        put_row2(Ks, t, cb, k8);
        put_col8(Vt, t, cb, mask8(in.v[0], on));
        put_mat2(St, in.s0[0], tid);
        put_mat2(Sl, in.s0l[0], tid);
        *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.t;
        float ksq = 0.f;
#pragma unroll
        for (int i = 0; i < NKB; ++i) ksq += sq8(k8.p[i]);
        sm.kk[cb][t] = ksq;
        if (w == 0) gates_derive(sm.gl, in.G, in.be, in.va, in.sg);
    }
    if (ci != (int)blockIdx.x) {  // the previous chunk's last block and token terms
        wout_store(a, ci - gridDim.x, NVB - 1, tid, sm);
        if (w == 0) wout_store_tok(a, ci - gridDim.x, tok);
    }
    wout_load<0>(a, cn, tn, in);
    __syncthreads();
    wout_load<1>(a, cn, tn, in);
    const RowGates rg = row_gates(sm.gl, tm);
    {  // P = Gam . QK^T (causal tiles) -> P^T hi/lo, once for both blocks
        f32x4 pq[2] = {zero4(), zero4()};
        if (tn0 <= tm) gemm2<KD, LDK, LDK>(pq, &Qs[(16 * tm) * LDK], Ks, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                pq[j][i] *= (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
            }
            store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq[j]);
        }
    }
#pragma unroll 1
    for (int vb = 0; vb < NVB; ++vb) {
        // Phase 1: R (-> Rt, lo over Vt) and gam Q S0 kept in registers; S0 as
        // hi + lo.
        f32x4 qs[2] = {zero4(), zero4()};
        {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2<KD, LDK, LDK>(x, &Ks[(16 * tm) * LDK], St, tn0);
            gemm2<KD, LDK, LDK>(qs, &Qs[(16 * tm) * LDK], St, tn0);
            gemm2<KD, LDK, LDK>(x, &Ks[(16 * tm) * LDK], Sl, tn0);
            gemm2<KD, LDK, LDK>(qs, &Qs[(16 * tm) * LDK], Sl, tn0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint16_t *vt = &Vt[(16 * (tn0 + j)) * LDB + 16 * tm];
                float vv[4];
                ld4_bf16(vt + acc_col() * LDB + 4 * (lane_id() >> 4), vv);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[j][i] = rg.beta[i] * (vv[i] - rg.gam[i] * x[j][i]);
                    qs[j][i] *= rg.gam[i];
                }
                store_tile_t_split(&Rt[(16 * (tn0 + j)) * LDB + 16 * tm], vt, LDB, x[j]);
            }
        }
        if (vb == 0) wout_load<2>(a, cn, tn, in);
        __syncthreads();
        // Phase 2: delta = T R (-> Dt/Dl) and |delta_t|^2 of the block.
        f32x4 dlt[2] = {zero4(), zero4()};
        {
            gemm2(dlt, &Tb[(16 * tm) * LDB], Rt, tn0);
            gemm2(dlt, &Tb[(16 * tm) * LDB], Vt, tn0);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = dlt[0][i] * dlt[0][i] + dlt[1][i] * dlt[1][i];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                store_tile_t_split(&Dt[(16 * (tn0 + j)) * LDB + 16 * tm],
                                   &Dl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, dlt[j]);
            row_reduce_store(p, sm.dd[vb][w & 1], tm);
        }
        __syncthreads();
        if (vb == NVB - 1 && w == 0) {  // the chunk's token terms, stored after the next staging
            float kk = 0.f, dd = 0.f;
#pragma unroll
            for (int q = 0; q < NW; ++q) kk += sm.kk[q][t];
            tok.kk = kk;
#pragma unroll
            for (int v2 = 0; v2 < NVB; ++v2) {
                tok.dd[v2] = sm.dd[v2][0][t] + sm.dd[v2][1][t];
                dd += tok.dd[v2];
            }
            tok.score = sm.gl.val[t] != 0.f ? sqrtf(kk * dd) : 0.f;
        }
        // delta (f32 rows) and O = gam Q S0 + P delta into their own tiles.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                sm.df[(16 * tm + acc_row(i)) * LDF + 16 * (tn0 + j) + acc_col()] = dlt[j][i];
        {
            f32x4 x[2] = {qs[0], qs[1]};
            gemm2_atr(x, Pt, 16 * tm, Dt, tn0);
            gemm2_atr(x, Pt, 16 * tm, Dl, tn0);
            gemm2_atr(x, Ptl, 16 * tm, Dt, tn0);
            if (a.out_bf16) {
#pragma unroll
                for (int j = 0; j < 2; ++j) store_tile_rm(&sm.os[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, x[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tq = t0 + 16 * tm + acc_row(i);
                        if (tq < a.T)
                            reinterpret_cast<float *>(a.out)[(((int64_t)b * a.T + tq) * a.H + h) * KD +
                                                             64 * vb + 16 * (tn0 + j) + acc_col()] = x[j][i];
                    }
            }
        }
        __syncthreads();  // delta and O rows complete; V, S0 and R of the block read
        if (vb == 0) {
            // Block 0's stores; block 1's V and S0 (loaded one chunk ahead) staged.
            wout_store(a, ci, 0, tid, sm);
            put_col8(Vt, t, cb, mask8(in.v[1], on));
            put_mat2(St, in.s0[1], tid);
            put_mat2(Sl, in.s0l[1], tid);
            wout_load<3>(a, cn, tn, in);
            __syncthreads();
        }
    }
    }
    {
        const int tid = threadIdx.x;
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        wout_store(a, last, NVB - 1, tid, sm);
        if ((tid >> 6) == 0) wout_store_tok(a, last, tok);
    }
}

// ---- backward prep: N of the adjoint map ---------------------------------------
// dS0 = M dS_C + N with M = A_c^T and N = Y - W^T X, Y = (gam Q)^T dO,
// X = P^T dO + diag(c) delta, W = T diag(beta gam) K (formed again from T and K
// with prep's operands and products).  One workgroup per chunk: W and P once,
// Y, X and N for both value blocks.
namespace {
struct WBPrepSmem {
    uint16_t q[KTILE], k[KTILE];  // Q, K rows; X^T hi/lo of block 0 (row stride LDB) from phase 2
    union {
        struct {
            uint16_t tb[TILE];    // T rows
            uint16_t kbg[KTILE];  // beta gam K rows (hi)
            uint16_t kbgl[KTILE];  // their lo parts
        } p1;
        uint16_t wt[2][KD * LDB];  // W^T hi/lo ([k][t]) from phase 2
    } u;
    uint16_t dos[NVB][TILE];       // dO rows of each block; X^T hi/lo of block 1 from phase 2
    uint16_t pt[TILE], ptl[TILE];  // P^T hi/lo
    GateLds gl;
    float dsc[C];
};
}  // namespace

// One chunk's inputs to bprep (rows past the sequence end read the last row; a
// missing dO reads q and a missing score adjoint the delta checkpoint, which
// holds more than B*T*H floats; the staging zeroes what is not used), so the
// loads take no branch.  Part P: 0 q, k; 1 dO; 2 T, the gates, the score adjoint.
struct WBPrepIn {
    Row2 q, k;
    uint4 dO[NVB];
    uint4 t;
    float G, be, va, dsc;
    int sg;
};
template <int P>
__device__ __forceinline__ void wbprep_load(const ChunkArgs &a, int ci, int tid, WBPrepIn &x) {
    const int bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tg = c * C + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    if constexpr (P == 0) {
        x.q = load_row2(a.q, a.qs, b, tr, h, cb, true);
        x.k = load_row2(a.k, a.ks, b, tr, h, cb, true);
    } else if constexpr (P == 1) {
        const uint16_t *dop = a.dout ? a.dout : a.q;
        const int64_t *dos = a.dout ? a.ds : a.qs;
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) x.dO[vb] = load8(dop + 64 * vb, dos, b, tr, h, cb, true);
    } else {
        x.t = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
        const GateBlock *gb = a.ck_gate + ci;
        x.G = gb->G[t], x.be = gb->beta[t], x.va = gb->val[t];
        x.sg = gb->seg[t];
        x.dsc = (a.dscores ? a.dscores : a.ck_delta)[((int64_t)b * a.T + tr) * a.H + h];
    }
}

// N of chunk ci from the registers it was formed in (transposed: Nt[col][row]).
__device__ __forceinline__ void wbprep_store(const ChunkArgs &a, int ci, int tm, int tn0,
                                             const f32x4 (&n)[NVB][NKB][2]) {
    float *Nt = a.ws_n + (int64_t)ci * KD * KD;
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<float4 *>(&Nt[(64 * vb + 16 * (tn0 + j) + acc_col()) * KD + 16 * (tm + 4 * kb) +
                                                acc_row(0)]) =
                    make_float4(n[vb][kb][j][0], n[vb][kb][j][1], n[vb][kb][j][2], n[vb][kb][j][3]);
}

// One workgroup per CU walks chunks blockIdx.x, blockIdx.x + gridDim.x, ...; the
// next chunk's inputs are loaded into registers while the current one computes,
// and a chunk's N (formed in the registers of Y) is stored after the next
// chunk's staging, so that no chunk but a workgroup's first waits on its loads
// or on the previous chunk's stores.
// SCORE: a score adjoint is given (the c delta term and its norms are compiled
// in only then).
template <bool SCORE>
__global__ void __launch_bounds__(NT) wide_bprep_kernel(ChunkArgs a, int nchunks) {
    __shared__ WBPrepSmem sm;
    uint16_t *Qs = sm.q, *Ks = sm.k, *Tb = sm.u.p1.tb, *KBGs = sm.u.p1.kbg, *KBGl = sm.u.p1.kbgl;
    uint16_t *Pt = sm.pt, *Ptl = sm.ptl;
    uint16_t *Wt = sm.u.wt[0], *Wtl = sm.u.wt[1];  // over the phase-1 operands
    // X^T hi/lo of each block, over Q/K (block 0) and the dO rows (block 1) after phase 2
    uint16_t *Xt[NVB] = {sm.q, sm.dos[0]}, *Xtl[NVB] = {sm.k, sm.dos[1]};
    constexpr bool score_adj = SCORE;
    WBPrepIn in;
    wbprep_load<0>(a, blockIdx.x, threadIdx.x, in);
    wbprep_load<1>(a, blockIdx.x, threadIdx.x, in);
    wbprep_load<2>(a, blockIdx.x, threadIdx.x, in);
    // Y, then N = Y - W^T X in place; held until the next chunk's staging is done.
    f32x4 yacc[NVB][NKB][2];
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the lane- and wave-dependent address arithmetic inside
    // the loop (hoisted, it would stay live across it and exhaust the registers).
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);
    const float *dck = a.ck_delta + (int64_t)ci * C * KD;
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    // The next chunk.  Past the end the loads need no branch either: every lane
    // addresses this chunk as thread 0 would, so each load instruction touches
    // a line or two that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    {
        const bool on = in.va != 0.f;
        const float gam = in.sg == 0 ? __expf(in.G) : 0.f, bg = in.be * gam;
        const Row2 q8 = mask_row2(in.q, on), k8 = mask_row2(in.k, on);
        put_row2(Qs, t, cb, q8);
        put_row2(Ks, t, cb, k8);
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) put_row8(sm.dos[vb], t, cb, mask8(in.dO[vb], on && a.dout));
#pragma unroll
        for (int i = 0; i < NKB; ++i) {
            uint4 kh, kl;
            scale8_split(k8.p[i], bg, kh, kl);
            put_row8(KBGs, t, cb + 8 * i, kh, LDK);
            put_row8(KBGl, t, cb + 8 * i, kl, LDK);
        }
        *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.t;
        if (w == 0) {
            gates_derive(sm.gl, in.G, in.be, in.va, in.sg);
            sm.dsc[t] = score_adj ? in.dsc : 0.f;
        }
    }
    if (ci != (int)blockIdx.x) wbprep_store(a, ci - gridDim.x, tm, tn0, yacc);  // the previous chunk's N
    wbprep_load<0>(a, cn, tn, in);
    __syncthreads();
    wbprep_load<1>(a, cn, tn, in);
    const RowGates rg = row_gates(sm.gl, tm);
    // Phase 1: W = T (beta gam K) and both blocks' Y = (gam Q)^T dO in registers; P^T hi/lo.
    f32x4 wacc[NKB][2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        wacc[kb][0] = wacc[kb][1] = zero4();
        gemm2_tr<64, LDB, LDK>(wacc[kb], &Tb[(16 * tm) * LDB], KBGs, tn0 + 4 * kb);
        gemm2_tr<64, LDB, LDK>(wacc[kb], &Tb[(16 * tm) * LDB], KBGl, tn0 + 4 * kb);
        const int mt = tm + 4 * kb;  // row tile of Y (key channel)
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) yacc[vb][kb][0] = yacc[vb][kb][1] = zero4();
#pragma unroll
        for (int r = 0; r < 64; r += 32) {  // Y[k][v] = sum_t (gam Q)[t][k] dO[t][v], gam Q hi/lo
            bf16x8_t x, xl;
            frag_tr_scaled_split<LDK>(Qs, sm.gl.gam, r, 16 * mt, x, xl);
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const bf16x8_t ob = frag_tr(sm.dos[vb], r, 16 * (tn0 + j));
                    yacc[vb][kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, ob, yacc[vb][kb][j], 0, 0, 0);
                    yacc[vb][kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, ob, yacc[vb][kb][j], 0, 0, 0);
                }
        }
    }
    {
        f32x4 pq[2] = {zero4(), zero4()};
        if (tn0 <= tm) gemm2<KD, LDK, LDK>(pq, &Qs[(16 * tm) * LDK], Ks, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                pq[j][i] *= (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
            }
            store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq[j]);
        }
    }
    __syncthreads();
    wbprep_load<2>(a, cn, tn, in);
    // Phase 2: W^T hi/lo; both blocks' X = P^T dO + diag(c) delta in registers, then
    // stored transposed (hi/lo) once every wave has read the dO rows.
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile_t_split(&Wt[(16 * (tn0 + 4 * kb + j)) * LDB + 16 * tm],
                               &Wtl[(16 * (tn0 + 4 * kb + j)) * LDB + 16 * tm], LDB, wacc[kb][j]);
    f32x4 xx[NVB][2];
    float cs[4] = {0.f, 0.f, 0.f, 0.f};
    if (score_adj) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ss = r0 + i;
            float dq = 0.f;
#pragma unroll
            for (int v2 = 0; v2 < NVB; ++v2) dq += a.ck_ddp[((int64_t)ci * NVB + v2) * C + ss];
            const float nk = sqrtf(a.ck_kk[(int64_t)ci * C + ss]), nd = sqrtf(dq);
            cs[i] = (nk > 0.f && nd > 0.f) ? sm.dsc[ss] * nk / nd : 0.f;
        }
    }
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
        xx[vb][0] = xx[vb][1] = zero4();
        gemm2_tr(xx[vb], &Pt[(16 * tm) * LDB], sm.dos[vb], tn0);  // B[v][t] = dO[t][v]
        gemm2_tr(xx[vb], &Ptl[(16 * tm) * LDB], sm.dos[vb], tn0);
        if (score_adj) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xx[vb][j][i] += cs[i] * dck[(r0 + i) * KD + 64 * vb + 16 * (tn0 + j) + acc_col()];
        }
    }
    __syncthreads();  // Q, K and dO rows read: X^T takes their tiles
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile_t_split(&Xt[vb][(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Xtl[vb][(16 * (tn0 + j)) * LDB + 16 * tm], LDB, xx[vb][j]);
    __syncthreads();
    // Phase 3: N = Y - W^T X, both blocks' 64 columns, all KD rows, in Y's registers.
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const int mt = tm + 4 * kb;
            f32x4 x[2] = {zero4(), zero4()};
            gemm2(x, &Wt[(16 * mt) * LDB], Xt[vb], tn0);
            gemm2(x, &Wt[(16 * mt) * LDB], Xtl[vb], tn0);
            gemm2(x, &Wtl[(16 * mt) * LDB], Xt[vb], tn0);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) yacc[vb][kb][j][e] -= x[j][e];
        }
    __syncthreads();  // W^T and X^T read: the next chunk's staging takes their tiles
    }
    {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        wbprep_store(a, last, w >> 1, 2 * (w & 1), yacc);
    }
}

// ---- bgrad: every gradient of one chunk ------------------------------------------
// The phases of gdn2_chunk.hip's gradient kernel with the value side cut into
// the two value blocks of 64 columns, which one workgroup walks in turn.  What
// does not depend on the values (gates, T, KK^T, QK^T and P) is formed once.
// What a value block contributes to dq, dk, dbeta and dG is a sum over its
// columns and stays in registers across the blocks: dO S0^T, the dK terms, dA
// and dP before their masks, and the row-sum partials.  The masked dA and dP,
// their products with K and Q (phase G), the dG reverse scan and the dq/dk
// stores then run once.
namespace {
struct WBGradSmem {
    uint16_t q[KTILE];    // Q rows
    uint16_t k[KTILE];    // K rows
    uint16_t s0t[KTILE];  // S0^T rows of block vb; with dos: dK^T [KD][LDB] after the blocks
    uint16_t dos[TILE];   // dO rows of block vb
    uint16_t dst[KTILE];  // dS^T rows of block vb (A..D); dR rows (E..F)
    uint16_t vr[TILE];    // V rows of block vb (..E); the last block's dV^T (F..)
    uint16_t tr[TILE];    // T rows; MA^T (F..G)
    uint16_t dh[TILE], dlo[TILE];  // delta rows hi/lo of block vb (..F); dQ^T [KD][LDB] over both at the end
    uint16_t pt[TILE], ptl[TILE];  // P^T hi/lo (until read into registers); ddelta^T (D..E);
                                   // block 0's dV^T over pt (its F .. block 1's D) and dR lo
                                   // rows over ptl (F); MP^T (after the blocks)
    uint16_t xl[KTILE];            // dS^T lo rows of block vb (A..D); S0^T lo rows (F)
    GateLds gl;
    float dsc[C];
    float g1[2][C], ku[2][C], b1[2][C], b2[2][C], zr[2][C], zc[4][C], dlam[2][C];
    float frob[NW];
};

// A value block's inputs as loaded: dO, S0^T and dS^T rows, V, delta (f32).
struct VbRaw {
    uint4 dor, vr;
    Mat2 s0, ds, dsl;  // S0^T rows (hi), dS^T rows (hi and lo)
    float4 d0, d1;
};
}  // namespace

// SCORE: a score adjoint is given (its terms c delta and c' k and the norms
// behind them are compiled in only then; without it they would hold registers
// that the kernel has none to spare for).
template <bool SCORE>
__global__ void __launch_bounds__(NT) wide_bgrad_kernel(ChunkArgs a) {
    __shared__ WBGradSmem sm;
    uint16_t *Qs = sm.q, *Ks = sm.k, *dOs = sm.dos, *S0t = sm.s0t, *dSt = sm.dst;
    uint16_t *Vr = sm.vr, *Tr = sm.tr, *Dh = sm.dh, *Dlo = sm.dlo, *Pt = sm.pt, *Ptl = sm.ptl;
    uint16_t *Dd = sm.pt, *Ddl = sm.ptl;  // ddelta^T, D..E
    uint16_t *dRr = sm.dst;               // dR rows, E..F
    uint16_t *MAt = sm.tr, *MPt = sm.pt, *MPtl = sm.ptl;
    uint16_t *dQt = sm.dh, *dKt = sm.s0t;
    uint16_t *Xl = sm.xl;  // dS^T lo (A..D), then S0^T lo (E..F)
    uint16_t *dRl = sm.ptl;  // dR rows' lo part (F): ddelta^T lo is read by then
    // dV^T of a block ([value][token]): block 0 over P^T's tiles (free from its
    // phase F until block 1's phase D), block 1 over its V rows (free after E).
    auto dVt = [&](int vb) { return vb == 0 ? sm.pt : sm.vr; };
    static_assert(sizeof(sm.dh) + sizeof(sm.dlo) >= KD * LDB * 2, "dQ^T over dh, dlo");
    static_assert(sizeof(sm.s0t) + sizeof(sm.dos) >= KD * LDB * 2, "dK^T over s0t, dos");
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);
    const int tg = c * C + t;
    const bool inb = tg < a.T;
    const GateBlock *gb = a.ck_gate + ci;
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    auto load_vb = [&](int vb, VbRaw &r) {
        const float *dck = a.ck_delta + (int64_t)ci * C * KD + 64 * vb;
        r.dor = a.dout ? load8(a.dout + 64 * vb, a.ds, b, tg, h, cb, inb) : make_uint4(0, 0, 0, 0);
        r.s0 = load_mat2(a.ck_state + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
        r.ds = load_mat2(a.ws_dstate + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
        r.dsl = load_mat2(a.ws_dstate_lo + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
        r.vr = load8(a.v + 64 * vb, a.vs, b, tg, h, cb, inb);
        r.d0 = ld_off<float4>(dck, 4u * (uint32_t)(t * KD + 8 * cb));
        r.d1 = ld_off<float4>(dck, 4u * (uint32_t)(t * KD + 8 * cb + 4));
    };
    const Row2 qr = load_row2(a.q, a.qs, b, tg, h, cb, inb);
    const Row2 kr = load_row2(a.k, a.ks, b, tg, h, cb, inb);
    VbRaw raw;
    load_vb(0, raw);
    const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
    const int sg = gb->seg[t];
    const float dsc = (a.dscores && inb && w == 0) ? a.dscores[((int64_t)b * a.T + tg) * a.H + h] : 0.f;
    constexpr bool score_adj = SCORE;
    const uint4 trw = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C +
                                                      (tid >> 3) * C + 8 * (tid & 7));
    const bool on = va != 0.f;
    float frob = 0.f;  // this thread's part of <S0, dS> over both blocks
    // A block's dO, S0^T and dS^T rows (hi; dS^T lo over xl) into LDS (the first
    // stage of each block); S0^T lo comes in phase E.
    auto stage_vb_a = [&](const VbRaw &r) {
        put_row8(dOs, t, cb, mask8(r.dor, on));
        put_mat2(S0t, r.s0, tid);
        put_mat2(dSt, r.ds, tid);
        put_mat2(Xl, r.dsl, tid);
#pragma unroll
        for (int i = 0; i < NKB; ++i)
            frob += dot8_bf16(r.s0.p[i], r.ds.p[i]) + dot8_bf16(r.s0.p[i], r.dsl.p[i]);
    };
    // A block's V rows and delta rows (hi/lo): read from phase D on.
    auto stage_vb_b = [&](const VbRaw &r) {
        put_row8(Vr, t, cb, mask8(r.vr, on));
        const float x[8] = {r.d0.x, r.d0.y, r.d0.z, r.d0.w, r.d1.x, r.d1.y, r.d1.z, r.d1.w};
        Pack8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; ++e) split_bf16(x[e], ph.h[e], pl.h[e]);
        put_row8(Dh, t, cb, ph.u);
        put_row8(Dlo, t, cb, pl.u);
    };
    put_row2(Qs, t, cb, mask_row2(qr, on));
    put_row2(Ks, t, cb, mask_row2(kr, on));
    *reinterpret_cast<uint4 *>(&Tr[(tid >> 3) * LDB + 8 * (tid & 7)]) = trw;
    stage_vb_a(raw);
    stage_vb_b(raw);
    if (w == 0) {
        gates_derive(sm.gl, G, be, va, sg);
        sm.dsc[t] = dsc;
    }
    __syncthreads();
    // lam, beta and gam at this lane's rows, read from LDS where they are used (held
    // in registers across the block loop, they would spill).
    auto row4 = [&](const float *v) {
        const float4 x = lds_f4(&v[r0]);
        return f32x4{x.x, x.y, x.z, x.w};
    };
    float cs[4] = {0.f, 0.f, 0.f, 0.f}, ck[4] = {0.f, 0.f, 0.f, 0.f};
    if (score_adj) {  // c and c' from the forward's |k|^2 and both blocks' |delta|^2
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ss = r0 + i;
            float dq = 0.f;
#pragma unroll
            for (int v2 = 0; v2 < NVB; ++v2) dq += a.ck_ddp[((int64_t)ci * NVB + v2) * C + ss];
            const float nk = sqrtf(a.ck_kk[(int64_t)ci * C + ss]), nd = sqrtf(dq);
            const bool ok = nk > 0.f && nd > 0.f;
            cs[i] = ok ? sm.dsc[ss] * nk / nd : 0.f;
            ck[i] = ok ? sm.dsc[ss] * nd / nk : 0.f;
        }
    }
    // The Gam mask at this wave's tiles (formed here and again after the blocks).
    auto gam_mask = [&](float (&gm)[2][4]) {
        const RowGates rg = row_gates(sm.gl, tm);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                gm[j][i] = (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
            }
        }
    };
    // P = Gam . QK^T, transposed (hi/lo) -> LDS, read by each block's phase D.
    // Formed again for the second block (its tiles hold the first block's
    // ddelta^T and dV^T in between): held in registers across the block loop,
    // its fragments would spill.
    auto stage_p = [&]() {
        float gm[2][4];
        gam_mask(gm);
        f32x4 qk[2] = {zero4(), zero4()};
        if (tn0 <= tm) gemm2<KD, LDK, LDK>(qk, &Qs[(16 * tm) * LDK], Ks, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f32x4 pq;
#pragma unroll
            for (int i = 0; i < 4; ++i) pq[i] = qk[j][i] * gm[j][i];
            store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq);
        }
    };
    stage_p();
    __syncthreads();
    // Sums over both blocks, in registers: dO S0^T (-> dQ), the dK terms, dA and
    // dP before their masks, and the row-sum partials of the gate gradients.
    f32x4 dos[NKB][2], dka[NKB][2], da[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) dos[kb][0] = dos[kb][1] = dka[kb][0] = dka[kb][1] = zero4();
    da[0] = da[1] = dp[0] = dp[1] = zero4();
    // A block's dV rows out of its staged transposed tile: lane (token 16 (w%4) +
    // l%16, values 32 (w/4) + 8 (l/16) ..) stores one 16-byte piece.
    auto dv_out = [&](int vb) {
        const int l = lane_id(), tq = c * C + 16 * (w & 3) + (l & 15);
        const bf16x8_t gv = frag_tr(dVt(vb), 32 * (w >> 2), 16 * (w & 3));
        if (tq < a.T && a.dv)
            *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dv) +
                                          (((int64_t)b * a.T + tq) * a.H + h) * KD + 64 * vb +
                                          32 * (w >> 2) + 8 * (l >> 4)) = gv;
    };
    // Rolled: unrolled, the second block's loads are hoisted into the first
    // block's phases and the registers spill.
#pragma unroll 1
    for (int vb = 0; vb < NVB; ++vb) {
        if (vb > 0) {
            load_vb(1, raw);  // vb == 1: a constant block, so the addresses stay scalar
            __syncthreads();  // the previous block's phase F has read dO, S0^T, dR and delta
            dv_out(vb - 1);
            stage_vb_a(raw);
            stage_vb_b(raw);
            __syncthreads();  // the first block's dV^T is out of P's tiles
            stage_p();
            __syncthreads();
        }
        // Phase A: dO S0^T (key tiles of both key blocks), lam K dS.  Row-sum
        // partials of the gate gradients add into their LDS rows block by block.
        f32x4 kds[2] = {zero4(), zero4()};
        float pg1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2_tr<64, LDB, LDK>(x, &dOs[(16 * tm) * LDB], S0t, tn0 + 4 * kb);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float qv[4];
                ld4_rm_tr<LDK>(Qs, 16 * tm, 16 * (tn0 + 4 * kb + j), qv);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pg1[i] += qv[i] * x[j][i];  // q_t . (dO S0^T)_t
                    dos[kb][j][i] += x[j][i];
                }
            }
        }
        row_reduce_accum(pg1, sm.g1[w & 1], tm, vb > 0);
        gemm2<KD, LDK, LDK>(kds, &Ks[(16 * tm) * LDK], dSt, tn0);
        gemm2<KD, LDK, LDK>(kds, &Ks[(16 * tm) * LDK], Xl, tn0);
        {
            const f32x4 lmv = row4(sm.gl.lam);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) kds[j][i] *= lmv[i];
        }
        // Phase D: delta dS^T (-> dlam, dK), ddelta = P^T dO + lam K dS + c delta.
        f32x4 xd[2] = {kds[0], kds[1]};
        float pdl[4] = {0.f, 0.f, 0.f, 0.f};
        const f32x4 lmv = row4(sm.gl.lam);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2_tr<64, LDB, LDK>(x, &Dh[(16 * tm) * LDB], dSt, tn0 + 4 * kb);
            gemm2_tr<64, LDB, LDK>(x, &Dlo[(16 * tm) * LDB], dSt, tn0 + 4 * kb);
            gemm2_tr<64, LDB, LDK>(x, &Dh[(16 * tm) * LDB], Xl, tn0 + 4 * kb);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float kv[4];
                ld4_rm_tr<LDK>(Ks, 16 * tm, 16 * (tn0 + 4 * kb + j), kv);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pdl[i] += kv[i] * x[j][i];
                    dka[kb][j][i] += lmv[i] * x[j][i];
                }
            }
        }
        row_reduce_accum(pdl, sm.dlam[w & 1], tm, vb > 0);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            // this wave's rows of P^T (hi, lo): the A operand of P^T dO
            const bf16x8_t ph = frag(&Pt[(16 * tm) * LDB], LDB, 32 * k2);
            const bf16x8_t pl = frag(&Ptl[(16 * tm) * LDB], LDB, 32 * k2);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const bf16x8_t ob = frag_tr(dOs, 32 * k2, 16 * (tn0 + j));  // B[v][t] = dO[t][v]
                xd[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, ob, xd[j], 0, 0, 0);
                xd[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, ob, xd[j], 0, 0, 0);
            }
        }
        if (score_adj) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float dh[4], dlo[4];
                ld4_rm_tr(Dh, 16 * tm, 16 * (tn0 + j), dh);
                ld4_rm_tr(Dlo, 16 * tm, 16 * (tn0 + j), dlo);
#pragma unroll
                for (int i = 0; i < 4; ++i) xd[j][i] += cs[i] * (dh[i] + dlo[i]);
            }
        }
        // S0^T lo rows again (phase F's operand, staged over dS^T lo in phase E;
        // an L2 hit, issued here so that phase E hides it)
        const Mat2 s0lr = load_mat2(a.ck_state_lo + (int64_t)ci * KD * KD + 64 * vb * KD, tid);
        __syncthreads();  // P^T and delta read by every wave before ddelta^T takes P's tiles
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile_t_split(&Dd[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ddl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, xd[j]);
#pragma unroll
        for (int i = 0; i < NKB; ++i) {  // <S0 lo, dS hi> at this thread's staging positions
            const int p = tid + NT * i, r = p / (KD / 8), c0 = 8 * (p % (KD / 8));
            frob += dot8_bf16(s0lr.p[i], *reinterpret_cast<const uint4 *>(&dSt[r * LDK + c0]));
        }
        __syncthreads();
        // Phase E: dR = T^T ddelta -> dV, the sum_v dR v part of dbeta, dR rows.
        {
            const f32x4 bt = row4(sm.gl.beta);
            f32x4 x[2] = {zero4(), zero4()};
#pragma unroll
            for (int r = 0; r < 64; r += 32) {
                const bf16x8_t tt = frag_tr(Tr, r, 16 * tm);  // A[s][t] = T[t][s]
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint16_t *Yh = &Dd[(16 * (tn0 + j)) * LDB], *Yl = &Ddl[(16 * (tn0 + j)) * LDB];
                    x[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tt, frag(Yh, LDB, r), x[j], 0, 0, 0);
                    x[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tt, frag(Yl, LDB, r), x[j], 0, 0, 0);
                }
            }
            f32x4 dvv[2];
            float pb2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float vv[4];
                ld4_rm_tr(Vr, 16 * tm, 16 * (tn0 + j), vv);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pb2[i] += x[j][i] * vv[i];
                    dvv[j][i] = sm.gl.val[r0 + i] != 0.f ? bt[i] * x[j][i] : 0.f;  // bt: beta rows
                }
                store_tile_rm(&dRr[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, x[j]);
            }
            row_reduce_accum(pb2, sm.b2[w & 1], tm, vb > 0);
            put_mat2(Xl, s0lr, tid);  // dS^T lo was last read in phase D
            __syncthreads();  // V and ddelta^T read: their tiles take this block's dV^T and dR's lo rows
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                store_tile_t(&dVt(vb)[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, dvv[j]);
                f32x4 lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) lo[i] = x[j][i] - bf16_val(bf16_bits(x[j][i]));
                store_tile_rm(&dRl[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, lo);
            }
            __syncthreads();
        }
        // Phase F: dR S0^T (-> dK, dbeta, dgam); dR delta^T and dO delta^T summed.
        float pku[4] = {0.f, 0.f, 0.f, 0.f};
        const f32x4 bt = row4(sm.gl.beta), gm = row4(sm.gl.gam);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            f32x4 drs[2] = {zero4(), zero4()};
            gemm2_tr<64, LDB, LDK>(drs, &dRr[(16 * tm) * LDB], S0t, tn0 + 4 * kb);
            gemm2_tr<64, LDB, LDK>(drs, &dRr[(16 * tm) * LDB], Xl, tn0 + 4 * kb);
            gemm2_tr<64, LDB, LDK>(drs, &dRl[(16 * tm) * LDB], S0t, tn0 + 4 * kb);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float kv[4];
                ld4_rm_tr<LDK>(Ks, 16 * tm, 16 * (tn0 + 4 * kb + j), kv);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pku[i] += kv[i] * drs[j][i];
                    dka[kb][j][i] -= bt[i] * gm[i] * drs[j][i];  // beta gam
                }
            }
        }
        row_reduce_accum(pku, sm.ku[w & 1], tm, vb > 0);
        {  // phase A's dO S0^T with S0's lo part, which xl holds now
            float pg1l[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                f32x4 x[2] = {zero4(), zero4()};
                gemm2_tr<64, LDB, LDK>(x, &dOs[(16 * tm) * LDB], Xl, tn0 + 4 * kb);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    float qv[4];
                    ld4_rm_tr<LDK>(Qs, 16 * tm, 16 * (tn0 + 4 * kb + j), qv);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        pg1l[i] += qv[i] * x[j][i];
                        dos[kb][j][i] += x[j][i];
                    }
                }
            }
            row_reduce_accum(pg1l, sm.g1[w & 1], tm, true);
        }
        if (tn0 <= tm) {
            gemm2(da, &dRr[(16 * tm) * LDB], Dh, tn0);
            gemm2(da, &dRr[(16 * tm) * LDB], Dlo, tn0);
            gemm2(da, &dRl[(16 * tm) * LDB], Dh, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dh, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dlo, tn0);
        }
    }
    frob = wave_sum(frob);
    if (lane_id() == 0) sm.frob[w] = frob;
    __syncthreads();  // the last block's phase F has read dR's lo rows: MP^T takes their tile
    const RowGates rg = row_gates(sm.gl, tm);
    // dA and dP masked -> MA^T, MP^T, and the gate-gradient partial sums (KK^T,
    // QK^T and the mask formed again here rather than held through the blocks).
    {
        float gmA[2][4];
        gam_mask(gmA);
        f32x4 kk[2] = {zero4(), zero4()}, qk[2] = {zero4(), zero4()};
        if (tn0 <= tm) {
            gemm2<KD, LDK, LDK>(kk, &Ks[(16 * tm) * LDK], Ks, tn0);
            gemm2<KD, LDK, LDK>(qk, &Qs[(16 * tm) * LDK], Ks, tn0);
        }
        float pb[4] = {0.f, 0.f, 0.f, 0.f}, pz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            f32x4 ma, mp, z;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                const float gm = gmA[j][i];
                const float dA = ss < tt ? -da[j][i] : 0.f;
                const float dP = dp[j][i];
                ma[i] = dA * rg.beta[i] * gm;
                mp[i] = dP * gm;
                pb[i] += dA * gm * kk[j][i];
                z[i] = (dA * rg.beta[i] * kk[j][i] + dP * qk[j][i]) * gm;
                pz[i] += z[i];
            }
            store_tile_t(&MAt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, ma);
            store_tile_t_split(&MPt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &MPtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, mp);
            const float zc = col_reduce(z);
            if ((lane_id() >> 4) == 0) sm.zc[tm][ss] = zc;
        }
        row_reduce_store(pb, sm.b1[w & 1], tm);
        row_reduce_store(pz, sm.zr[w & 1], tm);
    }
    __syncthreads();
    // Phase G: dQ = MP K + gam dO S0^T and dK = (MA + MA^T) K + MP^T Q + lam delta
    // dS^T - beta gam dR S0^T (+ c' k), masked, staged transposed with dV.
    {
        f32x4 x[NKB][2], y[NKB][2];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) x[kb][0] = x[kb][1] = y[kb][0] = y[kb][1] = zero4();
#pragma unroll
        for (int r = 0; r < 64; r += 32) {
            const bf16x8_t mp = frag_tr(MPt, r, 16 * tm), mpl = frag_tr(MPtl, r, 16 * tm);
            const bf16x8_t ma = frag_tr(MAt, r, 16 * tm), mat = frag(&MAt[(16 * tm) * LDB], LDB, r);
            const bf16x8_t pt = frag(&MPt[(16 * tm) * LDB], LDB, r), ptl = frag(&MPtl[(16 * tm) * LDB], LDB, r);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int tn = 16 * (tn0 + 4 * kb + j);
                    const bf16x8_t kbf = frag_tr<LDK>(Ks, r, tn);  // B[k][s] = K[s][k]
                    const bf16x8_t qbf = frag_tr<LDK>(Qs, r, tn);  // B[k][t] = Q[t][k]
                    x[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mp, kbf, x[kb][j], 0, 0, 0);
                    x[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mpl, kbf, x[kb][j], 0, 0, 0);
                    y[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ma, kbf, y[kb][j], 0, 0, 0);
                    y[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mat, kbf, y[kb][j], 0, 0, 0);
                    y[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pt, qbf, y[kb][j], 0, 0, 0);
                    y[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ptl, qbf, y[kb][j], 0, 0, 0);
                }
        }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float kv[4] = {0.f, 0.f, 0.f, 0.f};
                if (score_adj) ld4_rm_tr<LDK>(Ks, 16 * tm, 16 * (tn0 + 4 * kb + j), kv);
                f32x4 gq, gk;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool von = sm.gl.val[r0 + i] != 0.f;
                    gq[i] = von ? x[kb][j][i] + rg.gam[i] * dos[kb][j][i] : 0.f;
                    gk[i] = von ? y[kb][j][i] + dka[kb][j][i] + ck[i] * kv[i] : 0.f;
                }
                // Transposed gradient tiles ([channel][token]) in slots phase G does not read.
                store_tile_t(&dQt[(16 * (tn0 + 4 * kb + j)) * LDB + 16 * tm], LDB, gq);
                store_tile_t(&dKt[(16 * (tn0 + 4 * kb + j)) * LDB + 16 * tm], LDB, gk);
            }
    }
    __syncthreads();
    dv_out(NVB - 1);
    // Rows out: lane (token 16 (w%4) + l%16, channels 32 (w/4) + 8 (l/16) ..) of
    // every 64-channel block stores one 16-byte piece per gradient.
    {
        const int l = lane_id();
        const int tq = c * C + 16 * (w & 3) + (l & 15);
        const int64_t row = ((int64_t)b * a.T + tq) * a.H + h;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const bf16x8_t gq = frag_tr(dQt, 64 * kb + 32 * (w >> 2), 16 * (w & 3));
            const bf16x8_t gk = frag_tr(dKt, 64 * kb + 32 * (w >> 2), 16 * (w & 3));
            const int64_t o = row * KD + 64 * kb + 32 * (w >> 2) + 8 * (l >> 4);
            if (tq < a.T && a.dq) *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dq) + o) = gq;
            if (tq < a.T && a.dk) *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dk) + o) = gk;
        }
    }
    // Phase H: gate gradients (wave 0, lane == token; lane t holds token 63 - t).
    if (w == 0) {
        const int s = 63 - t, ts = c * C + s;
        const float gam = sm.gl.gam[s], lam = sm.gl.lam[s], bet = sm.gl.beta[s];
        const float dlam = sm.dlam[0][s] + sm.dlam[1][s];
        const float u = sm.ku[0][s] + sm.ku[1][s];
        float dG = sm.zr[0][s] + sm.zr[1][s] -
                   (sm.zc[0][s] + sm.zc[1][s] + sm.zc[2][s] + sm.zc[3][s]) +
                   gam * (sm.g1[0][s] + sm.g1[1][s] - bet * u) - lam * dlam;
        const float tail = wave_sum(lam * dlam);
        if (s == 63) {
            float fr = 0.f;
#pragma unroll
            for (int q = 0; q < NW; ++q) fr += sm.frob[q];
            dG += tail + sm.gl.gamC * fr;
        }
        const float db = sm.b1[0][s] + sm.b1[1][s] + sm.b2[0][s] + sm.b2[1][s] - gam * u;
        const float x = wave_scan_add(dG);
        const bool von = sm.gl.val[s] != 0.f;
        const bool rs = von && (s == 0 ? sm.gl.seg[0] == 1 : sm.gl.seg[s] != sm.gl.seg[s - 1]);
        if (ts < a.T) {
            const int64_t o = ((int64_t)b * a.T + ts) * a.H + h;
            if (a.dg) a.dg[o] = (von && !rs) ? x : 0.f;
            if (a.dbeta) a.dbeta[o] = von ? db : 0.f;
        }
    }
}

static inline void wmark(const hipEvent_t *ev, int i, hipStream_t stream) {
    if (ev) (void)hipEventRecord(ev[i], stream);
}

// The factored scan over a head's chunks: forward (states, U of prep) or
// reverse (state adjoints, N of bprep).
static hipError_t wide_scan(const ChunkArgs &a, bool reverse, hipStream_t stream) {
    LrScanArgs p{};
    p.nc = a.nc;
    p.B = a.B;
    p.H = a.H;
    p.vd = KD;
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
        p.x0.s0 = (int64_t)a.H * KD * KD;
        p.x0.s1 = (int64_t)KD * KD;
        p.x0.s2 = KD;
        p.x0.s3 = 1;
        p.xout = a.dinitial;
    }
    return launch_lr_scan(p, KD, C, stream);
}

hipError_t launch_wide_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nch = a.B * a.H * a.nc;
    wmark(ev, 0, stream);
    hipLaunchKernelGGL(wide_prep_kernel, dim3(nch), dim3(NT), 0, stream, a);
    wmark(ev, 1, stream);
    wmark(ev, 2, stream);
    const hipError_t e = wide_scan(a, false, stream);
    if (e != hipSuccess) return e;
    wmark(ev, 3, stream);
    wmark(ev, 4, stream);
    hipLaunchKernelGGL(wide_out_kernel, dim3(std::min(nch, device_cus())), dim3(NT), 0, stream, a, nch);
    wmark(ev, 5, stream);
    return hipGetLastError();
}

hipError_t launch_wide_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nch = a.B * a.H * a.nc;
    wmark(ev, 0, stream);
    if (a.dscores)
        hipLaunchKernelGGL(wide_bprep_kernel<true>, dim3(std::min(nch, device_cus())), dim3(NT), 0, stream, a, nch);
    else
        hipLaunchKernelGGL(wide_bprep_kernel<false>, dim3(std::min(nch, device_cus())), dim3(NT), 0, stream, a, nch);
    wmark(ev, 1, stream);
    wmark(ev, 2, stream);
    const hipError_t e = wide_scan(a, true, stream);
    if (e != hipSuccess) return e;
    wmark(ev, 3, stream);
    wmark(ev, 4, stream);
    if (a.dscores)
        hipLaunchKernelGGL(wide_bgrad_kernel<true>, dim3(nch), dim3(NT), 0, stream, a);
    else
        hipLaunchKernelGGL(wide_bgrad_kernel<false>, dim3(nch), dim3(NT), 0, stream, a);
    wmark(ev, 5, stream);
    return hipGetLastError();
}

}  // namespace gdn2
