// Chunk-WY scalar-gate gated delta rule on gfx950 MFMA.
//
// Recurrence per valid token t (the GDN-2 recurrence of
// crates/mixers/src/reference.rs:68-111 with alpha = exp(g_t) on every key
// channel and erase = write = beta_t):
//   S_t = a_t S_{t-1} + b_t k_t (v_t - a_t S_{t-1}^T k_t)^T,  o_t = S_t^T q_t.
// Per chunk of C = 64 tokens with start state S0 (G = chunk-local cumsum of g,
// segments split at resets so decays never cross a reset):
//   gam_t = exp(G_t)            lam_s = exp(G_63 - G_s)      Gam_ts = exp(G_t - G_s)
//   A   = strict_lower(beta_t Gam_ts k_t.k_s)     T = (I + A)^-1   (UT/WY inverse)
//   R   = diag(beta) (V - diag(gam) K S0)         delta = T R     (the edits)
//   O   = diag(gam) Q S0 + lower(Gam .* Q K^T) delta
//   S_C = gam_63 S0 + (diag(lam) K)^T delta,      score_t = |k_t| |delta_t|
// This is the chunk form of crates/mixers/src/chunk.rs:155-241 with the
// nilpotent series replaced by a blocked substitution inverse (C > 16).
//
// Forward = three launches:
//   prep  (one workgroup per chunk): gates, A, T -> checkpoint (T bf16, gates)
//   state (one workgroup per (batch, head), chunks in order): the only
//         sequential part; fp32 S lives in MFMA accumulators, next chunk's
//         K/V/T/gates are prefetched into registers; writes S at each chunk start
//   out   (one workgroup per chunk): delta from the chunk-start state, O, scores
// Workgroups are 8 waves; wave w owns output tiles (w/2, 2(w%2)) and
// (w/2, 2(w%2)+1) of every 64x64 product.  All GEMMs are
// v_mfma_f32_16x16x32_bf16 on LDS tiles; the inverse is fp32 (diagonal 16x16
// blocks by forward substitution, off-diagonal blocks by a 2x2 recursion on
// v_mfma_f32_16x16x4_f32).  R, delta and P enter the GEMMs that consume them
// as two-term bf16 splits (hi + lo); S0, T, Q, K, V as single bf16 terms.
#include "gdn2_chunk_tile.h"

#include <algorithm>
#include <atomic>

namespace gdn2 {

namespace {

struct PrepSmem {
    uint16_t slot[4][TILE];  // K rows (then T), beta gam K rows (hi, lo), beta V rows
    struct {
        float Af[C * LDF];
        float Tf[C * LDF];
    } inv;
    GateLds gl;
};

struct OutSmem {
    uint16_t slot[8][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[2][C];
};

}  // namespace

// ---- prep: gates, the UT inverse and the dense state map of every chunk -------
// W = T diag(beta gam) K and U = T diag(beta) V give the chunk's state map
//   S_C = A_c S0 + B_c,  A_c = gam_63 I - Ktil^T W,  B_c = Ktil^T U  (Ktil = lam K),
// formed from hi/lo pairs of Ktil, W and U and stored for the scans: A_c rows
// and A_c^T rows as bf16 hi and lo, B_c^T in f32.
__global__ void __launch_bounds__(NT) chunk_prep_kernel(ChunkArgs a) {
    __shared__ PrepSmem sm;
    // beta gam K and beta V are staged as scaled rows; the products that need
    // them transposed read across them.
    uint16_t *Ks = sm.slot[0], *KBGs = sm.slot[1], *KBGl = sm.slot[3], *VBs = sm.slot[2];
    uint16_t *Tb = sm.slot[0];  // over K once A is formed
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tg = c * C + t;
    const int tm = w >> 1, tn0 = 2 * (w & 1);
    const bool inb = tg < a.T;
    // Every load issued up front; masks are applied once the values arrive.
    const uint4 kraw = load8(a.k, a.ks, b, tg, h, cb, inb);
    const uint4 vraw = load8(a.v, a.vs, b, tg, h, cb, inb);
    const float vld = inb ? ld4<float>(a.valid, b, tg, 0, 0) : 0.f;
    float rst = 0.f, gt = 0.f, bt = 0.f;
    if (w == 0 && inb) {
        rst = ld4<float>(a.reset, b, tg, 0, 0);
        gt = ld4<float>(a.g, b, tg, h, 0);
        bt = ld4<float>(a.beta, b, tg, h, 0);
    }
    const bool on = vld != 0.f;
    const uint4 k8 = mask8(kraw, on), v8 = mask8(vraw, on);
    put_row8(Ks, t, cb, k8);
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
    uint4 ktil_hi, ktil_lo;  // Ktil = lam K rows (hi, lo), staged once the inverse is done
    {  // beta gam K rows (hi, lo) for the W product
        const float bg = sm.gl.beta[t] * sm.gl.gam[t], la = sm.gl.lam[t];
        Pack8 kp;
        kp.u = k8;
        uint32_t kb[4], kbl[4], kh[4], kl[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float k0 = bf16_val(kp.h[e]), k1 = bf16_val(kp.h[e + 1]);
            uint16_t h0, l0, h1, l1;
            split_bf16(bg * k0, h0, l0);
            split_bf16(bg * k1, h1, l1);
            kb[e / 2] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            kbl[e / 2] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            split_bf16(la * k0, h0, l0);
            split_bf16(la * k1, h1, l1);
            kh[e / 2] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            kl[e / 2] = (uint32_t)l0 | ((uint32_t)l1 << 16);
        }
        put_row8(KBGs, t, cb, make_uint4(kb[0], kb[1], kb[2], kb[3]));
        put_row8(KBGl, t, cb, make_uint4(kbl[0], kbl[1], kbl[2], kbl[3]));
        ktil_hi = make_uint4(kh[0], kh[1], kh[2], kh[3]);
        ktil_lo = make_uint4(kl[0], kl[1], kl[2], kl[3]);
    }
    // A = strict_lower(beta_t Gam_ts k_t.k_s) in f32 (tiles with tn <= tm only).
    if (tn0 <= tm) {
        f32x4 kk[2] = {zero4(), zero4()};
        gemm2(kk, &Ks[(16 * tm) * LDB], Ks, tn0);
        const RowGates rg = row_gates(sm.gl, tm);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                sm.inv.Af[tt * LDF + ss] = (ss < tt && rg.seg[i] == sgs)
                                                 ? rg.beta[i] * __expf(rg.G[i] - Gs) * kk[j][i]
                                                 : 0.f;
            }
        }
    }
    __syncthreads();
    ut_inverse(sm.inv.Af, sm.inv.Tf, w);
    // T (bf16, row-major, zero above the diagonal): LDS operand and checkpoint.
    {
        const int r = tid >> 3, c0 = 8 * (tid & 7);
        // Two 16-byte reads; the blocks above the diagonal hold stale data and are
        // masked after the read.
        const float4 f0 = *reinterpret_cast<const float4 *>(&sm.inv.Tf[r * LDF + c0]);
        const float4 f1 = *reinterpret_cast<const float4 *>(&sm.inv.Tf[r * LDF + c0 + 4]);
        const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s0 = c0 + 2 * e;
            pk[e] = bf16_pack2(s0 <= r ? f[2 * e] : 0.f, s0 + 1 <= r ? f[2 * e + 1] : 0.f);
        }
        const uint4 v = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *reinterpret_cast<uint4 *>(a.ck_t + (int64_t)ci * C * C + r * C + c0) = v;
        *reinterpret_cast<uint4 *>(&Tb[r * LDB + c0]) = v;
    }
    {  // beta V rows for U, written once the inverse no longer needs the time
        const float be = sm.gl.beta[t];
        Pack8 vp;
        vp.u = v8;
        uint32_t vb[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            vb[e / 2] = bf16_pack2(be * bf16_val(vp.h[e]), be * bf16_val(vp.h[e + 1]));
        put_row8(VBs, t, cb, make_uint4(vb[0], vb[1], vb[2], vb[3]));
    }
    __syncthreads();  // T staged; the inverse's scratch is free: Ktil rows (hi, lo) take it
    uint16_t *KLs = reinterpret_cast<uint16_t *>(sm.inv.Af), *KLl = KLs + TILE;
    static_assert(sizeof(sm.inv) >= 2 * TILE * sizeof(uint16_t), "Ktil hi/lo over the inverse's scratch");
    put_row8(KLs, t, cb, ktil_hi);
    put_row8(KLl, t, cb, ktil_lo);
    // W = T (beta gam K), U = T (beta V) in registers ...
    f32x4 x[2] = {zero4(), zero4()}, y[2] = {zero4(), zero4()};
    gemm2_tr(x, &Tb[(16 * tm) * LDB], KBGs, tn0);  // B[k][t] = (beta gam K)[t][k]
    gemm2_tr(x, &Tb[(16 * tm) * LDB], KBGl, tn0);
    gemm2_tr(y, &Tb[(16 * tm) * LDB], VBs, tn0);   // B[v][t] = (beta V)[t][v]
    __syncthreads();  // T, beta gam K and beta V read: W^T and U^T (hi, lo) take their slots
    uint16_t *Wt = sm.slot[0], *Wtl = sm.slot[1], *Ut = sm.slot[2], *Utl = sm.slot[3];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        store_tile_t_split(&Wt[(16 * (tn0 + j)) * LDB + 16 * tm], &Wtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        store_tile_t_split(&Ut[(16 * (tn0 + j)) * LDB + 16 * tm], &Utl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, y[j]);
    }
    __syncthreads();
    // ... then A_c = gam_63 I - Ktil^T W and B_c = Ktil^T U over the three terms
    // of the hi/lo pairs (tile rows: key 16 tm + .., columns 16 (tn0 + j) + ..).
    f32x4 am[2] = {zero4(), zero4()}, bm[2] = {zero4(), zero4()};
    gemm2_atr(am, KLs, 16 * tm, Wt, tn0);  // A[k][t] = Ktil[t][k]
    gemm2_atr(am, KLs, 16 * tm, Wtl, tn0);
    gemm2_atr(am, KLl, 16 * tm, Wt, tn0);
    gemm2_atr(bm, KLs, 16 * tm, Ut, tn0);
    gemm2_atr(bm, KLs, 16 * tm, Utl, tn0);
    gemm2_atr(bm, KLl, 16 * tm, Ut, tn0);
    {
        const float gC = sm.gl.gamC;
        float *Bt = a.map_b + (int64_t)ci * D * D;  // B_c^T [value][key]
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int cc = 16 * (tn0 + j) + acc_col();
#pragma unroll
            for (int i = 0; i < 4; ++i) am[j][i] = (16 * tm + acc_row(i) == cc ? gC : 0.f) - am[j][i];
            *reinterpret_cast<float4 *>(&Bt[cc * D + 16 * tm + acc_row(0)]) =
                make_float4(bm[j][0], bm[j][1], bm[j][2], bm[j][3]);
        }
    }
    __syncthreads();  // W^T and U^T read: A_c^T (hi, lo) takes their slots
    uint16_t *Mt = sm.slot[0], *Mtl = sm.slot[1];
#pragma unroll
    for (int j = 0; j < 2; ++j)
        store_tile_t_split(&Mt[(16 * (tn0 + j)) * LDB + 16 * tm], &Mtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, am[j]);
    __syncthreads();
    // Rows out, hi then lo: M = A_c^T row by row (the adjoint scan's map), and A_c
    // (the state scan's) read across it: lane (row 16 (w%4) + l%16, columns
    // 32 (w/4) + 8 (l/16) ..) stores one 16-byte row piece.
    {
        const int r = tid >> 3, c0 = 8 * (tid & 7), l = lane_id();
        uint16_t *mt = a.map_mt + (int64_t)ci * 2 * D * D, *mm = a.map_m + (int64_t)ci * 2 * D * D;
        const int64_t fo = (int64_t)(16 * (w & 3) + (l & 15)) * D + 32 * (w >> 2) + 8 * (l >> 4);
#pragma unroll
        for (int part = 0; part < 2; ++part) {
            const uint16_t *src = part == 0 ? Mt : Mtl;
            *reinterpret_cast<uint4 *>(mt + part * D * D + r * D + c0) =
                *reinterpret_cast<const uint4 *>(&src[r * LDB + c0]);
            *reinterpret_cast<bf16x8_t *>(mm + part * D * D + fo) = frag_tr(src, 32 * (w >> 2), 16 * (w & 3));
        }
    }
}

// ---- out: outputs and scores of every chunk --------------------------------------
__global__ void __launch_bounds__(NT) chunk_out_kernel(ChunkArgs a) {
    __shared__ OutSmem sm;
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *Vt = sm.slot[2], *Tb = sm.slot[3];
    uint16_t *St = sm.slot[4], *Rt = sm.slot[5], *Pt = sm.slot[6], *Ptl = sm.slot[7];  // P^T hi/lo
    uint16_t *Dt = sm.slot[0], *Dl = sm.slot[1];  // over Q/K after phase 1
    uint16_t *Os = sm.slot[4];                    // over S0^T after phase 1
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, t0 = c * C, tg = t0 + t;
    const int tm = w >> 1, tn0 = 2 * (w & 1);
    const GateBlock *gb = a.ck_gate + ci;
    const bool inb = tg < a.T;
    // T is read only from phase 2: its load is issued last and written to LDS
    // after phase 1.
    const uint4 qr = load8(a.q, a.qs, b, tg, h, cb, inb);
    const uint4 kr = load8(a.k, a.ks, b, tg, h, cb, inb);
    const uint4 vr = load8(a.v, a.vs, b, tg, h, cb, inb);
    const uint4 s0r = *reinterpret_cast<const uint4 *>(a.ck_state + (int64_t)ci * D * D +
                                                       (tid >> 3) * D + 8 * (tid & 7));
    // S0's lo part enters the K S0 and Q S0 products straight from the
    // checkpoint as B fragments: S0^T row 16 (tn0 + j) + l % 16, keys 32 i + 8 (l / 16).
    bf16x8_t s0l[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
            s0l[j][i] = *reinterpret_cast<const bf16x8_t *>(
                a.ck_state_lo + (int64_t)ci * D * D + (16 * (tn0 + j) + (tid & 15)) * D + 32 * i +
                8 * ((tid & 63) >> 4));
    const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
    const int sg = gb->seg[t];
    const uint4 trw =
        *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
    {
        const bool on = va != 0.f;
        const uint4 k8 = mask8(kr, on);
        put_row8(Qs, t, cb, mask8(qr, on));
        put_row8(Ks, t, cb, k8);
        put_col8(Vt, t, cb, mask8(vr, on));
        *reinterpret_cast<uint4 *>(&St[(tid >> 3) * LDB + 8 * (tid & 7)]) = s0r;  // S0^T rows
        Pack8 kp;
        kp.u = k8;
        float ksq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float kf = bf16_val(kp.h[e]);
            ksq += kf * kf;
        }
        sm.kk[cb][t] = ksq;
        if (w == 0) gates_derive(sm.gl, G, be, va, sg);
    }
    __syncthreads();
    // Phase 1: R (-> Rt, lo over Vt), P (hi/lo), and gam Q S0 kept in registers.
    f32x4 qs[2] = {zero4(), zero4()};
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2(x, &Ks[(16 * tm) * LDB], St, tn0);
        gemm2(qs, &Qs[(16 * tm) * LDB], St, tn0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const bf16x8_t kf = frag(&Ks[(16 * tm) * LDB], LDB, 32 * i);
            const bf16x8_t qf = frag(&Qs[(16 * tm) * LDB], LDB, 32 * i);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                x[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, s0l[j][i], x[j], 0, 0, 0);
                qs[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf, s0l[j][i], qs[j], 0, 0, 0);
            }
        }
        f32x4 pq[2] = {zero4(), zero4()};
        if (tn0 <= tm) gemm2(pq, &Qs[(16 * tm) * LDB], Ks, tn0);
        const RowGates rg = row_gates(sm.gl, tm);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
            uint16_t *vt = &Vt[(16 * (tn0 + j)) * LDB + 16 * tm];
            float vv[4];
            ld4_bf16(vt + acc_col() * LDB + 4 * (lane_id() >> 4), vv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                x[j][i] = rg.beta[i] * (vv[i] - rg.gam[i] * x[j][i]);
                qs[j][i] *= rg.gam[i];
                pq[j][i] *= (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
            }
            store_tile_t_split(&Rt[(16 * (tn0 + j)) * LDB + 16 * tm], vt, LDB, x[j]);
            store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq[j]);
        }
    }
    *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = trw;
    __syncthreads();
    // Phase 2: delta = T R (-> Dt/Dl over the Q/K slots) and |delta_t|^2; delta
    // itself stays in registers for the checkpoint.
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
        row_reduce_store(p, sm.dd[w & 1], tm);
    }
    __syncthreads();
    // delta (f32, row-major) over the R^T-lo and T slots, dead from here on; it
    // leaves for the checkpoint as 16-byte row pieces after the last barrier.
    float *Df = reinterpret_cast<float *>(sm.slot[2]);
    static_assert(C * LDF * sizeof(float) <= 2 * sizeof(sm.slot[0]), "delta tile spans two slots");
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) Df[(16 * tm + acc_row(i)) * LDF + 16 * (tn0 + j) + acc_col()] = dlt[j][i];
    // Phase 3: O = gam Q S0 + P delta, staged through LDS for coalesced stores.
    {
        f32x4 x[2] = {qs[0], qs[1]};
        gemm2_atr(x, Pt, 16 * tm, Dt, tn0);  // A[t][s] = P^T[s][t]
        gemm2_atr(x, Pt, 16 * tm, Dl, tn0);
        gemm2_atr(x, Ptl, 16 * tm, Dt, tn0);
        if (a.out_bf16) {
#pragma unroll
            for (int j = 0; j < 2; ++j) store_tile_rm(&Os[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, x[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tq = t0 + 16 * tm + acc_row(i);
                    if (tq < a.T)
                        reinterpret_cast<float *>(a.out)[(((int64_t)b * a.T + tq) * a.H + h) * D +
                                                         16 * (tn0 + j) + acc_col()] = x[j][i];
                }
        }
    }
    if (tid < 64 && tg < a.T) {
        float kk = 0.f;
#pragma unroll
        for (int q = 0; q < NW; ++q) kk += sm.kk[q][t];
        const float dd = sm.dd[0][t] + sm.dd[1][t];
        a.scores[((int64_t)b * a.T + tg) * a.H + h] = sm.gl.val[t] != 0.f ? sqrtf(kk * dd) : 0.f;
    }
    __syncthreads();
    {
        const int r = tid >> 3, c0 = 8 * (tid & 7), tq = t0 + r;
        float *dck = a.ck_delta + (int64_t)ci * C * D + r * D + c0;  // checkpoint for the backward
        *reinterpret_cast<float4 *>(dck) = *reinterpret_cast<const float4 *>(&Df[r * LDF + c0]);
        *reinterpret_cast<float4 *>(dck + 4) = *reinterpret_cast<const float4 *>(&Df[r * LDF + c0 + 4]);
        if (a.out_bf16 && tq < a.T)
            *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.out) +
                                       (((int64_t)b * a.T + tq) * a.H + h) * D + c0) =
                *reinterpret_cast<const uint4 *>(&Os[r * LDB + c0]);
    }
}

// ---- affine scan: the sequential part -------------------------------------------
// X_next = M_c X + N_c over the chunks of one (batch, head): forward (M = A_c,
// N = B_c; X0 = the initial state; X before each step = the chunk-start state)
// or reverse (M = A_c^T, N from bprep; X0 = the final-state adjoint; X before
// each step = the chunk-end state adjoint).  X before each step goes to the
// checkpoint transposed (X^T rows), as bf16 hi and lo.  The state's columns
// evolve independently, so each head's scan is split over AS_SPLIT workgroups
// of 16 AS_CW columns each (the workgroups of one head read the same maps; their
// block indices differ by a multiple of B*H, so with B*H a multiple of the XCD
// count they share an L2).  AS_CW + 3 waves per workgroup:
//   waves 0 .. AS_CW-1  compute: wave w owns state columns j0 + 16 w .. + 15 in
//              MFMA accumulators; per step it writes X^T hi/lo into its LDS
//              tiles (the B operand of the product and the writer's source),
//              passes the step's barrier and forms N + M_hi X_hi + M_hi X_lo +
//              M_lo X_hi (24 MFMAs, four independent accumulator tiles);
//   wave AS_CW      streams M (hi, then lo) into an LDS ring with LDS-DMA loads,
//              AS_MRING - 1 chunks ahead;
//   wave AS_CW + 1  streams the workgroup's rows of N^T (f32) the same way;
//   wave AS_CW + 2  copies each step's X^T tiles to the checkpoint.
// The compute waves issue no global memory operations inside the loop.  LDS
// rows are swizzled by 16-byte chunk against bank conflicts.
namespace {
constexpr int AS_CW = 2;               // compute waves per workgroup
constexpr int AS_SPLIT = 4 / AS_CW;    // workgroups per head
constexpr int AS_MRING = 3;
constexpr int AS_NRING = 3;
constexpr int AS_MOPS = 2 * D * D * 2 / 1024;       // LDS-DMA instructions per map (hi + lo, 1 KiB each)
constexpr int AS_NOPS = 16 * AS_CW * D * 4 / 1024;  // per workgroup's rows of N^T (f32)
constexpr int AS_THREADS = (AS_CW + 3) * 64;

struct AsArgs {
    int nc, B, H;
    const uint16_t *m;  // per chunk: M rows, bf16 hi [64][64] then lo [64][64]
    const float *n;     // per chunk: N^T rows, f32 [64][64]
    uint16_t *ckpt, *ckpt_lo;  // X^T per chunk, bf16 hi and lo
    View x0;            // [B,H,64,64] strided (data may be null: zero)
    float *xout;        // [B,H,64,64] dense (may be null)
};

struct AsSmem {
    uint4 m[AS_MRING][2 * D * D / 8];       // row r (hi rows 0..63, lo rows 64..127): chunk x at x ^ (r & 7)
    uint4 n[AS_NRING][16 * AS_CW * D / 4];  // N^T row j0 + j: chunk x (four f32) at x ^ (j & 15)
    uint16_t xs[2][AS_CW][2][16 * LDB];     // [step parity][compute wave][hi, lo]: X^T [col][row]
};

// s_waitcnt immediates (gfx9 encoding): vmcnt <= n only; lgkmcnt == 0 only.
constexpr int as_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int AS_LGKMCNT_ZERO = 15 | (3 << 14) | (7 << 4);

__device__ __forceinline__ void as_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
}  // namespace

// REV: the reverse scan (chunks walked from the last).
template <bool REV>
__global__ void __launch_bounds__(AS_THREADS) affine_scan_kernel(AsArgs p) {
    extern __shared__ __align__(1024) char as_lds[];
    AsSmem &sm = *reinterpret_cast<AsSmem *>(as_lds);
    const int nbh = p.B * p.H, bh = blockIdx.x % nbh, j0 = 16 * AS_CW * (blockIdx.x / nbh);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
    typedef __attribute__((address_space(1))) const void *gptr;
    typedef __attribute__((address_space(3))) void *lptr;
    auto chunk_of = [&](int s) {
        const int sc = min(s, p.nc - 1);
        return (int64_t)bh * p.nc + (REV ? p.nc - 1 - sc : sc);
    };
    if (w == AS_CW) {  // producer: M (hi and lo), AS_MRING - 1 chunks ahead
        auto issue = [&](int s) {
            const uint16_t *M = p.m + chunk_of(s) * 2 * D * D;
            uint4 *slot = sm.m[s % AS_MRING];
#pragma unroll
            for (int i = 0; i < AS_MOPS; ++i) {
                const int q = 64 * i + l, r = q >> 3, x = q & 7;
                __builtin_amdgcn_global_load_lds((gptr)(M + r * D + 8 * (x ^ (r & 7))), (lptr)(slot + 64 * i), 16,
                                                 0, 0);
            }
        };
        for (int s = 0; s < AS_MRING - 1; ++s) issue(s);
        for (int s = 0; s < p.nc; ++s) {
            // chunk s has landed once no more than the AS_MRING - 2 later maps are in flight
            __builtin_amdgcn_s_waitcnt(as_vmcnt((AS_MRING - 2) * AS_MOPS));
            as_barrier();
            issue(s + AS_MRING - 1);  // into the slot that step s - 1 read
        }
        __builtin_amdgcn_s_waitcnt(as_vmcnt(0));
        return;
    }
    if (w == AS_CW + 1) {  // producer: this workgroup's rows of N^T, AS_NRING - 1 chunks ahead
        auto issue = [&](int s) {
            const float *N = p.n + chunk_of(s) * D * D + j0 * D;
            uint4 *slot = sm.n[s % AS_NRING];
#pragma unroll
            for (int i = 0; i < AS_NOPS; ++i) {
                const int q = 64 * i + l, jj = q >> 4, x = q & 15;
                __builtin_amdgcn_global_load_lds((gptr)(N + jj * D + 4 * (x ^ (jj & 15))), (lptr)(slot + 64 * i), 16,
                                                 0, 0);
            }
        };
        for (int s = 0; s < AS_NRING - 1; ++s) issue(s);
        for (int s = 0; s < p.nc; ++s) {
            __builtin_amdgcn_s_waitcnt(as_vmcnt((AS_NRING - 2) * AS_NOPS));
            as_barrier();
            issue(s + AS_NRING - 1);
        }
        __builtin_amdgcn_s_waitcnt(as_vmcnt(0));
        return;
    }
    if (w == AS_CW + 2) {  // writer: X^T before step s -> the checkpoint of chunk c(s)
        for (int s = 0; s < p.nc; ++s) {
            as_barrier();
            const int64_t co = chunk_of(s) * D * D;
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                uint16_t *ck = part == 0 ? p.ckpt : p.ckpt_lo;
#pragma unroll
                for (int i = 0; i < 2 * AS_CW; ++i) {  // AS_CW compute waves x 16 columns x 64 rows
                    const int q = 64 * i + l, cw = q >> 7, col = (q >> 3) & 15, r8 = 8 * (q & 7);
                    const uint4 v = *reinterpret_cast<const uint4 *>(&sm.xs[s & 1][cw][part][col * LDB + r8]);
                    *reinterpret_cast<uint4 *>(&ck[co + (j0 + 16 * cw + col) * D + r8]) = v;
                }
            }
        }
        return;
    }
    const int b = bh / p.H, h = bh % p.H, g = l >> 4, n = l & 15;
    const int jl = 16 * w + n, j = j0 + jl;  // this lane's state column (in the workgroup, in the state)
    f32x4 X[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int i = 0; i < 4; ++i) X[tm][i] = p.x0.data ? ld4<float>(p.x0, b, h, 16 * tm + 4 * g + i, j) : 0.f;
    for (int s = 0; s < p.nc; ++s) {
        uint16_t *xh = sm.xs[s & 1][w][0], *xl = sm.xs[s & 1][w][1];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) store_tile_t_split(xh + 16 * tm, xl + 16 * tm, LDB, X[tm]);
        // The writer wave reads these tiles after the barrier, and the LDS writes of
        // different waves may complete out of issue order: wait until they landed.
        __builtin_amdgcn_s_waitcnt(AS_LGKMCNT_ZERO);
        as_barrier();  // this step's M and N are in their slots; the writer may read X^T
        const uint4 *slot = sm.m[s % AS_MRING];
        const float4 *nslot = reinterpret_cast<const float4 *>(sm.n[s % AS_NRING]);
        f32x4 Y[4], Z[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {  // N[16 tm + 4 g + i][j]: chunk 4 tm + g of N^T row j
            const float4 nv = nslot[jl * 16 + ((4 * tm + g) ^ (jl & 15))];
            Y[tm] = f32x4{nv.x, nv.y, nv.z, nv.w};
            Z[tm] = zero4();
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const bf16x8_t bh_ = frag(xh, LDB, 32 * kk), bl_ = frag(xl, LDB, 32 * kk);
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                const int r = 16 * tm + n, q = 4 * kk + g;
                const bf16x8_t mh = __builtin_bit_cast(bf16x8_t, slot[r * 8 + (q ^ (r & 7))]);
                const bf16x8_t ml = __builtin_bit_cast(bf16x8_t, slot[512 + r * 8 + (q ^ (r & 7))]);
                Y[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, bh_, Y[tm], 0, 0, 0);
                Z[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, bl_, Z[tm], 0, 0, 0);
                Z[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ml, bh_, Z[tm], 0, 0, 0);
            }
        }
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int i = 0; i < 4; ++i) X[tm][i] = Y[tm][i] + Z[tm][i];
    }
    if (p.xout)
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int i = 0; i < 4; ++i) p.xout[((int64_t)bh * D + 16 * tm + 4 * g + i) * D + j] = X[tm][i];
}

// The scan over a head's chunks: forward (chunk-start states and their lo
// parts, A_c and B_c^T from prep) or reverse (chunk-end state adjoints and
// their lo parts, A_c^T and N^T from bprep).
hipError_t launch_chunk_scan(const ChunkArgs &a, bool reverse, hipStream_t stream) {
    AsArgs p{};
    p.nc = a.nc;
    p.B = a.B;
    p.H = a.H;
    if (!reverse) {
        p.m = a.map_m;
        p.n = a.map_b;
        p.ckpt = a.ck_state;
        p.ckpt_lo = a.ck_state_lo;
        p.x0 = a.initial;
        p.xout = a.final_state;
    } else {
        p.m = a.map_mt;
        p.n = a.ws_n;
        p.ckpt = a.ws_dstate;
        p.ckpt_lo = a.ws_dstate_lo;
        p.x0.data = a.dfinal;
        p.x0.s0 = (int64_t)a.H * D * D;
        p.x0.s1 = D * D;
        p.x0.s2 = D;
        p.x0.s3 = 1;
        p.xout = a.dinitial;
    }
    constexpr size_t lds = sizeof(AsSmem);
    static_assert(lds <= 160 * 1024, "rings and staging fit LDS");
    // The kernel's dynamic LDS limit, raised once per process (a function-local
    // static: initialised exactly once even with concurrent first callers).
    static const hipError_t attr = [] {
        const hipError_t e = hipFuncSetAttribute((const void *)affine_scan_kernel<false>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        return e != hipSuccess ? e
                               : hipFuncSetAttribute((const void *)affine_scan_kernel<true>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }();
    if (attr != hipSuccess) return attr;
    if (reverse)
        hipLaunchKernelGGL(affine_scan_kernel<true>, dim3(a.B * a.H * AS_SPLIT), dim3(AS_THREADS), lds, stream, p);
    else
        hipLaunchKernelGGL(affine_scan_kernel<false>, dim3(a.B * a.H * AS_SPLIT), dim3(AS_THREADS), lds, stream, p);
    return hipGetLastError();
}

static inline void mark(const hipEvent_t *ev, int i, hipStream_t stream) {
    if (ev) (void)hipEventRecord(ev[i], stream);
}

hipError_t launch_chunk_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nchunks = a.B * a.H * a.nc;
    mark(ev, 0, stream);
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(nchunks), dim3(NT), 0, stream, a);
    mark(ev, 1, stream);
    mark(ev, 2, stream);
    (void)launch_chunk_scan(a, false, stream);
    mark(ev, 3, stream);
    mark(ev, 4, stream);
    hipLaunchKernelGGL(chunk_out_kernel, dim3(nchunks), dim3(NT), 0, stream, a);
    mark(ev, 5, stream);
    return hipGetLastError();
}

// ---- backward -------------------------------------------------------------------
// Given the chunk-start state S0 (forward checkpoint) and the adjoint dS of the
// state at the chunk end, with delta = T R, R = diag(beta)(V - diag(gam) K S0),
// O = diag(gam) Q S0 + P delta, S_C = gam_63 S0 + (lam K)^T delta:
//   ddelta = P^T dO + diag(lam) K dS^T + diag(c) delta,   c_s = dscore_s |k_s|/|delta_s|
//   dR     = T^T ddelta;  dV = diag(beta) dR
//   dS0    = gam_63 dS + (gam Q)^T dO - (beta gam K)^T dR
//   dA     = -strict_lower(dR delta^T);  dP = lower(dO delta^T)
//   dQ     = (dP.Gam) K + diag(gam) dO S0^T
//   dK     = (dA.beta Gam) K + (dA.beta Gam)^T K + (dP.Gam)^T Q - diag(beta gam) dR S0^T
//            + diag(lam) delta dS^T + diag(dscore |delta|/|k|) K
//   dbeta  = rowsum(dA.Gam.KK^T) + rowsum(dR.(V - gam K S0))
//   dG_t   = rowsum_t(Z) - colsum_t(Z) + gam_t (q_t.(dO S0^T)_t - beta_t k_t.(dR S0^T)_t)
//            - lam_t dlam_t [+ at t=63: sum_s lam_s dlam_s + gam_63 <S0, dS>],
//            Z = (dA beta KK^T + dP QK^T) . Gam,  dlam_s = k_s.(delta dS^T)_s;
//   dg_u   = sum_{t >= u} dG_t (zero on padding and reset tokens).
// bstate walks the chunks backwards carrying dS (fp32, MFMA accumulators) and
// writes dS at every chunk end; bgrad then produces all token gradients of
// every chunk in parallel.

namespace {

struct BPrepSmem {  // fits twice in one CU's LDS
    uint16_t slot[8][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[NW][C];
    float dsc[C];
};

struct BGradSmem {
    uint16_t slot[16][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[NW][C];
    float dsc[C];
    float g1[2][C], ku[2][C], b1[2][C], b2[2][C], zr[2][C], zc[4][C], dlam[2][C];
    float frob[NW];
    // Per token, from phase G: dG without the chunk-end term, dbeta, lam dlam, and
    // 1 where dg is kept (valid, not a reset); the |S0 dS| total.
    float hdg[C], hdb[C], hld[C], hkeep[C];
    float frs;
};

__device__ __forceinline__ uint4 load_mat(const uint16_t *src, int tid) {
    return *reinterpret_cast<const uint4 *>(src + (tid >> 3) * D + 8 * (tid & 7));
}

// One chunk's global inputs to bgrad, held in registers.  A workgroup walks
// several chunks and loads the next chunk's inputs while it computes the
// current one, in five parts spread over the phases so that no phase issues
// more than a few memory instructions per wave (a burst of them stalls issue
// for the whole CU).
struct BgradIn {
    uint4 q, k, dO, s0, ds, s0l, dsl;  // S0^T and dS^T rows: bf16 hi and lo
    float G, be, va, dsc;
    int sg;
    uint4 v, t;
    float4 d0, d1;
};

struct ChunkPos {
    int b, h, c;
};
__device__ __forceinline__ ChunkPos chunk_pos(const ChunkArgs &a, int ci) {
    const int bh = ci / a.nc;
    return ChunkPos{bh / a.H, bh % a.H, ci % a.nc};
}

// Part P of chunk ci's inputs: 0 q, k; 1 dO, S0^T; 2 dS^T, the gates, the score
// adjoint; 3 V, T; 4 delta.  The loads take no branch, so that the compiler's
// memory-counter waits stay exact across the chunk loop: a row past the
// sequence end reads the last row (the gate block marks such tokens invalid,
// and the staging zeroes invalid rows), a missing dO reads q (zeroed at the
// staging) and a missing score adjoint reads the delta checkpoint, which holds
// more than B*T*H floats (the value is then never used).
template <int P>
__device__ __forceinline__ void bgrad_load(const ChunkArgs &a, int ci, const ChunkPos &p, int tid,
                                           BgradIn &x) {
    const int t = tid & 63, cb = tid >> 6, tg = p.c * C + t;
    const int tr = tg < a.T ? tg : a.T - 1;
    if constexpr (P == 0) {
        x.q = *reinterpret_cast<const uint4 *>(row_ptr(a.q, a.qs, p.b, tr, p.h) + 8 * cb);
        x.k = *reinterpret_cast<const uint4 *>(row_ptr(a.k, a.ks, p.b, tr, p.h) + 8 * cb);
    } else if constexpr (P == 1) {
        const uint16_t *dop = a.dout ? a.dout : a.q;
        const int64_t *dos = a.dout ? a.ds : a.qs;
        x.dO = *reinterpret_cast<const uint4 *>(row_ptr(dop, dos, p.b, tr, p.h) + 8 * cb);
        x.s0 = load_mat(a.ck_state + (int64_t)ci * D * D, tid);
        x.s0l = load_mat(a.ck_state_lo + (int64_t)ci * D * D, tid);
    } else if constexpr (P == 2) {
        x.ds = load_mat(a.ws_dstate + (int64_t)ci * D * D, tid);
        x.dsl = load_mat(a.ws_dstate_lo + (int64_t)ci * D * D, tid);
        const GateBlock *gb = a.ck_gate + ci;
        x.G = gb->G[t], x.be = gb->beta[t], x.va = gb->val[t];
        x.sg = gb->seg[t];
        x.dsc = (a.dscores ? a.dscores : a.ck_delta)[((int64_t)p.b * a.T + tr) * a.H + p.h];
    } else if constexpr (P == 3) {
        x.v = *reinterpret_cast<const uint4 *>(row_ptr(a.v, a.vs, p.b, tr, p.h) + 8 * cb);
        x.t = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
    } else {
        const float *dck = a.ck_delta + (int64_t)ci * C * D + t * D + 8 * cb;
        x.d0 = *reinterpret_cast<const float4 *>(dck);
        x.d1 = *reinterpret_cast<const float4 *>(dck + 4);
    }
}

}  // namespace

// The backward state recurrence is affine too: with
//   X = P^T dO + diag(c) delta,  Y = (gam Q)^T dO,  W = T diag(beta gam) K,
//   ddelta = X + diag(lam) K dS_C  and  dS0 = gam_63 dS_C + Y - W^T ddelta,
// so dS0 = M dS_C + N with M = gam_63 I - W^T diag(lam) K = A_c^T and
// N = Y - W^T X.  M and T come from the forward prep, delta from the forward
// output kernel; bprep forms W = T (beta gam K) again (the same operands and
// products as prep, so the same bits) and builds N for every chunk in parallel.
__global__ void __launch_bounds__(NT) chunk_bprep_kernel(ChunkArgs a) {
    __shared__ BPrepSmem sm;
    // Tiles are staged as rows and read across with transpose reads where a
    // product needs them transposed.
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *dOs = sm.slot[2];
    uint16_t *Tb = sm.slot[3], *KBGs = sm.slot[4], *Pt = sm.slot[5], *Ptl = sm.slot[6];
    uint16_t *KBGl = sm.slot[7];  // beta gam K lo rows
    uint16_t *Xt = sm.slot[0], *Xtl = sm.slot[1];  // over Q/K after phase 1
    uint16_t *Wt = sm.slot[3], *Wtl = sm.slot[4];  // over T and beta gam K after phase 1
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);
    const int tg = c * C + t;
    const bool inb = tg < a.T;
    const GateBlock *gb = a.ck_gate + ci;
    const float *dck = a.ck_delta + (int64_t)ci * C * D;
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    // Loads in order of use: phase 1's operands (T among them), then delta
    // (phase 2); W is formed in phase 1 and written to LDS in phase 2.
    const uint4 qr = load8(a.q, a.qs, b, tg, h, cb, inb);
    const uint4 kr = load8(a.k, a.ks, b, tg, h, cb, inb);
    const uint4 dor = a.dout ? load8(a.dout, a.ds, b, tg, h, cb, inb) : make_uint4(0, 0, 0, 0);
    const uint4 trow = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C +
                                                         (tid >> 3) * C + 8 * (tid & 7));
    const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
    const int sg = gb->seg[t];
    const float dsc = (a.dscores && inb && w == 0) ? a.dscores[((int64_t)b * a.T + tg) * a.H + h] : 0.f;
    // The score adjoint's term c delta (and the norms c needs) only exists when a
    // score adjoint is given; a.dscores is uniform, so the branches cost nothing.
    const bool score_adj = a.dscores != nullptr;
    float4 d0 = make_float4(0.f, 0.f, 0.f, 0.f), d1 = d0;
    float dl[2][4] = {};  // delta at this wave's X tile, used in phase 2
    if (score_adj) {
        d0 = *reinterpret_cast<const float4 *>(dck + t * D + 8 * cb);
        d1 = *reinterpret_cast<const float4 *>(dck + t * D + 8 * cb + 4);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) dl[j][i] = dck[(r0 + i) * D + 16 * (tn0 + j) + acc_col()];
    }
    {
        const bool on = va != 0.f;
        const float gam = sg == 0 ? __expf(G) : 0.f, bg = be * gam;
        Pack8 qp, kp;
        qp.u = mask8(qr, on);
        kp.u = mask8(kr, on);
        put_row8(Qs, t, cb, qp.u);
        put_row8(Ks, t, cb, kp.u);
        put_row8(dOs, t, cb, mask8(dor, on));
        float ksq = 0.f;
        uint32_t kb[4], kbl[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float k0 = bf16_val(kp.h[e]), k1 = bf16_val(kp.h[e + 1]);
            uint16_t h0, l0, h1, l1;
            split_bf16(bg * k0, h0, l0);
            split_bf16(bg * k1, h1, l1);
            kb[e / 2] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            kbl[e / 2] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            ksq += k0 * k0 + k1 * k1;
        }
        put_row8(KBGs, t, cb, make_uint4(kb[0], kb[1], kb[2], kb[3]));
        put_row8(KBGl, t, cb, make_uint4(kbl[0], kbl[1], kbl[2], kbl[3]));
        *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = trow;
        if (score_adj) sm.kk[cb][t] = ksq;
        if (w == 0) {
            gates_derive(sm.gl, G, be, va, sg);
            sm.dsc[t] = dsc;
        }
    }
    __syncthreads();
    const RowGates rg = row_gates(sm.gl, tm);
    // Phase 1: P (causal tiles, masked) -> P^T hi/lo; Y = (gam Q)^T dO and
    // W = T (beta gam K) in registers.
    f32x4 yacc[2] = {zero4(), zero4()}, wacc[2] = {zero4(), zero4()};
    gemm2_tr(wacc, &Tb[(16 * tm) * LDB], KBGs, tn0);  // B[k][t] = (beta gam K)[t][k]
    gemm2_tr(wacc, &Tb[(16 * tm) * LDB], KBGl, tn0);
    {
        f32x4 pq[2] = {zero4(), zero4()};
#pragma unroll
        for (int r = 0; r < 64; r += 32) {  // Y[k][v] = sum_t (gam Q)[t][k] dO[t][v], gam Q hi/lo
            bf16x8_t x, xl;
            frag_tr_scaled_split(Qs, sm.gl.gam, r, 16 * tm, x, xl);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const bf16x8_t ob = frag_tr(dOs, r, 16 * (tn0 + j));
                yacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, ob, yacc[j], 0, 0, 0);
                yacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, ob, yacc[j], 0, 0, 0);
            }
        }
        if (tn0 <= tm) gemm2(pq, &Qs[(16 * tm) * LDB], Ks, tn0);
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
    if (score_adj)
        sm.dd[cb][t] = d0.x * d0.x + d0.y * d0.y + d0.z * d0.z + d0.w * d0.w + d1.x * d1.x +
                       d1.y * d1.y + d1.z * d1.z + d1.w * d1.w;
    __syncthreads();
    // Phase 2: X = P^T dO + diag(c) delta, stored transposed (hi/lo); W^T hi/lo.
#pragma unroll
    for (int j = 0; j < 2; ++j)
        store_tile_t_split(&Wt[(16 * (tn0 + j)) * LDB + 16 * tm],
                           &Wtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, wacc[j]);
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2_tr(x, &Pt[(16 * tm) * LDB], dOs, tn0);  // B[v][t] = dO[t][v]
        gemm2_tr(x, &Ptl[(16 * tm) * LDB], dOs, tn0);
        if (score_adj) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ss = r0 + i;
                float kq = 0.f, dq = 0.f;
#pragma unroll
                for (int q = 0; q < NW; ++q) {
                    kq += sm.kk[q][ss];
                    dq += sm.dd[q][ss];
                }
                const float nk = sqrtf(kq), nd = sqrtf(dq);
                const float cs = (nk > 0.f && nd > 0.f) ? sm.dsc[ss] * nk / nd : 0.f;
#pragma unroll
                for (int j = 0; j < 2; ++j) x[j][i] += cs * dl[j][i];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            store_tile_t_split(&Xt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Xtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        }
    }
    __syncthreads();
    // Phase 3: N = Y - W^T X.
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2(x, &Wt[(16 * tm) * LDB], Xt, tn0);
        gemm2(x, &Wt[(16 * tm) * LDB], Xtl, tn0);
        gemm2(x, &Wtl[(16 * tm) * LDB], Xt, tn0);
        float *Nt = a.ws_n + (int64_t)ci * D * D;  // N transposed: Nt[col][row], f32
#pragma unroll
        for (int j = 0; j < 2; ++j)
            *reinterpret_cast<float4 *>(&Nt[(16 * (tn0 + j) + acc_col()) * D + 16 * tm + acc_row(0)]) =
                make_float4(yacc[j][0] - x[j][0], yacc[j][1] - x[j][1], yacc[j][2] - x[j][2],
                            yacc[j][3] - x[j][3]);
    }
}

// The stores of one bgrad chunk.  dq, dk, dv: lane (token 16 (w%4) + l%16,
// channels 32 (w/4) + 8 (l/16) ..) reads its eight channels across the
// transposed gradient tile (every lane runs the transpose reads) and stores one
// 16-byte row piece; dg, dbeta from wave 0's registers (lane l: token 63 - l).
__device__ __forceinline__ bf16x8_t bgrad_grad_frag(const uint16_t *tile, int w) {
    return frag_tr(tile, 32 * (w >> 2), 16 * (w & 3));
}
__device__ __forceinline__ void bgrad_store_rows(const ChunkArgs &a, const ChunkPos &p, int w,
                                                 bf16x8_t gq, bf16x8_t gk, bf16x8_t gv) {
    const int l = lane_id();
    const int tq = p.c * C + 16 * (w & 3) + (l & 15);
    if (tq < a.T) {
        const int64_t o = (((int64_t)p.b * a.T + tq) * a.H + p.h) * D + 32 * (w >> 2) + 8 * (l >> 4);
        if (a.dq) *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dq) + o) = gq;
        if (a.dk) *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dk) + o) = gk;
        if (a.dv) *reinterpret_cast<bf16x8_t *>(reinterpret_cast<uint16_t *>(a.dv) + o) = gv;
    }
}
__device__ __forceinline__ void bgrad_store_gates(const ChunkArgs &a, const ChunkPos &p, int w,
                                                  float dg, float db) {
    const int ts = p.c * C + 63 - lane_id();
    if (w == 0 && ts < a.T) {
        const int64_t o = ((int64_t)p.b * a.T + ts) * a.H + p.h;
        if (a.dg) a.dg[o] = dg;
        if (a.dbeta) a.dbeta[o] = db;
    }
}

// bgrad: every gradient of one chunk, given S0, the edits delta (forward
// checkpoint) and dS at the chunk end (adjoint scan).  Phases between barriers:
//   A  dO S0^T, K dS, KK^T, QK^T (registers); P^T -> LDS
//   D  delta dS^T (-> dlam); ddelta = P^T dO + lam K dS + c delta -> LDS
//   E  dR = T^T ddelta -> dV, dbeta (sum dR v), dR rows
//   F  dR S0^T (-> dK, dbeta, dgam); dA, dP masked -> MA^T, MP^T
//   G  dQ = MP K + gam dO S0^T;  dK = (MA + MA^T) K + MP^T Q + ...
//   H  gate gradients: dbeta, and dg by a reverse scan of dG (wave 0)
// The grid holds one workgroup per CU (the LDS allows no more), each walking
// chunks blockIdx.x, blockIdx.x + gridDim.x, ...: the next chunk's inputs are
// loaded into registers while the current chunk computes, so the load latency
// that starts every chunk is paid once per workgroup instead of once per chunk.
// A chunk's stores are issued after the next chunk's staging, so that the
// staging's wait on its (older) loads never waits on stores.
// SCORE: a score adjoint is given; its terms (c delta in ddelta, c' k in dk and the
// norms behind them) are compiled in only then.
template <bool SCORE>
__global__ void __launch_bounds__(NT) chunk_bgrad_kernel(ChunkArgs a, int nchunks) {
    __shared__ BGradSmem sm;
    // Every input tile is staged once, in the orientation it is stored in (rows
    // of Q, K, dO, V, T; S0^T and dS^T as checkpointed), and read the other way
    // with transpose reads.
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *dOs = sm.slot[2];
    uint16_t *Vr = sm.slot[6], *Tr = sm.slot[7];     // V rows, T rows (T[t][s])
    uint16_t *S0t = sm.slot[8], *dSt = sm.slot[9];   // S0^T, dS^T rows (bf16 hi)
    uint16_t *S0lt = sm.slot[15];                    // S0^T lo, staging..F
    uint16_t *dSlt = sm.slot[10];                    // dS^T lo, staging..D
    uint16_t *Dh = sm.slot[11], *Dlo = sm.slot[12];  // delta rows (hi/lo)
    uint16_t *Pt = sm.slot[13], *Ptl = sm.slot[14];  // A..D
    // Later tenants of free or dead slots.
    uint16_t *Dd = sm.slot[3], *Ddl = sm.slot[4];  // ddelta^T, D..E
    uint16_t *dRr = sm.slot[9], *dRl = sm.slot[14];  // dR rows (hi, lo), E..F
    // F..G: MA and MP are stored transposed only; phase G reads them both ways.
    uint16_t *MAt = sm.slot[4], *MAtl = sm.slot[6], *MPt = sm.slot[7], *MPtl = sm.slot[10];
    // Gradients, G to the next chunk's staging: slots that phase G does not read and
    // the staging does not write.
    uint16_t *dQt = sm.slot[3], *dKt = sm.slot[5], *dVt = sm.slot[13];
    constexpr bool score_adj = SCORE;
    BgradIn in;
    {
        const ChunkPos p0 = chunk_pos(a, blockIdx.x);
        bgrad_load<0>(a, blockIdx.x, p0, threadIdx.x, in);
        bgrad_load<1>(a, blockIdx.x, p0, threadIdx.x, in);
        bgrad_load<2>(a, blockIdx.x, p0, threadIdx.x, in);
        bgrad_load<3>(a, blockIdx.x, p0, threadIdx.x, in);
        bgrad_load<4>(a, blockIdx.x, p0, threadIdx.x, in);
    }
    float pdg = 0.f, pdb = 0.f;  // wave 0: the previous chunk's dg, dbeta (lane t: token 63 - t)
    for (int ci = blockIdx.x; ci < nchunks; ci += gridDim.x) {
    // An opaque zero keeps the wave- and lane-dependent address arithmetic of
    // the body inside the loop: hoisted out, it would stay live across it and
    // exhaust the registers.
    int zero;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
    const ChunkArgs &a = chunk_args_reloaded();
    const int tid = threadIdx.x + zero, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    // The next chunk of this workgroup.  Past the end the loads need no branch
    // either: every lane of a load reads the first element of this chunk's
    // source (thread index 0 for the addressing), so each load instruction
    // touches one cache line that the chunk itself has just read.
    const bool live = ci + (int)gridDim.x < nchunks;
    const int cn = live ? ci + (int)gridDim.x : ci, tn = live ? tid : 0;
    const ChunkPos pn = chunk_pos(a, cn);
    // The previous chunk (stored during this one) and whether there is one.
    const bool prev = ci != (int)blockIdx.x;
    const ChunkPos pp = chunk_pos(a, prev ? ci - (int)gridDim.x : ci);
    // Phase A's tiles go to LDS before the first barrier; the rest (V, T, delta)
    // after phase A.  Each part's registers then take the next chunk's loads.
    const bool on = in.va != 0.f;
    {
        const uint4 q8 = mask8(in.q, on), k8 = mask8(in.k, on), d8 = mask8(in.dO, on && a.dout);
        put_row8(Qs, t, cb, q8);
        put_row8(Ks, t, cb, k8);
        put_row8(dOs, t, cb, d8);
        if (score_adj) {
            Pack8 kp;
            kp.u = k8;
            float ksq = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float kf = bf16_val(kp.h[e]);
                ksq += kf * kf;
            }
            sm.kk[cb][t] = ksq;
        }
        *reinterpret_cast<uint4 *>(&S0t[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.s0;
        *reinterpret_cast<uint4 *>(&dSt[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.ds;
        *reinterpret_cast<uint4 *>(&S0lt[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.s0l;
        *reinterpret_cast<uint4 *>(&dSlt[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.dsl;
        if (w == 0) {
            gates_derive(sm.gl, in.G, in.be, in.va, in.sg);
            sm.dsc[t] = in.dsc;
        }
    }
    // |S0 dS| partial; written after the barrier, when the previous chunk's phase H
    // (wave 0) has read the last one.
    const float fr = wave_sum(dot8_bf16(in.s0, in.ds) + dot8_bf16(in.s0l, in.ds) + dot8_bf16(in.s0, in.dsl));
    // The previous chunk's dv tile is read now: phase A writes P^T over it.
    const bf16x8_t gv = bgrad_grad_frag(dVt, w);
    bgrad_load<0>(a, cn, pn, tn, in);
    __syncthreads();
    if (lane_id() == 0) sm.frob[w] = fr;
    const RowGates rg = row_gates(sm.gl, tm);
    float lmv[4];
    {
        const float4 lm = lds_f4(&sm.gl.lam[r0]);
        lmv[0] = lm.x, lmv[1] = lm.y, lmv[2] = lm.z, lmv[3] = lm.w;
    }
    // Phase A: dO S0^T, lam K dS, KK^T, QK^T in registers; P^T (hi/lo) -> LDS.
    float gmA[2][4];  // Gam at this wave's tiles, formed here and reused in phase F
    f32x4 dos[2] = {zero4(), zero4()}, kds[2] = {zero4(), zero4()};
    f32x4 kk[2] = {zero4(), zero4()}, qk[2] = {zero4(), zero4()};
    gemm2_tr(dos, &dOs[(16 * tm) * LDB], S0t, tn0);  // B[k][v] = S0^T[v][k]
    gemm2_tr(dos, &dOs[(16 * tm) * LDB], S0lt, tn0);
    gemm2(kds, &Ks[(16 * tm) * LDB], dSt, tn0);
    gemm2(kds, &Ks[(16 * tm) * LDB], dSlt, tn0);
    if (tn0 <= tm) {
        gemm2(kk, &Ks[(16 * tm) * LDB], Ks, tn0);
        gemm2(qk, &Qs[(16 * tm) * LDB], Ks, tn0);
    }
    {
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
            float qv[4];
            ld4_rm_tr(Qs, 16 * tm, 16 * (tn0 + j), qv);
            f32x4 pq = qk[j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                kds[j][i] *= lmv[i];
                p[i] += qv[i] * dos[j][i];  // q_t . (dO S0^T)_t
                gmA[j][i] = (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
                pq[i] *= gmA[j][i];
            }
            store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq);
        }
        row_reduce_store(p, sm.g1[w & 1], tm);
    }
    {  // second half of the staging: operands of phases D-G that A does not read
        put_row8(Vr, t, cb, mask8(in.v, on));
        *reinterpret_cast<uint4 *>(&Tr[(tid >> 3) * LDB + 8 * (tid & 7)]) = in.t;
        const float x[8] = {in.d0.x, in.d0.y, in.d0.z, in.d0.w, in.d1.x, in.d1.y, in.d1.z, in.d1.w};
        Pack8 ph, pl;
        float dsq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            split_bf16(x[e], ph.h[e], pl.h[e]);
            dsq += x[e] * x[e];
        }
        put_row8(Dh, t, cb, ph.u);
        put_row8(Dlo, t, cb, pl.u);
        if (score_adj) sm.dd[cb][t] = dsq;
    }
    // The previous chunk's dq, dk, dv rows, then the next chunk's V and T.
    if (prev) bgrad_store_rows(a, pp, w, bgrad_grad_frag(dQt, w), bgrad_grad_frag(dKt, w), gv);
    bgrad_load<3>(a, cn, pn, tn, in);
    __syncthreads();
    bgrad_load<1>(a, cn, pn, tn, in);
    if (prev) bgrad_store_gates(a, pp, w, pdg, pdb);
    // Phase D: delta dS^T (-> dlam), ddelta = P^T dO + lam K dS + c delta (-> ddelta^T).
    float cs[4] = {0.f, 0.f, 0.f, 0.f}, ck[4] = {0.f, 0.f, 0.f, 0.f};
    if (score_adj) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ss = r0 + i;
            float kq = 0.f, dq = 0.f;
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                kq += sm.kk[q][ss];
                dq += sm.dd[q][ss];
            }
            const float nk = sqrtf(kq), nd = sqrtf(dq);
            const bool ok = nk > 0.f && nd > 0.f;
            cs[i] = ok ? sm.dsc[ss] * nk / nd : 0.f;
            ck[i] = ok ? sm.dsc[ss] * nd / nk : 0.f;
        }
    }
    // dK accumulates lam (delta dS^T) here, -beta gam dR S0^T in F, the rest in G.
    f32x4 dka[2] = {zero4(), zero4()};
    {
        gemm2_tr(dka, &Dh[(16 * tm) * LDB], dSt, tn0);  // B[k][v] = dS^T[v][k]
        gemm2_tr(dka, &Dlo[(16 * tm) * LDB], dSt, tn0);
        gemm2_tr(dka, &Dh[(16 * tm) * LDB], dSlt, tn0);
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4];
            ld4_rm_tr(Ks, 16 * tm, 16 * (tn0 + j), kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] += kv[i] * dka[j][i];
                dka[j][i] *= lmv[i];
            }
        }
        row_reduce_store(p, sm.dlam[w & 1], tm);
        f32x4 x[2] = {kds[0], kds[1]};
        gemm2_tr(x, &Pt[(16 * tm) * LDB], dOs, tn0);  // B[v][t] = dO[t][v]
        gemm2_tr(x, &Ptl[(16 * tm) * LDB], dOs, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (score_adj) {
                float dh[4], dlo[4];  // delta at this tile: hi + lo rows
                ld4_rm_tr(Dh, 16 * tm, 16 * (tn0 + j), dh);
                ld4_rm_tr(Dlo, 16 * tm, 16 * (tn0 + j), dlo);
#pragma unroll
                for (int i = 0; i < 4; ++i) x[j][i] += cs[i] * (dh[i] + dlo[i]);
            }
            store_tile_t_split(&Dd[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ddl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        }
    }
    __syncthreads();
    bgrad_load<2>(a, cn, pn, tn, in);
    // Phase E: dR = T^T ddelta -> dV (kept for the stores), dbeta (sum_v dR v part), dR rows.
    f32x4 dvv[2];
    {
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
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float vv[4];
            ld4_rm_tr(Vr, 16 * tm, 16 * (tn0 + j), vv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] += x[j][i] * vv[i];
                dvv[j][i] = sm.gl.val[r0 + i] != 0.f ? rg.beta[i] * x[j][i] : 0.f;
            }
            store_tile_rm_split(&dRr[(16 * tm) * LDB + 16 * (tn0 + j)], &dRl[(16 * tm) * LDB + 16 * (tn0 + j)],
                                LDB, x[j]);
        }
        row_reduce_store(p, sm.b2[w & 1], tm);
    }
    __syncthreads();
    bgrad_load<4>(a, cn, pn, tn, in);
    // Phase F: dR S0^T (-> dK; sum_k k dR S0^T -> dbeta and dgam), dA and dP
    // (masked) -> MA^T, MP^T, and the gate-gradient partial sums.
    f32x4 drs[2] = {zero4(), zero4()};
    gemm2_tr(drs, &dRr[(16 * tm) * LDB], S0t, tn0);  // B[k][v] = S0^T[v][k]
    gemm2_tr(drs, &dRr[(16 * tm) * LDB], S0lt, tn0);
    gemm2_tr(drs, &dRl[(16 * tm) * LDB], S0t, tn0);
    {
        float p2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4];
            ld4_rm_tr(Ks, 16 * tm, 16 * (tn0 + j), kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p2[i] += kv[i] * drs[j][i];
                dka[j][i] -= rg.beta[i] * rg.gam[i] * drs[j][i];
            }
        }
        row_reduce_store(p2, sm.ku[w & 1], tm);
    }
    {
        f32x4 da[2] = {zero4(), zero4()}, dp[2] = {zero4(), zero4()};
        if (tn0 <= tm) {
            gemm2(da, &dRr[(16 * tm) * LDB], Dh, tn0);
            gemm2(da, &dRr[(16 * tm) * LDB], Dlo, tn0);
            gemm2(da, &dRl[(16 * tm) * LDB], Dh, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dh, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dlo, tn0);
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
            store_tile_t_split(&MAt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &MAtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, ma);
            store_tile_t_split(&MPt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &MPtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, mp);
            const float zc = col_reduce(z);
            if ((lane_id() >> 4) == 0) sm.zc[tm][ss] = zc;
        }
        row_reduce_store(pb, sm.b1[w & 1], tm);
        row_reduce_store(pz, sm.zr[w & 1], tm);
    }
    __syncthreads();
    // Every per-token term of the gate gradients is in LDS now: each wave sums
    // those of 8 tokens while phase G's products run.  With u_t = k_t . (dR S0^T)_t:
    //   dbeta_t = sum dA Gam KK^T + sum_v dR v - gam_t u_t,
    //   dG_t   = row - column sums of Z + gam_t (q_t . (dO S0^T)_t - beta_t u_t) - lam_t dlam_t
    // (plus, for the last token, the chunk-end term added in phase H).
    {  // straight-line (every lane computes token 8w + l%8), so it interleaves with phase G
        const int s = 8 * w + (lane_id() & 7);
        const float gam = sm.gl.gam[s], lam = sm.gl.lam[s], bet = sm.gl.beta[s];
        const float dlam = sm.dlam[0][s] + sm.dlam[1][s];
        const float u = sm.ku[0][s] + sm.ku[1][s];
        const float dG = sm.zr[0][s] + sm.zr[1][s] - (sm.zc[0][s] + sm.zc[1][s] + sm.zc[2][s] + sm.zc[3][s]) +
                         gam * (sm.g1[0][s] + sm.g1[1][s] - bet * u) - lam * dlam;
        const bool on = sm.gl.val[s] != 0.f;
        const int sgp = sm.gl.seg[s > 0 ? s - 1 : 0];
        const bool rs = on && (s == 0 ? sm.gl.seg[0] == 1 : sm.gl.seg[s] != sgp);
        const float db = on ? sm.b1[0][s] + sm.b1[1][s] + sm.b2[0][s] + sm.b2[1][s] - gam * u : 0.f;
        float fr = 0.f;
#pragma unroll
        for (int q = 0; q < NW; ++q) fr += sm.frob[q];
        if (lane_id() < 8) {
            sm.hdg[s] = dG;
            sm.hdb[s] = db;
            sm.hld[s] = lam * dlam;
            sm.hkeep[s] = (on && !rs) ? 1.f : 0.f;
            if (s == 0) sm.frs = fr;
        }
    }
    // Phase G: dQ and dK.
    {
        f32x4 x[2] = {zero4(), zero4()}, y[2] = {zero4(), zero4()};
#pragma unroll
        for (int r = 0; r < 64; r += 32) {
            // MP and MA rows, read across their transposes.
            const bf16x8_t mp = frag_tr(MPt, r, 16 * tm), mpl = frag_tr(MPtl, r, 16 * tm);
            const bf16x8_t ma = frag_tr(MAt, r, 16 * tm), mat = frag(&MAt[(16 * tm) * LDB], LDB, r);
            const bf16x8_t mal = frag_tr(MAtl, r, 16 * tm), matl = frag(&MAtl[(16 * tm) * LDB], LDB, r);
            const bf16x8_t pt = frag(&MPt[(16 * tm) * LDB], LDB, r), ptl = frag(&MPtl[(16 * tm) * LDB], LDB, r);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const bf16x8_t kb = frag_tr(Ks, r, 16 * (tn0 + j));  // B[k][s] = K[s][k]
                const bf16x8_t qb = frag_tr(Qs, r, 16 * (tn0 + j));  // B[k][t] = Q[t][k]
                x[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mp, kb, x[j], 0, 0, 0);
                x[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mpl, kb, x[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ma, kb, y[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mat, kb, y[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mal, kb, y[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(matl, kb, y[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pt, qb, y[j], 0, 0, 0);
                y[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ptl, qb, y[j], 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4] = {0.f, 0.f, 0.f, 0.f};
            if (score_adj) ld4_rm_tr(Ks, 16 * tm, 16 * (tn0 + j), kv);
            f32x4 gq, gk;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool on = sm.gl.val[r0 + i] != 0.f;
                gq[i] = on ? x[j][i] + rg.gam[i] * dos[j][i] : 0.f;
                gk[i] = on ? y[j][i] + dka[j][i] + ck[i] * kv[i] : 0.f;
            }
            // Transposed gradient tiles ([channel][token]) in slots phase G does not read.
            store_tile_t(&dQt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, gq);
            store_tile_t(&dKt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, gk);
            store_tile_t(&dVt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, dvv[j]);
        }
    }
    __syncthreads();  // gradient tiles complete: the next iteration stores them
    // Phase H (wave 0): dg by a reverse scan of dG.  Lane t holds token s = 63 - t,
    // so a forward scan over lanes sums suffixes: dg_s = sum_{r >= s} dG_r.
    if (w == 0) {
        const int s = 63 - t;
        float dG = sm.hdg[s];
        const float tail = wave_sum(sm.hld[s]);
        if (s == 63) dG += tail + sm.gl.gamC * sm.frs;
        const float x = wave_scan_add(dG);
        pdg = sm.hkeep[s] != 0.f ? x : 0.f;
        pdb = sm.hdb[s];
    }
    // No barrier here: the next staging writes no LDS that the stores or phase H
    // read (the per-token sums phase H reads are rewritten only in the next
    // chunk's phase G, after a barrier that wave 0 reaches after phase H).
    }
    {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int last = blockIdx.x + (nchunks - 1 - (int)blockIdx.x) / (int)gridDim.x * gridDim.x;
        const ChunkArgs &a = chunk_args_reloaded();
        const ChunkPos pl = chunk_pos(a, last);
        bgrad_store_rows(a, pl, w, bgrad_grad_frag(dQt, w), bgrad_grad_frag(dKt, w), bgrad_grad_frag(dVt, w));
        bgrad_store_gates(a, pl, w, pdg, pdb);
    }
}

int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            return 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t launch_chunk_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev) {
    const int nchunks = a.B * a.H * a.nc;
    mark(ev, 0, stream);
    hipLaunchKernelGGL(chunk_bprep_kernel, dim3(nchunks), dim3(NT), 0, stream, a);
    mark(ev, 1, stream);
    mark(ev, 2, stream);
    (void)launch_chunk_scan(a, true, stream);
    mark(ev, 3, stream);
    mark(ev, 4, stream);
    if (a.dscores)
        hipLaunchKernelGGL(chunk_bgrad_kernel<true>, dim3(std::min(nchunks, device_cus())), dim3(NT), 0, stream, a,
                           nchunks);
    else
        hipLaunchKernelGGL(chunk_bgrad_kernel<false>, dim3(std::min(nchunks, device_cus())), dim3(NT), 0, stream,
                           a, nchunks);
    mark(ev, 5, stream);
    return hipGetLastError();
}

}  // namespace gdn2
