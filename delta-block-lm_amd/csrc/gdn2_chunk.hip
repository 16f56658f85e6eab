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
#include "gdn2_chunk.h"
#include "gdn2_mfma.h"

namespace gdn2 {

namespace {

constexpr int C = CHUNK;
constexpr int D = CHUNK_D;
constexpr int NW = 8, NT = 64 * NW;
constexpr int LDB = 72;  // bf16 row stride of a 64x64 LDS tile
constexpr int LDF = 68;  // fp32 row stride
constexpr int LDX = 17;
constexpr int TILE = 64 * LDB;

struct GateLds {
    float G[C], beta[C], val[C], gam[C], lam[C];
    int seg[C];
    float gamC;
};

union Pack8 {
    uint4 u;
    uint16_t h[8];
};

__device__ __forceinline__ const uint16_t *row_ptr(const uint16_t *base, const int64_t *s, int b,
                                                   int t, int h) {
    return base + (int64_t)b * s[0] + (int64_t)t * s[1] + (int64_t)h * s[2];
}

// Channels [8cb, 8cb+8) of token tg; zero beyond the sequence.
__device__ __forceinline__ uint4 load8(const uint16_t *base, const int64_t *s, int b, int tg, int h,
                                       int cb, bool inb) {
    return inb ? *reinterpret_cast<const uint4 *>(row_ptr(base, s, b, tg, h) + 8 * cb)
               : make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ uint4 mask8(uint4 v, bool on) {
    return on ? v : make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ void put_row8(uint16_t *tile, int t, int cb, uint4 v) {
    *reinterpret_cast<uint4 *>(&tile[t * LDB + 8 * cb]) = v;
}

__device__ __forceinline__ void put_col8(uint16_t *tile, int t, int cb, uint4 v) {
    Pack8 p;
    p.u = v;
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[(8 * cb + e) * LDB + t] = p.h[e];
}

// Inclusive wave scans (64 lanes).
__device__ __forceinline__ float wave_scan_add(float x) {
    const int l = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d);
        if (l >= d) x += y;
    }
    return x;
}
__device__ __forceinline__ int wave_scan_add(int x) {
    const int l = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (l >= d) x += y;
    }
    return x;
}

// Wave 0 (lane == token): decays derived from a gate block.
__device__ __forceinline__ void gates_derive(GateLds &gl, float G, float beta, float val, int seg) {
    const int t = lane_id();
    const float G63 = __shfl(G, 63);
    const int seg63 = __shfl(seg, 63);
    gl.G[t] = G;
    gl.beta[t] = beta;
    gl.val[t] = val;
    gl.seg[t] = seg;
    gl.gam[t] = seg == 0 ? __expf(G) : 0.f;
    gl.lam[t] = seg == seg63 ? __expf(G63 - G) : 0.f;
    if (t == 0) gl.gamC = seg63 == 0 ? __expf(G63) : 0.f;
}

// Per-lane view of the four accumulator rows (tokens) a tile covers.
struct RowGates {
    float G[4], beta[4], gam[4];
    int seg[4];
};
__device__ __forceinline__ RowGates row_gates(const GateLds &gl, int tm) {
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    RowGates r;
    const float4 G = *reinterpret_cast<const float4 *>(&gl.G[r0]);
    const float4 be = *reinterpret_cast<const float4 *>(&gl.beta[r0]);
    const float4 ga = *reinterpret_cast<const float4 *>(&gl.gam[r0]);
    const int4 sg = *reinterpret_cast<const int4 *>(&gl.seg[r0]);
    r.G[0] = G.x, r.G[1] = G.y, r.G[2] = G.z, r.G[3] = G.w;
    r.beta[0] = be.x, r.beta[1] = be.y, r.beta[2] = be.z, r.beta[3] = be.w;
    r.gam[0] = ga.x, r.gam[1] = ga.y, r.gam[2] = ga.z, r.gam[3] = ga.w;
    r.seg[0] = sg.x, r.seg[1] = sg.y, r.seg[2] = sg.z, r.seg[3] = sg.w;
    return r;
}

// acc[j] += X[16 rows][0:64] * Y[16 rows of tile (tn0 + j)][0:64]^T, j = 0, 1.
__device__ __forceinline__ void gemm2(f32x4 (&acc)[2], const uint16_t *X, const uint16_t *Y,
                                      int tn0) {
    const uint16_t *Y0 = Y + (16 * tn0) * LDB, *Y1 = Y0 + 16 * LDB;
    const bf16x8_t x0 = frag(X, LDB, 0), x1 = frag(X, LDB, 32);
    const bf16x8_t a0 = frag(Y0, LDB, 0), a1 = frag(Y0, LDB, 32);
    const bf16x8_t b0 = frag(Y1, LDB, 0), b1 = frag(Y1, LDB, 32);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, a0, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, b0, acc[1], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, a1, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, b1, acc[1], 0, 0, 0);
}

// Four consecutive bf16 of one LDS row as floats.
__device__ __forceinline__ void ld4_bf16(const uint16_t *p, float (&o)[4]) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    o[0] = bf16_val((uint16_t)(v.x & 0xffff));
    o[1] = bf16_val((uint16_t)(v.x >> 16));
    o[2] = bf16_val((uint16_t)(v.y & 0xffff));
    o[3] = bf16_val((uint16_t)(v.y >> 16));
}

// T = (I + A)^-1 for the strictly lower 64x64 A in Af; result in Tf (lower
// blocks).  Called by all waves; ends with a barrier.  Blocks are 16x16:
//   1. diagonal blocks T_bb = (I + A_bb)^-1 by forward substitution (waves 0-3,
//      four lanes per column share each row's dot product);
//   2. T_10 = -T_11 A_10 T_00 and T_32 = -T_33 A_32 T_22;
//   3. T_21 (32x32, blocks r = 2,3 x c = 0,1) = -T_22(32) A_21(32) T_11(32).
__device__ void ut_inverse(const float *Af, float *Tf, float (*Xs)[16 * LDX], int w) {
    const int l = lane_id();
    if (w < 4) {
        // Lane (col, part) holds rows part, part+4, part+8, part+12 of column col;
        // the four parts of a column split each row's dot product.
        const int col = l & 15, part = l >> 4;
        const float *Ab = Af + (16 * w) * LDF + 16 * w;
        float Tq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int s = part + 4 * m;
                if (s < r) acc += Ab[r * LDF + s] * Tq[m];
            }
            acc += __shfl_xor(acc, 16);
            acc += __shfl_xor(acc, 32);
            if ((r & 3) == part) Tq[r >> 2] = (r == col ? 1.f : 0.f) - acc;
        }
        float *Tb = Tf + (16 * w) * LDF + 16 * w;
#pragma unroll
        for (int m = 0; m < 4; ++m) Tb[(part + 4 * m) * LDF + col] = Tq[m];
    }
    __syncthreads();
    auto blkA = [&](int r, int c) { return Af + (16 * r) * LDF + 16 * c; };
    auto blkT = [&](int r, int c) { return Tf + (16 * r) * LDF + 16 * c; };
    if (w < 2) {  // X = A_{2w+1,2w} T_{2w,2w}
        f32x4 x = zero4();
        mm16_f32(x, blkA(2 * w + 1, 2 * w), LDF, blkT(2 * w, 2 * w), LDF);
#pragma unroll
        for (int i = 0; i < 4; ++i) Xs[w][acc_row(i) * LDX + acc_col()] = x[i];
    }
    __syncthreads();
    if (w < 2) {  // T_{2w+1,2w} = -T_{2w+1,2w+1} X
        f32x4 y = zero4();
        mm16_f32(y, blkT(2 * w + 1, 2 * w + 1), LDF, Xs[w], LDX);
        float *dst = blkT(2 * w + 1, 2 * w);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[acc_row(i) * LDF + acc_col()] = -y[i];
    }
    __syncthreads();
    const int r = 2 + (w >> 1), c = w & 1;
    if (w < 4) {  // Y_rc = sum_{m=c..1} A_rm T_mc
        f32x4 x = zero4();
        for (int m = c; m < 2; ++m) mm16_f32(x, blkA(r, m), LDF, blkT(m, c), LDF);
#pragma unroll
        for (int i = 0; i < 4; ++i) Xs[w][acc_row(i) * LDX + acc_col()] = x[i];
    }
    __syncthreads();
    if (w < 4) {  // T_rc = -sum_{m=2..r} T_rm Y_mc
        f32x4 y = zero4();
        for (int m = 2; m <= r; ++m) mm16_f32(y, blkT(r, m), LDF, Xs[2 * (m - 2) + c], LDX);
        float *dst = blkT(r, c);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[acc_row(i) * LDF + acc_col()] = -y[i];
    }
    __syncthreads();
}

struct PrepSmem {
    uint16_t Ks[TILE];
    float Af[C * LDF];
    float Tf[C * LDF];
    float Xs[4][16 * LDX];
    GateLds gl;
};

struct StateSmem {
    uint16_t Ks[TILE];  // [t][i]
    uint16_t Kl[TILE];  // [i][t] = lam_t k_t[i]
    uint16_t Vt[TILE];  // [j][t]; then the low half of R^T (in place)
    uint16_t Tb[TILE];  // [t][s]
    uint16_t St[TILE];  // [j][i] = S0[i][j]
    uint16_t Rt[TILE];  // [j][t] high half of R^T
    uint16_t Dt[TILE];  // [j][t] high half of delta^T
    uint16_t Dl[TILE];  // low half
    float gam[C], beta[C];
    float gamC;
};

struct OutSmem {
    uint16_t slot[8][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[2][C];
};

// Chunk-start state, transposed to bf16 St[j][i], from a row-major f32 64x64.
__device__ __forceinline__ void load_state_t(uint16_t *St, const float *S0, int tid) {
    const int i = tid >> 3, j0 = 8 * (tid & 7);
    const float4 *src = reinterpret_cast<const float4 *>(S0 + i * D + j0);
    const float4 v0 = src[0], v1 = src[1];
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) St[(j0 + e) * LDB + i] = bf16_bits(v[e]);
}

}  // namespace

// ---- prep: gates and the UT inverse of every chunk ----------------------------
__global__ void __launch_bounds__(NT) chunk_prep_kernel(ChunkArgs a) {
    __shared__ PrepSmem sm;
    const int tid = threadIdx.x, w = tid >> 6;
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tg = c * C + t;
    const bool inb = tg < a.T;
    // Every load issued up front; masks are applied once the values arrive.
    const uint4 kraw = load8(a.k, a.ks, b, tg, h, cb, inb);
    const float vld = inb ? ld4<float>(a.valid, b, tg, 0, 0) : 0.f;
    float rst = 0.f, gt = 0.f, bt = 0.f;
    if (w == 0 && inb) {
        rst = ld4<float>(a.reset, b, tg, 0, 0);
        gt = ld4<float>(a.g, b, tg, h, 0);
        bt = ld4<float>(a.beta, b, tg, h, 0);
    }
    const bool on = vld != 0.f;
    put_row8(sm.Ks, t, cb, mask8(kraw, on));
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
    // A = strict_lower(beta_t Gam_ts k_t.k_s) in f32 (tiles with tn <= tm only).
    {
        const int tm = w >> 1, tn0 = 2 * (w & 1);
        if (tn0 <= tm) {
            f32x4 kk[2] = {zero4(), zero4()};
            gemm2(kk, &sm.Ks[(16 * tm) * LDB], sm.Ks, tn0);
            const RowGates rg = row_gates(sm.gl, tm);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int ss = 16 * (tn0 + j) + acc_col();
                const float Gs = sm.gl.G[ss];
                const int sgs = sm.gl.seg[ss];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tt = 16 * tm + acc_row(i);
                    const float v = (ss < tt && rg.seg[i] == sgs)
                                        ? rg.beta[i] * __expf(rg.G[i] - Gs) * kk[j][i]
                                        : 0.f;
                    sm.Af[tt * LDF + ss] = v;
                }
            }
        }
    }
    __syncthreads();
    ut_inverse(sm.Af, sm.Tf, sm.Xs, w);
    // T (bf16, row-major, zero above the diagonal) to the checkpoint.
    {
        const int r = tid >> 3, c0 = 8 * (tid & 7);
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s0 = c0 + 2 * e;
            pk[e] = bf16_pack2(s0 <= r ? sm.Tf[r * LDF + s0] : 0.f,
                               s0 + 1 <= r ? sm.Tf[r * LDF + s0 + 1] : 0.f);
        }
        *reinterpret_cast<uint4 *>(a.ck_t + (int64_t)ci * C * C + r * C + c0) =
            make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
}

// ---- state: the sequential inter-chunk recurrence -------------------------------
__global__ void __launch_bounds__(NT) chunk_state_kernel(ChunkArgs a) {
    __shared__ StateSmem sm;
    const int tid = threadIdx.x, w = tid >> 6;
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6;
    const int tm = w >> 1, tn0 = 2 * (w & 1);

    f32x4 Sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            Sacc[j][i] = a.initial.data ? ld4<float>(a.initial, b, h, 16 * tm + acc_row(i),
                                                     16 * (tn0 + j) + acc_col())
                                        : 0.f;

    // Register prefetch of one chunk: K/V rows, a T row segment, gate scalars.
    // None of these loads depends on another, so one chunk costs one latency.
    uint4 kr, vr, tr;
    float pG, pBeta, pVal, pG63;
    int pSeg, pSeg63;
    auto fetch = [&](int c) {
        const int64_t ci = (int64_t)bh * a.nc + c;
        const GateBlock *gb = a.ck_gate + ci;
        const int tg = c * C + t;
        kr = load8(a.k, a.ks, b, tg, h, cb, tg < a.T);
        vr = load8(a.v, a.vs, b, tg, h, cb, tg < a.T);
        tr = *reinterpret_cast<const uint4 *>(a.ck_t + ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
        pG = gb->G[t];
        pBeta = gb->beta[t];
        pVal = gb->val[t];
        pSeg = gb->seg[t];
        pG63 = gb->G[63];
        pSeg63 = gb->seg[63];
    };
    fetch(0);
    for (int c = 0; c < a.nc; ++c) {
        const int64_t ci = (int64_t)bh * a.nc + c;
        // Stage the prefetched chunk.
        {
            const bool on = pVal != 0.f;
            const uint4 k8 = mask8(kr, on);
            put_row8(sm.Ks, t, cb, k8);
            put_col8(sm.Vt, t, cb, mask8(vr, on));
            const float lam = pSeg == pSeg63 ? __expf(pG63 - pG) : 0.f;
            Pack8 kp;
            kp.u = k8;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                sm.Kl[(8 * cb + e) * LDB + t] = bf16_bits(lam * bf16_val(kp.h[e]));
            *reinterpret_cast<uint4 *>(&sm.Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = tr;
            if (w == 0) {
                sm.gam[t] = pSeg == 0 ? __expf(pG) : 0.f;
                sm.beta[t] = pBeta;
                if (t == 0) sm.gamC = pSeg63 == 0 ? __expf(pG63) : 0.f;
            }
        }
        // Chunk-start state: checkpoint (f32) and the bf16 transposed operand.
        float *ck = a.ck_state + ci * D * D;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ck[(16 * tm + acc_row(i)) * D + 16 * (tn0 + j) + acc_col()] = Sacc[j][i];
            store_tile_t(&sm.St[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, Sacc[j]);
        }
        if (c + 1 < a.nc) fetch(c + 1);
        __syncthreads();
        // R = beta (V - gam K S0), stored transposed (hi; lo over V^T in place).
        {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2(x, &sm.Ks[(16 * tm) * LDB], sm.St, tn0);
            const int r0 = 16 * tm + 4 * (lane_id() >> 4);
            const float4 be = *reinterpret_cast<const float4 *>(&sm.beta[r0]);
            const float4 ga = *reinterpret_cast<const float4 *>(&sm.gam[r0]);
            const float bev[4] = {be.x, be.y, be.z, be.w}, gav[4] = {ga.x, ga.y, ga.z, ga.w};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint16_t *vt = &sm.Vt[(16 * (tn0 + j)) * LDB + 16 * tm];
                float vv[4];
                ld4_bf16(vt + acc_col() * LDB + 4 * (lane_id() >> 4), vv);
#pragma unroll
                for (int i = 0; i < 4; ++i) x[j][i] = bev[i] * (vv[i] - gav[i] * x[j][i]);
                // Each lane overwrites exactly the V^T entries it just read.
                store_tile_t_split(&sm.Rt[(16 * (tn0 + j)) * LDB + 16 * tm], vt, LDB, x[j]);
            }
        }
        __syncthreads();
        // delta = T R.
        {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2(x, &sm.Tb[(16 * tm) * LDB], sm.Rt, tn0);
            gemm2(x, &sm.Tb[(16 * tm) * LDB], sm.Vt, tn0);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                store_tile_t_split(&sm.Dt[(16 * (tn0 + j)) * LDB + 16 * tm],
                                   &sm.Dl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        }
        __syncthreads();
        // S_C = gam_C S0 + (lam K)^T delta, in the accumulators.
        const float gC = sm.gamC;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) Sacc[j][i] *= gC;
        gemm2(Sacc, &sm.Kl[(16 * tm) * LDB], sm.Dt, tn0);
        gemm2(Sacc, &sm.Kl[(16 * tm) * LDB], sm.Dl, tn0);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a.final_state[((int64_t)bh * D + 16 * tm + acc_row(i)) * D + 16 * (tn0 + j) +
                          acc_col()] = Sacc[j][i];
}

// ---- out: outputs and scores of every chunk --------------------------------------
__global__ void __launch_bounds__(NT) chunk_out_kernel(ChunkArgs a) {
    __shared__ OutSmem sm;
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *Vt = sm.slot[2], *Tb = sm.slot[3];
    uint16_t *St = sm.slot[4], *Rt = sm.slot[5], *P = sm.slot[6], *Pl = sm.slot[7];
    uint16_t *Dt = sm.slot[0], *Dl = sm.slot[1];  // over Q/K after phase 1
    uint16_t *Os = sm.slot[4];                    // over S0^T after phase 1
    const int tid = threadIdx.x, w = tid >> 6;
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, t0 = c * C, tg = t0 + t;
    const int tm = w >> 1, tn0 = 2 * (w & 1);
    const GateBlock *gb = a.ck_gate + ci;
    const bool inb = tg < a.T;
    {
        const uint4 qr = load8(a.q, a.qs, b, tg, h, cb, inb);
        const uint4 kr = load8(a.k, a.ks, b, tg, h, cb, inb);
        const uint4 vr = load8(a.v, a.vs, b, tg, h, cb, inb);
        const uint4 trw =
            *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C + (tid >> 3) * C + 8 * (tid & 7));
        load_state_t(St, a.ck_state + (int64_t)ci * D * D, tid);
        const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
        const int sg = gb->seg[t];
        const bool on = va != 0.f;
        const uint4 k8 = mask8(kr, on);
        put_row8(Qs, t, cb, mask8(qr, on));
        put_row8(Ks, t, cb, k8);
        put_col8(Vt, t, cb, mask8(vr, on));
        *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = trw;
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
            store_tile_rm_split(&P[(16 * tm) * LDB + 16 * (tn0 + j)],
                                &Pl[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, pq[j]);
        }
    }
    __syncthreads();
    // Phase 2: delta = T R (-> Dt/Dl over the Q/K slots) and |delta_t|^2.
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2(x, &Tb[(16 * tm) * LDB], Rt, tn0);
        gemm2(x, &Tb[(16 * tm) * LDB], Vt, tn0);
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = x[0][i] * x[0][i] + x[1][i] * x[1][i];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile_t_split(&Dt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Dl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) p[i] += __shfl_xor(p[i], m);
            if (acc_col() == 0) sm.dd[w & 1][16 * tm + acc_row(i)] = p[i];
        }
    }
    __syncthreads();
    // Phase 3: O = gam Q S0 + P delta, staged through LDS for coalesced stores.
    {
        f32x4 x[2] = {qs[0], qs[1]};
        gemm2(x, &P[(16 * tm) * LDB], Dt, tn0);
        gemm2(x, &P[(16 * tm) * LDB], Dl, tn0);
        gemm2(x, &Pl[(16 * tm) * LDB], Dt, tn0);
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
    if (a.out_bf16) {
        __syncthreads();
        const int r = tid >> 3, c0 = 8 * (tid & 7), tq = t0 + r;
        if (tq < a.T)
            *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.out) +
                                       (((int64_t)b * a.T + tq) * a.H + h) * D + c0) =
                *reinterpret_cast<const uint4 *>(&Os[r * LDB + c0]);
    }
}

hipError_t launch_chunk_fwd(const ChunkArgs &a, hipStream_t stream) {
    const int nchunks = a.B * a.H * a.nc;
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(nchunks), dim3(NT), 0, stream, a);
    hipLaunchKernelGGL(chunk_state_kernel, dim3(a.B * a.H), dim3(NT), 0, stream, a);
    hipLaunchKernelGGL(chunk_out_kernel, dim3(nchunks), dim3(NT), 0, stream, a);
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

struct BStateSmem {
    uint16_t slot[13][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[2][C];
    float dsc[C];
};

struct BGradSmem {
    uint16_t slot[14][TILE];
    GateLds gl;
    float kk[NW][C];
    float dd[2][C];
    float dsc[C];
    float g1[2][C], g2[2][C], b1[2][C], b2[2][C], zr[2][C], zc[4][C], dlam[2][C];
    float frob[NW];
};

__device__ __forceinline__ float4 lds_f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Row partial sums p[i] over this lane's 16 tile columns -> dst[row] (lanes of column 0).
__device__ __forceinline__ void row_reduce_store(float (&p)[4], float *dst, int tm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) p[i] += __shfl_xor(p[i], m);
        if (acc_col() == 0) dst[16 * tm + acc_row(i)] = p[i];
    }
}

// Column sum over the 16 rows of a tile (value per lane column) -> all lanes.
__device__ __forceinline__ float col_reduce(const f32x4 &x) {
    float s = x[0] + x[1] + x[2] + x[3];
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    return s;
}

// Stage a row-major f32 64x64 matrix (row i = tid>>3, 8 columns) into the
// bf16 transposed tile dstT[j][i] and (optionally) the row-major tile dst[i][j].
__device__ __forceinline__ void stage_mat(uint16_t *dstT, uint16_t *dst, const float4 (&v)[2],
                                          int tid) {
    const int i = tid >> 3, j0 = 8 * (tid & 7);
    const float x[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) dstT[(j0 + e) * LDB + i] = bf16_bits(x[e]);
    if (dst)
        *reinterpret_cast<uint4 *>(&dst[i * LDB + j0]) =
            make_uint4(bf16_pack2(x[0], x[1]), bf16_pack2(x[2], x[3]), bf16_pack2(x[4], x[5]),
                       bf16_pack2(x[6], x[7]));
}

__device__ __forceinline__ void load_mat(float4 (&v)[2], const float *src, int tid) {
    const float4 *p = reinterpret_cast<const float4 *>(src + (tid >> 3) * D + 8 * (tid & 7));
    v[0] = p[0];
    v[1] = p[1];
}

__device__ __forceinline__ void store_grad(void *dst, int64_t idx, float x) {
    reinterpret_cast<uint16_t *>(dst)[idx] = bf16_bits(x);
}

}  // namespace

__global__ void __launch_bounds__(NT) chunk_bstate_kernel(ChunkArgs a) {
    __shared__ BStateSmem sm;
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *Vt = sm.slot[2], *Tb = sm.slot[3];
    uint16_t *Ttb = sm.slot[4], *St = sm.slot[5], *dSt = sm.slot[6], *dOt = sm.slot[7];
    uint16_t *QGt = sm.slot[8], *KBGt = sm.slot[9], *Rt = sm.slot[10], *Pt = sm.slot[11];
    uint16_t *Ptl = sm.slot[12];
    uint16_t *Dd = sm.slot[10], *Ddl = sm.slot[2];  // ddelta^T (hi, lo) after phase B
    uint16_t *dRt = sm.slot[3];                      // dR^T after phase C
    const int tid = threadIdx.x, w = tid >> 6;
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);

    f32x4 dS[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dS[j][i] = a.dfinal ? a.dfinal[((int64_t)bh * D + 16 * tm + acc_row(i)) * D +
                                           16 * (tn0 + j) + acc_col()]
                                : 0.f;

    for (int c = a.nc - 1; c >= 0; --c) {
        const int64_t ci = (int64_t)bh * a.nc + c;
        const int tg = c * C + t;
        const bool inb = tg < a.T;
        const GateBlock *gb = a.ck_gate + ci;
        const uint4 qr = load8(a.q, a.qs, b, tg, h, cb, inb);
        const uint4 kr = load8(a.k, a.ks, b, tg, h, cb, inb);
        const uint4 vr = load8(a.v, a.vs, b, tg, h, cb, inb);
        const uint4 dor = a.dout ? load8(a.dout, a.ds, b, tg, h, cb, inb) : make_uint4(0, 0, 0, 0);
        const uint4 trw = *reinterpret_cast<const uint4 *>(a.ck_t + ci * C * C + (tid >> 3) * C +
                                                          8 * (tid & 7));
        float4 s0[2];
        load_mat(s0, a.ck_state + ci * D * D, tid);
        const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
        const int sg = gb->seg[t];
        const float dsc = (a.dscores && inb && w == 0) ? a.dscores[((int64_t)b * a.T + tg) * a.H + h] : 0.f;
        // dS at the chunk end: workspace copy (f32) and the bf16 transposed operand.
        float *wd = a.ws_dstate + ci * D * D;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wd[(16 * tm + acc_row(i)) * D + 16 * (tn0 + j) + acc_col()] = dS[j][i];
            store_tile_t(&dSt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, dS[j]);
        }
        stage_mat(St, nullptr, s0, tid);
        {
            const bool on = va != 0.f;
            const float gam = sg == 0 ? __expf(G) : 0.f;
            Pack8 qp, kp;
            qp.u = mask8(qr, on);
            kp.u = mask8(kr, on);
            put_row8(Qs, t, cb, qp.u);
            put_row8(Ks, t, cb, kp.u);
            put_col8(Vt, t, cb, mask8(vr, on));
            put_col8(dOt, t, cb, mask8(dor, on));
            float ksq = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float qf = bf16_val(qp.h[e]), kf = bf16_val(kp.h[e]);
                QGt[(8 * cb + e) * LDB + t] = bf16_bits(gam * qf);
                KBGt[(8 * cb + e) * LDB + t] = bf16_bits(-be * gam * kf);
                ksq += kf * kf;
            }
            sm.kk[cb][t] = ksq;
            Pack8 tp;
            tp.u = trw;
            *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = trw;
#pragma unroll
            for (int e = 0; e < 8; ++e) Ttb[(8 * (tid & 7) + e) * LDB + (tid >> 3)] = tp.h[e];
            if (w == 0) {
                gates_derive(sm.gl, G, be, va, sg);
                sm.dsc[t] = dsc;
            }
        }
        __syncthreads();
        // Phase A: R (Rt hi, lo over V^T), P^T (hi/lo), lam K dS^T in registers.
        const RowGates rg = row_gates(sm.gl, tm);
        f32x4 kds[2] = {zero4(), zero4()};
        {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2(x, &Ks[(16 * tm) * LDB], St, tn0);
            gemm2(kds, &Ks[(16 * tm) * LDB], dSt, tn0);
            f32x4 pq[2] = {zero4(), zero4()};
            if (tn0 <= tm) gemm2(pq, &Qs[(16 * tm) * LDB], Ks, tn0);
            const float4 lm = lds_f4(&sm.gl.lam[16 * tm + 4 * (lane_id() >> 4)]);
            const float lmv[4] = {lm.x, lm.y, lm.z, lm.w};
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
                    pq[j][i] *= (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
                    kds[j][i] *= lmv[i];
                }
                store_tile_t_split(&Rt[(16 * (tn0 + j)) * LDB + 16 * tm], vt, LDB, x[j]);
                store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                                   &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq[j]);
            }
        }
        __syncthreads();
        // Phase B: delta = T R (registers) and |delta_s|^2.
        f32x4 dl[2] = {zero4(), zero4()};
        {
            gemm2(dl, &Tb[(16 * tm) * LDB], Rt, tn0);
            gemm2(dl, &Tb[(16 * tm) * LDB], Vt, tn0);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = dl[0][i] * dl[0][i] + dl[1][i] * dl[1][i];
            row_reduce_store(p, sm.dd[w & 1], tm);
        }
        __syncthreads();
        // Phase C: ddelta = P^T dO + lam K dS^T + c delta, stored transposed (hi/lo).
        {
            float cs[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ss = 16 * tm + acc_row(i);
                float kk = 0.f;
#pragma unroll
                for (int q = 0; q < NW; ++q) kk += sm.kk[q][ss];
                const float nk = sqrtf(kk), nd = sqrtf(sm.dd[0][ss] + sm.dd[1][ss]);
                cs[i] = (nk > 0.f && nd > 0.f) ? sm.dsc[ss] * nk / nd : 0.f;
            }
            f32x4 x[2] = {kds[0], kds[1]};
            gemm2(x, &Pt[(16 * tm) * LDB], dOt, tn0);
            gemm2(x, &Ptl[(16 * tm) * LDB], dOt, tn0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int i = 0; i < 4; ++i) x[j][i] += cs[i] * dl[j][i];
                store_tile_t_split(&Dd[(16 * (tn0 + j)) * LDB + 16 * tm],
                                   &Ddl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
            }
        }
        __syncthreads();
        // Phase D: dR = T^T ddelta, stored transposed.
        {
            f32x4 x[2] = {zero4(), zero4()};
            gemm2(x, &Ttb[(16 * tm) * LDB], Dd, tn0);
            gemm2(x, &Ttb[(16 * tm) * LDB], Ddl, tn0);
#pragma unroll
            for (int j = 0; j < 2; ++j) store_tile_t(&dRt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        }
        __syncthreads();
        // Phase E: dS <- gam_63 dS + (gam Q)^T dO - (beta gam K)^T dR.
        {
            const float gC = sm.gl.gamC;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) dS[j][i] *= gC;
            gemm2(dS, &QGt[(16 * tm) * LDB], dOt, tn0);
            gemm2(dS, &KBGt[(16 * tm) * LDB], dRt, tn0);
        }
        __syncthreads();
    }
    if (a.dinitial)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a.dinitial[((int64_t)bh * D + 16 * tm + acc_row(i)) * D + 16 * (tn0 + j) +
                           acc_col()] = dS[j][i];
}

__global__ void __launch_bounds__(NT) chunk_bgrad_kernel(ChunkArgs a) {
    __shared__ BGradSmem sm;
    uint16_t *Qs = sm.slot[0], *Ks = sm.slot[1], *dOs = sm.slot[2], *Qt = sm.slot[3];
    uint16_t *Kt = sm.slot[4], *dOt = sm.slot[5], *Vt = sm.slot[6], *Tb = sm.slot[7];
    uint16_t *Ttb = sm.slot[8], *S0t = sm.slot[9], *S0b = sm.slot[10], *dSt = sm.slot[11];
    uint16_t *dSb = sm.slot[12];
    // Later tenants of dead slots.
    uint16_t *Pt = sm.slot[0], *Ptl = sm.slot[11];                    // phase B..D
    uint16_t *Rt = sm.slot[1], *Rl = sm.slot[6];                      // phase B..C
    uint16_t *Dh = sm.slot[9], *Dlo = sm.slot[13];                    // delta rows, C..F
    uint16_t *Dd = sm.slot[7], *Ddl = sm.slot[1];                     // ddelta^T, D..E
    uint16_t *dRr = sm.slot[6];                                       // dR rows, E..F
    uint16_t *MA = sm.slot[0], *MAt = sm.slot[11];                    // F..G
    uint16_t *MP = sm.slot[5], *MPl = sm.slot[8], *MPt = sm.slot[7], *MPtl = sm.slot[1];
    const int tid = threadIdx.x, w = tid >> 6;
    const int ci = blockIdx.x, bh = ci / a.nc, c = ci % a.nc, b = bh / a.H, h = bh % a.H;
    const int t = tid & 63, cb = tid >> 6, tm = w >> 1, tn0 = 2 * (w & 1);
    const int tg = c * C + t;
    const bool inb = tg < a.T;
    const GateBlock *gb = a.ck_gate + ci;
    {
        const uint4 qr = load8(a.q, a.qs, b, tg, h, cb, inb);
        const uint4 kr = load8(a.k, a.ks, b, tg, h, cb, inb);
        const uint4 vr = load8(a.v, a.vs, b, tg, h, cb, inb);
        const uint4 dor = a.dout ? load8(a.dout, a.ds, b, tg, h, cb, inb) : make_uint4(0, 0, 0, 0);
        const uint4 trw = *reinterpret_cast<const uint4 *>(a.ck_t + (int64_t)ci * C * C +
                                                          (tid >> 3) * C + 8 * (tid & 7));
        float4 s0[2], ds[2];
        load_mat(s0, a.ck_state + (int64_t)ci * D * D, tid);
        load_mat(ds, a.ws_dstate + (int64_t)ci * D * D, tid);
        const float G = gb->G[t], be = gb->beta[t], va = gb->val[t];
        const int sg = gb->seg[t];
        const float dsc = (a.dscores && inb && w == 0) ? a.dscores[((int64_t)b * a.T + tg) * a.H + h] : 0.f;
        const bool on = va != 0.f;
        const uint4 q8 = mask8(qr, on), k8 = mask8(kr, on), d8 = mask8(dor, on);
        put_row8(Qs, t, cb, q8);
        put_row8(Ks, t, cb, k8);
        put_row8(dOs, t, cb, d8);
        put_col8(Qt, t, cb, q8);
        put_col8(Kt, t, cb, k8);
        put_col8(dOt, t, cb, d8);
        put_col8(Vt, t, cb, mask8(vr, on));
        Pack8 kp, tp;
        kp.u = k8;
        tp.u = trw;
        float ksq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float kf = bf16_val(kp.h[e]);
            ksq += kf * kf;
        }
        sm.kk[cb][t] = ksq;
        *reinterpret_cast<uint4 *>(&Tb[(tid >> 3) * LDB + 8 * (tid & 7)]) = trw;
#pragma unroll
        for (int e = 0; e < 8; ++e) Ttb[(8 * (tid & 7) + e) * LDB + (tid >> 3)] = tp.h[e];
        stage_mat(S0t, S0b, s0, tid);
        stage_mat(dSt, dSb, ds, tid);
        float fr = s0[0].x * ds[0].x + s0[0].y * ds[0].y + s0[0].z * ds[0].z + s0[0].w * ds[0].w +
                   s0[1].x * ds[1].x + s0[1].y * ds[1].y + s0[1].z * ds[1].z + s0[1].w * ds[1].w;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) fr += __shfl_xor(fr, m);
        if (lane_id() == 0) sm.frob[w] = fr;
        if (w == 0) {
            gates_derive(sm.gl, G, be, va, sg);
            sm.dsc[t] = dsc;
        }
    }
    __syncthreads();
    const RowGates rg = row_gates(sm.gl, tm);
    const int r0 = 16 * tm + 4 * (lane_id() >> 4);
    float lmv[4];
    {
        const float4 lm = lds_f4(&sm.gl.lam[r0]);
        lmv[0] = lm.x, lmv[1] = lm.y, lmv[2] = lm.z, lmv[3] = lm.w;
    }
    // Phase A (registers only): dO S0^T, lam K dS^T, KK^T, QK^T, V - gam K S0.
    f32x4 dos[2] = {zero4(), zero4()}, kds[2] = {zero4(), zero4()};
    f32x4 kk[2] = {zero4(), zero4()}, qk[2] = {zero4(), zero4()}, vmk[2] = {zero4(), zero4()};
    gemm2(dos, &dOs[(16 * tm) * LDB], S0b, tn0);
    gemm2(kds, &Ks[(16 * tm) * LDB], dSt, tn0);
    gemm2(vmk, &Ks[(16 * tm) * LDB], S0t, tn0);
    if (tn0 <= tm) {
        gemm2(kk, &Ks[(16 * tm) * LDB], Ks, tn0);
        gemm2(qk, &Qs[(16 * tm) * LDB], Ks, tn0);
    }
    {
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float vv[4], qv[4];
            ld4_bf16(&Vt[(16 * (tn0 + j) + acc_col()) * LDB + r0], vv);
            ld4_bf16(&Qt[(16 * (tn0 + j) + acc_col()) * LDB + r0], qv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                vmk[j][i] = vv[i] - rg.gam[i] * vmk[j][i];
                kds[j][i] *= lmv[i];
                p[i] += qv[i] * dos[j][i];  // q_t . (dO S0^T)_t
            }
        }
        row_reduce_store(p, sm.g1[w & 1], tm);
    }
    __syncthreads();
    // Phase B: P^T (hi/lo) over Q/dS^T, R (hi over K, lo over V^T).
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int ss = 16 * (tn0 + j) + acc_col();
        const float Gs = sm.gl.G[ss];
        const int sgs = sm.gl.seg[ss];
        f32x4 pq = qk[j], x;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tt = 16 * tm + acc_row(i);
            pq[i] *= (ss <= tt && rg.seg[i] == sgs) ? __expf(rg.G[i] - Gs) : 0.f;
            x[i] = rg.beta[i] * vmk[j][i];
        }
        store_tile_t_split(&Pt[(16 * (tn0 + j)) * LDB + 16 * tm],
                           &Ptl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, pq);
        store_tile_t_split(&Rt[(16 * (tn0 + j)) * LDB + 16 * tm],
                           &Rl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x);
    }
    __syncthreads();
    // Phase C: delta = T R -> registers and rows (hi/lo); |delta_s|^2.
    f32x4 dl[2] = {zero4(), zero4()};
    {
        gemm2(dl, &Tb[(16 * tm) * LDB], Rt, tn0);
        gemm2(dl, &Tb[(16 * tm) * LDB], Rl, tn0);
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = dl[0][i] * dl[0][i] + dl[1][i] * dl[1][i];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile_rm_split(&Dh[(16 * tm) * LDB + 16 * (tn0 + j)],
                                &Dlo[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, dl[j]);
        row_reduce_store(p, sm.dd[w & 1], tm);
    }
    __syncthreads();
    // Phase D: delta dS^T (-> dlam), ddelta = P^T dO + lam K dS^T + c delta (-> ddelta^T).
    float cs[4], ck[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ss = r0 + i;
        float kq = 0.f;
#pragma unroll
        for (int q = 0; q < NW; ++q) kq += sm.kk[q][ss];
        const float nk = sqrtf(kq), nd = sqrtf(sm.dd[0][ss] + sm.dd[1][ss]);
        const bool ok = nk > 0.f && nd > 0.f;
        cs[i] = ok ? sm.dsc[ss] * nk / nd : 0.f;
        ck[i] = ok ? sm.dsc[ss] * nd / nk : 0.f;
    }
    f32x4 dkl[2] = {zero4(), zero4()};
    {
        gemm2(dkl, &Dh[(16 * tm) * LDB], dSb, tn0);
        gemm2(dkl, &Dlo[(16 * tm) * LDB], dSb, tn0);
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4];
            ld4_bf16(&Kt[(16 * (tn0 + j) + acc_col()) * LDB + r0], kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] += kv[i] * dkl[j][i];
        }
        row_reduce_store(p, sm.dlam[w & 1], tm);
        f32x4 x[2] = {kds[0], kds[1]};
        gemm2(x, &Pt[(16 * tm) * LDB], dOt, tn0);
        gemm2(x, &Ptl[(16 * tm) * LDB], dOt, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] += cs[i] * dl[j][i];
            store_tile_t_split(&Dd[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &Ddl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, x[j]);
        }
    }
    __syncthreads();
    // Phase E: dR = T^T ddelta -> dV, dbeta (R part), dR rows.
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2(x, &Ttb[(16 * tm) * LDB], Dd, tn0);
        gemm2(x, &Ttb[(16 * tm) * LDB], Ddl, tn0);
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] += x[j][i] * vmk[j][i];
                const int tq = c * C + r0 + i;
                if (a.dv && tq < a.T)
                    store_grad(a.dv, (((int64_t)b * a.T + tq) * a.H + h) * D + 16 * (tn0 + j) + acc_col(),
                               sm.gl.val[r0 + i] != 0.f ? rg.beta[i] * x[j][i] : 0.f);
            }
            store_tile_rm(&dRr[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, x[j]);
        }
        row_reduce_store(p, sm.b2[w & 1], tm);
    }
    __syncthreads();
    // Phase F: dR S0^T (-> dK, dgam), dA and dP (masked) -> MA, MP (+ transposes),
    // and the gate-gradient partial sums.
    f32x4 drs[2] = {zero4(), zero4()};
    gemm2(drs, &dRr[(16 * tm) * LDB], S0b, tn0);
    {
        float p2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4];
            ld4_bf16(&Kt[(16 * (tn0 + j) + acc_col()) * LDB + r0], kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) p2[i] -= rg.beta[i] * kv[i] * drs[j][i];
        }
        row_reduce_store(p2, sm.g2[w & 1], tm);
    }
    {
        f32x4 da[2] = {zero4(), zero4()}, dp[2] = {zero4(), zero4()};
        if (tn0 <= tm) {
            gemm2(da, &dRr[(16 * tm) * LDB], Dh, tn0);
            gemm2(da, &dRr[(16 * tm) * LDB], Dlo, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dh, tn0);
            gemm2(dp, &dOs[(16 * tm) * LDB], Dlo, tn0);
        }
        float pb[4] = {0.f, 0.f, 0.f, 0.f}, pz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ss = 16 * (tn0 + j) + acc_col();
            const float Gs = sm.gl.G[ss];
            const int sgs = sm.gl.seg[ss];
            f32x4 ma, mp, z;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 16 * tm + acc_row(i);
                const bool same = rg.seg[i] == sgs;
                const float gm = (ss <= tt && same) ? __expf(rg.G[i] - Gs) : 0.f;
                const float dA = ss < tt ? -da[j][i] : 0.f;
                const float dP = dp[j][i];
                ma[i] = dA * rg.beta[i] * gm;
                mp[i] = dP * gm;
                pb[i] += dA * gm * kk[j][i];
                z[i] = (dA * rg.beta[i] * kk[j][i] + dP * qk[j][i]) * gm;
                pz[i] += z[i];
            }
            store_tile_rm(&MA[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, ma);
            store_tile_t(&MAt[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, ma);
            store_tile_rm_split(&MP[(16 * tm) * LDB + 16 * (tn0 + j)],
                                &MPl[(16 * tm) * LDB + 16 * (tn0 + j)], LDB, mp);
            store_tile_t_split(&MPt[(16 * (tn0 + j)) * LDB + 16 * tm],
                               &MPtl[(16 * (tn0 + j)) * LDB + 16 * tm], LDB, mp);
            const float zc = col_reduce(z);
            if ((lane_id() >> 4) == 0) sm.zc[tm][ss] = zc;
        }
        row_reduce_store(pb, sm.b1[w & 1], tm);
        row_reduce_store(pz, sm.zr[w & 1], tm);
    }
    __syncthreads();
    // Phase G: dQ and dK.
    {
        f32x4 x[2] = {zero4(), zero4()};
        gemm2(x, &MP[(16 * tm) * LDB], Kt, tn0);
        gemm2(x, &MPl[(16 * tm) * LDB], Kt, tn0);
        f32x4 y[2] = {zero4(), zero4()};
        gemm2(y, &MA[(16 * tm) * LDB], Kt, tn0);
        gemm2(y, &MAt[(16 * tm) * LDB], Kt, tn0);
        gemm2(y, &MPt[(16 * tm) * LDB], Qt, tn0);
        gemm2(y, &MPtl[(16 * tm) * LDB], Qt, tn0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float kv[4];
            ld4_bf16(&Kt[(16 * (tn0 + j) + acc_col()) * LDB + r0], kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tq = c * C + r0 + i;
                const bool on = sm.gl.val[r0 + i] != 0.f;
                const float dq = x[j][i] + rg.gam[i] * dos[j][i];
                const float dk = y[j][i] - rg.beta[i] * rg.gam[i] * drs[j][i] +
                                 lmv[i] * dkl[j][i] + ck[i] * kv[i];
                if (tq < a.T) {
                    const int64_t o = (((int64_t)b * a.T + tq) * a.H + h) * D + 16 * (tn0 + j) + acc_col();
                    if (a.dq) store_grad(a.dq, o, on ? dq : 0.f);
                    if (a.dk) store_grad(a.dk, o, on ? dk : 0.f);
                }
            }
        }
    }
    __syncthreads();
    // Phase H: gate gradients (wave 0, lane == token).
    if (w == 0) {
        const float gam = sm.gl.gam[t], lam = sm.gl.lam[t];
        const float dlam = sm.dlam[0][t] + sm.dlam[1][t];
        float dG = sm.zr[0][t] + sm.zr[1][t] -
                   (sm.zc[0][t] + sm.zc[1][t] + sm.zc[2][t] + sm.zc[3][t]) +
                   gam * (sm.g1[0][t] + sm.g1[1][t] + sm.g2[0][t] + sm.g2[1][t]) - lam * dlam;
        float tail = lam * dlam;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) tail += __shfl_xor(tail, m);
        if (t == 63) {
            float fr = 0.f;
#pragma unroll
            for (int q = 0; q < NW; ++q) fr += sm.frob[q];
            dG += tail + sm.gl.gamC * fr;
        }
        // reverse inclusive scan: dg_u = sum_{t >= u} dG_t
        float x = dG;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const float y = __shfl_down(x, d);
            if (t + d < 64) x += y;
        }
        const bool on = sm.gl.val[t] != 0.f;
        const bool rs = on && (t == 0 ? sm.gl.seg[0] == 1 : sm.gl.seg[t] != sm.gl.seg[t - 1]);
        if (tg < a.T) {
            const int64_t o = ((int64_t)b * a.T + tg) * a.H + h;
            if (a.dg) a.dg[o] = (on && !rs) ? x : 0.f;
            if (a.dbeta) a.dbeta[o] = on ? sm.b1[0][t] + sm.b1[1][t] + sm.b2[0][t] + sm.b2[1][t] : 0.f;
        }
    }
}

hipError_t launch_chunk_bwd(const ChunkArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(chunk_bstate_kernel, dim3(a.B * a.H), dim3(NT), 0, stream, a);
    hipLaunchKernelGGL(chunk_bgrad_kernel, dim3(a.B * a.H * a.nc), dim3(NT), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gdn2
