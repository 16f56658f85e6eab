// LDS tile helpers shared by the chunk-WY kernels (gfx950): operand staging,
// DPP wave reductions and scans, gate blocks, 16x16x32 bf16 MFMA tile products
// over row-major LDS tiles (direct and transposed reads) and the blocked UT
// inverse.  Every helper is private to the translation unit that includes it.
#pragma once

#include "gdn2_chunk.h"
#include "gdn2_mfma.h"

namespace gdn2 {

namespace {

constexpr int C = CHUNK;
constexpr int D = CHUNK_D;
constexpr int NW = 8, NT = 64 * NW;
constexpr int LDB = 72;  // bf16 row stride of a 64x64 LDS tile
constexpr int LDF = 68;  // fp32 row stride
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

__device__ __forceinline__ void put_row8(uint16_t *tile, int t, int cb, uint4 v, int ld = LDB) {
    *reinterpret_cast<uint4 *>(&tile[t * ld + 8 * cb]) = v;
}

__device__ __forceinline__ void put_col8(uint16_t *tile, int t, int cb, uint4 v, int ld = LDB) {
    Pack8 p;
    p.u = v;
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[(8 * cb + e) * ld + t] = p.h[e];
}

// DPP lane moves (gfx9 controls): lanes whose source is outside the pattern,
// or whose row is masked off, read 0.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, false);
}

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15), left in every lane:
// quad swaps (lane ^ 1, lane ^ 2) then half-row and row mirrors.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x;
}

// Sum over the 64 lanes of a wave, left in every lane.
__device__ __forceinline__ float wave_sum(float x) {
    const int r = __builtin_bit_cast(int, row16_sum(x));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 16)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 32)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 48));
}

// Inclusive scan over the 64 lanes of a wave: shifts right by 1, 2, 4, 8 within
// each row, then lane 15 of rows 0/2 into rows 1/3 and lane 31 into rows 2-3.
template <typename Tv>
__device__ __forceinline__ Tv wave_scan_add(Tv x) {
    x += dpp<0x111>(x);
    x += dpp<0x112>(x);
    x += dpp<0x114>(x);
    x += dpp<0x118>(x);
    x += dpp<0x142, 0xA>(x);
    x += dpp<0x143, 0xC>(x);
    return x;
}

// Row sums of an accumulator tile: p[i] is this lane's term of row 4(l/16) + i;
// the sum over the 16 lanes of each DPP row goes to dst[16 tm + row].  An
// exchange butterfly: across lane bit 3 each lane keeps two rows (rows 0, 1 if
// the bit is clear, else 2, 3) and sends the other two; across the half-row
// mirror (which flips lane bit 2) it keeps one of those; two quad steps finish.
// Lanes with l % 4 == 0 then hold row 2 b3 + b2 and store it.
__device__ __forceinline__ void row_reduce_store(const float (&p)[4], float *dst, int tm) {
    const int n = lane_id() & 15;
    const bool b3 = (n & 8) != 0, b2 = (n & 4) != 0;
    const float s0 = b3 ? p[0] : p[2], s1 = b3 ? p[1] : p[3];
    const float a0 = (b3 ? p[2] : p[0]) + dpp<0x128>(s0);  // row_ror:8, lane n ^ 8
    const float a1 = (b3 ? p[3] : p[1]) + dpp<0x128>(s1);
    float x = (b2 ? a1 : a0) + dpp<0x141>(b2 ? a0 : a1);  // row_half_mirror
    x += dpp<0x4E>(x);
    x += dpp<0xB1>(x);
    if ((n & 3) == 0) dst[16 * tm + 4 * (lane_id() >> 4) + 2 * b3 + b2] = x;
}

// As row_reduce_store, adding to dst when add is set (the lane that stores a
// row's sum is the same for every call with the same tm).
__device__ __forceinline__ void row_reduce_accum(const float (&p)[4], float *dst, int tm, bool add) {
    const int n = lane_id() & 15;
    const bool b3 = (n & 8) != 0, b2 = (n & 4) != 0;
    const float s0 = b3 ? p[0] : p[2], s1 = b3 ? p[1] : p[3];
    const float a0 = (b3 ? p[2] : p[0]) + dpp<0x128>(s0);
    const float a1 = (b3 ? p[3] : p[1]) + dpp<0x128>(s1);
    float x = (b2 ? a1 : a0) + dpp<0x141>(b2 ? a0 : a1);
    x += dpp<0x4E>(x);
    x += dpp<0xB1>(x);
    float *d = &dst[16 * tm + 4 * (lane_id() >> 4) + 2 * b3 + b2];
    if ((n & 3) == 0) *d = add ? *d + x : x;
}

// Wave 0 (lane == token): decays derived from a gate block.
__device__ __forceinline__ void gates_derive(GateLds &gl, float G, float beta, float val, int seg) {
    const int t = lane_id();
    const float G63 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, G), 63));
    const int seg63 = __builtin_amdgcn_readlane(seg, 63);
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

// acc[j] += X[16 rows][0:R] * Y[16 rows of tile (tn0 + j)][0:R]^T, j = 0, 1
// (row strides LDX, LDY).
template <int R = 64, int LDX = LDB, int LDY = LDB>
__device__ __forceinline__ void gemm2(f32x4 (&acc)[2], const uint16_t *X, const uint16_t *Y,
                                      int tn0) {
    const uint16_t *Y0 = Y + (16 * tn0) * LDY, *Y1 = Y0 + 16 * LDY;
    bf16x8_t x[R / 32], a[R / 32], b[R / 32];
#pragma unroll
    for (int i = 0; i < R / 32; ++i) x[i] = frag(X, LDX, 32 * i);
#pragma unroll
    for (int i = 0; i < R / 32; ++i) a[i] = frag(Y0, LDY, 32 * i);
#pragma unroll
    for (int i = 0; i < R / 32; ++i) b[i] = frag(Y1, LDY, 32 * i);
#pragma unroll
    for (int i = 0; i < R / 32; ++i) {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[i], a[i], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[i], b[i], acc[1], 0, 0, 0);
    }
}

// Four consecutive bf16 of one LDS row as floats.
__device__ __forceinline__ void ld4_bf16(const uint16_t *p, float (&o)[4]) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    o[0] = bf16_val((uint16_t)(v.x & 0xffff));
    o[1] = bf16_val((uint16_t)(v.x >> 16));
    o[2] = bf16_val((uint16_t)(v.y & 0xffff));
    o[3] = bf16_val((uint16_t)(v.y >> 16));
}

typedef short v4s __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: in each 16-lane group, lane i supplies the address of
// four 16-bit elements M[i][0..3]; lane j receives M[4e + j/4][j%4], e < 4.
__device__ __forceinline__ v4s lds_tr16(const uint16_t *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)p);
}

// Accumulator-layout values (rows row0 + 4(l/16) + e, column col0 + l%16) of a
// row-major bf16 LDS tile, with one transpose read.
template <int LDZ = LDB>
__device__ __forceinline__ void ld4_rm_tr(const uint16_t *Z, int row0, int col0, float (&o)[4]) {
    const int l = lane_id(), i = l & 15;
    const v4s v = lds_tr16(Z + (row0 + 4 * (l >> 4) + (i >> 2)) * LDZ + col0 + 4 * (i & 3));
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = bf16_val((uint16_t)v[e]);
}

// MFMA operand fragment of a tile held in the other orientation: lane
// (n = l%16, g = l/16) receives Z[r0 + 8g + e][c0 + n], e < 8, i.e. the
// fragment of the matrix Y[n][r] = Z[r][n] at reduction offset r0 and row block
// c0.  Two transpose reads of four rows each; like lds_tr16, every lane of the
// wave runs it.
template <int LDZ = LDB>
__device__ __forceinline__ bf16x8_t frag_tr(const uint16_t *Z, int r0, int c0) {
    const int l = lane_id(), i = l & 15;
    const uint16_t *p = Z + (r0 + 8 * (l >> 4) + (i >> 2)) * LDZ + c0 + 4 * (i & 3);
    const v4s x = lds_tr16(p), y = lds_tr16(p + 4 * LDZ);
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
    return __builtin_bit_cast(bf16x8_t, v);
}

// acc[j] += X[16 rows][0:R] * Y_j[16 rows][0:R]^T with Y_j[n][r] =
// Z[r][16 (tn0 + j) + n]: the B operand is read across a row-major tile Z.
template <int R = 64, int LDX = LDB, int LDZ = LDB>
__device__ __forceinline__ void gemm2_tr(f32x4 (&acc)[2], const uint16_t *X, const uint16_t *Z,
                                         int tn0) {
#pragma unroll
    for (int r = 0; r < R; r += 32) {
        const bf16x8_t x = frag(X, LDX, r);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, frag_tr<LDZ>(Z, r, 16 * (tn0 + j)),
                                                             acc[j], 0, 0, 0);
    }
}

// acc[j] += X * Y_j^T with the A operand read across a row-major tile Z
// (X[m][r] = Z[r][m0 + m]) and Y_j the row tile (tn0 + j) of Y.
template <int R = 64, int LDZ = LDB, int LDY = LDB>
__device__ __forceinline__ void gemm2_atr(f32x4 (&acc)[2], const uint16_t *Z, int m0,
                                          const uint16_t *Y, int tn0) {
#pragma unroll
    for (int r = 0; r < R; r += 32) {
        const bf16x8_t x = frag_tr<LDZ>(Z, r, m0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                x, frag(Y + (16 * (tn0 + j)) * LDY, LDY, r), acc[j], 0, 0, 0);
    }
}

// frag_tr(Z, r0, c0) with row r of Z scaled by s[r], as a two-term bf16 split
// (hi + lo carries ~16 mantissa bits of s[r] Z[r][c]).  Lane (n, g) holds rows
// r0 + 8g .. r0 + 8g + 7, so it reads those eight scales (s 16-byte aligned,
// r0 a multiple of 8).  Used where a per-token scale falls on the reduction
// index, so it cannot be applied to the product's accumulator instead.
template <int LDZ = LDB>
__device__ __forceinline__ void frag_tr_scaled_split(const uint16_t *Z, const float *s, int r0, int c0,
                                                     bf16x8_t &hi, bf16x8_t &lo) {
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s z = __builtin_bit_cast(v8s, frag_tr<LDZ>(Z, r0, c0));
    const float *sr = s + r0 + 8 * (lane_id() >> 4);
    const float4 s0 = *reinterpret_cast<const float4 *>(sr), s1 = *reinterpret_cast<const float4 *>(sr + 4);
    const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    v8s h, o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint16_t hh, ll;
        split_bf16(sc[e] * bf16_val((uint16_t)z[e]), hh, ll);
        h[e] = (short)hh;
        o[e] = (short)ll;
    }
    hi = __builtin_bit_cast(bf16x8_t, h);
    lo = __builtin_bit_cast(bf16x8_t, o);
}

// T = (I + A)^-1 for the strictly lower 64x64 A in Af; result in Tf (lower
// blocks).  Called by all waves; ends with a barrier.  Blocks are 16x16:
//   1. diagonal blocks T_bb = (I + A_bb)^-1 by forward substitution: wave 0,
//      lane (block l/16, column l%16) walks its column down the 16 rows with
//      FMAs on its own registers (the A values are LDS broadcasts);
//   2. T_10 = -T_11 A_10 T_00 and T_32 = -T_33 A_32 T_22;
//   3. T_21 (32x32, blocks r = 2,3 x c = 0,1) = -T_22(32) A_21(32) T_11(32).
// Products chain through registers (the second factor of each step is an
// accumulator tile), so the three steps take three barriers.
__device__ __forceinline__ void ut_inverse(const float *Af, float *Tf, int w) {
    const int l = lane_id();
    if (w == 0) {
        const int bk = l >> 4, col = l & 15;
        const float *Ab = Af + (16 * bk) * LDF + 16 * bk;
        // Row r of the block, L[r][0..r-1], as (r + 3) / 4 float4 reads (the entries
        // at and above the diagonal are zero), issued PD rows ahead of its use so
        // that the LDS latency overlaps the substitution instead of preceding each row.
        constexpr int PD = 4;
        float4 Lr[16][4];
        auto load_row = [&](int r) {
#pragma unroll
            for (int v = 0; v < (r + 3) / 4; ++v) Lr[r][v] = *reinterpret_cast<const float4 *>(Ab + r * LDF + 4 * v);
        };
#pragma unroll
        for (int r = 1; r <= PD; ++r) load_row(r);
        float Tc[16];  // T_bb[r][col]; rows above col come out 0
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (r >= 1 && r + PD < 16) load_row(r + PD);
            __builtin_amdgcn_sched_barrier(0);  // keeps the reads ahead of this row's FMAs
            float e0 = 0.f, e1 = 0.f;  // two chains halve the dependent FMA latency
#pragma unroll
            for (int q = 0; q < r; ++q) {
                const float4 &v4 = Lr[r][q >> 2];
                const float a = (q & 3) == 0 ? v4.x : (q & 3) == 1 ? v4.y : (q & 3) == 2 ? v4.z : v4.w;
                if (q & 1) e1 += a * Tc[q];
                else e0 += a * Tc[q];
            }
            Tc[r] = (r == col ? 1.f : 0.f) - (e0 + e1);
        }
        float *Tb = Tf + (16 * bk) * LDF + 16 * bk;
#pragma unroll
        for (int r = 0; r < 16; ++r) Tb[r * LDF + col] = Tc[r];
    }
    __syncthreads();
    auto blkA = [&](int r, int c) { return Af + (16 * r) * LDF + 16 * c; };
    auto blkT = [&](int r, int c) { return Tf + (16 * r) * LDF + 16 * c; };
    // acc += Z[16x16] Y with Y an accumulator tile: instruction i reduces over
    // Y's rows 4(l/16) + i (the rows lane l holds), Z read at the same columns.
    auto mm_acc = [&](f32x4 &acc, const float *Z, const f32x4 &Y) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Z[(l & 15) * LDF + 4 * (l >> 4) + i], Y[i], acc,
                                                       0, 0, 0);
    };
    if (w < 2) {  // T_{2w+1,2w} = -T_{2w+1,2w+1} (A_{2w+1,2w} T_{2w,2w})
        f32x4 x = zero4(), y = zero4();
        mm16_f32(x, blkA(2 * w + 1, 2 * w), LDF, blkT(2 * w, 2 * w), LDF);
        mm_acc(y, blkT(2 * w + 1, 2 * w + 1), x);
        float *dst = blkT(2 * w + 1, 2 * w);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[acc_row(i) * LDF + acc_col()] = -y[i];
    }
    __syncthreads();
    if (w < 4) {  // T_rc = -sum_{m=2..r} T_rm Y_mc, Y_mc = sum_{m'=c..1} A_mm' T_m'c (own Y's)
        const int r = 2 + (w >> 1), c = w & 1;
        f32x4 y2 = zero4(), y3 = zero4(), t = zero4();
        for (int m = c; m < 2; ++m) mm16_f32(y2, blkA(2, m), LDF, blkT(m, c), LDF);
        if (r == 3)
            for (int m = c; m < 2; ++m) mm16_f32(y3, blkA(3, m), LDF, blkT(m, c), LDF);
        mm_acc(t, blkT(r, 2), y2);
        if (r == 3) mm_acc(t, blkT(3, 3), y3);
        float *dst = blkT(r, c);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[acc_row(i) * LDF + acc_col()] = -t[i];
    }
    __syncthreads();
}

__device__ __forceinline__ float4 lds_f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Column sum over the 16 rows of a tile (value per lane column) -> all lanes.
__device__ __forceinline__ float col_reduce(const f32x4 &x) {
    float s = x[0] + x[1] + x[2] + x[3];
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    return s;
}

// sum_e a[e] b[e] over eight bf16 pairs.
__device__ __forceinline__ float dot8_bf16(const uint4 a, const uint4 b) {
    Pack8 pa, pb;
    pa.u = a;
    pb.u = b;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += bf16_val(pa.h[e]) * bf16_val(pb.h[e]);
    return s;
}

}  // namespace

}  // namespace gdn2
