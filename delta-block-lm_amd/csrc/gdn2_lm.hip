// Fused operators of the lm512 training step (the GDN language model of the
// configuration-4 workload) on gfx950.  None has a counterpart in the
// reference, whose model composes the f32 custom ops one by one
// (crates/mixers/src/lib.rs:456-525, crates/experiment/src/model.rs:300-364);
// these fold the casts, slices, residual adds and pointwise ops of a bf16
// training step into the kernels that already touch the data:
//   * lm_norm: RMSNorm over rows (width 128 or 256 NV) with the residual add in front
//     (u = x + r, r in bf16) and a bf16 output; its VJP adds the residual
//     gradient and writes the input gradient in f32 and bf16;
//   * lm_mixer_in: from the packed projection z (bf16, per token
//     [q | k | v | gate | beta | decay]) the depthwise causal convolution with
//     SiLU, the per-head L2 norm of q and k, and the scalar gates
//     beta = sigmoid(z_beta), g = -exp(decay_scale) softplus(z_decay + decay_bias);
//     its VJP writes the bf16 gradient columns of z directly;
//   * lm_mixer_out: y = rms_norm(o) * silu(gate) per head, in bf16;
//   * lm_swiglu: silu(h_gate) * h_up with the model's bf16 rounding points.
// Every kernel computes in f32 and rounds where the bf16 model rounds: the
// fused step keeps the rounding points of the unfused composition.  Parameter
// gradients are reduced in two deterministic passes (partials per workgroup,
// then a fixed-order sum).
#include <math.h>

#include <algorithm>

#include "gdn2_common.h"
#include "gdn2_status.h"

namespace gdn2 {
namespace {

constexpr int kSegRows = 32;        // time steps per convolution segment (one workgroup)
constexpr int kWaveRows = 8;        // time steps per wave of a segment
constexpr int kInWaves = kSegRows / kWaveRows;
constexpr int kBwdBlocks = 1024;    // workgroups of the persistent row VJPs (fixed: deterministic)
constexpr int kSumWaves = 16;

template <int CTRL>
__device__ __forceinline__ float dpp_mv(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over each row of 16 lanes (every lane of the row gets it).
__device__ __forceinline__ float sum16(float x) {
    x += dpp_mv<0xB1>(x);
    x += dpp_mv<0x4E>(x);
    x += dpp_mv<0x141>(x);
    x += dpp_mv<0x140>(x);
    return x;
}

// Sum over the wave (every lane).
__device__ __forceinline__ float sum64(float x) {
    x = sum16(x);
    return readlane_f(x, 0) + readlane_f(x, 16) + readlane_f(x, 32) + readlane_f(x, 48);
}

// The pointwise ops use the hardware exp2 / reciprocal / reciprocal square
// root (v_exp_f32, v_rcp_f32, v_rsq_f32, about 1 ulp each): these kernels
// would otherwise be bound by the VALU work of IEEE division and libm exp,
// and the results are rounded to bf16 anyway (relative error ~1e-6 at most,
// against bf16's 2^-9).
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float frsq(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float sigm(float x) { return frcp(1.f + fexp(-x)); }
// SiLU, x / (1 + exp(-x)).
__device__ __forceinline__ float silu_div(float x) { return x * frcp(1.f + fexp(-x)); }
// up * d silu(x) / dx.
__device__ __forceinline__ float silu_vjp(float x, float up) {
    const float s = sigm(x);
    return up * s * (1.f + x * (1.f - s));
}

__device__ __forceinline__ float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_f(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}
__device__ __forceinline__ float rbf(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ float4 ld_bf4(const bf16_t *p) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p);
    return make_float4(lo_f(u.x), hi_f(u.x), lo_f(u.y), hi_f(u.y));
}
__device__ __forceinline__ void st_bf4(bf16_t *p, float4 f) {
    *reinterpret_cast<uint2 *>(p) = make_uint2(pack2(f.x, f.y), pack2(f.z, f.w));
}
__device__ __forceinline__ float4 ld_f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st_f4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// out[i] = sum_s part[s * n + i] for s < segs: 64 columns per workgroup, its
// 16 waves each summing every 16th segment, then the waves in order.
__global__ void __launch_bounds__(64 * kSumWaves) lm_colsum_kernel(const float *part, int64_t n,
                                                                  int64_t segs, float *out) {
    __shared__ float red[kSumWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (i < n) {
#pragma unroll 16
        for (int64_t k = w; k < segs; k += kSumWaves) s += part[k * n + i];
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && i < n) {
        float t = red[0][lane];
        for (int j = 1; j < kSumWaves; ++j) t += red[j][lane];
        out[i] = t;
    }
}

void colsum(const float *part, int64_t n, int64_t segs, float *out, hipStream_t st) {
    hipLaunchKernelGGL(lm_colsum_kernel, dim3((unsigned)((n + 63) / 64)), dim3(64 * kSumWaves), 0,
                       st, part, n, segs, out);
}

// ---- RMSNorm with residual ----------------------------------------------------------
struct NormArgs {
    int64_t rows;
    int W;
    float eps;
    const float *x;
    const bf16_t *res;
    const float *w;
    float *u;
    bf16_t *y;
    float *inv;
    const float *inv_in;
    const bf16_t *dy;
    const float *dres;
    float *dx;
    bf16_t *dxb;
    float *part;
};

// Sum over each group of G lanes (16, 32 or 64; aligned), in every lane of it.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    x = sum16(x);
    if (G == 32) x += __shfl_xor(x, 16);
    if (G == 64) x = readlane_f(x, 0) + readlane_f(x, 16) + readlane_f(x, 32) + readlane_f(x, 48);
    return x;
}

// G lanes per row (256 / G rows per workgroup); lane owns the float4 columns
// 4 (G k + lane), k < NV: width = 4 G NV.  A spare lane group past the last
// row redoes that row and stores nothing.
template <int G, int NV>
__global__ void __launch_bounds__(256) lm_norm_fwd_kernel(NormArgs a) {
    constexpr int RPB = 256 / G;
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / G;
    const bool live = row < a.rows;
    const int64_t base = (live ? row : a.rows - 1) * a.W;
    float4 z[NV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * G + lane) * 4;
        z[k] = ld_f4(a.x + base + c);
        if (a.res) {
            const float4 r = ld_bf4(a.res + base + c);
            z[k] = make_float4(z[k].x + r.x, z[k].y + r.y, z[k].z + r.z, z[k].w + r.w);
        }
        ss += dot4(z[k], z[k]);
    }
    ss = group_sum<G>(ss);
    const float inv = frsq(ss * (1.f / (float)a.W) + a.eps);
    if (!live) return;
    if (lane == 0) a.inv[row] = inv;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * G + lane) * 4;
        if (a.u) st_f4(a.u + base + c, z[k]);
        const float4 w = ld_f4(a.w + c), v = z[k];
        st_bf4(a.y + base + c,
               make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w));
    }
}

// dx = dres + J^T dy per row; weight-gradient partial sums per workgroup
// (persistent grid; the lane groups of a workgroup are added in order).
template <int G, int NV>
__global__ void __launch_bounds__(256) lm_norm_bwd_kernel(NormArgs a) {
    constexpr int RPB = 256 / G, W = 4 * G * NV;
    __shared__ float red[RPB][W];
    const int lane = threadIdx.x % G, slot = threadIdx.x / G;
    float4 w[NV], acc[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        w[k] = ld_f4(a.w + (k * G + lane) * 4);
        acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int64_t r0 = (int64_t)blockIdx.x * RPB; r0 < a.rows; r0 += (int64_t)gridDim.x * RPB) {
        const int64_t row = r0 + slot;
        const bool live = row < a.rows;
        const int64_t base = (live ? row : a.rows - 1) * W;
        float4 z[NV], up[NV], uw[NV];
        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c = (k * G + lane) * 4;
            z[k] = ld_f4(a.x + base + c);
            up[k] = ld_bf4(a.dy + base + c);
            uw[k] = make_float4(up[k].x * w[k].x, up[k].y * w[k].y, up[k].z * w[k].z,
                                up[k].w * w[k].w);
            dot += dot4(uw[k], z[k]);
        }
        dot = group_sum<G>(dot);
        if (!live) continue;
        const float inv = a.inv_in[row];
        const float corr = dot * inv * inv / (float)W;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c = (k * G + lane) * 4;
            float4 d = make_float4((uw[k].x - z[k].x * corr) * inv, (uw[k].y - z[k].y * corr) * inv,
                                   (uw[k].z - z[k].z * corr) * inv, (uw[k].w - z[k].w * corr) * inv);
            if (a.dres) {
                const float4 r = ld_f4(a.dres + base + c);
                d = make_float4(r.x + d.x, r.y + d.y, r.z + d.z, r.w + d.w);
            }
            st_f4(a.dx + base + c, d);
            if (a.dxb) st_bf4(a.dxb + base + c, d);
            acc[k].x += up[k].x * z[k].x * inv;
            acc[k].y += up[k].y * z[k].y * inv;
            acc[k].z += up[k].z * z[k].z * inv;
            acc[k].w += up[k].w * z[k].w * inv;
        }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) st_f4(&red[slot][(k * G + lane) * 4], acc[k]);
    __syncthreads();
    for (int c = threadIdx.x; c < W; c += 256) {
        float s = red[0][c];
        for (int j = 1; j < RPB; ++j) s += red[j][c];
        a.part[(int64_t)blockIdx.x * W + c] = s;
    }
}

// ---- mixer input: convolution, SiLU, L2 of q / k, scalar gates ----------------------
struct InArgs {
    int64_t B, T, zs;  // zs: elements between token rows of z and dz
    int H, K, V, C;    // C = 2 H K + H V convolution channels
    const bf16_t *z;
    const float *w;  // [taps, C]
    const float *valid, *docs;  // [B, T]
    const float *dscale, *dbias;  // [H]
    bf16_t *qkv;  // [B, T, C]
    float *beta, *g;  // [B, T, H]
    const bf16_t *dq, *dk, *dv;  // [B, T, H, K|V]
    const float *dbeta, *dg;
    bf16_t *dz;
    float *wpart;  // [B nseg][taps][C]
    float *gpart;  // [B nseg][2 H]
};

__host__ __device__ inline int64_t in_segments(int64_t T) { return (T + kSegRows - 1) / kSegRows; }

// The rows a segment reads, fetched up front: slot i is row tb + i of this
// thread's channel (rows outside [0, T) read as zero).  The lag masks are
// wave-uniform, so they live in LDS: mk[r][l] = mask of the lag from slot
// r - l to slot r, valid[s] valid[r] [docs[s] == docs[r]] (0 past the window
// or outside [0, T)); lane r computes row r's W masks.
template <int W>
constexpr int mask_pitch() { return (W + 3) & ~3; }

template <int NR, int W>
struct Rows {
    float x[NR];
    float (*mk)[mask_pitch<W>()];

    __device__ __forceinline__ void fetch(const InArgs &a, int64_t b, int64_t tb, int c,
                                          float (*lds)[mask_pitch<W>()]) {
        mk = lds;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int64_t t = tb + i;
            const int64_t tc = t < 0 ? 0 : (t >= a.T ? a.T - 1 : t);  // in bounds; masked below
            x[i] = bf16_to_f32(a.z[(b * a.T + tc) * a.zs + c]);
        }
        const int lane = threadIdx.x & 63;
        if (lane < NR) {
            auto row = [&](int64_t t, float &d, float &v) {
                const bool in = t >= 0 && t < a.T;
                d = in ? a.docs[b * a.T + t] : 0.f;
                v = in ? a.valid[b * a.T + t] : 0.f;
            };
            float dr, vr;
            row(tb + lane, dr, vr);
#pragma unroll
            for (int l = 0; l < W; ++l) {
                float ds = 0.f, vs = 0.f;
                if (lane - l >= 0) row(tb + lane - l, ds, vs);
                mk[lane][l] = ds == dr ? vs * vr : 0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const bool in = tb + i >= 0 && tb + i < a.T;
            x[i] = in ? x[i] : 0.f;
        }
    }
    // Pre-activation output of slot r (r >= W - 1).
    __device__ __forceinline__ float pre(const float *w, int r) const {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < W; ++l) s += x[r - l] * w[l] * mk[r][l];
        return s;
    }
};

// Gate columns of one (batch, segment): lane h = lane % H handles every
// (t, h) with the same h, so the per-head sums need no atomics.
__device__ void gates_forward(const InArgs &a, int64_t b, int64_t t0, int64_t t1, int lane) {
    const int H = a.H;
    const int64_t cb = a.C + (int64_t)H * a.V;  // beta column; decay follows at cb + H
    for (int i = lane; i < kSegRows * H; i += 64) {
        const int64_t t = t0 + i / H;
        const int h = i % H;
        if (t >= t1) break;
        const bf16_t *zr = a.z + (b * a.T + t) * a.zs;
        const float zb = bf16_to_f32(zr[cb + h]), zd = bf16_to_f32(zr[cb + H + h]);
        const float x = zd + a.dbias[h];
        const float sp = x > 20.f ? x : log1pf(expf(x));
        const int64_t o = (b * a.T + t) * H + h;
        a.beta[o] = sigm(zb);
        a.g[o] = -expf(a.dscale[h]) * sp;
    }
}

// Grid (B nseg, C / 64 + 1): block column y < C / 64 holds 64 channels (one
// head of q, k or v), its 4 waves 8 time steps each; the last column does the
// gates (wave 0).
template <int W>
__global__ void __launch_bounds__(64 * kInWaves) lm_in_fwd_kernel(InArgs a) {
    constexpr int NR = kWaveRows + W - 1;
    const int64_t nseg = in_segments(a.T);
    const int64_t b = blockIdx.x / nseg, t0 = (blockIdx.x % nseg) * kSegRows;
    const int64_t t1 = min(t0 + kSegRows, a.T);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if ((int)blockIdx.y == a.C / 64) {
        if (wv == 0) gates_forward(a, b, t0, t1, lane);
        return;
    }
    const int c = blockIdx.y * 64 + lane;
    const bool l2 = c < 2 * a.H * a.K;  // q and k heads (64 channels each): wave-uniform
    float w[W];
#pragma unroll
    for (int l = 0; l < W; ++l) w[l] = a.w[l * a.C + c];
    __shared__ __align__(16) float mk[kInWaves][NR][mask_pitch<W>()];
    const int64_t tw = t0 + kWaveRows * wv;  // this wave's first row
    Rows<NR, W> rw;
    rw.fetch(a, b, tw - (W - 1), c, mk[wv]);
#pragma unroll
    for (int i = 0; i < kWaveRows; ++i) {
        const int64_t t = tw + i;
        if (t >= t1) continue;  // wave-uniform
        const float p = rw.pre(w, i + W - 1);
        float s = p * sigm(p);
        if (l2) s = s * frsq(sum64(s * s) + 1e-6f);
        a.qkv[(b * a.T + t) * a.C + c] = f32_to_bf16(s);
    }
}

__device__ void gates_backward(const InArgs &a, int64_t b, int64_t t0, int64_t t1, int lane) {
    const int H = a.H;
    const int64_t cb = a.C + (int64_t)H * a.V;
    float pb = 0.f, ps = 0.f;
    for (int i = lane; i < kSegRows * H; i += 64) {
        const int64_t t = t0 + i / H;
        const int h = i % H;
        if (t >= t1) break;
        const int64_t row = b * a.T + t;
        const bf16_t *zr = a.z + row * a.zs;
        bf16_t *dzr = a.dz + row * a.zs;
        const float zb = bf16_to_f32(zr[cb + h]), zd = bf16_to_f32(zr[cb + H + h]);
        const float be = sigm(zb);
        dzr[cb + h] = f32_to_bf16(a.dbeta[row * H + h] * (1.f - be) * be);
        const float x = zd + a.dbias[h];
        const float ex = expf(x), sp = x > 20.f ? x : log1pf(ex);
        const float dg = a.dg[row * H + h];
        const float dsp = dg * -expf(a.dscale[h]);
        const float dx = x > 20.f ? dsp : dsp * ex / (ex + 1.f);
        dzr[cb + H + h] = f32_to_bf16(dx);
        pb += dx;
        ps += dg * sp;
    }
    // Lanes l, l + H, l + 2H, ... share head l % H (H a power of two).
    for (int off = H; off < 64; off <<= 1) {
        pb += __shfl_xor(pb, off);
        ps += __shfl_xor(ps, off);
    }
    if (lane < H) {
        a.gpart[(int64_t)blockIdx.x * 2 * H + lane] = pb;
        a.gpart[(int64_t)blockIdx.x * 2 * H + H + lane] = ps;
    }
}

// VJP of lm_in_fwd_kernel (the VJP of a convolution): with gr the gradient at
// the pre-activation of row t (recomputed: window, SiLU, L2),
//   dz[t]  = sum_l gr[t + l] w[l] mask(t -> t + l)
//   dw[l] += gr[t] z[t - l] mask(t - l -> t)     (t in this segment)
// Each wave computes gr for its 8 rows into LDS (the last wave also for the
// next segment's first W - 1 rows), then emits dz and dw for its rows; the
// waves' dw are added in order into one partial per workgroup.
template <int W>
__global__ void __launch_bounds__(64 * kInWaves) lm_in_bwd_kernel(InArgs a) {
    constexpr int NG = kWaveRows + W - 1;  // gradient rows of the last wave
    constexpr int NR = NG + W - 1;         // rows read: tw - (W - 1) .. tw + NG - 1
    const int64_t nseg = in_segments(a.T);
    const int64_t b = blockIdx.x / nseg, t0 = (blockIdx.x % nseg) * kSegRows;
    const int64_t t1 = min(t0 + kSegRows, a.T);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if ((int)blockIdx.y == a.C / 64) {
        if (wv == 0) gates_backward(a, b, t0, t1, lane);
        return;
    }
    const int c = blockIdx.y * 64 + lane;
    const int HK = a.H * a.K;
    const bool l2 = c < 2 * HK;
    const bf16_t *src;
    int64_t width;
    int col;
    if (c < HK) {
        src = a.dq;
        width = HK;
        col = c;
    } else if (c < 2 * HK) {
        src = a.dk;
        width = HK;
        col = c - HK;
    } else {
        src = a.dv;
        width = (int64_t)a.H * a.V;
        col = c - 2 * HK;
    }
    float w[W];
#pragma unroll
    for (int l = 0; l < W; ++l) w[l] = a.w[l * a.C + c];
    __shared__ __align__(16) float mk[kInWaves][NR][mask_pitch<W>()];
    __shared__ float gsh[kSegRows + W - 1][64];  // gr of row t0 + j
    __shared__ float dwr[kInWaves][W][64];
    const int64_t tw = t0 + kWaveRows * wv;  // this wave's first row; slot i + W - 1 is row tw + i
    Rows<NR, W> rw;
    rw.fetch(a, b, tw - (W - 1), c, mk[wv]);
    const int ng = wv == kInWaves - 1 ? NG : kWaveRows;  // wave-uniform
    float up[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int64_t t = tw + i;
        up[i] = i < ng ? bf16_to_f32(src[(b * a.T + (t < a.T ? t : a.T - 1)) * width + col]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        if (i >= ng) continue;  // wave-uniform
        float gv = 0.f;
        if (tw + i < a.T) {  // wave-uniform
            const float p = rw.pre(w, i + W - 1);
            const float sg = sigm(p), s = p * sg;
            float u = up[i];
            if (l2) {
                const float inv = frsq(sum64(s * s) + 1e-6f);
                const float corr = sum64(u * s) * inv * inv;
                u = (u - s * corr) * inv;
            }
            gv = u * sg * (1.f + p * (1.f - sg));
        }
        gsh[kWaveRows * wv + i][lane] = gv;
    }
    __syncthreads();
    float dw[W];
#pragma unroll
    for (int l = 0; l < W; ++l) dw[l] = 0.f;
#pragma unroll
    for (int i = 0; i < kWaveRows; ++i) {
        if (tw + i >= t1) continue;  // wave-uniform
        const int r = i + W - 1, j = kWaveRows * wv + i;
        const float g0 = gsh[j][lane];
#pragma unroll
        for (int l = 0; l < W; ++l) dw[l] += g0 * rw.x[r - l] * rw.mk[r][l];
        float sum = 0.f;
#pragma unroll
        for (int l = 0; l < W; ++l) {
            const float m = rw.mk[r + l][l];  // lag from row tw + i to row tw + i + l
            if (m != 0.f) sum += gsh[j + l][lane] * w[l] * m;
        }
        a.dz[(b * a.T + tw + i) * a.zs + c] = f32_to_bf16(sum);
    }
#pragma unroll
    for (int l = 0; l < W; ++l) dwr[wv][l][lane] = dw[l];
    __syncthreads();
    if (wv == 0) {
        float *part = a.wpart + (int64_t)blockIdx.x * W * a.C;
#pragma unroll
        for (int l = 0; l < W; ++l) {
            float t = dwr[0][l][lane];
            for (int q = 1; q < kInWaves; ++q) t += dwr[q][l][lane];
            part[l * a.C + c] = t;
        }
    }
}

// ddecay_bias[h] = sum of the decay-column gradients; ddecay_scale[h] =
// -(sum dg softplus) exp(decay_scale[h]).  One workgroup, lane = column of
// the [segments][2 H] partials.
__global__ void __launch_bounds__(64 * kSumWaves) lm_gate_sum_kernel(const float *part, int H,
                                                                    int64_t segs,
                                                                    const float *dscale,
                                                                    float *ddbias, float *ddscale) {
    __shared__ float red[kSumWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = 2 * H;
    float s = 0.f;
    if (lane < n) {
#pragma unroll 8
        for (int64_t k = w; k < segs; k += kSumWaves) s += part[k * n + lane];
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && lane < n) {
        float t = red[0][lane];
        for (int j = 1; j < kSumWaves; ++j) t += red[j][lane];
        if (lane < H) ddbias[lane] = t;
        else ddscale[lane - H] = -t * expf(dscale[lane - H]);
    }
}

// ---- mixer output gate ------------------------------------------------------------
// Rows r = (b t) H + h of V = 64 values: 16 lanes per row, 4 values per lane.
struct OutArgs {
    int64_t rows, zs;
    int H, gcol;  // gate column of head 0 in z
    float eps;
    const bf16_t *o, *z;
    const float *w;
    bf16_t *y;
    float *inv;
    const float *inv_in;
    const bf16_t *dy;
    bf16_t *d_o, *dz;
    float *part;
};

__global__ void __launch_bounds__(256) lm_out_fwd_kernel(OutArgs a) {
    const int lane = threadIdx.x & 15;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool live = row < a.rows;
    const int64_t r = live ? row : a.rows - 1;  // a spare row group redoes the last row, stores nothing
    const int64_t bt = r / a.H;
    const int h = (int)(r % a.H);
    const float4 o = ld_bf4(a.o + r * 64 + 4 * lane);
    const float ss = sum16(dot4(o, o));
    const float inv = frsq(ss * (1.f / 64.f) + a.eps);
    if (!live) return;
    const float4 w = ld_f4(a.w + 4 * lane);
    const float4 g = ld_bf4(a.z + bt * a.zs + a.gcol + h * 64 + 4 * lane);
    const float4 y = make_float4(o.x * inv * w.x * silu_div(g.x), o.y * inv * w.y * silu_div(g.y),
                                 o.z * inv * w.z * silu_div(g.z), o.w * inv * w.w * silu_div(g.w));
    st_bf4(a.y + r * 64 + 4 * lane, y);
    if (lane == 0) a.inv[row] = inv;
}

struct OutGrad {
    float dn, dg;
};

// Per value: n = o inv w, y = n silu(g); returns dn = dy silu(g) and the gate gradient.
__device__ __forceinline__ OutGrad out_grad(float dy, float o, float inv, float w, float g) {
    const float n = o * inv * w;
    return {dy * silu_div(g), silu_vjp(g, dy * n)};
}

__global__ void __launch_bounds__(256) lm_out_bwd_kernel(OutArgs a) {
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const float4 w = ld_f4(a.w + 4 * lane);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t r0 = (int64_t)blockIdx.x * 16; r0 < a.rows; r0 += (int64_t)gridDim.x * 16) {
        const int64_t row = r0 + slot;
        const bool live = row < a.rows;
        const int64_t r = live ? row : a.rows - 1;
        const int64_t bt = r / a.H;
        const int h = (int)(r % a.H);
        const float4 o = ld_bf4(a.o + r * 64 + 4 * lane);
        const float4 dy = ld_bf4(a.dy + r * 64 + 4 * lane);
        const float4 g = ld_bf4(a.z + bt * a.zs + a.gcol + h * 64 + 4 * lane);
        const float inv = a.inv_in[r];
        const OutGrad ex = out_grad(dy.x, o.x, inv, w.x, g.x), ey = out_grad(dy.y, o.y, inv, w.y, g.y),
                      ez = out_grad(dy.z, o.z, inv, w.z, g.z), ew = out_grad(dy.w, o.w, inv, w.w, g.w);
        const float4 uw = make_float4(ex.dn * w.x, ey.dn * w.y, ez.dn * w.z, ew.dn * w.w);
        const float dot = sum16(dot4(uw, o));
        if (!live) continue;
        const float corr = dot * inv * inv / 64.f;
        st_bf4(a.d_o + r * 64 + 4 * lane,
               make_float4((uw.x - o.x * corr) * inv, (uw.y - o.y * corr) * inv,
                           (uw.z - o.z * corr) * inv, (uw.w - o.w * corr) * inv));
        st_bf4(a.dz + bt * a.zs + a.gcol + h * 64 + 4 * lane, make_float4(ex.dg, ey.dg, ez.dg, ew.dg));
        acc.x += ex.dn * o.x * inv;
        acc.y += ey.dn * o.y * inv;
        acc.z += ez.dn * o.z * inv;
        acc.w += ew.dn * o.w * inv;
    }
    st_f4(&red[slot][4 * lane], acc);
    __syncthreads();
    if (threadIdx.x < 64) {
        float s = red[0][threadIdx.x];
        for (int j = 1; j < 16; ++j) s += red[j][threadIdx.x];
        a.part[(int64_t)blockIdx.x * 64 + threadIdx.x] = s;
    }
}

// ---- SwiGLU -------------------------------------------------------------------------
// h [rows, 2M] = [gate | up]; 8 values per thread.
struct GluArgs {
    int64_t rows, M;
    const bf16_t *h, *da;
    bf16_t *a, *dh;
};

__device__ __forceinline__ void unpack8(uint4 u, float *f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = lo_f(w[i]);
        f[2 * i + 1] = hi_f(w[i]);
    }
}
__device__ __forceinline__ uint4 pack8(const float *f) {
    return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
}

__global__ void __launch_bounds__(256) lm_glu_fwd_kernel(GluArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per = a.M / 8;
    if (i >= a.rows * per) return;
    const int64_t r = i / per, j = (i % per) * 8;
    float g[8], u[8], y[8];
    unpack8(*reinterpret_cast<const uint4 *>(a.h + r * 2 * a.M + j), g);
    unpack8(*reinterpret_cast<const uint4 *>(a.h + r * 2 * a.M + a.M + j), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = rbf(silu_div(g[e])) * u[e];
    *reinterpret_cast<uint4 *>(a.a + r * a.M + j) = pack8(y);
}

__global__ void __launch_bounds__(256) lm_glu_bwd_kernel(GluArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per = a.M / 8;
    if (i >= a.rows * per) return;
    const int64_t r = i / per, j = (i % per) * 8;
    float g[8], u[8], d[8], dg[8], du[8];
    unpack8(*reinterpret_cast<const uint4 *>(a.h + r * 2 * a.M + j), g);
    unpack8(*reinterpret_cast<const uint4 *>(a.h + r * 2 * a.M + a.M + j), u);
    unpack8(*reinterpret_cast<const uint4 *>(a.da + r * a.M + j), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float s = rbf(silu_div(g[e]));
        du[e] = d[e] * s;
        dg[e] = silu_vjp(g[e], rbf(d[e] * u[e]));
    }
    *reinterpret_cast<uint4 *>(a.dh + r * 2 * a.M + j) = pack8(dg);
    *reinterpret_cast<uint4 *>(a.dh + r * 2 * a.M + a.M + j) = pack8(du);
}

// ---- host helpers ------------------------------------------------------------------
bool al(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

int check_in_shape(const gdn2_lm_mixer_shape *s) {
    if (!s) return fail(GDN2_ERR_ARGUMENT, "shape is null");
    if (s->batch <= 0 || s->time <= 0 || s->heads <= 0)
        return fail(GDN2_ERR_SHAPE, "mixer shape requires nonempty axes");
    if (s->keys != 64 || s->values != 64)
        return fail(GDN2_ERR_SHAPE, "the fused mixer operators take keys = values = 64");
    if (s->heads > 32 || (s->heads & (s->heads - 1)))
        return fail(GDN2_ERR_SHAPE, "heads must be a power of two up to 32 (got %lld)",
                    (long long)s->heads);
    if (s->taps < 1 || s->taps > 8) return fail(GDN2_ERR_SHAPE, "taps must be 1..8");
    const int64_t width = 4 * s->heads * 64 + 2 * s->heads;
    if (s->z_stride < width || s->z_stride % 4)
        return fail(GDN2_ERR_SHAPE, "z_stride must be >= %lld and a multiple of 4",
                    (long long)width);
    if (s->batch * s->time * s->z_stride > ((int64_t)1 << 38))
        return fail(GDN2_ERR_SHAPE, "mixer tensors too large");
    return GDN2_OK;
}

InArgs in_args(const gdn2_lm_mixer_shape *s, const void *z, const float *conv_w,
               const float *valid, const float *docs, const float *dscale, const float *dbias) {
    InArgs a{};
    a.B = s->batch;
    a.T = s->time;
    a.zs = s->z_stride;
    a.H = (int)s->heads;
    a.K = 64;
    a.V = 64;
    a.C = 3 * a.H * 64;
    a.z = static_cast<const bf16_t *>(z);
    a.w = conv_w;
    a.valid = valid;
    a.docs = docs;
    a.dscale = dscale;
    a.dbias = dbias;
    return a;
}

template <template <int> class K>
void launch_taps(int W, dim3 grid, hipStream_t st, const InArgs &a) {
    switch (W) {
        case 1: hipLaunchKernelGGL(K<1>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 2: hipLaunchKernelGGL(K<2>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 3: hipLaunchKernelGGL(K<3>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 4: hipLaunchKernelGGL(K<4>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 5: hipLaunchKernelGGL(K<5>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 6: hipLaunchKernelGGL(K<6>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        case 7: hipLaunchKernelGGL(K<7>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
        default: hipLaunchKernelGGL(K<8>::fn, grid, dim3(64 * kInWaves), 0, st, a); break;
    }
}
template <int W> struct InFwd { static constexpr auto fn = lm_in_fwd_kernel<W>; };
template <int W> struct InBwd { static constexpr auto fn = lm_in_bwd_kernel<W>; };

dim3 in_grid(const InArgs &a) {
    return dim3((unsigned)(a.B * in_segments(a.T)), (unsigned)(a.C / 64 + 1));
}

// Row widths of the norm kernels: 4 G NV with G = 64 (multiples of 256 up to
// 1024) or G = 32 (width 128).
int check_norm_shape(int64_t rows, int64_t width) {
    if (rows <= 0) return fail(GDN2_ERR_SHAPE, "rows must be positive");
    if (width != 128 && (width <= 0 || width % 256 || width > 1024))
        return fail(GDN2_ERR_SHAPE, "width must be 128 or a multiple of 256 up to 1024 (got %lld)",
                    (long long)width);
    if (rows * width > ((int64_t)1 << 38)) return fail(GDN2_ERR_SHAPE, "rows too large");
    return GDN2_OK;
}

int norm_lanes(int64_t width) { return width == 128 ? 32 : 64; }

int64_t norm_blocks(int64_t rows, int64_t width) {
    const int64_t rpb = 256 / norm_lanes(width);
    return std::max<int64_t>(1, std::min<int64_t>((rows + rpb - 1) / rpb, kBwdBlocks));
}
int64_t out_blocks(int64_t rows) {
    return std::max<int64_t>(1, std::min<int64_t>((rows + 15) / 16, kBwdBlocks));
}

}  // namespace
}  // namespace gdn2

using namespace gdn2;

extern "C" {

int gdn2_lm_norm_forward(int64_t rows, int64_t width, float epsilon, const float *x,
                         const void *residual, const float *weight, float *u, void *y,
                         float *inverse, void *stream) {
    GDN2_TRY(check_norm_shape(rows, width));
    if (!(epsilon > 0.f) || !isfinite(epsilon))
        return fail(GDN2_ERR_ARGUMENT, "epsilon must be finite and positive");
    if (!x || !weight || !y || !inverse) return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!al(x, 16) || !al(weight, 16) || (u && !al(u, 16)) || !al(y, 8) ||
        (residual && !al(residual, 8)))
        return fail(GDN2_ERR_ARGUMENT, "operands must be 16-byte (f32) / 8-byte (bf16) aligned");
    NormArgs a{};
    a.rows = rows;
    a.W = (int)width;
    a.eps = epsilon;
    a.x = x;
    a.res = static_cast<const bf16_t *>(residual);
    a.w = weight;
    a.u = u;
    a.y = static_cast<bf16_t *>(y);
    a.inv = inverse;
    const int G = norm_lanes(width);
    const dim3 grid((unsigned)((rows + 256 / G - 1) / (256 / G)));
    hipStream_t st = (hipStream_t)stream;
    if (G == 32) {
        hipLaunchKernelGGL((lm_norm_fwd_kernel<32, 1>), grid, dim3(256), 0, st, a);
    } else {
        switch (width / 256) {
            case 1: hipLaunchKernelGGL((lm_norm_fwd_kernel<64, 1>), grid, dim3(256), 0, st, a); break;
            case 2: hipLaunchKernelGGL((lm_norm_fwd_kernel<64, 2>), grid, dim3(256), 0, st, a); break;
            case 3: hipLaunchKernelGGL((lm_norm_fwd_kernel<64, 3>), grid, dim3(256), 0, st, a); break;
            default: hipLaunchKernelGGL((lm_norm_fwd_kernel<64, 4>), grid, dim3(256), 0, st, a); break;
        }
    }
    return launch_status(hipGetLastError(), "gdn2_lm_norm_forward");
}

size_t gdn2_lm_norm_workspace_bytes(int64_t rows, int64_t width) {
    if (rows <= 0 || width <= 0) return 0;
    return (size_t)norm_blocks(rows, width) * width * sizeof(float);
}

int gdn2_lm_norm_backward(int64_t rows, int64_t width, const float *x, const float *weight,
                          const float *inverse, const void *dy, const float *dres, float *dx,
                          void *dx_bf16, float *dweight, void *workspace, size_t workspace_bytes,
                          void *stream) {
    GDN2_TRY(check_norm_shape(rows, width));
    if (!x || !weight || !inverse || !dy || !dx || !dweight)
        return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!al(x, 16) || !al(weight, 16) || !al(dx, 16) || (dres && !al(dres, 16)) || !al(dy, 8) ||
        (dx_bf16 && !al(dx_bf16, 8)))
        return fail(GDN2_ERR_ARGUMENT, "operands must be 16-byte (f32) / 8-byte (bf16) aligned");
    if (!workspace || workspace_bytes < gdn2_lm_norm_workspace_bytes(rows, width))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn2_lm_norm_workspace_bytes(rows, width), workspace_bytes);
    NormArgs a{};
    a.rows = rows;
    a.W = (int)width;
    a.x = x;
    a.w = weight;
    a.inv_in = inverse;
    a.dy = static_cast<const bf16_t *>(dy);
    a.dres = dres;
    a.dx = dx;
    a.dxb = static_cast<bf16_t *>(dx_bf16);
    a.part = static_cast<float *>(workspace);
    const int64_t nb = norm_blocks(rows, width);
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)nb);
    if (norm_lanes(width) == 32) {
        hipLaunchKernelGGL((lm_norm_bwd_kernel<32, 1>), grid, dim3(256), 0, st, a);
    } else {
        switch (width / 256) {
            case 1: hipLaunchKernelGGL((lm_norm_bwd_kernel<64, 1>), grid, dim3(256), 0, st, a); break;
            case 2: hipLaunchKernelGGL((lm_norm_bwd_kernel<64, 2>), grid, dim3(256), 0, st, a); break;
            case 3: hipLaunchKernelGGL((lm_norm_bwd_kernel<64, 3>), grid, dim3(256), 0, st, a); break;
            default: hipLaunchKernelGGL((lm_norm_bwd_kernel<64, 4>), grid, dim3(256), 0, st, a); break;
        }
    }
    colsum(a.part, width, nb, dweight, st);
    return launch_status(hipGetLastError(), "gdn2_lm_norm_backward");
}

int gdn2_lm_mixer_in_forward(const gdn2_lm_mixer_shape *shape, const void *z, const float *conv_w,
                             const float *valid, const float *docs, const float *decay_scale,
                             const float *decay_bias, void *qkv, float *beta, float *g,
                             void *stream) {
    GDN2_TRY(check_in_shape(shape));
    if (!z || !conv_w || !valid || !docs || !decay_scale || !decay_bias || !qkv || !beta || !g)
        return fail(GDN2_ERR_ARGUMENT, "null operand");
    InArgs a = in_args(shape, z, conv_w, valid, docs, decay_scale, decay_bias);
    a.qkv = static_cast<bf16_t *>(qkv);
    a.beta = beta;
    a.g = g;
    launch_taps<InFwd>((int)shape->taps, in_grid(a), (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_lm_mixer_in_forward");
}

size_t gdn2_lm_mixer_in_workspace_bytes(const gdn2_lm_mixer_shape *shape) {
    if (!shape || shape->batch < 1 || shape->time < 1 || shape->heads < 1 || shape->taps < 1)
        return 0;
    const int64_t segs = shape->batch * in_segments(shape->time);
    const int64_t C = 3 * shape->heads * 64;
    return (size_t)segs * (shape->taps * C + 2 * shape->heads) * sizeof(float);
}

int gdn2_lm_mixer_in_backward(const gdn2_lm_mixer_shape *shape, const void *z,
                              const float *conv_w, const float *valid, const float *docs,
                              const float *decay_scale, const float *decay_bias, const void *dq,
                              const void *dk, const void *dv, const float *dbeta, const float *dg,
                              void *dz, float *dconv_w, float *ddecay_scale, float *ddecay_bias,
                              void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_in_shape(shape));
    if (!z || !conv_w || !valid || !docs || !decay_scale || !decay_bias || !dq || !dk || !dv ||
        !dbeta || !dg || !dz || !dconv_w || !ddecay_scale || !ddecay_bias)
        return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!workspace || workspace_bytes < gdn2_lm_mixer_in_workspace_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn2_lm_mixer_in_workspace_bytes(shape), workspace_bytes);
    InArgs a = in_args(shape, z, conv_w, valid, docs, decay_scale, decay_bias);
    a.dq = static_cast<const bf16_t *>(dq);
    a.dk = static_cast<const bf16_t *>(dk);
    a.dv = static_cast<const bf16_t *>(dv);
    a.dbeta = dbeta;
    a.dg = dg;
    a.dz = static_cast<bf16_t *>(dz);
    const int64_t segs = a.B * in_segments(a.T);
    a.wpart = static_cast<float *>(workspace);
    a.gpart = a.wpart + segs * shape->taps * a.C;
    hipStream_t st = (hipStream_t)stream;
    launch_taps<InBwd>((int)shape->taps, in_grid(a), st, a);
    colsum(a.wpart, shape->taps * a.C, segs, dconv_w, st);
    hipLaunchKernelGGL(lm_gate_sum_kernel, dim3(1), dim3(64 * kSumWaves), 0, st, a.gpart, a.H,
                       segs, decay_scale, ddecay_bias, ddecay_scale);
    return launch_status(hipGetLastError(), "gdn2_lm_mixer_in_backward");
}

int gdn2_lm_mixer_out_forward(const gdn2_lm_mixer_shape *shape, const void *o, const void *z,
                              const float *norm_w, float epsilon, void *y, float *inverse,
                              void *stream) {
    GDN2_TRY(check_in_shape(shape));
    if (!o || !z || !norm_w || !y || !inverse) return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!(epsilon > 0.f) || !isfinite(epsilon))
        return fail(GDN2_ERR_ARGUMENT, "epsilon must be finite and positive");
    if (!al(o, 8) || !al(z, 8) || !al(y, 8) || !al(norm_w, 16))
        return fail(GDN2_ERR_ARGUMENT, "operands must be 8-byte (bf16) / 16-byte (f32) aligned");
    OutArgs a{};
    a.rows = shape->batch * shape->time * shape->heads;
    a.zs = shape->z_stride;
    a.H = (int)shape->heads;
    a.gcol = 3 * a.H * 64;
    a.eps = epsilon;
    a.o = static_cast<const bf16_t *>(o);
    a.z = static_cast<const bf16_t *>(z);
    a.w = norm_w;
    a.y = static_cast<bf16_t *>(y);
    a.inv = inverse;
    hipLaunchKernelGGL(lm_out_fwd_kernel, dim3((unsigned)((a.rows + 15) / 16)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_lm_mixer_out_forward");
}

size_t gdn2_lm_mixer_out_workspace_bytes(const gdn2_lm_mixer_shape *shape) {
    if (!shape || shape->batch < 1 || shape->time < 1 || shape->heads < 1) return 0;
    return (size_t)out_blocks(shape->batch * shape->time * shape->heads) * 64 * sizeof(float);
}

int gdn2_lm_mixer_out_backward(const gdn2_lm_mixer_shape *shape, const void *o, const void *z,
                               const float *norm_w, const float *inverse, const void *dy,
                               void *d_o, void *dz, float *dnorm_w, void *workspace,
                               size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_in_shape(shape));
    if (!o || !z || !norm_w || !inverse || !dy || !d_o || !dz || !dnorm_w)
        return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!al(o, 8) || !al(z, 8) || !al(dy, 8) || !al(d_o, 8) || !al(dz, 8) || !al(norm_w, 16))
        return fail(GDN2_ERR_ARGUMENT, "operands must be 8-byte (bf16) / 16-byte (f32) aligned");
    if (!workspace || workspace_bytes < gdn2_lm_mixer_out_workspace_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn2_lm_mixer_out_workspace_bytes(shape), workspace_bytes);
    OutArgs a{};
    a.rows = shape->batch * shape->time * shape->heads;
    a.zs = shape->z_stride;
    a.H = (int)shape->heads;
    a.gcol = 3 * a.H * 64;
    a.o = static_cast<const bf16_t *>(o);
    a.z = static_cast<const bf16_t *>(z);
    a.w = norm_w;
    a.inv_in = inverse;
    a.dy = static_cast<const bf16_t *>(dy);
    a.d_o = static_cast<bf16_t *>(d_o);
    a.dz = static_cast<bf16_t *>(dz);
    a.part = static_cast<float *>(workspace);
    const int64_t nb = out_blocks(a.rows);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(lm_out_bwd_kernel, dim3((unsigned)nb), dim3(256), 0, st, a);
    colsum(a.part, 64, nb, dnorm_w, st);
    return launch_status(hipGetLastError(), "gdn2_lm_mixer_out_backward");
}

int gdn2_lm_swiglu_forward(int64_t rows, int64_t width, const void *h, void *a, void *stream) {
    if (rows <= 0 || width <= 0 || width % 8)
        return fail(GDN2_ERR_SHAPE, "rows must be positive and width a positive multiple of 8");
    if (rows * width > ((int64_t)1 << 38)) return fail(GDN2_ERR_SHAPE, "rows too large");
    if (!h || !a) return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!al(h, 16) || !al(a, 16)) return fail(GDN2_ERR_ARGUMENT, "operands must be 16-byte aligned");
    GluArgs g{};
    g.rows = rows;
    g.M = width;
    g.h = static_cast<const bf16_t *>(h);
    g.a = static_cast<bf16_t *>(a);
    const int64_t n = rows * (width / 8);
    hipLaunchKernelGGL(lm_glu_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, g);
    return launch_status(hipGetLastError(), "gdn2_lm_swiglu_forward");
}

int gdn2_lm_swiglu_backward(int64_t rows, int64_t width, const void *h, const void *da, void *dh,
                            void *stream) {
    if (rows <= 0 || width <= 0 || width % 8)
        return fail(GDN2_ERR_SHAPE, "rows must be positive and width a positive multiple of 8");
    if (rows * width > ((int64_t)1 << 38)) return fail(GDN2_ERR_SHAPE, "rows too large");
    if (!h || !da || !dh) return fail(GDN2_ERR_ARGUMENT, "null operand");
    if (!al(h, 16) || !al(da, 16) || !al(dh, 16))
        return fail(GDN2_ERR_ARGUMENT, "operands must be 16-byte aligned");
    GluArgs g{};
    g.rows = rows;
    g.M = width;
    g.h = static_cast<const bf16_t *>(h);
    g.da = static_cast<const bf16_t *>(da);
    g.dh = static_cast<bf16_t *>(dh);
    const int64_t n = rows * (width / 8);
    hipLaunchKernelGGL(lm_glu_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, g);
    return launch_status(hipGetLastError(), "gdn2_lm_swiglu_backward");
}

}  // extern "C"
