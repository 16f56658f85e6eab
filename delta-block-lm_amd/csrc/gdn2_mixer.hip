// Mixer prologue / epilogue operators on gfx950: depthwise causal convolution
// (with optional fused SiLU), L2 / RMS / sigmoid-gated RMS row normalization,
// and the decay gate, each with its VJP.
//
// Semantics follow the reference custom ops (crates/kernels/src/conv.rs,
// norm.rs, decay.rs) and their scalar-f64 checks
// (crates/mixers/src/convolution_checks.rs, normalization_checks.rs).
//
// These operators move a few bytes per flop, so each is laid out for HBM:
//   * the convolution gives each thread one channel (consecutive channels on
//     consecutive lanes) and a segment of kConvRows time steps, swept in order
//     with the tap window in registers: every input element is loaded once, and
//     the backward produces dx and the weight-gradient partials in one pass;
//   * row normalizations of contiguous rows (width a multiple of 64 up to 256,
//     or of 256 up to 1024) give each row 16 or 64 lanes with 16-byte accesses
//     and reduce with DPP; other layouts take a one-wave-per-row kernel;
//   * parameter gradients (conv weight, norm weight, decay bias/scale) are
//     reduced in two deterministic passes: partial sums per row segment into
//     the caller's workspace, then a fixed-order sum over segments.
#include <math.h>

#include <algorithm>

#include "gdn2_status.h"

namespace gdn2 {
namespace {

constexpr int64_t kMaxSegments = 1024;  // row segments of the parameter-gradient reductions
constexpr int kMaxTaps = 8;
constexpr int kMaxNormWidth = 1024;

__device__ __forceinline__ float ldv(const gdn2_view &v, int64_t i0, int64_t i1, int64_t i2 = 0,
                                     int64_t i3 = 0) {
    return reinterpret_cast<const float *>(v.data)[i0 * v.stride[0] + i1 * v.stride[1] +
                                                   i2 * v.stride[2] + i3 * v.stride[3]];
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave, in every lane (DPP within rows, readlane across).
__device__ __forceinline__ float wave_total(float x) {
    x += dpp_move<0xB1>(x);
    x += dpp_move<0x4E>(x);
    x += dpp_move<0x141>(x);
    x += dpp_move<0x140>(x);
    const int r = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 16)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 32)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 48));
}

// Row segments of about 32 rows each (at most kMaxSegments), and rows per segment.
int64_t segment_count(int64_t rows) {
    return std::max<int64_t>(1, std::min<int64_t>((rows + 31) / 32, kMaxSegments));
}
int64_t segment_rows(int64_t rows) {
    const int64_t s = segment_count(rows);
    return (rows + s - 1) / s;
}

// out[i] = sum_s part[s * n + i] over s < segments: 64 outputs per workgroup,
// each of its 16 waves summing every 16th segment, then the waves in order.
constexpr int kColumnWaves = 16;
__global__ void __launch_bounds__(64 * kColumnWaves) column_sum_kernel(const float *part, int64_t n,
                                                                      int64_t segments, float *out) {
    __shared__ float red[kColumnWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (i < n) {
#pragma unroll 8
        for (int64_t k = w; k < segments; k += kColumnWaves) s += part[k * n + i];
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && i < n) {
        float t = red[0][lane];
        for (int j = 1; j < kColumnWaves; ++j) t += red[j][lane];
        out[i] = t;
    }
}

void column_sum(const float *part, int64_t n, int64_t segments, float *out, hipStream_t st) {
    hipLaunchKernelGGL(column_sum_kernel, dim3((unsigned)((n + 63) / 64)), dim3(64 * kColumnWaves),
                       0, st, part, n, segments, out);
}

// out[g] = sum_s sum_{j < group} part[s * n + g * group + j]  (n = groups * group).
__global__ void segment_group_sum_kernel(const float *part, int64_t groups, int64_t group,
                                         int segments, float *out) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const int64_t n = groups * group;
    float s = 0.f;
    for (int k = 0; k < segments; ++k)
        for (int64_t j = 0; j < group; ++j) s += part[(int64_t)k * n + g * group + j];
    out[g] = s;
}

// ---- convolution ------------------------------------------------------------
struct ConvArgs {
    int64_t B, T, C;
    int W, act;
    gdn2_view x, w, valid, docs, dy;
    float *y, *dx, *dw_part;
};

// d(act(p))/dp times the upstream value.
__device__ __forceinline__ float act_grad(int act, float p, float up) {
    if (!act) return up;
    const float s = sigmoidf(p);
    return up * s * (1.f + p * (1.f - s));
}

constexpr int kConvRows = 32;  // time steps per thread (one segment)

__host__ __device__ inline int64_t conv_segments(int64_t T) { return (T + kConvRows - 1) / kConvRows; }

// A thread's sliding window over time: slot l holds row t - l of its channel
// (input value, document id, valid flag).  Rows before 0 or from T on read as
// zero input, invalid.
template <int W>
struct ConvWindow {
    float x[W], d[W], v[W];

    __device__ __forceinline__ void clear() {
#pragma unroll
        for (int l = 0; l < W; ++l) x[l] = d[l] = v[l] = 0.f;
    }
    __device__ __forceinline__ void push(const ConvArgs &a, int64_t b, int64_t t, int64_t c) {
#pragma unroll
        for (int l = W - 1; l > 0; --l) {
            x[l] = x[l - 1];
            d[l] = d[l - 1];
            v[l] = v[l - 1];
        }
        const bool in = t >= 0 && t < a.T;
        x[0] = in ? ldv(a.x, b, t, c) : 0.f;
        d[0] = in ? ldv(a.docs, b, t) : 0.f;
        v[0] = in ? ldv(a.valid, b, t) : 0.f;
    }
    // Mask of the lag from slot s (source) to slot r (destination).
    __device__ __forceinline__ float mask(int s, int r) const {
        return d[s] == d[r] ? v[s] * v[r] : 0.f;
    }
    // Pre-activation output of the row in slot 0.
    __device__ __forceinline__ float pre(const float *w) const {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < W; ++l) s += x[l] * w[l] * mask(l, 0);
        return s;
    }
};

// Grid (batch * segments, channel blocks of 64); one wave per workgroup.
template <int W>
__global__ void __launch_bounds__(64) conv_forward_kernel(ConvArgs a) {
    const int64_t c = (int64_t)blockIdx.y * 64 + threadIdx.x;
    const int64_t nseg = conv_segments(a.T);
    const int64_t b = blockIdx.x / nseg, t0 = (blockIdx.x % nseg) * kConvRows;
    const int64_t t1 = min(t0 + kConvRows, a.T);
    if (c >= a.C) return;
    float w[W];
#pragma unroll
    for (int l = 0; l < W; ++l) w[l] = ldv(a.w, l, c);
    ConvWindow<W> win;
    win.clear();
    for (int64_t t = t0 - (W - 1); t < t0; ++t) win.push(a, b, t, c);
#pragma unroll 4
    for (int64_t t = t0; t < t1; ++t) {
        win.push(a, b, t, c);
        const float p = win.pre(w);
        a.y[(b * a.T + t) * a.C + c] = a.act ? p * sigmoidf(p) : p;
    }
}

// dx and per-segment weight-gradient partials in one sweep.  With g the
// gradient at the pre-activation output:
//   dx[t]     = sum_l g[t + l] w[l] mask(t -> t + l)
//   dw[l]    += g[t] x[t - l] mask(t - l -> t)           (t in this segment)
// The sweep runs t' from t0 to t1 + W - 2, computing g[t'] (rows of the next
// segment recomputed, rows past T zero) and emitting dx[t' - W + 1].
template <int W>
__global__ void __launch_bounds__(64) conv_backward_kernel(ConvArgs a) {
    const int64_t c = (int64_t)blockIdx.y * 64 + threadIdx.x;
    const int64_t nseg = conv_segments(a.T);
    const int64_t b = blockIdx.x / nseg, t0 = (blockIdx.x % nseg) * kConvRows;
    const int64_t t1 = min(t0 + kConvRows, a.T);
    if (c >= a.C) return;
    float w[W], dw[W], g[W];  // g[k]: gradient of the row in window slot k
#pragma unroll
    for (int l = 0; l < W; ++l) {
        w[l] = ldv(a.w, l, c);
        dw[l] = 0.f;
        g[l] = 0.f;
    }
    ConvWindow<W> win;
    win.clear();
    for (int64_t t = t0 - (W - 1); t < t0; ++t) win.push(a, b, t, c);
#pragma unroll 4
    for (int64_t t = t0; t < t1 + W - 1; ++t) {
        win.push(a, b, t, c);
#pragma unroll
        for (int l = W - 1; l > 0; --l) g[l] = g[l - 1];
        g[0] = 0.f;
        if (t < a.T) {
            const float up = ldv(a.dy, b, t, c);
            g[0] = a.act ? act_grad(1, win.pre(w), up) : up;
        }
        if (a.dw_part && t < t1) {
#pragma unroll
            for (int l = 0; l < W; ++l) dw[l] += g[0] * win.x[l] * win.mask(l, 0);
        }
        const int64_t td = t - (W - 1);  // the row whose dx is now complete (slot W - 1)
        if (a.dx && td >= t0) {
            float s = 0.f;
#pragma unroll
            for (int l = 0; l < W; ++l) {
                const float m = win.mask(W - 1, W - 1 - l);
                if (m != 0.f) s += g[W - 1 - l] * w[l] * m;
            }
            a.dx[(b * a.T + td) * a.C + c] = s;
        }
    }
    if (a.dw_part) {
        float *part = a.dw_part + (int64_t)blockIdx.x * W * a.C;
#pragma unroll
        for (int l = 0; l < W; ++l) part[l * a.C + c] = dw[l];
    }
}

// ---- row normalization -------------------------------------------------------
struct NormArgs {
    int64_t B, T, H, W;
    int mode;
    float eps;
    gdn2_view x, weight, gate, dy;
    float *y, *inverse;
    const float *inv_in;
    float *dx, *dgate, *dw_part;
};

__device__ __forceinline__ void row_index(const NormArgs &a, int64_t row, int64_t &b, int64_t &t,
                                          int64_t &h) {
    h = row % a.H;
    t = row / a.H % a.T;
    b = row / (a.H * a.T);
}

// One wave per row, lanes over the width.
__global__ void __launch_bounds__(256) norm_forward_kernel(NormArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.B * a.T * a.H) return;
    int64_t b, t, h;
    row_index(a, row, b, t, h);
    float z[kMaxNormWidth / 64];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxNormWidth / 64; ++j) {
        const int64_t c = lane + 64 * j;
        z[j] = 0.f;
        if (c < a.W) {
            float v = ldv(a.x, b, t, h, c);
            if (a.mode == 2) v *= sigmoidf(ldv(a.gate, b, t, h, c));
            z[j] = v;
            ss += v * v;
        }
    }
    ss = wave_total(ss);
    const float div = a.mode == 0 ? 1.f : (float)a.W;
    const float inv = 1.f / sqrtf(ss / div + a.eps);
    if (lane == 0) a.inverse[row] = inv;
#pragma unroll
    for (int j = 0; j < kMaxNormWidth / 64; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < a.W) {
            float v = z[j] * inv;
            if (a.mode != 0) v *= ldv(a.weight, c, 0);
            a.y[row * a.W + c] = v;
        }
    }
}

__global__ void __launch_bounds__(256) norm_dx_kernel(NormArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.B * a.T * a.H) return;
    int64_t b, t, h;
    row_index(a, row, b, t, h);
    float z[kMaxNormWidth / 64], u[kMaxNormWidth / 64], sg[kMaxNormWidth / 64];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxNormWidth / 64; ++j) {
        const int64_t c = lane + 64 * j;
        z[j] = u[j] = 0.f;
        sg[j] = 1.f;
        if (c < a.W) {
            float v = ldv(a.x, b, t, h, c);
            if (a.mode == 2) {
                sg[j] = sigmoidf(ldv(a.gate, b, t, h, c));
                v *= sg[j];
            }
            z[j] = v;
            float up = ldv(a.dy, b, t, h, c);
            if (a.mode != 0) up *= ldv(a.weight, c, 0);
            u[j] = up;
            dot += up * v;
        }
    }
    dot = wave_total(dot);
    const float inv = a.inv_in[row];
    const float corr = dot * inv * inv / (a.mode == 0 ? 1.f : (float)a.W);
#pragma unroll
    for (int j = 0; j < kMaxNormWidth / 64; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < a.W) {
            const float dz = (u[j] - z[j] * corr) * inv;
            if (a.dx) a.dx[row * a.W + c] = dz * sg[j];
            if (a.mode == 2 && a.dgate) a.dgate[row * a.W + c] = dz * z[j] * (1.f - sg[j]);
        }
    }
}

// Partial weight gradients: block (column block, segment), lane = column.
__global__ void __launch_bounds__(64) norm_dw_partial_kernel(NormArgs a, int64_t seg_rows) {
    const int64_t c = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int seg = blockIdx.y;
    if (c >= a.W) return;
    const int64_t rows = a.B * a.T * a.H;
    const int64_t r0 = seg * seg_rows, r1 = min(r0 + seg_rows, rows);
    float acc = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
        int64_t b, t, h;
        row_index(a, r, b, t, h);
        float v = ldv(a.x, b, t, h, c);
        if (a.mode == 2) v *= sigmoidf(ldv(a.gate, b, t, h, c));
        acc += ldv(a.dy, b, t, h, c) * v * a.inv_in[r];
    }
    a.dw_part[(int64_t)seg * a.W + c] = acc;
}

// ---- row normalization, contiguous rows ---------------------------------------
// G lanes per row (16 or 64), NV float4 per lane: width = 4 G NV.  Row r is
// (b, t, h) = (r / (T H), r / H % T, r % H); every operand row starts on a
// 16-byte boundary.
struct NormFast {
    int64_t rows, T, H, W;
    const float *x, *gate, *dy;
    int64_t xs[3], gs[3], ds[3];  // element strides of b, t, h
    gdn2_view weight;
    int mode;
    float eps, div;
    float *y, *inverse, *dx, *dgate, *dw_part;
    const float *inv_in;
};

template <int G>
__device__ __forceinline__ float group_sum(float x) {
    x += dpp_move<0xB1>(x);
    x += dpp_move<0x4E>(x);
    x += dpp_move<0x141>(x);
    x += dpp_move<0x140>(x);
    if (G == 64) {
        const int r = __builtin_bit_cast(int, x);
        x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 16)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(r, 48));
    }
    return x;
}

__device__ __forceinline__ int64_t row_offset(const int64_t *st, int64_t r, int64_t T, int64_t H) {
    return r / (T * H) * st[0] + r / H % T * st[1] + r % H * st[2];
}

__device__ __forceinline__ float4 ld4f(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4f(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ float4 sig4(float4 g) {
    return make_float4(sigmoidf(g.x), sigmoidf(g.y), sigmoidf(g.z), sigmoidf(g.w));
}
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

template <int G, int NV>
__device__ __forceinline__ float4 weight4(const NormFast &a, int k, int lane) {
    if (a.mode == 0) return make_float4(1.f, 1.f, 1.f, 1.f);
    const int64_t c = (int64_t)(k * G + lane) * 4;
    return make_float4(ldv(a.weight, c, 0), ldv(a.weight, c + 1, 0), ldv(a.weight, c + 2, 0),
                       ldv(a.weight, c + 3, 0));
}

template <int G, int NV>
__global__ void __launch_bounds__(256) norm_forward_fast_kernel(NormFast a) {
    constexpr int RPB = 256 / G;
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / G;
    const bool live = row < a.rows;
    const int64_t r = live ? row : a.rows - 1;  // a spare group redoes the last row, stores nothing
    const float *x = a.x + row_offset(a.xs, r, a.T, a.H);
    const float *gt = a.mode == 2 ? a.gate + row_offset(a.gs, r, a.T, a.H) : nullptr;
    float4 z[NV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * G + lane) * 4;
        z[k] = ld4f(x + c);
        if (a.mode == 2) z[k] = mul4(z[k], sig4(ld4f(gt + c)));
        ss += dot4(z[k], z[k]);
    }
    ss = group_sum<G>(ss);
    const float inv = 1.f / sqrtf(ss / a.div + a.eps);
    if (!live) return;
    if (lane == 0) a.inverse[row] = inv;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const float4 w = weight4<G, NV>(a, k, lane);
        const float4 v = z[k];
        st4f(a.y + row * a.W + (k * G + lane) * 4,
             make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w));
    }
}

// dx (and dgate) per row, and the weight gradient sum_r dy z inv: each lane
// accumulates its columns over the rows its group visits, the groups of a
// workgroup are added in order in LDS, one partial row per workgroup.
template <int G, int NV>
__global__ void __launch_bounds__(256) norm_backward_fast_kernel(NormFast a) {
    constexpr int RPB = 256 / G;
    __shared__ float red[RPB * G * 4 * NV];
    const int lane = threadIdx.x % G, slot = threadIdx.x / G;
    float4 w[NV], acc[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        w[k] = weight4<G, NV>(a, k, lane);
        acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int64_t base = (int64_t)blockIdx.x * RPB; base < a.rows; base += (int64_t)gridDim.x * RPB) {
        const int64_t row = base + slot;
        const bool live = row < a.rows;
        const int64_t r = live ? row : a.rows - 1;
        const float *x = a.x + row_offset(a.xs, r, a.T, a.H);
        const float *dy = a.dy + row_offset(a.ds, r, a.T, a.H);
        const float *gt = a.mode == 2 ? a.gate + row_offset(a.gs, r, a.T, a.H) : nullptr;
        float4 z[NV], sg[NV], up[NV], u[NV];
        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c = (k * G + lane) * 4;
            z[k] = ld4f(x + c);
            sg[k] = make_float4(1.f, 1.f, 1.f, 1.f);
            if (a.mode == 2) {
                sg[k] = sig4(ld4f(gt + c));
                z[k] = mul4(z[k], sg[k]);
            }
            up[k] = ld4f(dy + c);
            u[k] = mul4(up[k], w[k]);
            dot += dot4(u[k], z[k]);
        }
        dot = group_sum<G>(dot);
        if (!live) continue;
        const float inv = a.inv_in[row];
        const float corr = dot * inv * inv / a.div;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t o = row * a.W + (k * G + lane) * 4;
            const float4 dz = make_float4((u[k].x - z[k].x * corr) * inv, (u[k].y - z[k].y * corr) * inv,
                                          (u[k].z - z[k].z * corr) * inv, (u[k].w - z[k].w * corr) * inv);
            if (a.dx) st4f(a.dx + o, mul4(dz, sg[k]));
            if (a.dgate)
                st4f(a.dgate + o, make_float4(dz.x * z[k].x * (1.f - sg[k].x),
                                              dz.y * z[k].y * (1.f - sg[k].y),
                                              dz.z * z[k].z * (1.f - sg[k].z),
                                              dz.w * z[k].w * (1.f - sg[k].w)));
            acc[k].x += up[k].x * z[k].x * inv;
            acc[k].y += up[k].y * z[k].y * inv;
            acc[k].z += up[k].z * z[k].z * inv;
            acc[k].w += up[k].w * z[k].w * inv;
        }
    }
    if (!a.dw_part) return;
    const int W = 4 * G * NV;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float *d = red + slot * W + (k * G + lane) * 4;
        d[0] = acc[k].x;
        d[1] = acc[k].y;
        d[2] = acc[k].z;
        d[3] = acc[k].w;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < W; c += 256) {
        float s = red[c];
        for (int j = 1; j < RPB; ++j) s += red[j * W + c];
        a.dw_part[(int64_t)blockIdx.x * W + c] = s;
    }
}

constexpr int kNormBlocks = 1024;  // workgroups of the fast backward (fixed: deterministic sums)

// ---- decay --------------------------------------------------------------------
struct DecayArgs {
    int64_t B, T, H, W;
    gdn2_view x, bias, scale, dy;
    float *y, *dx, *part_b, *part_s;
};

// softplus with the reference's threshold at 20 (decay.rs:13-19).
__device__ __forceinline__ float softplus20(float z) { return z > 20.f ? z : log1pf(expf(z)); }

__global__ void decay_forward_kernel(DecayArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.B * a.T * a.H * a.W) return;
    const int64_t c = i % a.W, h = i / a.W % a.H, r = i / (a.W * a.H);
    const int64_t t = r % a.T, b = r / a.T;
    const float z = ldv(a.x, b, t, h, c) + ldv(a.bias, h * a.W + c, 0);
    a.y[i] = expf(-softplus20(z) * expf(ldv(a.scale, h, 0)));
}

// dx for every element, plus per-segment partial sums of dbias (per (h, c))
// and of the dscale terms: block (column block over H*W, segment), lane = column.
__global__ void __launch_bounds__(64) decay_backward_kernel(DecayArgs a, int64_t seg_rows) {
    const int64_t hc = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int seg = blockIdx.y;
    const int64_t HW = a.H * a.W;
    if (hc >= HW) return;
    const int64_t h = hc / a.W, c = hc % a.W;
    const float bias = ldv(a.bias, hc, 0), es = expf(ldv(a.scale, h, 0));
    const int64_t r0 = seg * seg_rows, r1 = min(r0 + seg_rows, a.B * a.T);
    float pb = 0.f, ps = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t t = r % a.T, b = r / a.T;
        const float z = ldv(a.x, b, t, h, c) + bias;
        const float sp = softplus20(z);
        const float alpha = expf(-sp * es);
        const float deriv = z > 20.f ? 1.f : 1.f / (1.f + expf(-z));
        const float g = -ldv(a.dy, b, t, h, c) * alpha * es;
        const float dx = g * deriv;
        if (a.dx) a.dx[r * HW + hc] = dx;
        pb += dx;
        ps += g * sp;
    }
    a.part_b[(int64_t)seg * HW + hc] = pb;
    a.part_s[(int64_t)seg * HW + hc] = ps;
}

// ---- validation -----------------------------------------------------------------
int check_f32(const gdn2_view *v, const char *name) { return check_view(v, name, GDN2_F32, false); }

int blocks_for(int64_t n, int per) { return (int)((n + per - 1) / per); }

}  // namespace
}  // namespace gdn2

using namespace gdn2;

namespace {

int check_conv(const gdn2_conv_shape *s, const gdn2_view *x, const gdn2_view *w,
               const gdn2_view *valid, const gdn2_view *docs, int activation) {
    if (!s) return fail(GDN2_ERR_ARGUMENT, "shape is null");
    if (s->batch <= 0 || s->time <= 0 || s->channels <= 0)
        return fail(GDN2_ERR_SHAPE, "convolution requires nonempty axes");
    if (s->taps < 1 || s->taps > kMaxTaps)
        return fail(GDN2_ERR_SHAPE, "convolution taps must be 1..%d (got %lld)", kMaxTaps,
                    (long long)s->taps);
    if (activation != 0 && activation != 1) return fail(GDN2_ERR_ARGUMENT, "activation must be 0 or 1");
    if (s->batch * s->time * s->channels > ((int64_t)1 << 38) || s->channels > 64 * 65535)
        return fail(GDN2_ERR_SHAPE, "convolution too large");
    GDN2_TRY(check_f32(x, "x"));
    GDN2_TRY(check_f32(w, "w"));
    GDN2_TRY(check_f32(valid, "valid"));
    GDN2_TRY(check_f32(docs, "docs"));
    return GDN2_OK;
}

ConvArgs conv_args(const gdn2_conv_shape *s, const gdn2_view *x, const gdn2_view *w,
                   const gdn2_view *valid, const gdn2_view *docs, int activation) {
    ConvArgs a{};
    a.B = s->batch;
    a.T = s->time;
    a.C = s->channels;
    a.W = (int)s->taps;
    a.act = activation;
    a.x = *x;
    a.w = *w;
    a.valid = *valid;
    a.docs = *docs;
    return a;
}

int check_rows(const gdn2_rows_shape *s, int64_t max_width) {
    if (!s) return fail(GDN2_ERR_ARGUMENT, "shape is null");
    if (s->batch <= 0 || s->time <= 0 || s->heads <= 0 || s->width <= 0)
        return fail(GDN2_ERR_SHAPE, "rows require nonempty axes");
    if (s->width > max_width)
        return fail(GDN2_ERR_SHAPE, "row width must be <= %lld (got %lld)", (long long)max_width,
                    (long long)s->width);
    if (s->batch * s->time * s->heads * s->width > ((int64_t)1 << 38))
        return fail(GDN2_ERR_SHAPE, "tensor too large");
    return GDN2_OK;
}

int check_norm(const gdn2_rows_shape *s, int mode, const gdn2_view *x, const gdn2_view *weight,
               const gdn2_view *gate) {
    GDN2_TRY(check_rows(s, kMaxNormWidth));
    if (mode < 0 || mode > 2) return fail(GDN2_ERR_ARGUMENT, "mode must be 0, 1 or 2");
    GDN2_TRY(check_f32(x, "x"));
    if (mode >= 1) GDN2_TRY(check_f32(weight, "weight"));
    if (mode == 2) GDN2_TRY(check_f32(gate, "gate"));
    return GDN2_OK;
}

NormArgs norm_args(const gdn2_rows_shape *s, int mode, const gdn2_view *x, const gdn2_view *weight,
                   const gdn2_view *gate) {
    NormArgs a{};
    a.B = s->batch;
    a.T = s->time;
    a.H = s->heads;
    a.W = s->width;
    a.mode = mode;
    a.x = *x;
    if (mode >= 1) a.weight = *weight;
    if (mode == 2) a.gate = *gate;
    return a;
}

int check_decay(const gdn2_rows_shape *s, const gdn2_view *x, const gdn2_view *bias,
                const gdn2_view *scale) {
    GDN2_TRY(check_rows(s, (int64_t)1 << 20));
    GDN2_TRY(check_f32(x, "x"));
    GDN2_TRY(check_f32(bias, "bias"));
    GDN2_TRY(check_f32(scale, "scale"));
    return GDN2_OK;
}

DecayArgs decay_args(const gdn2_rows_shape *s, const gdn2_view *x, const gdn2_view *bias,
                     const gdn2_view *scale) {
    DecayArgs a{};
    a.B = s->batch;
    a.T = s->time;
    a.H = s->heads;
    a.W = s->width;
    a.x = *x;
    a.bias = *bias;
    a.scale = *scale;
    return a;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Rows of 4-float groups starting on 16-byte boundaries.
bool rows_fast(const gdn2_view *v) {
    return v && v->stride[3] == 1 && aligned16(v->data) && v->stride[0] % 4 == 0 &&
           v->stride[1] % 4 == 0 && v->stride[2] % 4 == 0;
}

// Widths of the contiguous-row kernels: 4 G NV with G = 64 (multiples of 256
// up to 1024) or G = 16 (multiples of 64 up to 192).
bool norm_fast_shape(int64_t W, int *G, int *NV) {
    if (W % 256 == 0 && W <= 1024) {
        *G = 64;
        *NV = (int)(W / 256);
        return true;
    }
    if (W % 64 == 0 && W < 256) {
        *G = 16;
        *NV = (int)(W / 64);
        return true;
    }
    return false;
}

int64_t norm_fast_blocks(int64_t rows, int G) {
    const int64_t rpb = 256 / G;
    return std::max<int64_t>(1, std::min<int64_t>((rows + rpb - 1) / rpb, kNormBlocks));
}

NormFast norm_fast(const gdn2_rows_shape *s, int mode, const gdn2_view *x, const gdn2_view *weight,
                   const gdn2_view *gate) {
    NormFast f{};
    f.rows = s->batch * s->time * s->heads;
    f.T = s->time;
    f.H = s->heads;
    f.W = s->width;
    f.mode = mode;
    f.div = mode == 0 ? 1.f : (float)s->width;
    f.x = static_cast<const float *>(x->data);
    for (int i = 0; i < 3; ++i) f.xs[i] = x->stride[i];
    if (mode >= 1) f.weight = *weight;
    if (mode == 2) {
        f.gate = static_cast<const float *>(gate->data);
        for (int i = 0; i < 3; ++i) f.gs[i] = gate->stride[i];
    }
    return f;
}

template <template <int, int> class K>
void launch_norm(int G, int NV, dim3 grid, hipStream_t st, const NormFast &f) {
    if (G == 16) {
        if (NV == 1) hipLaunchKernelGGL((K<16, 1>::fn), grid, dim3(256), 0, st, f);
        else if (NV == 2) hipLaunchKernelGGL((K<16, 2>::fn), grid, dim3(256), 0, st, f);
        else hipLaunchKernelGGL((K<16, 3>::fn), grid, dim3(256), 0, st, f);
    } else {
        if (NV == 1) hipLaunchKernelGGL((K<64, 1>::fn), grid, dim3(256), 0, st, f);
        else if (NV == 2) hipLaunchKernelGGL((K<64, 2>::fn), grid, dim3(256), 0, st, f);
        else if (NV == 3) hipLaunchKernelGGL((K<64, 3>::fn), grid, dim3(256), 0, st, f);
        else hipLaunchKernelGGL((K<64, 4>::fn), grid, dim3(256), 0, st, f);
    }
}
template <int G, int NV> struct NormFwd { static constexpr auto fn = norm_forward_fast_kernel<G, NV>; };
template <int G, int NV> struct NormBwd { static constexpr auto fn = norm_backward_fast_kernel<G, NV>; };

template <template <int> class K>
void launch_taps(int W, dim3 grid, hipStream_t st, const ConvArgs &a) {
    switch (W) {
        case 1: hipLaunchKernelGGL(K<1>::fn, grid, dim3(64), 0, st, a); break;
        case 2: hipLaunchKernelGGL(K<2>::fn, grid, dim3(64), 0, st, a); break;
        case 3: hipLaunchKernelGGL(K<3>::fn, grid, dim3(64), 0, st, a); break;
        case 4: hipLaunchKernelGGL(K<4>::fn, grid, dim3(64), 0, st, a); break;
        case 5: hipLaunchKernelGGL(K<5>::fn, grid, dim3(64), 0, st, a); break;
        case 6: hipLaunchKernelGGL(K<6>::fn, grid, dim3(64), 0, st, a); break;
        case 7: hipLaunchKernelGGL(K<7>::fn, grid, dim3(64), 0, st, a); break;
        default: hipLaunchKernelGGL(K<8>::fn, grid, dim3(64), 0, st, a); break;
    }
}
template <int W> struct ConvFwd { static constexpr auto fn = conv_forward_kernel<W>; };
template <int W> struct ConvBwd { static constexpr auto fn = conv_backward_kernel<W>; };

dim3 conv_grid(const ConvArgs &a) {
    return dim3((unsigned)(a.B * conv_segments(a.T)), (unsigned)blocks_for(a.C, 64));
}

}  // namespace

extern "C" {

int gdn2_conv_forward(const gdn2_conv_shape *shape, const gdn2_view *x, const gdn2_view *w,
                      const gdn2_view *valid, const gdn2_view *docs, int activation, float *y,
                      void *stream) {
    GDN2_TRY(check_conv(shape, x, w, valid, docs, activation));
    if (!y) return fail(GDN2_ERR_ARGUMENT, "y is null");
    ConvArgs a = conv_args(shape, x, w, valid, docs, activation);
    a.y = y;
    launch_taps<ConvFwd>(a.W, conv_grid(a), (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_conv_forward");
}

size_t gdn2_conv_workspace_bytes(const gdn2_conv_shape *shape) {
    if (!shape || shape->taps < 1 || shape->channels < 1 || shape->batch < 1 || shape->time < 1)
        return 0;
    return (size_t)shape->batch * conv_segments(shape->time) * shape->taps * shape->channels *
           sizeof(float);
}

int gdn2_conv_backward(const gdn2_conv_shape *shape, const gdn2_view *x, const gdn2_view *w,
                       const gdn2_view *valid, const gdn2_view *docs, int activation,
                       const gdn2_view *dy, float *dx, float *dw, void *workspace,
                       size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_conv(shape, x, w, valid, docs, activation));
    GDN2_TRY(check_f32(dy, "dy"));
    ConvArgs a = conv_args(shape, x, w, valid, docs, activation);
    a.dy = *dy;
    a.dx = dx;
    hipStream_t st = (hipStream_t)stream;
    if (dw) {
        if (!workspace || workspace_bytes < gdn2_conv_workspace_bytes(shape))
            return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                        gdn2_conv_workspace_bytes(shape), workspace_bytes);
        a.dw_part = static_cast<float *>(workspace);
    }
    if (!dx && !dw) return ok();
    launch_taps<ConvBwd>(a.W, conv_grid(a), st, a);
    if (dw) column_sum(a.dw_part, (int64_t)a.W * a.C, a.B * conv_segments(a.T), dw, st);
    return launch_status(hipGetLastError(), "gdn2_conv_backward");
}

int gdn2_norm_forward(const gdn2_rows_shape *shape, int mode, float epsilon, const gdn2_view *x,
                      const gdn2_view *weight, const gdn2_view *gate, float *y, float *inverse,
                      void *stream) {
    GDN2_TRY(check_norm(shape, mode, x, weight, gate));
    if (!(epsilon > 0.f) || !isfinite(epsilon))
        return fail(GDN2_ERR_ARGUMENT, "epsilon must be finite and positive");
    if (!y || !inverse) return fail(GDN2_ERR_ARGUMENT, "y and inverse must be non-null");
    hipStream_t st = (hipStream_t)stream;
    int G, NV;
    if (norm_fast_shape(shape->width, &G, &NV) && rows_fast(x) && (mode != 2 || rows_fast(gate)) &&
        aligned16(y)) {
        NormFast f = norm_fast(shape, mode, x, weight, gate);
        f.eps = epsilon;
        f.y = y;
        f.inverse = inverse;
        const dim3 grid((unsigned)blocks_for(f.rows, 256 / G));
        launch_norm<NormFwd>(G, NV, grid, st, f);
        return launch_status(hipGetLastError(), "gdn2_norm_forward");
    }
    NormArgs a = norm_args(shape, mode, x, weight, gate);
    a.eps = epsilon;
    a.y = y;
    a.inverse = inverse;
    hipLaunchKernelGGL(norm_forward_kernel, dim3(blocks_for(a.B * a.T * a.H, 4)), dim3(256), 0, st,
                       a);
    return launch_status(hipGetLastError(), "gdn2_norm_forward");
}

size_t gdn2_norm_workspace_bytes(const gdn2_rows_shape *shape) {
    if (!shape || shape->width < 1 || shape->batch < 1 || shape->time < 1 || shape->heads < 1)
        return 0;
    const int64_t rows = shape->batch * shape->time * shape->heads;
    const int64_t parts = std::max<int64_t>(segment_count(rows), norm_fast_blocks(rows, 64));
    return (size_t)parts * shape->width * sizeof(float);
}

int gdn2_norm_backward(const gdn2_rows_shape *shape, int mode, const gdn2_view *x,
                       const gdn2_view *weight, const gdn2_view *gate, const float *inverse,
                       const gdn2_view *dy, float *dx, float *dgate, float *dweight,
                       void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_norm(shape, mode, x, weight, gate));
    GDN2_TRY(check_f32(dy, "dy"));
    if (!inverse) return fail(GDN2_ERR_ARGUMENT, "inverse is null");
    const bool want_dw = mode >= 1 && dweight;
    if (want_dw && (!workspace || workspace_bytes < gdn2_norm_workspace_bytes(shape)))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn2_norm_workspace_bytes(shape), workspace_bytes);
    if (mode != 2) dgate = nullptr;
    hipStream_t st = (hipStream_t)stream;
    int G, NV;
    if (norm_fast_shape(shape->width, &G, &NV) && rows_fast(x) && rows_fast(dy) &&
        (mode != 2 || rows_fast(gate)) && aligned16(dx) && aligned16(dgate)) {
        if (!dx && !dgate && !want_dw) return ok();
        NormFast f = norm_fast(shape, mode, x, weight, gate);
        f.dy = static_cast<const float *>(dy->data);
        for (int i = 0; i < 3; ++i) f.ds[i] = dy->stride[i];
        f.inv_in = inverse;
        f.dx = dx;
        f.dgate = dgate;
        f.dw_part = want_dw ? static_cast<float *>(workspace) : nullptr;
        const int64_t nblk = norm_fast_blocks(f.rows, G);
        launch_norm<NormBwd>(G, NV, dim3((unsigned)nblk), st, f);
        if (want_dw) column_sum(f.dw_part, f.W, nblk, dweight, st);
        return launch_status(hipGetLastError(), "gdn2_norm_backward");
    }
    NormArgs a = norm_args(shape, mode, x, weight, gate);
    a.dy = *dy;
    a.inv_in = inverse;
    if (dx || dgate) {
        a.dx = dx;
        a.dgate = dgate;
        hipLaunchKernelGGL(norm_dx_kernel, dim3(blocks_for(a.B * a.T * a.H, 4)), dim3(256), 0, st,
                           a);
    }
    if (want_dw) {
        a.dw_part = static_cast<float *>(workspace);
        const int64_t rows = a.B * a.T * a.H;
        hipLaunchKernelGGL(norm_dw_partial_kernel, dim3(blocks_for(a.W, 64), segment_count(rows)),
                           dim3(64), 0, st, a, segment_rows(rows));
        column_sum(a.dw_part, a.W, segment_count(rows), dweight, st);
    }
    return launch_status(hipGetLastError(), "gdn2_norm_backward");
}

int gdn2_decay_forward(const gdn2_rows_shape *shape, const gdn2_view *x, const gdn2_view *bias,
                       const gdn2_view *scale, float *y, void *stream) {
    GDN2_TRY(check_decay(shape, x, bias, scale));
    if (!y) return fail(GDN2_ERR_ARGUMENT, "y is null");
    DecayArgs a = decay_args(shape, x, bias, scale);
    a.y = y;
    hipLaunchKernelGGL(decay_forward_kernel, dim3(blocks_for(a.B * a.T * a.H * a.W, 256)),
                       dim3(256), 0, (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_decay_forward");
}

size_t gdn2_decay_workspace_bytes(const gdn2_rows_shape *shape) {
    if (!shape || shape->heads < 1 || shape->width < 1 || shape->batch < 1 || shape->time < 1)
        return 0;
    const int64_t HW = shape->heads * shape->width;
    return (size_t)(2 * segment_count(shape->batch * shape->time) + 1) * HW * sizeof(float);
}

int gdn2_decay_backward(const gdn2_rows_shape *shape, const gdn2_view *x, const gdn2_view *bias,
                        const gdn2_view *scale, const gdn2_view *dy, float *dx, float *dbias,
                        float *dscale, void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_decay(shape, x, bias, scale));
    GDN2_TRY(check_f32(dy, "dy"));
    if (!workspace || workspace_bytes < gdn2_decay_workspace_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn2_decay_workspace_bytes(shape), workspace_bytes);
    DecayArgs a = decay_args(shape, x, bias, scale);
    a.dy = *dy;
    a.dx = dx;
    const int64_t HW = a.H * a.W;
    const int64_t nseg = segment_count(a.B * a.T);
    a.part_b = static_cast<float *>(workspace);
    a.part_s = a.part_b + nseg * HW;
    float *sum_s = a.part_s + nseg * HW;  // per (h, k) sums of the dscale terms
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(decay_backward_kernel, dim3(blocks_for(HW, 64), nseg), dim3(64), 0, st, a,
                       segment_rows(a.B * a.T));
    if (dbias) column_sum(a.part_b, HW, nseg, dbias, st);
    if (dscale) {
        column_sum(a.part_s, HW, nseg, sum_s, st);
        hipLaunchKernelGGL(segment_group_sum_kernel, dim3(blocks_for(a.H, 64)), dim3(64), 0, st,
                           sum_s, a.H, a.W, 1, dscale);
    }
    return launch_status(hipGetLastError(), "gdn2_decay_backward");
}

}  // extern "C"
