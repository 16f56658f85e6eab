// Mixer prologue / epilogue operators on gfx950: depthwise causal convolution
// (with optional fused SiLU), L2 / RMS / sigmoid-gated RMS row normalization,
// and the decay gate, each with its VJP.
//
// Semantics follow the reference custom ops (crates/kernels/src/conv.rs,
// norm.rs, decay.rs) and their scalar-f64 checks
// (crates/mixers/src/convolution_checks.rs, normalization_checks.rs).
//
// These operators move a few bytes per flop, so each is laid out for HBM:
//   * elementwise kernels (convolution, decay) put consecutive channels on
//     consecutive lanes, one (batch, time) row per group of lanes;
//   * row normalizations give one 64-lane wave to each row and reduce with DPP;
//   * parameter gradients (conv weight, norm weight, decay bias/scale) are
//     reduced in two deterministic passes: per row-segment partial sums into
//     the caller's workspace, then a sum over segments.
#include <math.h>

#include "gdn2_status.h"

namespace gdn2 {
namespace {

constexpr int kSegments = 64;  // row segments of the parameter-gradient reductions
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

int64_t segment_rows(int64_t rows) { return (rows + kSegments - 1) / kSegments; }

// out[i] = sum_s part[s * n + i], s < segments.
__global__ void segment_sum_kernel(const float *part, int64_t n, int segments, float *out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    for (int k = 0; k < segments; ++k) s += part[(int64_t)k * n + i];
    out[i] = s;
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

// Mask of a lag from source token s to destination token d of batch row b.
__device__ __forceinline__ float conv_mask(const ConvArgs &a, int64_t b, int64_t s, int64_t d) {
    return ldv(a.docs, b, s) == ldv(a.docs, b, d) ? ldv(a.valid, b, s) * ldv(a.valid, b, d) : 0.f;
}

// Pre-activation convolution output at (b, t, c).
__device__ __forceinline__ float conv_at(const ConvArgs &a, int64_t b, int64_t t, int64_t c) {
    float s = 0.f;
    for (int l = 0; l < a.W && l <= t; ++l)
        s += ldv(a.x, b, t - l, c) * ldv(a.w, l, c) * conv_mask(a, b, t - l, t);
    return s;
}

// d(act(p))/dp times the upstream value.
__device__ __forceinline__ float act_grad(int act, float p, float up) {
    if (!act) return up;
    const float s = sigmoidf(p);
    return up * s * (1.f + p * (1.f - s));
}

// One thread per element; channels contiguous across lanes.
__global__ void conv_forward_kernel(ConvArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.B * a.T * a.C) return;
    const int64_t c = i % a.C, t = i / a.C % a.T, b = i / (a.C * a.T);
    const float p = conv_at(a, b, t, c);
    a.y[i] = a.act ? p * sigmoidf(p) : p;
}

__global__ void conv_dx_kernel(ConvArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.B * a.T * a.C) return;
    const int64_t c = i % a.C, t = i / a.C % a.T, b = i / (a.C * a.T);
    float s = 0.f;
    for (int l = 0; l < a.W && t + l < a.T; ++l) {
        const float m = conv_mask(a, b, t, t + l);
        if (m == 0.f) continue;
        const float up = ldv(a.dy, b, t + l, c);
        const float g = a.act ? act_grad(1, conv_at(a, b, t + l, c), up) : up;
        s += g * ldv(a.w, l, c) * m;
    }
    a.dx[i] = s;
}

// Partial weight gradients: block (channel block, segment), lane = channel.
__global__ void __launch_bounds__(64) conv_dw_partial_kernel(ConvArgs a, int64_t seg_rows) {
    const int64_t c = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int seg = blockIdx.y;
    if (c >= a.C) return;
    float acc[kMaxTaps];
#pragma unroll
    for (int l = 0; l < kMaxTaps; ++l) acc[l] = 0.f;
    const int64_t r0 = seg * seg_rows, r1 = min(r0 + seg_rows, a.B * a.T);
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t b = r / a.T, t = r % a.T;
        const float up = ldv(a.dy, b, t, c);
        const float g = a.act ? act_grad(1, conv_at(a, b, t, c), up) : up;
#pragma unroll
        for (int l = 0; l < kMaxTaps; ++l)
            if (l < a.W && l <= t) acc[l] += g * ldv(a.x, b, t - l, c) * conv_mask(a, b, t - l, t);
    }
    for (int l = 0; l < a.W; ++l) a.dw_part[((int64_t)seg * a.W + l) * a.C + c] = acc[l];
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
    if (s->batch * s->time * s->channels > ((int64_t)1 << 38))
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

}  // namespace

extern "C" {

int gdn2_conv_forward(const gdn2_conv_shape *shape, const gdn2_view *x, const gdn2_view *w,
                      const gdn2_view *valid, const gdn2_view *docs, int activation, float *y,
                      void *stream) {
    GDN2_TRY(check_conv(shape, x, w, valid, docs, activation));
    if (!y) return fail(GDN2_ERR_ARGUMENT, "y is null");
    ConvArgs a = conv_args(shape, x, w, valid, docs, activation);
    a.y = y;
    hipLaunchKernelGGL(conv_forward_kernel, dim3(blocks_for(a.B * a.T * a.C, 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_conv_forward");
}

size_t gdn2_conv_workspace_bytes(const gdn2_conv_shape *shape) {
    if (!shape || shape->taps < 1 || shape->channels < 1) return 0;
    return (size_t)kSegments * shape->taps * shape->channels * sizeof(float);
}

int gdn2_conv_backward(const gdn2_conv_shape *shape, const gdn2_view *x, const gdn2_view *w,
                       const gdn2_view *valid, const gdn2_view *docs, int activation,
                       const gdn2_view *dy, float *dx, float *dw, void *workspace,
                       size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_conv(shape, x, w, valid, docs, activation));
    GDN2_TRY(check_f32(dy, "dy"));
    ConvArgs a = conv_args(shape, x, w, valid, docs, activation);
    a.dy = *dy;
    hipStream_t st = (hipStream_t)stream;
    if (dw) {
        if (!workspace || workspace_bytes < gdn2_conv_workspace_bytes(shape))
            return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                        gdn2_conv_workspace_bytes(shape), workspace_bytes);
        a.dw_part = static_cast<float *>(workspace);
        const int64_t seg_rows = segment_rows(a.B * a.T);
        hipLaunchKernelGGL(conv_dw_partial_kernel, dim3(blocks_for(a.C, 64), kSegments), dim3(64),
                           0, st, a, seg_rows);
        hipLaunchKernelGGL(segment_sum_kernel, dim3(blocks_for(a.W * a.C, 256)), dim3(256), 0, st,
                           a.dw_part, (int64_t)a.W * a.C, kSegments, dw);
    }
    if (dx) {
        a.dx = dx;
        hipLaunchKernelGGL(conv_dx_kernel, dim3(blocks_for(a.B * a.T * a.C, 256)), dim3(256), 0,
                           st, a);
    }
    return launch_status(hipGetLastError(), "gdn2_conv_backward");
}

int gdn2_norm_forward(const gdn2_rows_shape *shape, int mode, float epsilon, const gdn2_view *x,
                      const gdn2_view *weight, const gdn2_view *gate, float *y, float *inverse,
                      void *stream) {
    GDN2_TRY(check_norm(shape, mode, x, weight, gate));
    if (!(epsilon > 0.f) || !isfinite(epsilon))
        return fail(GDN2_ERR_ARGUMENT, "epsilon must be finite and positive");
    if (!y || !inverse) return fail(GDN2_ERR_ARGUMENT, "y and inverse must be non-null");
    NormArgs a = norm_args(shape, mode, x, weight, gate);
    a.eps = epsilon;
    a.y = y;
    a.inverse = inverse;
    hipLaunchKernelGGL(norm_forward_kernel, dim3(blocks_for(a.B * a.T * a.H, 4)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_norm_forward");
}

size_t gdn2_norm_workspace_bytes(const gdn2_rows_shape *shape) {
    if (!shape || shape->width < 1) return 0;
    return (size_t)kSegments * shape->width * sizeof(float);
}

int gdn2_norm_backward(const gdn2_rows_shape *shape, int mode, const gdn2_view *x,
                       const gdn2_view *weight, const gdn2_view *gate, const float *inverse,
                       const gdn2_view *dy, float *dx, float *dgate, float *dweight,
                       void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_norm(shape, mode, x, weight, gate));
    GDN2_TRY(check_f32(dy, "dy"));
    if (!inverse) return fail(GDN2_ERR_ARGUMENT, "inverse is null");
    NormArgs a = norm_args(shape, mode, x, weight, gate);
    a.dy = *dy;
    a.inv_in = inverse;
    hipStream_t st = (hipStream_t)stream;
    if (dx || (mode == 2 && dgate)) {
        a.dx = dx;
        a.dgate = mode == 2 ? dgate : nullptr;
        hipLaunchKernelGGL(norm_dx_kernel, dim3(blocks_for(a.B * a.T * a.H, 4)), dim3(256), 0, st,
                           a);
    }
    if (mode >= 1 && dweight) {
        if (!workspace || workspace_bytes < gdn2_norm_workspace_bytes(shape))
            return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                        gdn2_norm_workspace_bytes(shape), workspace_bytes);
        a.dw_part = static_cast<float *>(workspace);
        const int64_t seg_rows = segment_rows(a.B * a.T * a.H);
        hipLaunchKernelGGL(norm_dw_partial_kernel, dim3(blocks_for(a.W, 64), kSegments), dim3(64),
                           0, st, a, seg_rows);
        hipLaunchKernelGGL(segment_sum_kernel, dim3(blocks_for(a.W, 256)), dim3(256), 0, st,
                           a.dw_part, a.W, kSegments, dweight);
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
    if (!shape || shape->heads < 1 || shape->width < 1) return 0;
    return (size_t)2 * kSegments * shape->heads * shape->width * sizeof(float);
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
    a.part_b = static_cast<float *>(workspace);
    a.part_s = a.part_b + (int64_t)kSegments * HW;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(decay_backward_kernel, dim3(blocks_for(HW, 64), kSegments), dim3(64), 0, st,
                       a, segment_rows(a.B * a.T));
    if (dbias)
        hipLaunchKernelGGL(segment_sum_kernel, dim3(blocks_for(HW, 256)), dim3(256), 0, st,
                           a.part_b, HW, kSegments, dbias);
    if (dscale)
        hipLaunchKernelGGL(segment_group_sum_kernel, dim3(blocks_for(a.H, 64)), dim3(64), 0, st,
                           a.part_s, a.H, a.W, kSegments, dscale);
    return launch_status(hipGetLastError(), "gdn2_decay_backward");
}

}  // extern "C"
