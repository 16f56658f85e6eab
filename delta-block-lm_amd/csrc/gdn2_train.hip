// Training-step operators on gfx950: row cross entropy (forward, backward, and
// a fused forward + gradient) and AdamW with per-parameter gradient clipping
// over a whole parameter set.
//
// Semantics follow the reference's kernels (crates/kernels/src/cross_entropy.rs,
// update.rs); the layout is for HBM:
//   * cross entropy gives one 256-thread workgroup to each row; the row is read
//     with 16-byte loads, reduced to (max, sum of exponentials) online per
//     thread, then across the workgroup with DPP and LDS in a fixed order.  The
//     fused variant re-reads the row (from L2 / MALL) and writes the gradient in
//     the logits' own dtype, optionally over the logits;
//   * AdamW cuts every parameter tensor into 16384-element chunks, one
//     workgroup each: a first launch writes each chunk's sum of squared
//     gradients, the second reduces its tensor's partials in a fixed order
//     (deterministic clipping norm) and updates parameter and moments with
//     16-byte accesses, each element read once and written once.
#include <float.h>
#include <math.h>

#include "gdn2_common.h"
#include "gdn2_status.h"

namespace gdn2 {
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// ---- cross entropy -------------------------------------------------------------

constexpr int kCeThreads = 256;

struct CeArgs {
    const void *x;
    int64_t rs, cs;  // element strides between rows and between columns
    int64_t rows, width;
    const int64_t *target;
    int64_t ts;
    const float *stats_in;
    const float *upstream;
    int64_t us;
    float scale;
    float *loss;
    float *stats;
    void *dx;  // contiguous [rows, width] in x's dtype
    int vec;   // 16-byte loads: unit column stride, aligned rows, width % lanes == 0
};

// (m, s) running log-sum-exp state: s = sum exp(x - m).
struct Lse {
    float m, s;
};

__device__ __forceinline__ Lse lse_merge(Lse a, Lse b) {
    const float M = fmaxf(a.m, b.m);
    return {M, a.s * __expf(a.m - M) + b.s * __expf(b.m - M)};
}

template <int CTRL>
__device__ __forceinline__ Lse lse_dpp(Lse a) {
    return lse_merge(a, {dpp_f<CTRL>(a.m), dpp_f<CTRL>(a.s)});
}

// Row-wide (m, s) in every thread; fixed combination order (deterministic).
__device__ Lse lse_block(Lse a, Lse *red) {
    a = lse_dpp<0xB1>(a);   // quad: swap adjacent lanes
    a = lse_dpp<0x4E>(a);   // quad: swap pairs
    a = lse_dpp<0x141>(a);  // half-row mirror
    a = lse_dpp<0x140>(a);  // row mirror
    Lse w = {readlane_f(a.m, 0), readlane_f(a.s, 0)};
    w = lse_merge(w, {readlane_f(a.m, 16), readlane_f(a.s, 16)});
    w = lse_merge(w, {readlane_f(a.m, 32), readlane_f(a.s, 32)});
    w = lse_merge(w, {readlane_f(a.m, 48), readlane_f(a.s, 48)});
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = w;
    __syncthreads();
    Lse r = red[0];
    for (int i = 1; i < kCeThreads / 64; ++i) r = lse_merge(r, red[i]);
    return r;
}

template <typename T> struct Vec;
template <> struct Vec<float> {
    static constexpr int N = 4;
    static __device__ __forceinline__ void load(const void *p, int64_t i, float *v) {
        const float4 q = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(p) + i);
        v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
    }
    static __device__ __forceinline__ void store(void *p, int64_t i, const float *v) {
        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(p) + i) =
            make_float4(v[0], v[1], v[2], v[3]);
    }
};
template <> struct Vec<bf16_t> {
    static constexpr int N = 8;
    static __device__ __forceinline__ void load(const void *p, int64_t i, float *v) {
        const uint4 q = *reinterpret_cast<const uint4 *>(reinterpret_cast<const bf16_t *>(p) + i);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    }
    static __device__ __forceinline__ void store(void *p, int64_t i, const float *v) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = (uint32_t)f32_to_bf16(v[2 * j]) | ((uint32_t)f32_to_bf16(v[2 * j + 1]) << 16);
        *reinterpret_cast<uint4 *>(reinterpret_cast<bf16_t *>(p) + i) =
            make_uint4(w[0], w[1], w[2], w[3]);
    }
};

// Per-thread (m, s) over this thread's share of row r.
template <typename T>
__device__ Lse row_lse(const CeArgs &a, int64_t r) {
    Lse acc = {-FLT_MAX, 0.f};
    if (a.vec) {
        constexpr int N = Vec<T>::N;
        const int64_t base = r * a.rs;
        for (int64_t c = (int64_t)threadIdx.x * N; c < a.width; c += kCeThreads * N) {
            float v[N];
            Vec<T>::load(a.x, base + c, v);
            float cm = v[0];
#pragma unroll
            for (int j = 1; j < N; ++j) cm = fmaxf(cm, v[j]);
            const float M = fmaxf(acc.m, cm);
            float s = acc.s * __expf(acc.m - M);
#pragma unroll
            for (int j = 0; j < N; ++j) s += __expf(v[j] - M);
            acc = {M, s};
        }
    } else {
        for (int64_t c = threadIdx.x; c < a.width; c += kCeThreads) {
            const float v = Elem<T>::load(a.x, r * a.rs + c * a.cs);
            acc = lse_merge(acc, {v, 1.f});
        }
    }
    return acc;
}

// x[r, target[r]] (thread 0 only), or NaN for a label outside [0, width).  Read
// before the row's reduction barrier: the fused kernel overwrites x after it.
template <typename T>
__device__ float target_logit(const CeArgs &a, int64_t r) {
    if (threadIdx.x != 0) return 0.f;
    const int64_t label = a.target[r * a.ts];
    return label >= 0 && label < a.width ? Elem<T>::load(a.x, r * a.rs + label * a.cs)
                                         : __builtin_nanf("");
}

__device__ void write_row_loss(int64_t r, Lse t, float xl, float *loss, float *stats) {
    if (threadIdx.x != 0) return;
    const float logsum = logf(t.s);
    loss[r] = (t.m - xl) + logsum;
    if (stats) {
        stats[2 * r] = t.m;
        stats[2 * r + 1] = logsum;
    }
}

// dx[r, :] = (exp((x - m) - s) - onehot) * k, in T, contiguous.
template <typename T>
__device__ void write_row_grad(const CeArgs &a, int64_t r, float m, float logsum, float k) {
    const int64_t label = a.target[r * a.ts];
    const int64_t out = r * a.width;
    if (a.vec) {
        constexpr int N = Vec<T>::N;
        for (int64_t c = (int64_t)threadIdx.x * N; c < a.width; c += kCeThreads * N) {
            float v[N];
            Vec<T>::load(a.x, r * a.rs + c, v);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                float p = __expf((v[j] - m) - logsum);
                if (c + j == label) p -= 1.f;
                v[j] = p * k;
            }
            Vec<T>::store(a.dx, out + c, v);
        }
    } else {
        for (int64_t c = threadIdx.x; c < a.width; c += kCeThreads) {
            float p = __expf((Elem<T>::load(a.x, r * a.rs + c * a.cs) - m) - logsum);
            if (c == label) p -= 1.f;
            Elem<T>::store(a.dx, out + c, p * k);
        }
    }
}

template <typename T>
__global__ void __launch_bounds__(kCeThreads) ce_forward_kernel(CeArgs a) {
    __shared__ Lse red[kCeThreads / 64];
    const int64_t r = blockIdx.x;
    const float xl = target_logit<T>(a, r);
    const Lse t = lse_block(row_lse<T>(a, r), red);
    write_row_loss(r, t, xl, a.loss, a.stats);
}

template <typename T>
__global__ void __launch_bounds__(kCeThreads) ce_backward_kernel(CeArgs a) {
    const int64_t r = blockIdx.x;
    write_row_grad<T>(a, r, a.stats_in[2 * r], a.stats_in[2 * r + 1], a.upstream[r * a.us]);
}

template <typename T>
__global__ void __launch_bounds__(kCeThreads) ce_fused_kernel(CeArgs a) {
    __shared__ Lse red[kCeThreads / 64];
    const int64_t r = blockIdx.x;
    const float xl = target_logit<T>(a, r);
    const Lse t = lse_block(row_lse<T>(a, r), red);
    write_row_loss(r, t, xl, a.loss, nullptr);
    // Every thread has read its elements of row r, and thread 0 the target
    // logit, before lse_block's barrier; past it each element is rewritten
    // only by the thread that read it.
    write_row_grad<T>(a, r, t.m, logf(t.s), a.scale);
}

int check_ce(int64_t rows, int64_t width, const gdn2_view *x, const int64_t *target,
             CeArgs *a) {
    if (rows < 0 || width < 1) return fail(GDN2_ERR_SHAPE, "rows must be >= 0 and width >= 1");
    if (rows > 0x7FFFFFFF) return fail(GDN2_ERR_SHAPE, "at most 2^31 - 1 rows");
    GDN2_TRY(check_view(x, "x", -1, false));
    if (!target) return fail(GDN2_ERR_ARGUMENT, "target is null");
    *a = CeArgs{};
    a->x = x->data;
    a->rs = x->stride[0];
    a->cs = x->stride[1];
    a->rows = rows;
    a->width = width;
    a->target = target;
    const int n = x->dtype == GDN2_BF16 ? 8 : 4;
    const int es = x->dtype == GDN2_BF16 ? 2 : 4;
    a->vec = a->cs == 1 && width % n == 0 && ((uintptr_t)x->data & 15) == 0 &&
             (a->rs * es) % 16 == 0;
    return ok();
}

template <typename K>
int launch_ce(K kern_f32, K kern_bf16, int dtype, const CeArgs &a, void *stream, const char *what) {
    if (a.rows == 0) return ok();
    hipLaunchKernelGGL(dtype == GDN2_BF16 ? kern_bf16 : kern_f32, dim3((unsigned)a.rows),
                       dim3(kCeThreads), 0, (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), what);
}

// ---- AdamW ---------------------------------------------------------------------

constexpr int kAdamThreads = 256;
constexpr int64_t kAdamChunk = 16384;  // elements per workgroup
constexpr int kTableBatch = 16;        // descriptors written per table launch

struct AdamEntry {
    float *p;
    const float *g;
    float *m;
    float *v;
    int64_t numel;
    int32_t chunk0;  // first chunk of this tensor
    int32_t vec;     // all four pointers 16-byte aligned
};
static_assert(sizeof(AdamEntry) == 48, "descriptor layout");

struct TableBatch {
    AdamEntry e[kTableBatch];
    int first, n;
};

struct AdamArgs {
    const AdamEntry *table;
    int count;
    float *partial;
    int initialized;
    float c1, c2, b1c, b2c, decay, lr, clip;
};

__global__ void adam_table_kernel(AdamEntry *table, TableBatch b) {
    if ((int)threadIdx.x < b.n) table[b.first + threadIdx.x] = b.e[threadIdx.x];
}

// Tensor owning chunk c: the last entry whose chunk0 <= c.
__device__ __forceinline__ int find_tensor(const AdamEntry *table, int count, int c) {
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (table[mid].chunk0 <= c) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Sum over the workgroup in every thread (fixed order).
__device__ float block_sum(float x, float *red) {
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    x += dpp_f<0x141>(x);
    x += dpp_f<0x140>(x);
    const float w = ((readlane_f(x, 0) + readlane_f(x, 16)) + readlane_f(x, 32)) + readlane_f(x, 48);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kAdamThreads / 64; ++i) r += red[i];
    return r;
}

__global__ void __launch_bounds__(kAdamThreads) adam_square_kernel(AdamArgs a) {
    __shared__ float red[kAdamThreads / 64];
    const int c = blockIdx.x;
    const AdamEntry e = a.table[find_tensor(a.table, a.count, c)];
    const int64_t begin = (int64_t)(c - e.chunk0) * kAdamChunk;
    const int64_t end = min(begin + kAdamChunk, e.numel);
    float acc = 0.f;
    if (e.vec) {
        const int64_t body = begin + ((end - begin) & ~(int64_t)3);
        for (int64_t i = begin + 4 * (int64_t)threadIdx.x; i < body; i += 4 * kAdamThreads) {
            const float4 g = *reinterpret_cast<const float4 *>(e.g + i);
            acc += g.x * g.x;
            acc += g.y * g.y;
            acc += g.z * g.z;
            acc += g.w * g.w;
        }
        if (body + (int64_t)threadIdx.x < end) acc += e.g[body + threadIdx.x] * e.g[body + threadIdx.x];
    } else {
        for (int64_t i = begin + threadIdx.x; i < end; i += kAdamThreads) acc += e.g[i] * e.g[i];
    }
    const float s = block_sum(acc, red);
    if (threadIdx.x == 0) a.partial[c] = s;
}

// The reference's element update, every operation rounded separately: the
// pragma keeps each product and sum its own instruction (no fused multiply-add),
// and HIP's f32 division and square root are correctly rounded.
__device__ __forceinline__ void adam_one(const AdamArgs &a, float coef, float &p, float g, float &m,
                                         float &v) {
#pragma clang fp contract(off)
    g = g * coef;
    float nm = g * a.b1c;
    float nv = (g * g) * a.b2c;
    if (a.initialized) {
        nm = m * 0.9f + nm;
        nv = v * 0.999f + nv;
    }
    m = nm;
    v = nv;
    const float delta = (nm / a.c1) / (sqrtf(nv / a.c2) + 1e-5f);
    p = p * a.decay - delta * a.lr;
}

__global__ void __launch_bounds__(kAdamThreads) adam_update_kernel(AdamArgs a) {
    __shared__ float red[kAdamThreads / 64];
    const int c = blockIdx.x;
    const int t = find_tensor(a.table, a.count, c);
    const AdamEntry e = a.table[t];
    const int nch = (int)((e.numel + kAdamChunk - 1) / kAdamChunk);
    float acc = 0.f;
    for (int j = threadIdx.x; j < nch; j += kAdamThreads) acc += a.partial[e.chunk0 + j];
    const float sq = block_sum(acc, red);
    const float coef = fminf(a.clip / (sqrtf(sq) + FLT_MIN), 1.f);
    const int64_t begin = (int64_t)(c - e.chunk0) * kAdamChunk;
    const int64_t end = min(begin + kAdamChunk, e.numel);
    if (e.vec) {
        const int64_t body = begin + ((end - begin) & ~(int64_t)3);
        for (int64_t i = begin + 4 * (int64_t)threadIdx.x; i < body; i += 4 * kAdamThreads) {
            float4 p = *reinterpret_cast<const float4 *>(e.p + i);
            const float4 g = *reinterpret_cast<const float4 *>(e.g + i);
            float4 m = *reinterpret_cast<const float4 *>(e.m + i);
            float4 v = *reinterpret_cast<const float4 *>(e.v + i);
            adam_one(a, coef, p.x, g.x, m.x, v.x);
            adam_one(a, coef, p.y, g.y, m.y, v.y);
            adam_one(a, coef, p.z, g.z, m.z, v.z);
            adam_one(a, coef, p.w, g.w, m.w, v.w);
            *reinterpret_cast<float4 *>(e.p + i) = p;
            *reinterpret_cast<float4 *>(e.m + i) = m;
            *reinterpret_cast<float4 *>(e.v + i) = v;
        }
        const int64_t i = body + threadIdx.x;
        if (i < end) adam_one(a, coef, e.p[i], e.g[i], e.m[i], e.v[i]);
    } else {
        for (int64_t i = begin + threadIdx.x; i < end; i += kAdamThreads)
            adam_one(a, coef, e.p[i], e.g[i], e.m[i], e.v[i]);
    }
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// 0.9^time and 0.999^time by binary powering in f32 (compiler-rt's __powisf2,
// which Rust's f32::powi lowers to).
float powi_f32(float a, int64_t b) {
    float r = 1.f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return r;
}

}  // namespace
}  // namespace gdn2

using namespace gdn2;

extern "C" {

int gdn2_cross_entropy_forward(int64_t rows, int64_t width, const gdn2_view *x,
                               const int64_t *target, int64_t target_stride, float *loss,
                               float *stats, void *stream) {
    CeArgs a;
    GDN2_TRY(check_ce(rows, width, x, target, &a));
    if (!loss || !stats) return fail(GDN2_ERR_ARGUMENT, "loss and stats must be non-null");
    a.ts = target_stride;
    a.loss = loss;
    a.stats = stats;
    return launch_ce(ce_forward_kernel<float>, ce_forward_kernel<bf16_t>, x->dtype, a, stream,
                     "gdn2_cross_entropy_forward");
}

int gdn2_cross_entropy_backward(int64_t rows, int64_t width, const gdn2_view *x,
                                const int64_t *target, int64_t target_stride, const float *stats,
                                const float *upstream, int64_t upstream_stride, void *dx,
                                void *stream) {
    CeArgs a;
    GDN2_TRY(check_ce(rows, width, x, target, &a));
    if (!stats || !upstream || !dx)
        return fail(GDN2_ERR_ARGUMENT, "stats, upstream and dx must be non-null");
    a.ts = target_stride;
    a.stats_in = stats;
    a.upstream = upstream;
    a.us = upstream_stride;
    a.dx = dx;
    return launch_ce(ce_backward_kernel<float>, ce_backward_kernel<bf16_t>, x->dtype, a, stream,
                     "gdn2_cross_entropy_backward");
}

int gdn2_cross_entropy_fused(int64_t rows, int64_t width, const gdn2_view *x,
                             const int64_t *target, int64_t target_stride, float scale,
                             float *loss, void *dx, void *stream) {
    CeArgs a;
    GDN2_TRY(check_ce(rows, width, x, target, &a));
    if (!loss || !dx) return fail(GDN2_ERR_ARGUMENT, "loss and dx must be non-null");
    if (dx == x->data && !(a.cs == 1 && a.rs == width))
        return fail(GDN2_ERR_ARGUMENT, "dx may alias x only when x is contiguous");
    a.ts = target_stride;
    a.scale = scale;
    a.loss = loss;
    a.dx = dx;
    return launch_ce(ce_fused_kernel<float>, ce_fused_kernel<bf16_t>, x->dtype, a, stream,
                     "gdn2_cross_entropy_fused");
}

size_t gdn2_adamw_workspace_bytes(int32_t count, const gdn2_adamw_tensor *tensors) {
    if (count < 0 || (count > 0 && !tensors)) return 0;
    size_t chunks = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (tensors[i].numel < 0) return 0;
        chunks += (size_t)((tensors[i].numel + kAdamChunk - 1) / kAdamChunk);
    }
    return align256((size_t)count * sizeof(AdamEntry)) + chunks * sizeof(float) + 4;
}

int gdn2_adamw_update(int32_t count, const gdn2_adamw_tensor *tensors, int initialized,
                      int64_t time, double lr, float weight_decay, float clip, int reuse_table,
                      void *workspace, size_t workspace_bytes, void *stream) {
    if (count < 0 || (count > 0 && !tensors))
        return fail(GDN2_ERR_ARGUMENT, "count must be >= 0 with a tensor array");
    if (time < 1) return fail(GDN2_ERR_ARGUMENT, "time must be >= 1");
    if (!isfinite(lr) || !isfinite(weight_decay) || !(clip > 0.f) || !isfinite(clip))
        return fail(GDN2_ERR_ARGUMENT, "lr and weight_decay must be finite, clip positive");
    int64_t chunks = 0;
    for (int32_t i = 0; i < count; ++i) {
        const gdn2_adamw_tensor &t = tensors[i];
        if (t.numel < 0) return fail(GDN2_ERR_SHAPE, "tensor %d: negative numel", i);
        if (t.numel > 0 && (!t.param || !t.grad || !t.first || !t.second))
            return fail(GDN2_ERR_ARGUMENT, "tensor %d: null pointer", i);
        chunks += (t.numel + kAdamChunk - 1) / kAdamChunk;
    }
    if (chunks > 0x7FFFFFFF) return fail(GDN2_ERR_SHAPE, "too many elements");
    const size_t need = gdn2_adamw_workspace_bytes(count, tensors);
    if (!workspace || workspace_bytes < need)
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need,
                    workspace_bytes);
    if (((uintptr_t)workspace & 15) != 0)
        return fail(GDN2_ERR_ARGUMENT, "workspace must be 16-byte aligned");
    if (chunks == 0) return ok();
    hipStream_t st = (hipStream_t)stream;
    AdamEntry *table = reinterpret_cast<AdamEntry *>(workspace);
    if (!reuse_table) {
        TableBatch b{};
        int32_t chunk0 = 0;
        for (int32_t i = 0; i < count; ++i) {
            const gdn2_adamw_tensor &t = tensors[i];
            AdamEntry &e = b.e[b.n++];
            e.p = t.param;
            e.g = t.grad;
            e.m = t.first;
            e.v = t.second;
            e.numel = t.numel;
            e.chunk0 = chunk0;
            e.vec = (((uintptr_t)t.param | (uintptr_t)t.grad | (uintptr_t)t.first |
                      (uintptr_t)t.second) & 15) == 0;
            chunk0 += (int32_t)((t.numel + kAdamChunk - 1) / kAdamChunk);
            if (b.n == kTableBatch || i == count - 1) {
                hipLaunchKernelGGL(adam_table_kernel, dim3(1), dim3(kTableBatch), 0, st, table, b);
                GDN2_TRY(launch_status(hipGetLastError(), "gdn2_adamw_update (table)"));
                b.first += b.n;
                b.n = 0;
            }
        }
    }
    AdamArgs a{};
    a.table = table;
    a.count = count;
    a.partial = reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) +
                                          align256((size_t)count * sizeof(AdamEntry)));
    a.initialized = initialized != 0;
    a.c1 = 1.f - powi_f32(0.9f, time);
    a.c2 = 1.f - powi_f32(0.999f, time);
    a.b1c = 1.f - 0.9f;
    a.b2c = 1.f - 0.999f;
    a.decay = (float)(1.0 - lr * (double)weight_decay);
    a.lr = (float)lr;
    a.clip = clip;
    hipLaunchKernelGGL(adam_square_kernel, dim3((unsigned)chunks), dim3(kAdamThreads), 0, st, a);
    GDN2_TRY(launch_status(hipGetLastError(), "gdn2_adamw_update (norms)"));
    hipLaunchKernelGGL(adam_update_kernel, dim3((unsigned)chunks), dim3(kAdamThreads), 0, st, a);
    return launch_status(hipGetLastError(), "gdn2_adamw_update");
}

}  // extern "C"
