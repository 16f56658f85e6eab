// HOLA exact-memory cache read on gfx950: the downstream consumer of the GDN-2
// scores.  After every chunk of `chunk` tokens each (batch, head) keeps the
// `capacity` highest-scoring valid tokens of the document of the chunk's last
// physical slot (ties: earlier position); each valid query attends with
// softmax to the previous chunk's cache plus the causal tokens of its own
// chunk in its document, next to a learned zero-value sink logit.
//
// Semantics: crates/kernels/src/hola.rs (selection_kernel, forward_kernel,
// query/key VJPs) and the scalar oracle of crates/mixers/src/hola_checks.rs.
//
// Layout and work split:
//   * schedule: one wave per (batch, head), chunks in order; each candidate's
//     rank is the number of eligible candidates that beat it (exact top-k with
//     no sort); it writes the cache positions before/after every chunk and the
//     end of each key's visibility ("expiry");
//   * read, query VJP: one wave per (batch, head, chunk); the chunk's slots
//     (cache positions from the schedule + the chunk's own tokens) are gathered
//     once into LDS, then each query is a wave-wide softmax over <= 80 slots;
//   * key VJP: one wave per (batch, head, chunk) of keys.  A selected key stays
//     in the cache without interruption until it is evicted, so its visible
//     queries are the chunks from its own up to its expiry; the wave walks them
//     with a slot map per chunk and accumulates dk, dv in registers from the
//     (probability, logit gradient) pairs the query VJP saved.  No atomics.
//   * sink gradient: a fixed-order sum over tokens per head.
#include <float.h>
#include <math.h>

#include <algorithm>
#include <initializer_list>
#include <utility>

#include "gdn2_common.h"
#include "gdn2_status.h"

namespace gdn2 {
namespace {

constexpr int kMaxCapacity = 64;
constexpr int kMaxChunk = 16;
constexpr int kMaxSlots = kMaxCapacity + kMaxChunk;
constexpr int kMaxWidth = 128;

struct HolaArgs {
    int B, T, H, dk, dv, cap, chunk, nc, recency;
    float scale;
    View q, k, v, scores, valid, docs, sink, dout;
    float *schedule;         // [B*H][nc + 1][cap]
    float *expiry;           // [B*T*H]
    float *stats;            // [B*T*H][2]: softmax max, 1 / denominator
    float *out;              // [B*T*H][dv]
    const float *fwd_out;    // the forward output (backward)
    float *pairs;            // [B*T*H][cap + chunk][2]: probability, logit gradient
    float *aux;              // [B*T*H][2]: dO . o, sink gradient term
    float *gq, *gk, *gv, *gsink;  // dq, dk, dv, dsink
    float *final_positions;  // [B*H][cap] or null
};

__device__ __forceinline__ float ldf(const View &v, int64_t i0, int64_t i1 = 0, int64_t i2 = 0,
                                     int64_t i3 = 0) {
    return reinterpret_cast<const float *>(v.data)[i0 * v.s0 + i1 * v.s1 + i2 * v.s2 + i3 * v.s3];
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    x += dpp_f<0x141>(x);
    x += dpp_f<0x140>(x);
    return ((readlane_f(x, 0) + readlane_f(x, 16)) + readlane_f(x, 32)) + readlane_f(x, 48);
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));
    x = fmaxf(x, dpp_f<0x4E>(x));
    x = fmaxf(x, dpp_f<0x141>(x));
    x = fmaxf(x, dpp_f<0x140>(x));
    return fmaxf(fmaxf(readlane_f(x, 0), readlane_f(x, 16)),
                 fmaxf(readlane_f(x, 32), readlane_f(x, 48)));
}

__device__ __forceinline__ int64_t token(const HolaArgs &a, int b, int t, int h) {
    return ((int64_t)b * a.T + t) * a.H + h;
}

// ---- schedule ---------------------------------------------------------------------

__global__ void __launch_bounds__(64) hola_schedule_kernel(HolaArgs a) {
    __shared__ float cache[kMaxCapacity], next[kMaxCapacity];
    __shared__ float pos[kMaxSlots], pri[kMaxSlots];
    const int lane = threadIdx.x, bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int slots = a.cap + a.chunk;
    float *sched = a.schedule + (int64_t)bh * (a.nc + 1) * a.cap;
    if (lane < a.cap) {
        cache[lane] = -1.f;
        sched[lane] = -1.f;
    }
    __syncthreads();
    for (int c = 0; c < a.nc; ++c) {
        const int first = c * a.chunk, end = min(first + a.chunk, a.T);
        // The document of the chunk's last PHYSICAL slot, padding included.
        const float last_doc = ldf(a.docs, b, end - 1);
        if (lane < a.cap) next[lane] = -1.f;
        for (int s = lane; s < slots; s += 64) {
            float p = -1.f;
            if (s < a.cap) {
                p = cache[s];
            } else {
                const int t = first + s - a.cap;
                if (t < end) {
                    if (a.expiry) a.expiry[token(a, b, t, h)] = (float)end;
                    if (ldf(a.valid, b, t) >= 0.5f) p = (float)t;
                }
            }
            float score = 0.f;
            if (p >= 0.f) {
                const int t = (int)p;
                if (ldf(a.docs, b, t) == last_doc) score = a.recency ? p : ldf(a.scores, b, t, h);
                else p = -1.f;
            }
            pos[s] = p;
            pri[s] = score;
        }
        __syncthreads();
        for (int s = lane; s < slots; s += 64) {
            const float p = pos[s];
            if (p < 0.f) continue;
            const float sc = pri[s];
            int rank = 0;
            for (int o = 0; o < slots; ++o) {
                const float po = pos[o];
                if (po >= 0.f && (pri[o] > sc || (pri[o] == sc && po < p))) ++rank;
            }
            if (rank < a.cap) next[rank] = p;
        }
        __syncthreads();
        if (lane < a.cap) {
            const float p = next[lane];
            cache[lane] = p;
            sched[(int64_t)(c + 1) * a.cap + lane] = p;
            if (p >= 0.f && a.expiry)
                a.expiry[token(a, b, (int)p, h)] = (float)min(end + a.chunk, a.T);
        }
        __syncthreads();
    }
    if (a.final_positions && lane < a.cap) a.final_positions[(int64_t)bh * a.cap + lane] = cache[lane];
}

// ---- chunk slots ------------------------------------------------------------------

template <int DK, int DV>
struct SlotTiles {
    float K[kMaxSlots][DK + 1];  // +1: lanes reading different rows hit different banks
    float V[kMaxSlots][DV];
    float pos[kMaxSlots], doc[kMaxSlots];
};

// Slots of chunk c: the cache before the chunk, then the chunk's tokens.
// Empty or invalid slots get position -1 and zero rows.
template <int DK, int DV>
__device__ void stage_slots(const HolaArgs &a, int b, int h, int c, SlotTiles<DK, DV> &s) {
    const int lane = threadIdx.x, first = c * a.chunk, end = min(first + a.chunk, a.T);
    const int slots = a.cap + a.chunk;
    const float *sched = a.schedule + ((int64_t)(b * a.H + h) * (a.nc + 1) + c) * a.cap;
    for (int j = lane; j < slots; j += 64) {
        float p = -1.f;
        if (j < a.cap) {
            p = sched[j];
        } else {
            const int t = first + j - a.cap;
            if (t < end && ldf(a.valid, b, t) >= 0.5f) p = (float)t;
        }
        s.pos[j] = p;
        s.doc[j] = p >= 0.f ? ldf(a.docs, b, (int)p) : 0.f;
    }
    __syncthreads();
    for (int j = 0; j < slots; ++j) {
        const float p = s.pos[j];
        const int t = p >= 0.f ? (int)p : 0;
        for (int i = lane; i < DK; i += 64)
            s.K[j][i] = (p >= 0.f && i < a.dk) ? ldf(a.k, b, t, h, i) : 0.f;
        for (int i = lane; i < DV; i += 64)
            s.V[j][i] = (p >= 0.f && i < a.dv) ? ldf(a.v, b, t, h, i) : 0.f;
    }
    __syncthreads();
}

// Logit of query (in LDS) against slot j, or -FLT_MAX when j is not visible.
template <int DK, int DV>
__device__ __forceinline__ bool slot_logit(const HolaArgs &a, const SlotTiles<DK, DV> &s,
                                           const float *qs, int j, bool active, int t, float doc,
                                           float &logit) {
    logit = -FLT_MAX;
    const float p = s.pos[j];
    if (!(active && p >= 0.f && p <= (float)t && s.doc[j] == doc)) return false;
    float d = 0.f;
#pragma unroll 8
    for (int i = 0; i < DK; ++i) d += qs[i] * s.K[j][i];
    logit = d * a.scale;
    return true;
}

template <int DK, int DV>
__global__ void __launch_bounds__(64) hola_forward_kernel(HolaArgs a) {
    __shared__ SlotTiles<DK, DV> s;
    __shared__ float P[kMaxSlots];
    __shared__ float qs[DK];
    const int lane = threadIdx.x;
    const int c = blockIdx.x % a.nc, bh = blockIdx.x / a.nc, b = bh / a.H, h = bh % a.H;
    const int first = c * a.chunk, end = min(first + a.chunk, a.T), slots = a.cap + a.chunk;
    stage_slots<DK, DV>(a, b, h, c, s);
    const float sink = ldf(a.sink, h);
    for (int t = first; t < end; ++t) {
        const bool active = ldf(a.valid, b, t) >= 0.5f;
        const float doc = ldf(a.docs, b, t);
        for (int i = lane; i < DK; i += 64) qs[i] = i < a.dk ? ldf(a.q, b, t, h, i) : 0.f;
        __syncthreads();
        float lg[2];
        bool vis[2];
        float m = sink;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = lane + 64 * r;
            vis[r] = j < slots && slot_logit<DK, DV>(a, s, qs, j, active, t, doc, lg[r]);
            if (vis[r]) m = fmaxf(m, lg[r]);
        }
        m = wave_max(m);
        const float w0 = vis[0] ? expf(lg[0] - m) : 0.f;
        const float w1 = vis[1] ? expf(lg[1] - m) : 0.f;
        const float inv = 1.f / (wave_sum(w0 + w1) + expf(sink - m));
        // Normalised before the value product: finite values cannot overflow.
        if (lane < slots) P[lane] = w0 * inv;
        if (lane + 64 < slots) P[lane + 64] = w1 * inv;
        __syncthreads();
        const int64_t tok = token(a, b, t, h);
        for (int j = lane; j < a.dv; j += 64) {
            float o = 0.f;
            if (active)
                for (int k = 0; k < slots; ++k) o += P[k] * s.V[k][j];
            a.out[tok * a.dv + j] = o;
        }
        if (lane == 0) {
            a.stats[2 * tok] = m;
            a.stats[2 * tok + 1] = inv;
        }
        __syncthreads();
    }
}

// ---- backward ---------------------------------------------------------------------

template <int DK, int DV>
__global__ void __launch_bounds__(64) hola_query_backward_kernel(HolaArgs a) {
    __shared__ SlotTiles<DK, DV> s;
    __shared__ float D[kMaxSlots];
    __shared__ float qs[DK], gs[DV];
    const int lane = threadIdx.x;
    const int c = blockIdx.x % a.nc, bh = blockIdx.x / a.nc, b = bh / a.H, h = bh % a.H;
    const int first = c * a.chunk, end = min(first + a.chunk, a.T), slots = a.cap + a.chunk;
    stage_slots<DK, DV>(a, b, h, c, s);
    const float sink = ldf(a.sink, h);
    for (int t = first; t < end; ++t) {
        const bool active = ldf(a.valid, b, t) >= 0.5f;
        const float doc = ldf(a.docs, b, t);
        const int64_t tok = token(a, b, t, h);
        for (int i = lane; i < DK; i += 64) qs[i] = i < a.dk ? ldf(a.q, b, t, h, i) : 0.f;
        float dl = 0.f;
        for (int j = lane; j < DV; j += 64) {
            const float g = (j < a.dv && a.dout.data) ? ldf(a.dout, b, t, h, j) : 0.f;
            gs[j] = g;
            if (active && j < a.dv) dl += g * a.fwd_out[tok * a.dv + j];
        }
        const float delta = wave_sum(dl);
        const float m = a.stats[2 * tok], inv = a.stats[2 * tok + 1];
        if (lane == 0) {
            a.aux[2 * tok] = delta;
            a.aux[2 * tok + 1] = active ? -delta * expf(sink - m) * inv : 0.f;
        }
        __syncthreads();
        for (int j = lane; j < slots; j += 64) {
            float lg, p = 0.f, d = 0.f;
            if (slot_logit<DK, DV>(a, s, qs, j, active, t, doc, lg)) {
                p = expf(lg - m) * inv;
                float dot = 0.f;
#pragma unroll 8
                for (int i = 0; i < DV; ++i) dot += gs[i] * s.V[j][i];
                d = p * (dot - delta) * a.scale;
            }
            D[j] = d;
            float *pr = a.pairs + (tok * slots + j) * 2;
            pr[0] = p;
            pr[1] = d;
        }
        __syncthreads();
        for (int i = lane; i < a.dk; i += 64) {
            float g = 0.f;
            if (active)
                for (int j = 0; j < slots; ++j) g += D[j] * s.K[j][i];
            a.gq[tok * a.dk + i] = g;
        }
        __syncthreads();
    }
}

template <int DK, int DV>
__global__ void __launch_bounds__(64) hola_key_backward_kernel(HolaArgs a) {
    constexpr int RK = (DK + 63) / 64, RV = (DV + 63) / 64;
    __shared__ int map[kMaxChunk];
    const int lane = threadIdx.x;
    const int c = blockIdx.x % a.nc, bh = blockIdx.x / a.nc, b = bh / a.H, h = bh % a.H;
    const int first = c * a.chunk, end = min(first + a.chunk, a.T), n = end - first;
    const int slots = a.cap + a.chunk;
    const float *sched = a.schedule + (int64_t)bh * (a.nc + 1) * a.cap;
    float dka[kMaxChunk][RK], dva[kMaxChunk][RV];
#pragma unroll
    for (int j = 0; j < kMaxChunk; ++j) {
#pragma unroll
        for (int r = 0; r < RK; ++r) dka[j][r] = 0.f;
#pragma unroll
        for (int r = 0; r < RV; ++r) dva[j][r] = 0.f;
    }
    // Queries that can see a key of this chunk end at its expiry.
    int last = end;
    for (int j = 0; j < n; ++j) last = max(last, (int)a.expiry[token(a, b, first + j, h)]);
    for (int cq = c; cq * a.chunk < last; ++cq) {
        if (lane < kMaxChunk) map[lane] = -1;
        __syncthreads();
        if (cq == c) {
            if (lane < n) map[lane] = a.cap + lane;
        } else if (lane < a.cap) {
            const float p = sched[(int64_t)cq * a.cap + lane];
            if (p >= (float)first && p < (float)end) map[(int)p - first] = lane;
        }
        __syncthreads();
        int sl[kMaxChunk];
#pragma unroll
        for (int j = 0; j < kMaxChunk; ++j) sl[j] = j < n ? map[j] : -1;
        const int t1 = min(cq * a.chunk + a.chunk, a.T);
        for (int t = cq * a.chunk; t < t1; ++t) {
            const int64_t tok = token(a, b, t, h);
            float qv[RK], gv[RV];
#pragma unroll
            for (int r = 0; r < RK; ++r) {
                const int i = lane + 64 * r;
                qv[r] = i < a.dk ? ldf(a.q, b, t, h, i) : 0.f;
            }
#pragma unroll
            for (int r = 0; r < RV; ++r) {
                const int i = lane + 64 * r;
                gv[r] = (i < a.dv && a.dout.data) ? ldf(a.dout, b, t, h, i) : 0.f;
            }
            const float *pr = a.pairs + tok * slots * 2;
#pragma unroll
            for (int j = 0; j < kMaxChunk; ++j) {
                if (sl[j] < 0) continue;
                const float p = pr[2 * sl[j]], d = pr[2 * sl[j] + 1];
#pragma unroll
                for (int r = 0; r < RK; ++r) dka[j][r] += d * qv[r];
#pragma unroll
                for (int r = 0; r < RV; ++r) dva[j][r] += p * gv[r];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kMaxChunk; ++j) {
        if (j >= n) continue;
        const int64_t tok = token(a, b, first + j, h);
#pragma unroll
        for (int r = 0; r < RK; ++r) {
            const int i = lane + 64 * r;
            if (i < a.dk) a.gk[tok * a.dk + i] = dka[j][r];
        }
#pragma unroll
        for (int r = 0; r < RV; ++r) {
            const int i = lane + 64 * r;
            if (i < a.dv) a.gv[tok * a.dv + i] = dva[j][r];
        }
    }
}

// dsink[h] = sum over (b, t) of aux[.][1], in a fixed order.
__global__ void __launch_bounds__(1024) hola_sink_kernel(HolaArgs a) {
    __shared__ float red[16];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int64_t n = (int64_t)a.B * a.T;
    float s = 0.f;
    for (int64_t r = tid; r < n; r += 1024) s += a.aux[2 * (r * a.H + h) + 1];
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        float t = red[0];
        for (int i = 1; i < 16; ++i) t += red[i];
        a.gsink[h] = t;
    }
}

// ---- host ---------------------------------------------------------------------------

int pad_width(int64_t w) { return w <= 32 ? 32 : (w <= 64 ? 64 : 128); }

template <template <int, int> class K>
void launch_widths(const HolaArgs &a, dim3 grid, hipStream_t st) {
    const int kp = pad_width(a.dk), vp = pad_width(a.dv);
#define GDN2_HOLA_CASE(P, Q)                                                    \
    if (kp == P && vp == Q) {                                                   \
        hipLaunchKernelGGL((K<P, Q>::fn), grid, dim3(64), 0, st, a);            \
        return;                                                                 \
    }
    GDN2_HOLA_CASE(32, 32) GDN2_HOLA_CASE(32, 64) GDN2_HOLA_CASE(32, 128)
    GDN2_HOLA_CASE(64, 32) GDN2_HOLA_CASE(64, 64) GDN2_HOLA_CASE(64, 128)
    GDN2_HOLA_CASE(128, 32) GDN2_HOLA_CASE(128, 64) GDN2_HOLA_CASE(128, 128)
#undef GDN2_HOLA_CASE
}
template <int P, int Q> struct Fwd { static constexpr auto fn = hola_forward_kernel<P, Q>; };
template <int P, int Q> struct QBwd { static constexpr auto fn = hola_query_backward_kernel<P, Q>; };
template <int P, int Q> struct KBwd { static constexpr auto fn = hola_key_backward_kernel<P, Q>; };

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

int64_t chunks_of(const gdn2_hola_shape *s) { return (s->time + s->chunk - 1) / s->chunk; }

int check_hola_shape(const gdn2_hola_shape *s) {
    if (!s) return fail(GDN2_ERR_ARGUMENT, "shape is null");
    if (s->batch < 1 || s->time < 1 || s->heads < 1)
        return fail(GDN2_ERR_SHAPE, "HOLA requires nonempty batch, time and heads");
    if (s->keys < 1 || s->keys > kMaxWidth || s->values < 1 || s->values > kMaxWidth)
        return fail(GDN2_ERR_SHAPE, "HOLA key and value widths must be 1..%d", kMaxWidth);
    if (s->capacity < 1 || s->capacity > kMaxCapacity)
        return fail(GDN2_ERR_SHAPE, "HOLA capacity must be 1..%d (got %d)", kMaxCapacity,
                    s->capacity);
    if (s->chunk < 1 || s->chunk > kMaxChunk)
        return fail(GDN2_ERR_SHAPE, "HOLA chunk must be 1..%d (got %d)", kMaxChunk, s->chunk);
    if (s->batch * s->heads * chunks_of(s) > 0x7FFFFFFF || s->time > (1 << 24))
        return fail(GDN2_ERR_SHAPE, "HOLA problem too large");
    return ok();
}

struct CkLayout {
    size_t schedule, expiry, stats, total;
};

CkLayout ck_layout(const gdn2_hola_shape *s) {
    const int64_t bth = s->batch * s->time * s->heads;
    CkLayout l;
    l.schedule = 0;
    l.expiry = align256((size_t)s->batch * s->heads * (chunks_of(s) + 1) * s->capacity * 4);
    l.stats = l.expiry + align256((size_t)bth * 4);
    l.total = l.stats + align256((size_t)bth * 8);
    return l;
}

size_t ws_pairs_bytes(const gdn2_hola_shape *s) {
    return align256((size_t)s->batch * s->time * s->heads * (s->capacity + s->chunk) * 8);
}

HolaArgs hola_args(const gdn2_hola_shape *s, const gdn2_view *q, const gdn2_view *k,
                   const gdn2_view *v, const gdn2_view *valid, const gdn2_view *docs,
                   const gdn2_view *sink) {
    HolaArgs a{};
    a.B = (int)s->batch;
    a.T = (int)s->time;
    a.H = (int)s->heads;
    a.dk = (int)s->keys;
    a.dv = (int)s->values;
    a.cap = s->capacity;
    a.chunk = s->chunk;
    a.nc = (int)chunks_of(s);
    a.scale = 1.f / sqrtf((float)s->keys);
    a.q = make_view(q);
    a.k = make_view(k);
    a.v = make_view(v);
    a.valid = make_view(valid);
    a.docs = make_view(docs);
    a.sink = make_view(sink);
    return a;
}

int check_f32_views(std::initializer_list<std::pair<const gdn2_view *, const char *>> views) {
    for (auto &v : views) GDN2_TRY(check_view(v.first, v.second, GDN2_F32, false));
    return ok();
}

}  // namespace
}  // namespace gdn2

using namespace gdn2;

extern "C" {

int gdn2_hola_schedule(const gdn2_hola_shape *shape, int recency, const gdn2_view *scores,
                       const gdn2_view *valid, const gdn2_view *documents, float *schedule,
                       void *stream) {
    GDN2_TRY(check_hola_shape(shape));
    GDN2_TRY(check_f32_views({{scores, "scores"}, {valid, "valid"}, {documents, "documents"}}));
    if (!schedule) return fail(GDN2_ERR_ARGUMENT, "schedule is null");
    HolaArgs a = hola_args(shape, nullptr, nullptr, nullptr, valid, documents, nullptr);
    a.scores = make_view(scores);
    a.recency = recency != 0;
    a.schedule = schedule;
    hipLaunchKernelGGL(hola_schedule_kernel, dim3(a.B * a.H), dim3(64), 0, (hipStream_t)stream, a);
    return launch_status(hipGetLastError(), "gdn2_hola_schedule");
}

size_t gdn2_hola_checkpoint_bytes(const gdn2_hola_shape *shape) {
    if (check_hola_shape(shape)) return 0;
    return ck_layout(shape).total;
}

int gdn2_hola_read(const gdn2_hola_shape *shape, int recency, const gdn2_view *q,
                   const gdn2_view *k, const gdn2_view *v, const gdn2_view *scores,
                   const gdn2_view *valid, const gdn2_view *documents, const gdn2_view *sink,
                   float *output, float *final_positions, void *checkpoint,
                   size_t checkpoint_bytes, void *stream) {
    GDN2_TRY(check_hola_shape(shape));
    GDN2_TRY(check_f32_views({{q, "q"}, {k, "k"}, {v, "v"}, {scores, "scores"}, {valid, "valid"},
                              {documents, "documents"}, {sink, "sink"}}));
    if (!output) return fail(GDN2_ERR_ARGUMENT, "output is null");
    const CkLayout l = ck_layout(shape);
    if (!checkpoint || checkpoint_bytes < l.total)
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu", l.total,
                    checkpoint_bytes);
    HolaArgs a = hola_args(shape, q, k, v, valid, documents, sink);
    char *ck = static_cast<char *>(checkpoint);
    a.scores = make_view(scores);
    a.recency = recency != 0;
    a.schedule = reinterpret_cast<float *>(ck + l.schedule);
    a.expiry = reinterpret_cast<float *>(ck + l.expiry);
    a.stats = reinterpret_cast<float *>(ck + l.stats);
    a.out = output;
    a.final_positions = final_positions;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(hola_schedule_kernel, dim3(a.B * a.H), dim3(64), 0, st, a);
    GDN2_TRY(launch_status(hipGetLastError(), "gdn2_hola_read (schedule)"));
    launch_widths<Fwd>(a, dim3(a.B * a.H * a.nc), st);
    return launch_status(hipGetLastError(), "gdn2_hola_read");
}

size_t gdn2_hola_workspace_bytes(const gdn2_hola_shape *shape) {
    if (check_hola_shape(shape)) return 0;
    return ws_pairs_bytes(shape) +
           align256((size_t)shape->batch * shape->time * shape->heads * 8);
}

int gdn2_hola_backward(const gdn2_hola_shape *shape, const gdn2_view *q, const gdn2_view *k,
                       const gdn2_view *v, const gdn2_view *valid, const gdn2_view *documents,
                       const gdn2_view *sink, const void *checkpoint, size_t checkpoint_bytes,
                       const float *output, const gdn2_view *d_output, float *dq, float *dk,
                       float *dv, float *dsink, void *workspace, size_t workspace_bytes,
                       void *stream) {
    GDN2_TRY(check_hola_shape(shape));
    GDN2_TRY(check_f32_views({{q, "q"}, {k, "k"}, {v, "v"}, {valid, "valid"},
                              {documents, "documents"}, {sink, "sink"}}));
    if (d_output) GDN2_TRY(check_view(d_output, "d_output", GDN2_F32, true));
    if (!output || !dq || !dk || !dv || !dsink)
        return fail(GDN2_ERR_ARGUMENT, "output, dq, dk, dv and dsink must be non-null");
    const CkLayout l = ck_layout(shape);
    if (!checkpoint || checkpoint_bytes < l.total)
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu", l.total,
                    checkpoint_bytes);
    const size_t need = gdn2_hola_workspace_bytes(shape);
    if (!workspace || workspace_bytes < need)
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need,
                    workspace_bytes);
    HolaArgs a = hola_args(shape, q, k, v, valid, documents, sink);
    const char *ck = static_cast<const char *>(checkpoint);
    a.schedule = const_cast<float *>(reinterpret_cast<const float *>(ck + l.schedule));
    a.expiry = const_cast<float *>(reinterpret_cast<const float *>(ck + l.expiry));
    a.stats = const_cast<float *>(reinterpret_cast<const float *>(ck + l.stats));
    if (d_output) a.dout = make_view(d_output);
    a.fwd_out = output;
    a.pairs = static_cast<float *>(workspace);
    a.aux = reinterpret_cast<float *>(static_cast<char *>(workspace) + ws_pairs_bytes(shape));
    a.gq = dq;
    a.gk = dk;
    a.gv = dv;
    a.gsink = dsink;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(a.B * a.H * a.nc);
    launch_widths<QBwd>(a, grid, st);
    GDN2_TRY(launch_status(hipGetLastError(), "gdn2_hola_backward (queries)"));
    launch_widths<KBwd>(a, grid, st);
    GDN2_TRY(launch_status(hipGetLastError(), "gdn2_hola_backward (keys)"));
    hipLaunchKernelGGL(hola_sink_kernel, dim3(a.H), dim3(1024), 0, st, a);
    return launch_status(hipGetLastError(), "gdn2_hola_backward");
}

}  // extern "C"
