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
#include "gdn2_mfma.h"
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

// One wave per (batch, head), chunks in order.  The cache entries carry their
// ranking key and document in LDS, and the next chunk's token words (valid,
// document, score) are loaded while the current chunk is ranked, so a chunk
// costs LDS work only.
__global__ void __launch_bounds__(64) hola_schedule_kernel(HolaArgs a) {
    __shared__ float cpos[kMaxCapacity], cpri[kMaxCapacity], cdoc[kMaxCapacity];
    __shared__ float pos[kMaxSlots], pri[kMaxSlots], sdoc[kMaxSlots];
    __shared__ __align__(16) uint64_t key[kMaxSlots];
    __shared__ float npos[kMaxCapacity], npri[kMaxCapacity], ndoc[kMaxCapacity];
    const int lane = threadIdx.x, bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    float *sched = a.schedule + (int64_t)bh * (a.nc + 1) * a.cap;
    if (lane < a.cap) {
        cpos[lane] = -1.f;
        cpri[lane] = cdoc[lane] = 0.f;
        sched[lane] = -1.f;
    }
    // Candidate slots past capacity + chunk stay empty for good.
    for (int sl = lane; sl < kMaxSlots; sl += 64) {
        pos[sl] = -1.f;
        pri[sl] = 0.f;
        key[sl] = 0;
    }
    // Token words of a chunk: lane j < chunk holds token first + j.
    float tv = 0.f, td = 0.f, ts = 0.f;
    auto fetch = [&](int c) {
        const int t = c * a.chunk + lane;
        tv = td = ts = 0.f;
        if (lane < a.chunk && t < a.T) {
            tv = ldf(a.valid, b, t);
            td = ldf(a.docs, b, t);
            if (!a.recency) ts = ldf(a.scores, b, t, h);
        }
    };
    fetch(0);
    __syncthreads();
    for (int c = 0; c < a.nc; ++c) {
        const int first = c * a.chunk, end = min(first + a.chunk, a.T), n = end - first;
        const float mv = tv, md = td, ms = ts;
        if (c + 1 < a.nc) fetch(c + 1);
        // The document of the chunk's last PHYSICAL slot, padding included.
        const float last_doc = readlane_f(md, n - 1);
        if (lane < n && a.expiry) a.expiry[token(a, b, first + lane, h)] = (float)end;
        // Candidates: the cache, then the chunk's valid tokens; only the last
        // slot's document is eligible.
        if (lane < a.cap) {
            const float p = cpos[lane];
            const bool ok = p >= 0.f && cdoc[lane] == last_doc;
            pos[lane] = ok ? p : -1.f;
            pri[lane] = cpri[lane];
            sdoc[lane] = cdoc[lane];
        }
        if (lane < a.chunk) {
            const int t = first + lane;
            const bool ok = lane < n && mv >= 0.5f && md == last_doc;
            pos[a.cap + lane] = ok ? (float)t : -1.f;
            pri[a.cap + lane] = a.recency ? (float)t : ms;
            sdoc[a.cap + lane] = md;
        }
        if (lane < a.cap) npos[lane] = -1.f;
        __syncthreads();
        // Ranking keys: the order-preserving bits of the score (or position)
        // above the complemented position, so "beats" (higher key, ties to
        // the earlier position) is one unsigned compare; empty and ineligible
        // slots get key 0 and never beat.
        for (int sl = lane; sl < a.cap + a.chunk; sl += 64) {
            const float p = pos[sl];
            const uint32_t u = __float_as_uint(pri[sl]);
            const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            key[sl] = p >= 0.f ? ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)p) : 0;
        }
        __syncthreads();
        // Rank = number of eligible candidates that beat this one (higher key,
        // then earlier position): an exact top-capacity with no sort.  Each
        // lane ranks candidates lane and lane + 64 in one pass over the
        // candidate list, read four at a time (empty slots never beat).
        {
            const int s1 = lane + 64;
            const float p0 = pos[lane], c0 = pri[lane];
            const float p1 = s1 < kMaxSlots ? pos[s1] : -1.f, c1 = s1 < kMaxSlots ? pri[s1] : 0.f;
            const uint64_t k0 = key[lane], k1 = s1 < kMaxSlots ? key[s1] : 0;
            int r0 = 0, r1 = 0;
#pragma unroll 10
            for (int o = 0; o < kMaxSlots; o += 2) {
                const ulonglong2 ko = *reinterpret_cast<const ulonglong2 *>(&key[o]);
                r0 += (ko.x > k0) + (ko.y > k0);
                r1 += (ko.x > k1) + (ko.y > k1);
            }
            if (p0 >= 0.f && r0 < a.cap) {
                npos[r0] = p0;
                npri[r0] = c0;
                ndoc[r0] = sdoc[lane];
            }
            if (p1 >= 0.f && r1 < a.cap) {
                npos[r1] = p1;
                npri[r1] = c1;
                ndoc[r1] = sdoc[s1];
            }
        }
        __syncthreads();
        if (lane < a.cap) {
            const float p = npos[lane];
            cpos[lane] = p;
            cpri[lane] = npri[lane];
            cdoc[lane] = ndoc[lane];
            sched[(int64_t)(c + 1) * a.cap + lane] = p;
            if (p >= 0.f && a.expiry)
                a.expiry[token(a, b, (int)p, h)] = (float)min(end + a.chunk, a.T);
        }
        __syncthreads();
    }
    if (a.final_positions && lane < a.cap) a.final_positions[(int64_t)bh * a.cap + lane] = cpos[lane];
}

// ---- chunk slots ------------------------------------------------------------------

constexpr int kReadWaves = 4;  // waves per chunk in the read and the query VJP
constexpr int kReadThreads = 64 * kReadWaves;
constexpr int kWaveQueries = kMaxChunk / kReadWaves;

// Query tt of a chunk is handled by wave tt % 4 as its (tt / 4)-th query;
// transposed query tiles keep each wave's four queries of one channel in one
// 16-byte group.
__device__ __forceinline__ int query_slot(int tt) { return ((tt & 3) << 2) | (tt >> 2); }

// dst[j * LD + i] = x(b, pos_j, h, i) for rows j < MAXS (zero where j >= S,
// pos_j < 0 or i >= w), by NT threads.  Loads go out 16 per thread at a time
// before any is used, so a gather costs a few memory latencies rather than
// one per row.
template <int D, int LD, int MAXS, int NT = 64, bool TQ = false>
__device__ __forceinline__ void gather_rows(const View &x, int b, int h, int w, const float *pos,
                                            int S, float *dst) {
    constexpr int PER = MAXS * D / NT, BATCH = 16;
    static_assert(PER * NT == MAXS * D, "whole workgroups");
    const int lane = threadIdx.x;
    for (int n0 = 0; n0 < PER; n0 += BATCH) {
        float r[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int idx = lane + NT * (n0 + u), j = idx / D, i = idx % D;
            r[u] = 0.f;
            if (n0 + u < PER && j < S && i < w) {
                const float p = pos[j];
                if (p >= 0.f) r[u] = ldf(x, b, (int)p, h, i);
            }
        }
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int idx = lane + NT * (n0 + u), j = idx / D, i = idx % D;
            if (n0 + u < PER) {
                if (TQ) dst[i * MAXS + query_slot(j)] = r[u];
                else dst[j * LD + i] = r[u];
            }
        }
    }
}

// PAD = 1 (the read): lanes reading different rows of one column hit
// different banks.  PAD = 4 (the query VJP's MFMA products): an operand read
// of 16 rows x 4 columns hits 64 distinct banks, one of 4 rows x 16 columns
// (its dq product) each bank at most four times.
template <int DK, int DV, int PAD = 1>
struct SlotTiles {
    static constexpr int LK = DK + PAD, LV = DV + PAD;
    float K[kMaxSlots][LK];
    float V[kMaxSlots][LV];
    float QT[DK][kMaxChunk] __attribute__((aligned(16)));  // [channel][query_slot(tt)]
    float pos[kMaxSlots], doc[kMaxSlots];
    float tpos[kMaxChunk], tval[kMaxChunk], tdoc[kMaxChunk];
};

// Slots of chunk c (the cache before the chunk, then the chunk's tokens; empty
// or invalid slots get position -1 and zero rows), and the chunk's queries.
template <int DK, int DV, int PAD>
__device__ void stage_slots(const HolaArgs &a, int b, int h, int c, SlotTiles<DK, DV, PAD> &s) {
    const int lane = threadIdx.x, first = c * a.chunk, end = min(first + a.chunk, a.T);
    const int slots = a.cap + a.chunk;
    const float *sched = a.schedule + ((int64_t)(b * a.H + h) * (a.nc + 1) + c) * a.cap;
    for (int j = lane; j < slots; j += kReadThreads) {
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
    if (lane < kMaxChunk) {
        const int t = first + lane;
        const bool in = lane < a.chunk && t < end;
        s.tpos[lane] = in ? (float)t : -1.f;
        s.tval[lane] = in ? ldf(a.valid, b, t) : 0.f;
        s.tdoc[lane] = in ? ldf(a.docs, b, t) : 0.f;
    }
    __syncthreads();
    gather_rows<DK, DK + PAD, kMaxSlots, kReadThreads>(a.k, b, h, a.dk, s.pos, slots, &s.K[0][0]);
    gather_rows<DV, DV + PAD, kMaxSlots, kReadThreads>(a.v, b, h, a.dv, s.pos, slots, &s.V[0][0]);
    gather_rows<DK, DK, kMaxChunk, kReadThreads, true>(a.q, b, h, a.dk, s.tpos, kMaxChunk,
                                                      &s.QT[0][0]);
    __syncthreads();
}

// The four queries of a wave (tt = wave + 4u): token, activity, document.
struct WaveQueries {
    int t[kWaveQueries];
    bool on[kWaveQueries], act[kWaveQueries];
    float doc[kWaveQueries];
};

template <int DK, int DV, int PAD>
__device__ __forceinline__ WaveQueries wave_queries(const SlotTiles<DK, DV, PAD> &s, int wave, int first,
                                                    int n) {
    WaveQueries w;
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) {
        const int tt = wave + kReadWaves * u;
        w.t[u] = first + tt;
        w.on[u] = tt < n;
        w.act[u] = tt < n && s.tval[tt] >= 0.5f;
        w.doc[u] = tt < n ? s.tdoc[tt] : 0.f;
    }
    return w;
}

// Scaled logits of the wave's queries against slot j (-FLT_MAX where the slot
// is not visible: empty, later than the query, another document, or an
// inactive query).  One K read and one 16-byte query read per channel.
template <int DK, int DV>
__device__ __forceinline__ void wave_logits(const HolaArgs &a, const SlotTiles<DK, DV> &s,
                                            const WaveQueries &w, int wave, int j,
                                            float (&lg)[kWaveQueries]) {
    float acc[kWaveQueries] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int i = 0; i < DK; ++i) {
        const float kv = s.K[j][i];
        const float4 q4 = *reinterpret_cast<const float4 *>(&s.QT[i][4 * wave]);
        acc[0] += q4.x * kv;
        acc[1] += q4.y * kv;
        acc[2] += q4.z * kv;
        acc[3] += q4.w * kv;
    }
    const float p = s.pos[j], d = s.doc[j];
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) {
        const bool vis = w.act[u] && p >= 0.f && p <= (float)w.t[u] && d == w.doc[u];
        lg[u] = vis ? acc[u] * a.scale : -FLT_MAX;
    }
}

// [query slot][slot] tiles of a chunk (logits, probabilities, their adjoints):
// row stride 84 floats (20 mod 64), so an MFMA A-operand read (16 rows x 4
// columns) and an accumulator store hit 64 distinct banks.
constexpr int kLP = kMaxSlots + 4;

// Query tt of the chunk behind query slot qs (the inverse of query_slot).
__device__ __forceinline__ int slot_query(int qs) { return (qs >> 2) + 4 * (qs & 3); }

// X Y^T over the reduction width D on v_mfma_f32_16x16x4f32: X^T [D][16] in
// query-slot columns (the chunk's queries or their output adjoints), Y [slot]
// rows of stride LY (K or V); out[qs][slot] for the 16-slot tiles that cover
// the slots, wave w taking tiles w, w + 4, ...  Lane (lg, ln) reduces over
// k = 4 ks + lg and holds rows 4 lg + r of column 16 n + ln.
template <int D, int LY>
__device__ __forceinline__ void chunk_xyt(const float (*XT)[kMaxChunk], const float *Y, int slots, int wave,
                                          float (*out)[kLP]) {
    const int l = lane_id(), lg = l >> 4, ln = l & 15;
    for (int n = wave; 16 * n < slots; n += kReadWaves) {
        f32x4 acc = zero4();
#pragma unroll 4
        for (int ks = 0; ks < D / 4; ++ks)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(XT[4 * ks + lg][ln], Y[(16 * n + ln) * LY + 4 * ks + lg],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) out[4 * lg + r][16 * n + ln] = acc[r];
    }
}

// P Y over the slots on v_mfma_f32_16x16x4f32: P [qs][slot] (zero past the
// slots), Y [slot][channel] rows of stride LY (zero past the slots); wave w
// takes the 16-channel tiles w, w + 4, .. of the W used channels and stores row
// qs (query slot_query(qs) of the chunk) of each to dst[token][channel] when the
// query is inside the sequence, zero when it is inactive.
template <int D, int LY>
__device__ __forceinline__ void chunk_py(const HolaArgs &a, const float (*P)[kLP], const float *Y, int slots,
                                         int wave, int b, int h, int first, int n, const float *tval, int W,
                                         float *dst) {
    const int l = lane_id(), lg = l >> 4, ln = l & 15, nks = (slots + 3) >> 2;
    for (int ct = wave; ct < D / 16; ct += kReadWaves) {
        f32x4 acc = zero4();
        for (int ks = 0; ks < nks; ++ks)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(P[ln][4 * ks + lg], Y[(4 * ks + lg) * LY + 16 * ct + ln],
                                                       acc, 0, 0, 0);
        const int ch = 16 * ct + ln;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tt = slot_query(4 * lg + r);
            if (tt < n && ch < W)
                dst[token(a, b, first + tt, h) * W + ch] = tval[tt] >= 0.5f ? acc[r] : 0.f;
        }
    }
}

// Scaled logit of the wave's query u against slot j from the chunk's raw
// logits (-FLT_MAX where the slot is not visible: past the slots, empty, later
// than the query, another document, or an inactive query).
template <int DK, int DV, int PAD>
__device__ __forceinline__ float visible_logit(const HolaArgs &a, const SlotTiles<DK, DV, PAD> &s,
                                               const WaveQueries &w, const float (*L)[kLP], int wave, int u,
                                               int j, int slots) {
    if (j >= slots || !w.act[u]) return -FLT_MAX;
    const float p = s.pos[j];
    const bool vis = p >= 0.f && p <= (float)w.t[u] && s.doc[j] == w.doc[u];
    return vis ? L[4 * wave + u][j] * a.scale : -FLT_MAX;
}

template <int DK, int DV>
__global__ void __launch_bounds__(kReadThreads) hola_forward_kernel(HolaArgs a) {
    __shared__ SlotTiles<DK, DV> s;
    __shared__ float4 PT[kReadWaves][kMaxSlots];  // normalised probabilities, [slot][query]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x % a.nc, bh = blockIdx.x / a.nc, b = bh / a.H, h = bh % a.H;
    const int first = c * a.chunk, end = min(first + a.chunk, a.T), slots = a.cap + a.chunk;
    stage_slots<DK, DV>(a, b, h, c, s);
    const float sink = ldf(a.sink, h);
    const WaveQueries w = wave_queries(s, wave, first, end - first);
    float lg[2][kWaveQueries];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int j = lane + 64 * r;
        if (j < slots) wave_logits(a, s, w, wave, j, lg[r]);
        else
            for (int u = 0; u < kWaveQueries; ++u) lg[r][u] = -FLT_MAX;
    }
    float m[kWaveQueries], inv[kWaveQueries], p0[kWaveQueries], p1[kWaveQueries];
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) m[u] = wave_max(fmaxf(sink, fmaxf(lg[0][u], lg[1][u])));
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) {
        p0[u] = lg[0][u] > -FLT_MAX ? expf(lg[0][u] - m[u]) : 0.f;
        p1[u] = lg[1][u] > -FLT_MAX ? expf(lg[1][u] - m[u]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) {
        inv[u] = 1.f / (wave_sum(p0[u] + p1[u]) + expf(sink - m[u]));
        // Normalised before the value product: finite values cannot overflow.
        p0[u] *= inv[u];
        p1[u] *= inv[u];
    }
    if (lane < slots) PT[wave][lane] = make_float4(p0[0], p0[1], p0[2], p0[3]);
    if (lane + 64 < slots) PT[wave][lane + 64] = make_float4(p1[0], p1[1], p1[2], p1[3]);
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < a.dv; j += 64) {
        float o[kWaveQueries] = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < slots; ++k) {
            const float vv = s.V[k][j];
            const float4 p4 = PT[wave][k];
            o[0] += p4.x * vv;
            o[1] += p4.y * vv;
            o[2] += p4.z * vv;
            o[3] += p4.w * vv;
        }
#pragma unroll
        for (int u = 0; u < kWaveQueries; ++u)
            if (w.on[u]) a.out[token(a, b, w.t[u], h) * a.dv + j] = w.act[u] ? o[u] : 0.f;
    }
    if (lane == 0) {
#pragma unroll
        for (int u = 0; u < kWaveQueries; ++u) {
            if (!w.on[u]) continue;
            const int64_t tok = token(a, b, w.t[u], h);
            a.stats[2 * tok] = m[u];
            a.stats[2 * tok + 1] = inv[u];
        }
    }
}

// ---- backward ---------------------------------------------------------------------

template <int DK, int DV>
__global__ void __launch_bounds__(kReadThreads) hola_query_backward_kernel(HolaArgs a) {
    __shared__ SlotTiles<DK, DV, 4> s;
    __shared__ float L[kMaxChunk][kLP];   // logits, then logit gradients: [query slot][slot]
    __shared__ float Dt[kMaxChunk][kLP];  // dO . v_slot: [query slot][slot]
    __shared__ float GT[DV][kMaxChunk] __attribute__((aligned(16)));  // dO, [channel][query_slot]
    __shared__ float O[kMaxChunk][DV + 1];
    __shared__ float stat[kMaxChunk][2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x % a.nc, bh = blockIdx.x / a.nc, b = bh / a.H, h = bh % a.H;
    const int first = c * a.chunk, end = min(first + a.chunk, a.T), slots = a.cap + a.chunk;
    stage_slots<DK, DV>(a, b, h, c, s);
    // The chunk's output adjoints (transposed), forward outputs and softmax
    // statistics.
    {
        constexpr int PER = kMaxChunk * DV / kReadThreads;
        float g[PER], o[PER];
#pragma unroll
        for (int n = 0; n < PER; ++n) {
            const int idx = tid + kReadThreads * n, tt = idx / DV, j = idx % DV, t = first + tt;
            g[n] = o[n] = 0.f;
            if (tt < end - first && j < a.dv) {
                if (a.dout.data) g[n] = ldf(a.dout, b, t, h, j);
                o[n] = a.fwd_out[token(a, b, t, h) * a.dv + j];
            }
        }
#pragma unroll
        for (int n = 0; n < PER; ++n) {
            const int idx = tid + kReadThreads * n, tt = idx / DV, j = idx % DV;
            GT[j][query_slot(tt)] = g[n];
            O[tt][j] = o[n];
        }
        if (tid < 2 * kMaxChunk) {
            const int tt = tid >> 1, t = first + tt;
            stat[tt][tid & 1] = tt < end - first ? a.stats[2 * token(a, b, t, h) + (tid & 1)] : 0.f;
        }
    }
    __syncthreads();
    // Raw logits and dO . v for every (query, slot) on MFMA.
    chunk_xyt<DK, DK + 4>(s.QT, &s.K[0][0], slots, wave, L);
    chunk_xyt<DV, DV + 4>(GT, &s.V[0][0], slots, wave, Dt);
    const float sink = ldf(a.sink, h);
    const WaveQueries w = wave_queries(s, wave, first, end - first);
    float delta[kWaveQueries], m[kWaveQueries], inv[kWaveQueries];
#pragma unroll
    for (int u = 0; u < kWaveQueries; ++u) {
        const int tt = wave + kReadWaves * u;
        float dl = 0.f;
        if (w.act[u])
            for (int j = lane; j < DV; j += 64) dl += GT[j][query_slot(tt)] * O[tt][j];
        delta[u] = wave_sum(dl);
        m[u] = w.on[u] ? stat[tt][0] : 0.f;
        inv[u] = w.on[u] ? stat[tt][1] : 0.f;
    }
    if (lane == 0) {
#pragma unroll
        for (int u = 0; u < kWaveQueries; ++u) {
            if (!w.on[u]) continue;
            const int64_t tok = token(a, b, w.t[u], h);
            a.aux[2 * tok] = delta[u];
            a.aux[2 * tok + 1] = w.act[u] ? -delta[u] * expf(sink - m[u]) * inv[u] : 0.f;
        }
    }
    __syncthreads();
    // Per slot (lanes): p and the logit gradient d = p (dO . v - delta) / sqrt(d_k),
    // saved as pairs; the wave's rows of L take d (zero past the slots).
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int j = lane + 64 * r;
        if (j >= kMaxSlots) continue;
#pragma unroll
        for (int u = 0; u < kWaveQueries; ++u) {
            const float lgv = visible_logit(a, s, w, L, wave, u, j, slots);
            const float p = lgv > -FLT_MAX ? expf(lgv - m[u]) * inv[u] : 0.f;
            const float d = lgv > -FLT_MAX ? p * (Dt[4 * wave + u][j] - delta[u]) * a.scale : 0.f;
            if (w.on[u] && j < slots)
                reinterpret_cast<float2 *>(a.pairs)[token(a, b, w.t[u], h) * slots + j] = make_float2(p, d);
            L[4 * wave + u][j] = d;
        }
    }
    __syncthreads();
    chunk_py<DK, DK + 4>(a, L, &s.K[0][0], slots, wave, b, h, first, end - first, s.tval, a.dk, a.gq);
}

template <int DK, int DV>
__global__ void __launch_bounds__(64) hola_key_backward_kernel(HolaArgs a) {
    constexpr int RK = (DK + 63) / 64, RV = (DV + 63) / 64;
    __shared__ int map[kMaxChunk];
    __shared__ float Q[kMaxChunk][DK], G[kMaxChunk][DV];
    __shared__ float2 PD[kMaxChunk][kMaxChunk];  // (probability, logit gradient) [query][key]
    __shared__ float qpos[kMaxChunk];
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
    float lastf = (float)end;
    if (lane < n) lastf = fmaxf(lastf, a.expiry[token(a, b, first + lane, h)]);
    const int last = (int)wave_max(lastf);
    for (int cq = c; cq * a.chunk < last; ++cq) {
        const int q0 = cq * a.chunk, q1 = min(q0 + a.chunk, a.T), nq = q1 - q0;
        // Where this chunk's keys sit among the slots of query chunk cq.
        if (lane < kMaxChunk) {
            map[lane] = -1;
            qpos[lane] = lane < nq ? (float)(q0 + lane) : -1.f;
        }
        __syncthreads();
        if (cq == c) {
            if (lane < n) map[lane] = a.cap + lane;
        } else if (lane < a.cap) {
            const float p = sched[(int64_t)cq * a.cap + lane];
            if (p >= (float)first && p < (float)end) map[(int)p - first] = lane;
        }
        __syncthreads();
        // The chunk's queries, output adjoints and the pairs of the mapped slots.
        gather_rows<DK, DK, kMaxChunk>(a.q, b, h, a.dk, qpos, kMaxChunk, &Q[0][0]);
        if (a.dout.data) gather_rows<DV, DV, kMaxChunk>(a.dout, b, h, a.dv, qpos, kMaxChunk, &G[0][0]);
        else
            for (int idx = lane; idx < kMaxChunk * DV; idx += 64) G[idx / DV][idx % DV] = 0.f;
        {
            constexpr int PER = kMaxChunk * kMaxChunk / 64;
            float2 r[PER];
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int idx = lane + 64 * u, tq = idx / kMaxChunk, j = idx % kMaxChunk;
                const int sl = map[j];
                r[u] = make_float2(0.f, 0.f);
                if (tq < nq && sl >= 0)
                    r[u] = reinterpret_cast<const float2 *>(a.pairs)[token(a, b, q0 + tq, h) * slots + sl];
            }
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int idx = lane + 64 * u;
                PD[idx / kMaxChunk][idx % kMaxChunk] = r[u];
            }
        }
        __syncthreads();
        for (int tq = 0; tq < nq; ++tq) {
            float qv[RK], gv[RV];
#pragma unroll
            for (int r = 0; r < RK; ++r) qv[r] = lane + 64 * r < DK ? Q[tq][lane + 64 * r] : 0.f;
#pragma unroll
            for (int r = 0; r < RV; ++r) gv[r] = lane + 64 * r < DV ? G[tq][lane + 64 * r] : 0.f;
#pragma unroll
            for (int j = 0; j < kMaxChunk; ++j) {
                const float2 pd = PD[tq][j];
#pragma unroll
                for (int r = 0; r < RK; ++r) dka[j][r] += pd.y * qv[r];
#pragma unroll
                for (int r = 0; r < RV; ++r) dva[j][r] += pd.x * gv[r];
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
        hipLaunchKernelGGL((K<P, Q>::fn), grid, dim3(K<P, Q>::threads), 0, st, a); \
        return;                                                                 \
    }
    GDN2_HOLA_CASE(32, 32) GDN2_HOLA_CASE(32, 64) GDN2_HOLA_CASE(32, 128)
    GDN2_HOLA_CASE(64, 32) GDN2_HOLA_CASE(64, 64) GDN2_HOLA_CASE(64, 128)
    GDN2_HOLA_CASE(128, 32) GDN2_HOLA_CASE(128, 64) GDN2_HOLA_CASE(128, 128)
#undef GDN2_HOLA_CASE
}
template <int P, int Q> struct Fwd {
    static constexpr auto fn = hola_forward_kernel<P, Q>;
    static constexpr int threads = kReadThreads;
};
template <int P, int Q> struct QBwd {
    static constexpr auto fn = hola_query_backward_kernel<P, Q>;
    static constexpr int threads = kReadThreads;
};
template <int P, int Q> struct KBwd {
    static constexpr auto fn = hola_key_backward_kernel<P, Q>;
    static constexpr int threads = 64;
};

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
