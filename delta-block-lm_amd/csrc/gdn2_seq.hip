// Token-sequential GDN-2 scan for gfx950: the general channel-wise surface.
//
// Semantics follow crates/mixers/src/reference.rs:41-257 (forward and VJP),
// the stateful fused kernels crates/kernels/src/gdn_training.rs:12-284 and,
// with document limits, the forward of crates/mixers/src/gdn2_reference.rs:51-103
// (a token is live when end >= start and resets the state when start == t)
// with the exact VJP of that forward, as the reference's chunked kernels
// compute it (crates/kernels/src/gdn2.rs:24-65, :288-490): the adjoint never
// crosses a reset.
//
// One workgroup per (batch, head).  Value columns evolve independently in the
// recurrence, so each wave owns a block of value columns and walks the tokens
// without workgroup barriers; only the per-key gradients of the backward are
// summed across waves.
//
// Forward: thread tid owns value column j = tid / NG and the KR = 16 key rows
//   i0 = (tid % NG) * 16 .. i0 + 15 of the fp32 state (NG = K_pad / 16
//   adjacent lanes per column), so the two per-token key reductions (the edit
//   delta and the output) are DPP butterflies over NG lanes.
// Backward: lane l of wave w owns key rows RL*(l/4) .. +RL-1 (RL = K_pad/16)
//   and value columns 16w + 4(l%4) .. +3.  The edit adjoint (a sum over keys)
//   is four local terms per column plus a sum over the 16 lanes of one column
//   quad position; the per-key gradients (sums over value columns) are four
//   local terms plus a quad butterfly.  Each wave leaves its per-key partials
//   of FT tokens in LDS, and the workgroup sums them over waves and stores
//   dq/dk/dalpha/derase once per FT tokens.
//
// Token inputs are staged through LDS SEQ_CT tokens at a time.  The next
// block's global loads are issued before the current block's token loop and
// written to LDS after it, so their latency hides behind the loop.
//
// Checkpoints: the forward stores the state at the start of every block
// (row-major fp32), the edit delta of every token and the norms |k|, |delta|.
// The backward walks blocks in reverse and replays a block from its
// checkpoint with the forward's own deltas (the same rounded operations, so
// the replayed states are the forward's), keeping the pre-token states in a
// thread-major scratch area that the reverse token loop reads one token
// ahead.
#include "gdn2_seq.h"

namespace gdn2 {

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the NG adjacent lanes of a key group (NG = 2, 4 or 8), in all of
// them: DPP quad swaps, then the half-row mirror pairs the two quads.
template <int NG>
__device__ __forceinline__ float group_sum(float x) {
    x = dpp_add<0xB1>(x);                  // lane ^ 1
    if (NG >= 4) x = dpp_add<0x4E>(x);     // lane ^ 2
    if (NG >= 8) x = dpp_add<0x141>(x);    // quad <-> quad within 8 lanes
    return x;
}

// Sum over the 16 lanes of a DPP row, in all of them.
__device__ __forceinline__ float row16_sum(float x) {
    return dpp_add<0x140>(group_sum<8>(x));  // row mirror pairs the two halves
}

// x[l] + x[l ^ 16] and x[l] + x[l ^ 32] in every lane: a permlane swap of x
// with itself returns both halves of each pair.  Each result element is
// copied into a plain int before the bit cast: bit-casting an element of the
// returned vector directly reads element 0.
__device__ __forceinline__ float pair_sum(int a, int b) {
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap16_sum(float x) {
    const int i = __builtin_bit_cast(int, x);
    const auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    const int r0 = r[0], r1 = r[1];
    return pair_sum(r0, r1);
}
__device__ __forceinline__ float swap32_sum(float x) {
    const int i = __builtin_bit_cast(int, x);
    const auto r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    const int r0 = r[0], r1 = r[1];
    return pair_sum(r0, r1);
}

// x[l ^ 4]: the half-row mirror (l -> 7 - l) followed by a reversed quad.
__device__ __forceinline__ float xor4(float x) {
    const int m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false));
}

// Sum over the lanes of a wave congruent to this lane modulo S (S = 4 or 8),
// in all of them, as a balanced pairwise tree over the lane index (lane ^ 4
// for S = 4, then lane ^ 8 by a half-row rotation, then permlane swaps for
// lane ^ 16 and lane ^ 32).  Every step pairs two lanes symmetrically, so all
// the lanes of a group get bit-identical sums.
template <int S>
__device__ __forceinline__ float stride_sum(float x) {
    static_assert(S == 4 || S == 8, "stride");
    if (S == 4) x = x + xor4(x);
    x = dpp_add<0x128>(x);  // row_ror 8 == lane ^ 8
    return swap32_sum(swap16_sum(x));
}

// Balanced pairwise sum of p[0..N) in index order: the order in which the
// lane trees above combine row groups (pairs g ^ 1, then g ^ 2, ...).
template <int N>
__device__ __forceinline__ float tree_sum(float (&p)[N]) {
#pragma unroll
    for (int w = 1; w < N; w *= 2)
#pragma unroll
        for (int i = 0; i < N; i += 2 * w) p[i] = p[i] + p[i + w];
    return p[0];
}

template <int N>
__device__ __forceinline__ void lds_get(const float *p, float (&x)[N]) {
    static_assert(N % 2 == 0, "even runs");
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int m = 0; m < N; m += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(p + m);
            x[m] = v.x, x[m + 1] = v.y, x[m + 2] = v.z, x[m + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int m = 0; m < N; m += 2) {
            const float2 v = *reinterpret_cast<const float2 *>(p + m);
            x[m] = v.x, x[m + 1] = v.y;
        }
    }
}

template <int N>
__device__ __forceinline__ void lds_put(float *p, const float (&x)[N]) {
    static_assert(N % 2 == 0, "even runs");
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int m = 0; m < N; m += 4)
            *reinterpret_cast<float4 *>(p + m) = make_float4(x[m], x[m + 1], x[m + 2], x[m + 3]);
    } else {
#pragma unroll
        for (int m = 0; m < N; m += 2)
            *reinterpret_cast<float2 *>(p + m) = make_float2(x[m], x[m + 1]);
    }
}

template <typename TIN>
__device__ __forceinline__ void store_in(void *p, int64_t i, float x) {
    Elem<TIN>::store(p, i, x);
}

// One thread's share of a block of SEQ_CT tokens, held in registers between
// the global loads and the LDS stores.  Element n of an array is flat index
// tid + n * NT of the block's [SEQ_CT][width] tile.  The registers hold the
// raw loaded bits (bf16 inputs zero-extended): every conversion, exponential
// and flag test happens at the LDS store, so nothing waits for the loads
// until then.
template <int KP, int VP, int NT, bool BWD>
struct TokenRegs {
    static constexpr int NK = SEQ_CT * KP / NT, NV = SEQ_CT * VP / NT;
    static_assert(NK * NT == SEQ_CT * KP && NV * NT == SEQ_CT * VP, "block split");
    uint32_t q[NK], k[NK], a[NK], e[NK];
    uint32_t v[NV], w[NV];
    uint32_t dy[BWD ? NV : 1], d[BWD ? NV : 1];
    // Per-token words (threads tid < SEQ_CT): doc limits (start, end) or the
    // valid/reset masks; dscores and the forward's |k|, |delta|.
    uint32_t f0, f1, sa, nk, nd;
    bool in;
};

template <typename T>
__device__ __forceinline__ float raw_f(uint32_t r) {
    if constexpr (sizeof(T) == 2) return __uint_as_float(r << 16);
    else return __uint_as_float(r);
}

constexpr uint32_t NEG_INF_BITS = 0xff800000u;
constexpr uint32_t ONE_BITS = 0x3f800000u;

// One input of a (batch, head): element (t, c) at p[t * st + c * sc] (sc = 0
// broadcasts a per-token value over the channels).  Built once per
// workgroup, so the block loads carry two strides per input instead of the
// whole view.
struct Stream {
    const char *p;
    int64_t st, sc;
};

__device__ __forceinline__ Stream make_stream(const View &v, int b, int h, int esize,
                                              bool broadcast = false) {
    if (!v.data) return Stream{nullptr, 0, 0};
    return Stream{static_cast<const char *>(v.data) + ((int64_t)b * v.s0 + (int64_t)h * v.s2) * esize,
                  v.s1, broadcast ? 0 : v.s3};
}

// Token inputs of one (batch, head): q, k, the key gates a (alpha, or g in
// scalar mode) and e (erase, or beta), v, the write gate w (write, or beta),
// the output adjoint dy, and the per-token words f0/f1 (valid/reset masks,
// or the document limits start/end).
struct TokenSrc {
    Stream q, k, a, e, v, w, dy, f0, f1;
};

template <typename TIN>
__device__ __forceinline__ TokenSrc make_src(const SeqArgs &a, int b, int h) {
    TokenSrc s;
    s.q = make_stream(a.q, b, h, sizeof(TIN));
    s.k = make_stream(a.k, b, h, sizeof(TIN));
    s.a = a.scalar ? make_stream(a.g, b, h, 4, true) : make_stream(a.alpha, b, h, 4);
    s.e = a.scalar ? make_stream(a.beta, b, h, 4, true) : make_stream(a.erase, b, h, 4);
    s.v = make_stream(a.v, b, h, sizeof(TIN));
    s.w = a.scalar ? make_stream(a.beta, b, h, 4, true) : make_stream(a.write, b, h, 4);
    s.dy = make_stream(a.dout, b, h, sizeof(TIN));
    const View &f0 = a.doc ? a.doc_start : a.valid, &f1 = a.doc ? a.doc_end : a.reset;
    s.f0 = f0.data ? Stream{static_cast<const char *>(f0.data) + (int64_t)b * f0.s0 * 4, f0.s1, 0}
                   : Stream{nullptr, 0, 0};
    s.f1 = f1.data ? Stream{static_cast<const char *>(f1.data) + (int64_t)b * f1.s0 * 4, f1.s1, 0}
                   : Stream{nullptr, 0, 0};
    return s;
}

template <typename T>
__device__ __forceinline__ uint32_t ld_s(const Stream &s, int64_t t, int64_t c) {
    const int64_t i = t * s.st + c * s.sc;
    if constexpr (sizeof(T) == 2) return reinterpret_cast<const uint16_t *>(s.p)[i];
    else return reinterpret_cast<const uint32_t *>(s.p)[i];
}

// The per-workgroup scalars the block loads need besides the streams.
struct BlockCtx {
    int T, K, V, scalar, doc, H, b, h, bh;
    int64_t tp;
    const float *ck_delta, *ck_norm, *dscores;
};

__device__ __forceinline__ BlockCtx make_ctx(const SeqArgs &a, int b, int h, int bh) {
    return BlockCtx{a.T, a.K, a.V, a.scalar, a.doc, a.H, b, h, bh, (int64_t)a.nck * SEQ_CT,
                    a.ck_delta, a.ck_norm, a.dscores};
}

template <int KP, int VP, int NT, bool BWD, typename TIN>
__device__ __forceinline__ void load_tokens(const TokenSrc &src, const BlockCtx &x, int t0, int tid,
                                            TokenRegs<KP, VP, NT, BWD> &r) {
    using R = TokenRegs<KP, VP, NT, BWD>;
    // A thread's elements of a [SEQ_CT][width] tile share one channel and step
    // through the tokens NT / width apart.
    constexpr int KS = NT / KP, VS = NT / VP;
    static_assert(KS * KP == NT && VS * VP == NT, "token-major split");
    const int ck = tid % KP, tk = t0 + tid / KP, cv = tid % VP, tv = t0 + tid / VP;
#pragma unroll
    for (int n = 0; n < R::NK; ++n) {
        const int t = tk + n * KS;
        r.q[n] = r.k[n] = r.e[n] = 0u;
        r.a[n] = x.scalar ? NEG_INF_BITS : 0u;  // exp(-inf) = 0 beyond the sequence
        if (t < x.T && ck < x.K) {
            r.q[n] = ld_s<TIN>(src.q, t, ck);
            r.k[n] = ld_s<TIN>(src.k, t, ck);
            r.a[n] = ld_s<float>(src.a, t, ck);
            r.e[n] = ld_s<float>(src.e, t, ck);
        }
    }
#pragma unroll
    for (int n = 0; n < R::NV; ++n) {
        const int t = tv + n * VS;
        r.v[n] = r.w[n] = 0u;
        if constexpr (BWD) r.dy[n] = r.d[n] = 0u;
        if (t < x.T && cv < x.V) {
            r.v[n] = ld_s<TIN>(src.v, t, cv);
            r.w[n] = ld_s<float>(src.w, t, cv);
            if constexpr (BWD) {
                if (src.dy.p) r.dy[n] = ld_s<TIN>(src.dy, t, cv);
                r.d[n] = __float_as_uint(x.ck_delta[((int64_t)x.bh * x.tp + t) * VP + cv]);
            }
        }
    }
    const int t = t0 + tid;
    r.in = tid < SEQ_CT && t < x.T;
    r.f0 = x.doc ? 0u : ONE_BITS;
    r.f1 = r.sa = r.nk = r.nd = 0u;
    if (r.in) {
        if (src.f0.p) r.f0 = ld_s<float>(src.f0, t, 0);
        if (src.f1.p) r.f1 = ld_s<float>(src.f1, t, 0);
        if constexpr (BWD) {
            if (x.dscores) r.sa = __float_as_uint(x.dscores[((int64_t)x.b * x.T + t) * x.H + x.h]);
            r.nk = __float_as_uint(x.ck_norm[((int64_t)x.bh * x.tp + t) * 2]);
            r.nd = __float_as_uint(x.ck_norm[((int64_t)x.bh * x.tp + t) * 2 + 1]);
        }
    }
}

// Token flags (valid, reset) from a thread's per-token words.
template <int KP, int VP, int NT, bool BWD>
__device__ __forceinline__ void token_flags(const SeqArgs &a, const TokenRegs<KP, VP, NT, BWD> &r,
                                            int t, float &val, float &rst) {
    val = rst = 0.f;
    if (!r.in) return;
    if (a.doc) {
        const int32_t st = (int32_t)r.f0, en = (int32_t)r.f1;
        val = en >= st ? 1.f : 0.f;
        rst = st == t ? 1.f : 0.f;
    } else {
        val = __uint_as_float(r.f0);
        rst = __uint_as_float(r.f1);
    }
}

// ---- forward ---------------------------------------------------------------------

// Forward lane tile: RL key rows x CL value columns per lane, RGN row groups
// and CLN column lanes per wave (16 value columns per wave).  Eight row groups
// keep the per-token LDS reads of the key-side rows (a, e.k, k, q) at
// 4 RL floats per lane while the key sums stay three lane steps deep.
template <int KP>
struct FwdLayout {
    static constexpr int RGN = KP <= 64 ? 8 : 16;
    static constexpr int RL = KP / RGN;
    static constexpr int CLN = 64 / RGN;
    static constexpr int CL = 16 / CLN;
};

template <int KP, int VP>
struct FwdTokens {
    float q[SEQ_CT][KP], k[SEQ_CT][KP], a[SEQ_CT][KP], ek[SEQ_CT][KP];
    float wv[SEQ_CT][VP];
    float val[SEQ_CT], rst[SEQ_CT];
};

template <int KP, int VP>
struct alignas(16) SeqFwdSmem {
    FwdTokens<KP, VP> buf[2];
    float o[SEQ_CT][VP], d[SEQ_CT][VP];
};

template <int KP, int VP>
union SeqFwdShared {
    SeqFwdSmem<KP, VP> s;
    float st[KP * (VP + 1)];  // state transpose slab (row stride VP+1)
};

// Stage a block for the forward in two passes (a barrier between them): the
// token flags, then the operands with padding and resets folded in, so the
// token loop has no branches.  A padded token (or one beyond the sequence)
// gets a = 1 and zero e.k, k, q and w.v: the state passes unchanged and its
// edit and output are zero.  A reset token gets a = 0, which zeroes the
// carried state before the edit.
template <int KP, int VP, int NT, typename TIN>
__device__ __forceinline__ void store_fwd_flags(const SeqArgs &a,
                                                const TokenRegs<KP, VP, NT, false> &r,
                                                FwdTokens<KP, VP> &s, int t0, int tid) {
    if (tid < SEQ_CT) {
        float val, rst;
        token_flags(a, r, t0 + tid, val, rst);
        s.val[tid] = val;
        s.rst[tid] = rst;
    }
}

template <int KP, int VP, int NT, typename TIN>
__device__ __forceinline__ void store_fwd_data(const SeqArgs &a,
                                               const TokenRegs<KP, VP, NT, false> &r,
                                               FwdTokens<KP, VP> &s, int tid) {
    using R = TokenRegs<KP, VP, NT, false>;
#pragma unroll
    for (int n = 0; n < R::NK; ++n) {
        const int idx = tid + n * NT, tt = idx / KP, c = idx % KP;
        const bool on = s.val[tt] != 0.f, rs = s.rst[tt] != 0.f;
        const float kf = raw_f<TIN>(r.k[n]), af = __uint_as_float(r.a[n]);
        s.q[tt][c] = on ? raw_f<TIN>(r.q[n]) : 0.f;
        s.k[tt][c] = on ? kf : 0.f;
        s.a[tt][c] = on ? (rs ? 0.f : (a.scalar ? expf(af) : af)) : 1.f;
        s.ek[tt][c] = on ? __uint_as_float(r.e[n]) * kf : 0.f;
    }
#pragma unroll
    for (int n = 0; n < R::NV; ++n) {
        const int idx = tid + n * NT, tt = idx / VP, c = idx % VP;
        s.wv[tt][c] = s.val[tt] != 0.f ? __uint_as_float(r.w[n]) * raw_f<TIN>(r.v[n]) : 0.f;
    }
}

// One token's operands for a forward lane.
template <int RL, int CL>
struct FwdTok {
    float a[RL], ek[RL], k[RL], q[RL], wv[CL];
};

template <int KP, int VP, int RL, int CL>
__device__ __forceinline__ void fetch_fwd(const FwdTokens<KP, VP> &B, int tt, int r0, int c0,
                                          FwdTok<RL, CL> &x) {
    lds_get<RL>(&B.a[tt][r0], x.a);
    lds_get<RL>(&B.ek[tt][r0], x.ek);
    lds_get<RL>(&B.k[tt][r0], x.k);
    lds_get<RL>(&B.q[tt][r0], x.q);
    lds_get<CL>(&B.wv[tt][c0], x.wv);
}

#pragma clang fp contract(off)
template <int KP, int VP, typename TIN>
__global__ void __launch_bounds__(4 * VP) seq_fwd_kernel(SeqArgs a) {
    using L = FwdLayout<KP>;
    constexpr int RL = L::RL, CL = L::CL, CLN = L::CLN, NT = 4 * VP, CT = SEQ_CT;
    __shared__ SeqFwdShared<KP, VP> sh;
    SeqFwdSmem<KP, VP> &s = sh.s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rg = lane / CLN, cl = lane % CLN;
    const int r0 = RL * rg, c0 = 16 * w + CL * cl;  // first key row / value column of this lane
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int64_t tp = (int64_t)a.nck * CT;

    // Initial state, coalesced through the transpose slab.
    for (int idx = tid; idx < KP * VP; idx += NT) {
        const int i = idx / VP, c = idx % VP;
        sh.st[i * (VP + 1) + c] = (a.initial.data && i < a.K && c < a.V)
                                      ? ld4<float>(a.initial, b, h, i, c)
                                      : 0.f;
    }
    __syncthreads();
    float S[RL][CL];
#pragma unroll
    for (int ri = 0; ri < RL; ++ri)
#pragma unroll
        for (int cj = 0; cj < CL; ++cj) S[ri][cj] = sh.st[(r0 + ri) * (VP + 1) + c0 + cj];
    __syncthreads();

    const TokenSrc src = make_src<TIN>(a, b, h);
    const BlockCtx ctx = make_ctx(a, b, h, bh);
    TokenRegs<KP, VP, NT, false> nx;
    load_tokens<KP, VP, NT, false, TIN>(src, ctx, 0, tid, nx);
    store_fwd_flags<KP, VP, NT, TIN>(a, nx, s.buf[0], 0, tid);
    __syncthreads();
    store_fwd_data<KP, VP, NT, TIN>(a, nx, s.buf[0], tid);
    __syncthreads();

    for (int blk = 0; blk < a.nck; ++blk) {
        const int t0 = blk * CT, nt = min(CT, a.T - t0);
        const FwdTokens<KP, VP> &B = s.buf[blk & 1];
        if (a.ck) {
            float *ck = a.ck + ((int64_t)bh * a.nck + blk) * KP * VP;
#pragma unroll
            for (int ri = 0; ri < RL; ++ri) lds_put<CL>(ck + (r0 + ri) * VP + c0, S[ri]);
        }
        if (blk + 1 < a.nck) load_tokens<KP, VP, NT, false, TIN>(src, ctx, t0 + CT, tid, nx);
        // One token: S <- a S, delta = w v - S^T (e k), S += k delta^T,
        // o = S^T q.  Key sums keep two partial chains per column.
        auto step = [&](int tt, const FwdTok<RL, CL> &x) {
            float p0[CL], p1[CL], delta[CL], o[CL];
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) p0[cj] = p1[cj] = 0.f;
#pragma unroll
            for (int ri = 0; ri < RL; ++ri)
#pragma unroll
                for (int cj = 0; cj < CL; ++cj) {
                    S[ri][cj] = S[ri][cj] * x.a[ri];
                    if (ri & 1) p1[cj] = __builtin_fmaf(x.ek[ri], S[ri][cj], p1[cj]);
                    else p0[cj] = __builtin_fmaf(x.ek[ri], S[ri][cj], p0[cj]);
                }
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) {
                delta[cj] = x.wv[cj] - stride_sum<CLN>(p0[cj] + p1[cj]);
                p0[cj] = p1[cj] = 0.f;
            }
#pragma unroll
            for (int ri = 0; ri < RL; ++ri)
#pragma unroll
                for (int cj = 0; cj < CL; ++cj) {
                    S[ri][cj] = __builtin_fmaf(x.k[ri], delta[cj], S[ri][cj]);
                    if (ri & 1) p1[cj] = __builtin_fmaf(x.q[ri], S[ri][cj], p1[cj]);
                    else p0[cj] = __builtin_fmaf(x.q[ri], S[ri][cj], p0[cj]);
                }
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) o[cj] = stride_sum<CLN>(p0[cj] + p1[cj]);
            // Every row group holds the same sums; all lanes store them.
            lds_put<CL>(&s.o[tt][c0], o);
            lds_put<CL>(&s.d[tt][c0], delta);
        };
        if (nt == CT) {
            // A full block: straight-line code, two operand sets in turn so the
            // next token's LDS reads overlap this one.
            FwdTok<RL, CL> x[2];
            fetch_fwd<KP, VP, RL, CL>(B, 0, r0, c0, x[0]);
#pragma unroll
            for (int tt = 0; tt < CT; ++tt) {
                if (tt + 1 < CT) fetch_fwd<KP, VP, RL, CL>(B, tt + 1, r0, c0, x[(tt + 1) & 1]);
                step(tt, x[tt & 1]);
            }
        } else {  // the sequence's last, partial block (and decode steps)
            for (int tt = 0; tt < nt; ++tt) {
                FwdTok<RL, CL> x;
                fetch_fwd<KP, VP, RL, CL>(B, tt, r0, c0, x);
                step(tt, x);
            }
        }
        __syncthreads();
        // Stage the next block first: its loads are the oldest memory
        // operations still in flight, so waiting for them does not wait for
        // this block's output stores.
        if (blk + 1 < a.nck) {
            store_fwd_flags<KP, VP, NT, TIN>(a, nx, s.buf[(blk + 1) & 1], t0 + CT, tid);
            __syncthreads();
            store_fwd_data<KP, VP, NT, TIN>(a, nx, s.buf[(blk + 1) & 1], tid);
        }
        for (int idx = tid; idx < CT * VP; idx += NT) {
            const int tt = idx / VP, c = idx % VP;
            if (tt < nt) {
                if (c < a.V)
                    store_out(a.out, a.out_bf16, (((int64_t)b * a.T + t0 + tt) * a.H + h) * a.V + c,
                              s.o[tt][c]);
                if (a.ck) a.ck_delta[((int64_t)bh * tp + t0 + tt) * VP + c] = s.d[tt][c];
            }
        }
        // Scores |k| |delta| (zero on padding) and the checkpoint norms: one
        // 16-lane row per token.
        for (int tt = tid >> 4; tt < CT; tt += NT / 16) {
            const int l = tid & 15;
            float kk = 0.f, dd = 0.f;
            for (int c = l; c < KP; c += 16) kk = __builtin_fmaf(B.k[tt][c], B.k[tt][c], kk);
            for (int c = l; c < VP; c += 16) dd = __builtin_fmaf(s.d[tt][c], s.d[tt][c], dd);
            kk = row16_sum(kk);
            dd = row16_sum(dd);
            if (l == 0 && tt < nt) {
                const int t = t0 + tt;
                if (a.scores)
                    a.scores[((int64_t)b * a.T + t) * a.H + h] = B.val[tt] != 0.f ? sqrtf(kk * dd) : 0.f;
                if (a.ck) {
                    a.ck_norm[((int64_t)bh * tp + t) * 2] = sqrtf(kk);
                    a.ck_norm[((int64_t)bh * tp + t) * 2 + 1] = sqrtf(dd);
                }
            }
        }
        __syncthreads();
    }
    // Final state through the transpose slab.
#pragma unroll
    for (int ri = 0; ri < RL; ++ri)
#pragma unroll
        for (int cj = 0; cj < CL; ++cj) sh.st[(r0 + ri) * (VP + 1) + c0 + cj] = S[ri][cj];
    __syncthreads();
    if (a.final_state)
        for (int idx = tid; idx < a.K * a.V; idx += NT) {
            const int i = idx / a.V, c = idx % a.V;
            a.final_state[(int64_t)bh * a.K * a.V + idx] = sh.st[i * (VP + 1) + c];
        }
}
#pragma clang fp contract(on)

// ---- backward --------------------------------------------------------------------

template <int KP, int VP>
struct SeqBwdCfg {
    static constexpr int CL = VP == 128 ? 4 : 2;  // value columns per lane
    static constexpr int NW = VP / (4 * CL);      // waves (16 row groups x 4 column lanes)
    static constexpr int NT = 64 * NW;
    static constexpr int RL = KP / 16;            // key rows per lane
    static constexpr int FT0 = 4096 / (NW * KP);
    static constexpr int FT = FT0 >= SEQ_CT ? SEQ_CT : FT0;  // tokens per cross-wave sum
    static constexpr int RP = KP + 4;   // partial-sum row pitch (spreads LDS banks)
    // Up to 64 key rows the registers hold the next block's checkpoint and the
    // next token's LDS operands as well.
    static constexpr bool AHEAD = RL <= 4;
    static_assert(SEQ_CT % FT == 0, "flush groups tile a block");
};

template <int KP, int VP>
struct alignas(16) SeqBwdSmem {
    using Cfg = SeqBwdCfg<KP, VP>;
    float q[SEQ_CT][KP], k[SEQ_CT][KP], a[SEQ_CT][KP], e[SEQ_CT][KP];
    float v[SEQ_CT][VP], w[SEQ_CT][VP], dy[SEQ_CT][VP], d[SEQ_CT][VP];
    float dd[SEQ_CT][VP];  // edit adjoint of every token (zero on padding)
    float val[SEQ_CT], rst[SEQ_CT], cs[SEQ_CT], ks[SEQ_CT];
    // red[slot][wave][quantity][key]: per-wave sums over the wave's value
    // columns of the q-gradient, adj.delta, bar.ddelta and dalpha terms.
    float red[Cfg::FT][Cfg::NW][4][Cfg::RP];
};

// Stage a block for the backward in two passes (a barrier between them): the
// per-token flags and score-VJP coefficients, then the operands.  Padded
// tokens get a = 1 and zero q, k, e, dy (their delta is zero): the adjoint
// passes unchanged and every gradient but dalpha comes out zero (the flush
// zeroes dalpha).  A reset token gets a = 0, which cuts the adjoint.
template <int KP, int VP, int NT, typename TIN>
__device__ __forceinline__ void store_bwd_flags(const SeqArgs &a,
                                                const TokenRegs<KP, VP, NT, true> &r,
                                                SeqBwdSmem<KP, VP> &s, int t0, int tid) {
    if (tid < SEQ_CT) {
        float val, rst;
        token_flags(a, r, t0 + tid, val, rst);
        s.val[tid] = val;
        s.rst[tid] = rst;
        // Score VJP (zero subgradient at |k| |delta| = 0): ddelta += cs delta,
        // dk += ks k.
        const float sa = __uint_as_float(r.sa), nk = __uint_as_float(r.nk), nd = __uint_as_float(r.nd);
        const bool ok = val != 0.f && nk > 0.f && nd > 0.f;
        s.cs[tid] = ok ? sa * nk / nd : 0.f;
        s.ks[tid] = ok ? sa * nd / nk : 0.f;
    }
}

template <int KP, int VP, int NT, typename TIN>
__device__ __forceinline__ void store_bwd_data(const SeqArgs &a,
                                               const TokenRegs<KP, VP, NT, true> &r,
                                               SeqBwdSmem<KP, VP> &s, int tid) {
    using R = TokenRegs<KP, VP, NT, true>;
#pragma unroll
    for (int n = 0; n < R::NK; ++n) {
        const int idx = tid + n * NT, tt = idx / KP, c = idx % KP;
        const bool on = s.val[tt] != 0.f, cut = s.rst[tt] != 0.f;
        const float af = __uint_as_float(r.a[n]);
        s.q[tt][c] = on ? raw_f<TIN>(r.q[n]) : 0.f;
        s.k[tt][c] = on ? raw_f<TIN>(r.k[n]) : 0.f;
        s.a[tt][c] = on ? (cut ? 0.f : (a.scalar ? expf(af) : af)) : 1.f;
        s.e[tt][c] = on ? __uint_as_float(r.e[n]) : 0.f;
    }
#pragma unroll
    for (int n = 0; n < R::NV; ++n) {
        const int idx = tid + n * NT, tt = idx / VP, c = idx % VP;
        const bool on = s.val[tt] != 0.f;
        s.v[tt][c] = raw_f<TIN>(r.v[n]);
        s.w[tt][c] = __uint_as_float(r.w[n]);
        s.dy[tt][c] = on ? raw_f<TIN>(r.dy[n]) : 0.f;
        s.d[tt][c] = __uint_as_float(r.d[n]);
    }
}

template <int KP, int VP, int RL, int CL>
__device__ __forceinline__ void load_ck(const SeqArgs &a, int bh, int blk, int r0, int c0,
                                        float (&S)[RL][CL]) {
    const float *ck = a.ck + ((int64_t)bh * a.nck + blk) * KP * VP;
#pragma unroll
    for (int ri = 0; ri < RL; ++ri) lds_get<CL>(ck + (r0 + ri) * VP + c0, S[ri]);
}

// One token's operands for a backward lane.
template <int RL, int CL>
struct BwdTok {
    float q[RL], k[RL], a[RL], e[RL], dy[CL], d[CL];
    float cs;
};

template <int KP, int VP, int RL, int CL>
__device__ __forceinline__ void fetch_bwd(const SeqBwdSmem<KP, VP> &s, int tt, int r0, int c0,
                                          BwdTok<RL, CL> &x) {
    lds_get<RL>(&s.q[tt][r0], x.q);
    lds_get<RL>(&s.k[tt][r0], x.k);
    lds_get<RL>(&s.a[tt][r0], x.a);
    lds_get<RL>(&s.e[tt][r0], x.e);
    lds_get<CL>(&s.dy[tt][c0], x.dy);
    lds_get<CL>(&s.d[tt][c0], x.d);
    x.cs = s.cs[tt];
}

// Sum the per-wave partials of tokens g0 .. g0+FT-1 (those below nt) and
// store dq, dk, dalpha, derase, dv, dwrite; scalar-gate mode keeps derase and
// dalpha in the consumed e/a rows of LDS for the per-token chain rule.
template <int KP, int VP, typename TIN>
__device__ __forceinline__ void flush_group(const SeqArgs &a, SeqBwdSmem<KP, VP> &s, int b, int h,
                                            int t0, int g0, int nt, int tid) {
    using Cfg = SeqBwdCfg<KP, VP>;
    for (int idx = tid; idx < Cfg::FT * KP; idx += Cfg::NT) {
        const int sl = idx / KP, i = idx % KP, tt = g0 + sl;
        if (tt >= nt) continue;
        float gq = 0.f, gad = 0.f, gbd = 0.f, ga = 0.f;
#pragma unroll
        for (int wv = 0; wv < Cfg::NW; ++wv) {
            gq += s.red[sl][wv][0][i];
            gad += s.red[sl][wv][1][i];
            gbd += s.red[sl][wv][2][i];
            ga += s.red[sl][wv][3][i];
        }
        if (s.val[tt] == 0.f) ga = 0.f;  // padding: the adjoint passed through
        const float kr = s.k[tt][i], er = s.e[tt][i];
        const float dk = __builtin_fmaf(s.ks[tt], kr, __builtin_fmaf(-er, gbd, gad));
        const float de = -kr * gbd;
        if (i < a.K) {
            const int64_t o = (((int64_t)b * a.T + t0 + tt) * a.H + h) * a.K + i;
            if (a.dq) store_in<TIN>(a.dq, o, gq);
            if (a.dk) store_in<TIN>(a.dk, o, dk);
            if (a.dalpha) a.dalpha[o] = ga;
            if (a.derase) a.derase[o] = de;
        }
        if (a.scalar) {
            s.a[tt][i] = i < a.K ? ga : 0.f;
            s.e[tt][i] = i < a.K ? de : 0.f;
        }
    }
    for (int idx = tid; idx < Cfg::FT * VP; idx += Cfg::NT) {
        const int sl = idx / VP, j = idx % VP, tt = g0 + sl;
        if (tt >= nt || j >= a.V) continue;
        const float dd = s.dd[tt][j];
        const int64_t o = (((int64_t)b * a.T + t0 + tt) * a.H + h) * a.V + j;
        if (a.dv) store_in<TIN>(a.dv, o, s.w[tt][j] * dd);
        if (a.dwrite) a.dwrite[o] = s.v[tt][j] * dd;
    }
}

#pragma clang fp contract(off)
template <int KP, int VP, typename TIN>
__global__ void __launch_bounds__((SeqBwdCfg<KP, VP>::NT)) seq_bwd_kernel(SeqArgs a) {
    using Cfg = SeqBwdCfg<KP, VP>;
    constexpr int NT = Cfg::NT, RL = Cfg::RL, CL = Cfg::CL, FT = Cfg::FT, CT = SEQ_CT;
    constexpr bool AHEAD = Cfg::AHEAD;
    __shared__ SeqBwdSmem<KP, VP> s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rg = lane >> 2, cl = lane & 3;
    const int r0 = RL * rg, c0 = 4 * CL * w + CL * cl;  // first key row / value column of this lane
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int64_t KV = (int64_t)a.K * a.V;

    float adj[RL][CL];
#pragma unroll
    for (int ri = 0; ri < RL; ++ri)
#pragma unroll
        for (int cj = 0; cj < CL; ++cj) {
            const int i = r0 + ri, j = c0 + cj;
            adj[ri][cj] = (a.dfinal && i < a.K && j < a.V) ? a.dfinal[bh * KV + (int64_t)i * a.V + j]
                                                           : 0.f;
        }

    // Pre-token states of the current block: CL floats at
    // rp + ((tt * RL + ri) * NT + tid) * CL.
    float *rp = a.replay + (int64_t)bh * CT * KP * VP;

    const TokenSrc src = make_src<TIN>(a, b, h);
    const BlockCtx ctx = make_ctx(a, b, h, bh);
    TokenRegs<KP, VP, NT, true> nx;
    float ckn[RL][CL];
    load_tokens<KP, VP, NT, true, TIN>(src, ctx, (a.nck - 1) * CT, tid, nx);
    if (AHEAD) load_ck<KP, VP, RL, CL>(a, bh, a.nck - 1, r0, c0, ckn);
    store_bwd_flags<KP, VP, NT, TIN>(a, nx, s, (a.nck - 1) * CT, tid);
    __syncthreads();
    store_bwd_data<KP, VP, NT, TIN>(a, nx, s, tid);
    __syncthreads();

    for (int blk = a.nck - 1; blk >= 0; --blk) {
        const int t0 = blk * CT, nt = min(CT, a.T - t0);
        // Resets as a wave-uniform bit mask.
        const uint64_t rm = __ballot(lane < CT && s.rst[lane & (CT - 1)] != 0.f &&
                                     s.val[lane & (CT - 1)] != 0.f);
        if (!AHEAD) load_ck<KP, VP, RL, CL>(a, bh, blk, r0, c0, ckn);
        float S[RL][CL];
#pragma unroll
        for (int ri = 0; ri < RL; ++ri)
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) S[ri][cj] = ckn[ri][cj];
        // The earlier block's inputs: issued here, written to LDS after the
        // token loop.
        if (blk > 0) {
            load_tokens<KP, VP, NT, true, TIN>(src, ctx, t0 - CT, tid, nx);
            if (AHEAD) load_ck<KP, VP, RL, CL>(a, bh, blk - 1, r0, c0, ckn);
        }
        // Replay the block with the forward's deltas: padding leaves S as is
        // (a = 1, k = 0, delta = 0); a reset zeroes it first.
        for (int tt = 0; tt < nt; ++tt) {
            const bool rs = (rm >> tt) & 1;
#pragma unroll
            for (int ri = 0; ri < RL; ++ri)
#pragma unroll
                for (int cj = 0; cj < CL; ++cj) S[ri][cj] = rs ? 0.f : S[ri][cj];
#pragma unroll
            for (int ri = 0; ri < RL; ++ri) lds_put<CL>(rp + ((tt * RL + ri) * NT + tid) * CL, S[ri]);
            float dl[CL], al[RL], kr[RL];
            lds_get<CL>(&s.d[tt][c0], dl);
            lds_get<RL>(&s.a[tt][r0], al);
            lds_get<RL>(&s.k[tt][r0], kr);
#pragma unroll
            for (int ri = 0; ri < RL; ++ri)
#pragma unroll
                for (int cj = 0; cj < CL; ++cj)
                    S[ri][cj] = __builtin_fmaf(kr[ri], dl[cj], S[ri][cj] * al[ri]);
        }
        auto load_prev = [&](int tt, float (&p)[RL][CL]) {
#pragma unroll
            for (int ri = 0; ri < RL; ++ri) lds_get<CL>(rp + ((tt * RL + ri) * NT + tid) * CL, p[ri]);
        };
        // One token of the reverse sweep.
        auto step = [&](int tt, const float (&prev)[RL][CL], const BwdTok<RL, CL> &xin) {
            BwdTok<RL, CL> xl;
            if (!AHEAD) fetch_bwd<KP, VP, RL, CL>(s, tt, r0, c0, xl);
            const BwdTok<RL, CL> &x = AHEAD ? xin : xl;
            const int slot = tt % FT;
#pragma unroll
            for (int ri = 0; ri < RL; ++ri)
#pragma unroll
                for (int cj = 0; cj < CL; ++cj)
                    adj[ri][cj] = __builtin_fmaf(x.q[ri], x.dy[cj], adj[ri][cj]);
            // Edit adjoint ddelta_j = sum_i k_i adj_ij + cs delta_j.
            float dd[CL];
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) {
                float p = 0.f;
#pragma unroll
                for (int ri = 0; ri < RL; ++ri) p = __builtin_fmaf(x.k[ri], adj[ri][cj], p);
                dd[cj] = __builtin_fmaf(x.cs, x.d[cj], stride_sum<4>(p));
            }
            // Per-key terms summed over this lane's columns, then over the
            // column quad; lane cl keeps quantity cl.
            float *red = &s.red[slot][w][cl][r0];
#pragma unroll
            for (int ri = 0; ri < RL; ++ri) {
                const float ek = x.e[ri] * x.k[ri];
                float gq = 0.f, gad = 0.f, gbd = 0.f, ga = 0.f;
#pragma unroll
                for (int cj = 0; cj < CL; ++cj) {
                    const float p = prev[ri][cj];
                    const float bar = x.a[ri] * p;
                    gq = __builtin_fmaf(__builtin_fmaf(x.k[ri], x.d[cj], bar), x.dy[cj], gq);
                    gad = __builtin_fmaf(adj[ri][cj], x.d[cj], gad);
                    gbd = __builtin_fmaf(bar, dd[cj], gbd);
                    const float dbar = __builtin_fmaf(-ek, dd[cj], adj[ri][cj]);
                    ga = __builtin_fmaf(dbar, p, ga);
                    adj[ri][cj] = x.a[ri] * dbar;
                }
                gq = group_sum<4>(gq);
                gad = group_sum<4>(gad);
                gbd = group_sum<4>(gbd);
                ga = group_sum<4>(ga);
                red[ri] = cl == 0 ? gq : (cl == 1 ? gad : (cl == 2 ? gbd : ga));
            }
            // Every row group holds the same column sums; all lanes store them.
            lds_put<CL>(&s.dd[tt][c0], dd);
            if (slot == 0) {  // tokens tt .. tt+FT-1 are complete
                __syncthreads();
                flush_group<KP, VP, TIN>(a, s, b, h, t0, tt, nt, tid);
                __syncthreads();
            }
        };
        // Two sets of (pre-token state, operands) in turn: the next token's
        // scratch and LDS reads overlap this one.
        float pa[RL][CL], pb[RL][CL];
        BwdTok<RL, CL> xa, xb;
        load_prev(nt - 1, pa);
        if (AHEAD) fetch_bwd<KP, VP, RL, CL>(s, nt - 1, r0, c0, xa);
        for (int tt = nt - 1; tt >= 0; tt -= 2) {
            if (tt > 0) {
                load_prev(tt - 1, pb);
                if (AHEAD) fetch_bwd<KP, VP, RL, CL>(s, tt - 1, r0, c0, xb);
            }
            step(tt, pa, xa);
            if (tt == 0) break;
            if (tt > 1) {
                load_prev(tt - 2, pa);
                if (AHEAD) fetch_bwd<KP, VP, RL, CL>(s, tt - 2, r0, c0, xa);
            }
            step(tt - 1, pb, xb);
        }
        if (a.scalar) {  // chain rule onto beta and the log gate g
            for (int tt = tid >> 4; tt < CT; tt += NT / 16) {
                const int l = tid & 15;
                float de = 0.f, da = 0.f, dw = 0.f;
                for (int c = l; c < KP; c += 16) {
                    de += s.e[tt][c];
                    da += s.a[tt][c];
                }
                for (int c = l; c < VP; c += 16) dw = __builtin_fmaf(s.v[tt][c], s.dd[tt][c], dw);
                de = row16_sum(de);
                da = row16_sum(da);
                dw = row16_sum(dw);
                if (l == 0 && tt < nt) {
                    const int t = t0 + tt;
                    const int64_t tok = ((int64_t)b * a.T + t) * a.H + h;
                    const bool on = s.val[tt] != 0.f;
                    if (a.dbeta) a.dbeta[tok] = on ? de + dw : 0.f;
                    if (a.dg) a.dg[tok] = on ? expf(ld4<float>(a.g, b, t, h, 0)) * da : 0.f;
                }
            }
            __syncthreads();
        }
        if (blk > 0) {
            store_bwd_flags<KP, VP, NT, TIN>(a, nx, s, t0 - CT, tid);
            __syncthreads();
            store_bwd_data<KP, VP, NT, TIN>(a, nx, s, tid);
            __syncthreads();
        }
    }
    // Initial-state adjoint.
    if (a.dinitial) {
#pragma unroll
        for (int ri = 0; ri < RL; ++ri)
#pragma unroll
            for (int cj = 0; cj < CL; ++cj) {
                const int i = r0 + ri, j = c0 + cj;
                if (i < a.K && j < a.V) a.dinitial[bh * KV + (int64_t)i * a.V + j] = adj[ri][cj];
            }
    }
}
#pragma clang fp contract(on)

// ---- decode ----------------------------------------------------------------------

// One token on a carried state (T == 1): thread j owns value column j with
// all its key rows in registers, so the state is read and written once,
// coalesced across the columns.  Every sum follows the forward kernel's order
// (per row group two interleaved chains, then the balanced tree over row
// groups; the score norms as the forward's 16-lane trees), so a decode step
// is bit-identical to a one-token scan.
template <int KP, int VP, typename TIN>
__global__ void __launch_bounds__(VP < 64 ? 64 : VP) seq_decode_kernel(SeqArgs a) {
    using L = FwdLayout<KP>;
    constexpr int NTD = VP < 64 ? 64 : VP, RGN = L::RGN, RL = L::RL;
    __shared__ float sq[KP], sk[KP], sa[KP], sek[KP], sd[VP];
    const int j = threadIdx.x, bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const TokenSrc src = make_src<TIN>(a, b, h);
    const bool jin = j < a.V;
    float S[KP];
#pragma unroll
    for (int i = 0; i < KP; ++i)
        S[i] = (jin && i < a.K && a.initial.data) ? ld4<float>(a.initial, b, h, i, j) : 0.f;
    const float val = src.f0.p ? __uint_as_float(ld_s<float>(src.f0, 0, 0)) : 1.f;
    const float rst = src.f1.p ? __uint_as_float(ld_s<float>(src.f1, 0, 0)) : 0.f;
    const bool on = val != 0.f;
    // Operands staged as the forward stages them: padding folds to a = 1 and
    // zero q, k, e.k, w.v; a reset to a = 0.
    for (int i = j; i < KP; i += NTD) {
        float qf = 0.f, kf = 0.f, af = 0.f, ef = 0.f;
        if (i < a.K) {
            qf = raw_f<TIN>(ld_s<TIN>(src.q, 0, i));
            kf = raw_f<TIN>(ld_s<TIN>(src.k, 0, i));
            const float g = __uint_as_float(ld_s<float>(src.a, 0, i));
            af = a.scalar ? expf(g) : g;
            ef = __uint_as_float(ld_s<float>(src.e, 0, i));
        } else if (a.scalar) {
            af = 0.f;
        }
        sq[i] = on ? qf : 0.f;
        sk[i] = on ? kf : 0.f;
        sa[i] = on ? (rst != 0.f ? 0.f : af) : 1.f;
        sek[i] = on ? ef * kf : 0.f;
    }
    float wv = 0.f;
    if (jin && on) wv = __uint_as_float(ld_s<float>(src.w, 0, j)) * raw_f<TIN>(ld_s<TIN>(src.v, 0, j));
    __syncthreads();
    float pg[RGN], og[RGN];
#pragma unroll
    for (int g = 0; g < RGN; ++g) {
        float p0 = 0.f, p1 = 0.f;
#pragma unroll
        for (int ri = 0; ri < RL; ++ri) {
            const int i = g * RL + ri;
            S[i] = S[i] * sa[i];
            if (ri & 1) p1 = __builtin_fmaf(sek[i], S[i], p1);
            else p0 = __builtin_fmaf(sek[i], S[i], p0);
        }
        pg[g] = p0 + p1;
    }
    const float delta = wv - tree_sum(pg);
#pragma unroll
    for (int g = 0; g < RGN; ++g) {
        float p0 = 0.f, p1 = 0.f;
#pragma unroll
        for (int ri = 0; ri < RL; ++ri) {
            const int i = g * RL + ri;
            S[i] = __builtin_fmaf(sk[i], delta, S[i]);
            if (ri & 1) p1 = __builtin_fmaf(sq[i], S[i], p1);
            else p0 = __builtin_fmaf(sq[i], S[i], p0);
        }
        og[g] = p0 + p1;
    }
    const float o = tree_sum(og);
    const int64_t tok = (int64_t)b * a.T * a.H + h;
    if (jin) {
        store_out(a.out, a.out_bf16, tok * a.V + j, o);
        if (a.final_state) {
            float *fs = a.final_state + (int64_t)bh * a.K * a.V + j;
#pragma unroll
            for (int i = 0; i < KP; ++i)
                if (i < a.K) fs[(int64_t)i * a.V] = S[i];
        }
    }
    if (j < VP) sd[j] = delta;
    __syncthreads();
    // Score |k| |delta| with the forward's 16-lane sums.
    if (j == 0 && a.scores) {
        float kk[16], dd[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) {
            kk[l] = dd[l] = 0.f;
            for (int c = l; c < KP; c += 16) kk[l] = __builtin_fmaf(sk[c], sk[c], kk[l]);
            for (int c = l; c < VP; c += 16) dd[l] = __builtin_fmaf(sd[c], sd[c], dd[l]);
        }
        const float k2 = tree_sum(kk), d2 = tree_sum(dd);
        a.scores[tok] = on ? sqrtf(k2 * d2) : 0.f;
    }
}

template <int KP, int VP>
static hipError_t decode_typed(const SeqArgs &a, bool bf16, hipStream_t st) {
    constexpr int NTD = VP < 64 ? 64 : VP;
    if (bf16)
        hipLaunchKernelGGL((seq_decode_kernel<KP, VP, bf16_t>), dim3(a.B * a.H), dim3(NTD), 0, st, a);
    else
        hipLaunchKernelGGL((seq_decode_kernel<KP, VP, float>), dim3(a.B * a.H), dim3(NTD), 0, st, a);
    return hipGetLastError();
}

template <int KP, int VP>
static hipError_t fwd_typed(const SeqArgs &a, bool bf16, hipStream_t st) {
    constexpr int NT = 4 * VP;
    if (bf16)
        hipLaunchKernelGGL((seq_fwd_kernel<KP, VP, bf16_t>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    else
        hipLaunchKernelGGL((seq_fwd_kernel<KP, VP, float>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    return hipGetLastError();
}

template <int KP, int VP>
static hipError_t bwd_typed(const SeqArgs &a, bool bf16, hipStream_t st) {
    constexpr int NT = SeqBwdCfg<KP, VP>::NT;
    if (bf16)
        hipLaunchKernelGGL((seq_bwd_kernel<KP, VP, bf16_t>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    else
        hipLaunchKernelGGL((seq_bwd_kernel<KP, VP, float>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    return hipGetLastError();
}

#define GDN2_SEQ_DISPATCH(FN)                                              \
    const int kp = seq_pad(a.K), vp = seq_pad(a.V);                        \
    if (kp == 32 && vp == 32) return FN<32, 32>(a, bf16, st);              \
    if (kp == 32 && vp == 64) return FN<32, 64>(a, bf16, st);              \
    if (kp == 32 && vp == 128) return FN<32, 128>(a, bf16, st);            \
    if (kp == 64 && vp == 32) return FN<64, 32>(a, bf16, st);              \
    if (kp == 64 && vp == 64) return FN<64, 64>(a, bf16, st);              \
    if (kp == 64 && vp == 128) return FN<64, 128>(a, bf16, st);            \
    if (kp == 128 && vp == 32) return FN<128, 32>(a, bf16, st);            \
    if (kp == 128 && vp == 64) return FN<128, 64>(a, bf16, st);            \
    return FN<128, 128>(a, bf16, st);

hipError_t launch_seq_fwd(const SeqArgs &a, bool bf16, hipStream_t st) {
    GDN2_SEQ_DISPATCH(fwd_typed)
}

hipError_t launch_seq_decode(const SeqArgs &a, bool bf16, hipStream_t st) {
    if (a.T != 1 || a.doc) return hipErrorInvalidValue;
    GDN2_SEQ_DISPATCH(decode_typed)
}

hipError_t launch_seq_bwd(const SeqArgs &a, bool bf16, hipStream_t st) {
    if (!a.ck || !a.replay) return hipErrorInvalidValue;
    GDN2_SEQ_DISPATCH(bwd_typed)
}

}  // namespace gdn2
