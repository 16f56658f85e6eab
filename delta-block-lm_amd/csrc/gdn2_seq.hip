// Token-sequential GDN-2 scan for gfx950: the general channel-wise surface.
//
// Semantics follow crates/mixers/src/reference.rs:41-257 (forward and VJP)
// and the stateful fused kernels crates/kernels/src/gdn_training.rs:12-284.
//
// Work decomposition (one workgroup per (batch, head)):
//   thread tid owns value column j = tid / NG and the KR = 16 key rows
//   i0 = (tid % NG) * 16 .. i0 + 15 of the fp32 state, NG = KP / 16.  The NG
//   threads of one column are adjacent lanes of one wavefront, so the two
//   per-token reductions over keys (the edit delta and the output) are lane
//   butterflies with no LDS round trip and no barrier.  Token inputs are
//   staged through LDS 16 tokens at a time with coalesced strided loads;
//   outputs are staged back and stored coalesced.
//
// Checkpoints: the forward stores the state every SEQ_CT tokens in a private
// thread-major layout (one coalesced row per register).  The backward walks
// blocks in reverse, replays a block from its checkpoint (storing the 16
// pre-token states in a scratch buffer) and then runs the token VJP in
// reverse.  Per-key gradients are reduced over value columns with a wave
// butterfly, then across waves through a double-buffered LDS slab.
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

// Sum over the lanes of a wave that share a key group (lane % NG), in all of
// them: row rotations by multiples of NG sum the same-group lanes of each
// 16-lane row, then the four rows are combined with permlane swaps.
template <int NG>
__device__ __forceinline__ float column_sum(float x) {
    if (NG <= 2) x = dpp_add<0x122>(x);   // row_ror 2
    if (NG <= 4) x = dpp_add<0x124>(x);   // row_ror 4
    x = dpp_add<0x128>(x);                // row_ror 8
    return swap32_sum(swap16_sum(x));
}

template <int KP, int VP>
struct SeqFwdSmem {
    static constexpr int CT = SEQ_CT;
    float q[CT][KP], k[CT][KP], a[CT][KP], e[CT][KP];
    float v[CT][VP], w[CT][VP], o[CT][VP], d[CT][VP];
    float val[CT], rst[CT];
};

template <int KP, int VP>
union SeqFwdShared {
    SeqFwdSmem<KP, VP> s;
    float st[KP * (VP + 1)];  // state transpose slab (row stride VP+1)
};

// Stage SEQ_CT tokens starting at t0 into LDS as fp32 (zero beyond T/K/V).
template <int KP, int VP, int NT, typename TIN>
__device__ __forceinline__ void stage_tokens(const SeqArgs &a, int b, int h, int t0,
                                             float (*sq)[KP], float (*sk)[KP],
                                             float (*sa)[KP], float (*se)[KP],
                                             float (*sv)[VP], float (*sw)[VP],
                                             float *sval, float *srst, float *saclr, int tid) {
    constexpr int CT = SEQ_CT;
    for (int idx = tid; idx < CT * KP; idx += NT) {
        const int tt = idx / KP, c = idx % KP, t = t0 + tt;
        const bool in = t < a.T && c < a.K;
        sq[tt][c] = in ? ld4<TIN>(a.q, b, t, h, c) : 0.f;
        sk[tt][c] = in ? ld4<TIN>(a.k, b, t, h, c) : 0.f;
        if (a.scalar) {
            sa[tt][c] = in ? expf(ld4<float>(a.g, b, t, h, 0)) : 0.f;
            se[tt][c] = in ? ld4<float>(a.beta, b, t, h, 0) : 0.f;
        } else {
            sa[tt][c] = in ? ld4<float>(a.alpha, b, t, h, c) : 0.f;
            se[tt][c] = in ? ld4<float>(a.erase, b, t, h, c) : 0.f;
        }
    }
    for (int idx = tid; idx < CT * VP; idx += NT) {
        const int tt = idx / VP, c = idx % VP, t = t0 + tt;
        const bool in = t < a.T && c < a.V;
        sv[tt][c] = in ? ld4<TIN>(a.v, b, t, h, c) : 0.f;
        sw[tt][c] = in ? (a.scalar ? ld4<float>(a.beta, b, t, h, 0) : ld4<float>(a.write, b, t, h, c))
                       : 0.f;
    }
    if (tid < CT) {
        const int t = t0 + tid;
        float val = 0.f, rst = 0.f, clr = 0.f;
        if (t < a.T) {
            if (a.doc) {
                const int32_t st = reinterpret_cast<const int32_t *>(
                    a.doc_start.data)[b * a.doc_start.s0 + t * a.doc_start.s1];
                const int32_t en = reinterpret_cast<const int32_t *>(
                    a.doc_end.data)[b * a.doc_end.s0 + t * a.doc_end.s1];
                val = en >= st ? 1.f : 0.f;
                rst = st == t ? 1.f : 0.f;
                clr = en == t ? 1.f : 0.f;
            } else {
                val = a.valid.data ? ld4<float>(a.valid, b, t, 0, 0) : 1.f;
                rst = a.reset.data ? ld4<float>(a.reset, b, t, 0, 0) : 0.f;
            }
        }
        sval[tid] = val;
        srst[tid] = rst;
        if (saclr) saclr[tid] = clr;
    }
}

template <int KP, int VP, typename TIN>
__global__ void __launch_bounds__((KP / SEQ_KR) * VP) seq_fwd_kernel(SeqArgs a) {
    constexpr int NG = KP / SEQ_KR, NT = NG * VP, CT = SEQ_CT, KR = SEQ_KR;
    __shared__ SeqFwdShared<KP, VP> sh;
    SeqFwdSmem<KP, VP> &s = sh.s;
    const int tid = threadIdx.x;
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int ig = tid % NG, j = tid / NG, i0 = ig * KR;

    // Initial state, coalesced through the transpose slab.
    for (int idx = tid; idx < KP * VP; idx += NT) {
        const int i = idx / VP, c = idx % VP;
        sh.st[i * (VP + 1) + c] = (a.initial.data && i < a.K && c < a.V)
                                      ? ld4<float>(a.initial, b, h, i, c)
                                      : 0.f;
    }
    __syncthreads();
    float S[KR];
#pragma unroll
    for (int r = 0; r < KR; ++r) S[r] = sh.st[(i0 + r) * (VP + 1) + j];
    __syncthreads();

    for (int t0 = 0, blk = 0; t0 < a.T; t0 += CT, ++blk) {
        if (a.ck) {
            float *ck = a.ck + ((int64_t)bh * a.nck + blk) * KR * NT;
#pragma unroll
            for (int r = 0; r < KR; ++r) ck[r * NT + tid] = S[r];
        }
        stage_tokens<KP, VP, NT, TIN>(a, b, h, t0, s.q, s.k, s.a, s.e, s.v, s.w, s.val, s.rst,
                                      nullptr, tid);
        __syncthreads();
        const int nt = min(CT, a.T - t0);
        for (int tt = 0; tt < nt; ++tt) {
            if (s.val[tt] == 0.f) {  // padding: zero output/edit, frozen state
                if (ig == 0) {
                    s.o[tt][j] = 0.f;
                    s.d[tt][j] = 0.f;
                }
                continue;
            }
            if (s.rst[tt] != 0.f) {
#pragma unroll
                for (int r = 0; r < KR; ++r) S[r] = 0.f;
            }
            float part = 0.f;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                S[r] *= s.a[tt][i0 + r];
                part += s.e[tt][i0 + r] * s.k[tt][i0 + r] * S[r];
            }
            const float delta = s.w[tt][j] * s.v[tt][j] - group_sum<NG>(part);
            float o = 0.f;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                S[r] += s.k[tt][i0 + r] * delta;
                o += s.q[tt][i0 + r] * S[r];
            }
            o = group_sum<NG>(o);
            if (ig == 0) {
                s.o[tt][j] = o;
                s.d[tt][j] = delta;
            }
        }
        __syncthreads();
        for (int idx = tid; idx < nt * VP; idx += NT) {
            const int tt = idx / VP, c = idx % VP;
            if (c < a.V)
                store_out(a.out, a.out_bf16, (((int64_t)b * a.T + t0 + tt) * a.H + h) * a.V + c,
                          s.o[tt][c]);
        }
        if (a.scores && tid < nt) {
            float sc = 0.f;
            if (s.val[tid] != 0.f) {
                float kk = 0.f, dd = 0.f;
                for (int c = 0; c < a.K; ++c) kk += s.k[tid][c] * s.k[tid][c];
                for (int c = 0; c < a.V; ++c) dd += s.d[tid][c] * s.d[tid][c];
                sc = sqrtf(kk * dd);
            }
            a.scores[((int64_t)b * a.T + t0 + tid) * a.H + h] = sc;
        }
        __syncthreads();
    }
    // Final state through the transpose slab.
#pragma unroll
    for (int r = 0; r < KR; ++r) sh.st[(i0 + r) * (VP + 1) + j] = S[r];
    __syncthreads();
    if (a.final_state)
        for (int idx = tid; idx < a.K * a.V; idx += NT) {
            const int i = idx / a.V, c = idx % a.V;
            a.final_state[(int64_t)bh * a.K * a.V + idx] = sh.st[i * (VP + 1) + c];
        }
}

template <int KP, int VP>
struct SeqBwdSmem {
    static constexpr int CT = SEQ_CT, NW = (KP / SEQ_KR) * VP / 64;
    float q[CT][KP], k[CT][KP], a[CT][KP], e[CT][KP];
    float v[CT][VP], w[CT][VP], dy[CT][VP], d[CT][VP];
    float val[CT], rst[CT], aclr[CT], sa[CT], kk[CT], dd[CT];
    float red[2][NW][4][KP];
};

template <int KP, int VP>
union SeqBwdShared {
    SeqBwdSmem<KP, VP> s;
    float st[KP * (VP + 1)];
};

template <typename TIN>
__device__ __forceinline__ void store_in(void *p, int64_t i, float x) {
    Elem<TIN>::store(p, i, x);
}

template <int KP, int VP, typename TIN>
__global__ void __launch_bounds__((KP / SEQ_KR) * VP) seq_bwd_kernel(SeqArgs a) {
    constexpr int NG = KP / SEQ_KR, NT = NG * VP, CT = SEQ_CT, KR = SEQ_KR, NW = NT / 64;
    __shared__ SeqBwdShared<KP, VP> sh;
    SeqBwdSmem<KP, VP> &s = sh.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int ig = tid % NG, j = tid / NG, i0 = ig * KR;
    const int64_t KV = (int64_t)a.K * a.V;

    // Adjoint of the final state, coalesced through the transpose slab.
    for (int idx = tid; idx < KP * VP; idx += NT) {
        const int i = idx / VP, c = idx % VP;
        sh.st[i * (VP + 1) + c] =
            (a.dfinal && i < a.K && c < a.V) ? a.dfinal[bh * KV + (int64_t)i * a.V + c] : 0.f;
    }
    __syncthreads();
    float adj[KR];
#pragma unroll
    for (int r = 0; r < KR; ++r) adj[r] = sh.st[(i0 + r) * (VP + 1) + j];
    __syncthreads();

    float *rp = a.replay + (int64_t)bh * CT * KR * NT;
    int buf = 0;
    for (int blk = a.nck - 1; blk >= 0; --blk) {
        const int t0 = blk * CT, nt = min(CT, a.T - t0);
        stage_tokens<KP, VP, NT, TIN>(a, b, h, t0, s.q, s.k, s.a, s.e, s.v, s.w, s.val, s.rst,
                                      s.aclr, tid);
        for (int idx = tid; idx < CT * VP; idx += NT) {
            const int tt = idx / VP, c = idx % VP, t = t0 + tt;
            s.dy[tt][c] = (a.dout.data && t < a.T && c < a.V) ? ld4<TIN>(a.dout, b, t, h, c) : 0.f;
        }
        if (tid < CT) {
            const int t = t0 + tid;
            s.sa[tid] = (a.dscores && t < a.T) ? a.dscores[((int64_t)b * a.T + t) * a.H + h] : 0.f;
        }
        // Replay the block from its checkpoint; rp[tt] = state before token tt.
        float S[KR];
        const float *ck = a.ck + ((int64_t)bh * a.nck + blk) * KR * NT;
#pragma unroll
        for (int r = 0; r < KR; ++r) S[r] = ck[r * NT + tid];
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {
#pragma unroll
            for (int r = 0; r < KR; ++r) rp[((int64_t)tt * KR + r) * NT + tid] = S[r];
            if (s.val[tt] == 0.f) {
                if (ig == 0) s.d[tt][j] = 0.f;
                continue;
            }
            if (s.rst[tt] != 0.f) {
#pragma unroll
                for (int r = 0; r < KR; ++r) S[r] = 0.f;
            }
            float part = 0.f;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                S[r] *= s.a[tt][i0 + r];
                part += s.e[tt][i0 + r] * s.k[tt][i0 + r] * S[r];
            }
            const float delta = s.w[tt][j] * s.v[tt][j] - group_sum<NG>(part);
#pragma unroll
            for (int r = 0; r < KR; ++r) S[r] += s.k[tt][i0 + r] * delta;
            if (ig == 0) s.d[tt][j] = delta;
        }
        __syncthreads();
        if (tid < nt) {
            float kk = 0.f, dd = 0.f;
            for (int c = 0; c < a.K; ++c) kk += s.k[tid][c] * s.k[tid][c];
            for (int c = 0; c < a.V; ++c) dd += s.d[tid][c] * s.d[tid][c];
            s.kk[tid] = sqrtf(kk);
            s.dd[tid] = sqrtf(dd);
        }
        __syncthreads();

        for (int tt = nt - 1; tt >= 0; --tt) {
            const int t = t0 + tt;
            const int64_t tok = ((int64_t)b * a.T + t) * a.H + h;
            if (s.val[tt] == 0.f) {  // padding: exact zero gradients, adjoint passes through
                for (int idx = tid; idx < a.K; idx += NT) {
                    if (a.dq) store_in<TIN>(a.dq, tok * a.K + idx, 0.f);
                    if (a.dk) store_in<TIN>(a.dk, tok * a.K + idx, 0.f);
                    if (a.dalpha) a.dalpha[tok * a.K + idx] = 0.f;
                    if (a.derase) a.derase[tok * a.K + idx] = 0.f;
                }
                for (int idx = tid; idx < a.V; idx += NT) {
                    if (a.dv) store_in<TIN>(a.dv, tok * a.V + idx, 0.f);
                    if (a.dwrite) a.dwrite[tok * a.V + idx] = 0.f;
                }
                if (a.scalar && tid == 0) {
                    if (a.dbeta) a.dbeta[tok] = 0.f;
                    if (a.dg) a.dg[tok] = 0.f;
                }
                continue;
            }
            const bool rst = s.rst[tt] != 0.f;
            float prev[KR];
#pragma unroll
            for (int r = 0; r < KR; ++r) prev[r] = rst ? 0.f : rp[((int64_t)tt * KR + r) * NT + tid];
            const float dy = s.dy[tt][j], delta = s.d[tt][j];
            const float nk = s.kk[tt], nd = s.dd[tt], sadj = s.sa[tt];
            float dd = 0.f;
            if (nk > 0.f && nd > 0.f) dd = sadj * nk * delta / nd;  // score VJP, zero subgradient
            if (s.aclr[tt] != 0.f) {  // doc limits: a document ends here
#pragma unroll
                for (int r = 0; r < KR; ++r) adj[r] = 0.f;
            }
            float part = 0.f;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                adj[r] += s.q[tt][i0 + r] * dy;
                part += s.k[tt][i0 + r] * adj[r];
            }
            dd += group_sum<NG>(part);
            float gq[KR], gk[KR], ge[KR], ga[KR];
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                const float kr = s.k[tt][i0 + r], er = s.e[tt][i0 + r], ar = s.a[tt][i0 + r];
                const float bar = ar * prev[r];
                gq[r] = (bar + kr * delta) * dy;
                gk[r] = adj[r] * delta - er * bar * dd;
                ge[r] = -kr * bar * dd;
                const float dbar = adj[r] - er * kr * dd;
                ga[r] = dbar * prev[r];
                adj[r] = (rst && !a.doc) ? 0.f : ar * dbar;
            }
            // Sum over the value columns held by this wave (lanes sharing ig).
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                gq[r] = column_sum<NG>(gq[r]);
                gk[r] = column_sum<NG>(gk[r]);
                ge[r] = column_sum<NG>(ge[r]);
                ga[r] = column_sum<NG>(ga[r]);
            }
            if (lane < NG) {
#pragma unroll
                for (int r = 0; r < KR; ++r) {
                    s.red[buf][wave][0][i0 + r] = gq[r];
                    s.red[buf][wave][1][i0 + r] = gk[r];
                    s.red[buf][wave][2][i0 + r] = ga[r];
                    s.red[buf][wave][3][i0 + r] = ge[r];
                }
            }
            if (ig == 0 && j < a.V) {
                if (a.dv) store_in<TIN>(a.dv, tok * a.V + j, s.w[tt][j] * dd);
                if (a.dwrite) a.dwrite[tok * a.V + j] = s.v[tt][j] * dd;
                // Scalar mode keeps dwrite_j in the (already consumed) dy slot.
                if (a.scalar) s.dy[tt][j] = s.v[tt][j] * dd;
            }
            __syncthreads();
            const float kscale = (nk > 0.f && nd > 0.f) ? sadj * nd / nk : 0.f;
            for (int idx = tid; idx < 4 * a.K; idx += NT) {
                const int qn = idx / a.K, i = idx % a.K;
                float acc = 0.f;
#pragma unroll
                for (int w = 0; w < NW; ++w) acc += s.red[buf][w][qn][i];
                if (qn == 0) {
                    if (a.dq) store_in<TIN>(a.dq, tok * a.K + i, acc);
                } else if (qn == 1) {
                    if (a.dk) store_in<TIN>(a.dk, tok * a.K + i, acc + kscale * s.k[tt][i]);
                } else if (qn == 2) {
                    if (a.dalpha) a.dalpha[tok * a.K + i] = acc;
                    if (a.scalar) s.a[tt][i] = acc;  // alpha row of token tt is consumed
                } else {
                    if (a.derase) a.derase[tok * a.K + i] = acc;
                    if (a.scalar) s.e[tt][i] = acc;
                }
            }
            buf ^= 1;
        }
        __syncthreads();
        if (a.scalar) {  // chain rule onto beta and the log gate g
            if (tid < nt && s.val[tid] != 0.f) {
                const int t = t0 + tid;
                const int64_t tok = ((int64_t)b * a.T + t) * a.H + h;
                float de = 0.f, dw = 0.f, da = 0.f;
                for (int c = 0; c < a.K; ++c) {
                    de += s.e[tid][c];
                    da += s.a[tid][c];
                }
                for (int c = 0; c < a.V; ++c) dw += s.dy[tid][c];
                if (a.dbeta) a.dbeta[tok] = de + dw;
                if (a.dg) a.dg[tok] = expf(ld4<float>(a.g, b, t, h, 0)) * da;
            }
            __syncthreads();
        }
    }
    // Initial-state adjoint.
#pragma unroll
    for (int r = 0; r < KR; ++r) sh.st[(i0 + r) * (VP + 1) + j] = adj[r];
    __syncthreads();
    if (a.dinitial)
        for (int idx = tid; idx < a.K * a.V; idx += NT) {
            const int i = idx / a.V, c = idx % a.V;
            a.dinitial[bh * KV + idx] = sh.st[i * (VP + 1) + c];
        }
}

template <int KP, int VP>
static hipError_t fwd_typed(const SeqArgs &a, bool bf16, hipStream_t st) {
    constexpr int NT = (KP / SEQ_KR) * VP;
    if (bf16)
        hipLaunchKernelGGL((seq_fwd_kernel<KP, VP, bf16_t>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    else
        hipLaunchKernelGGL((seq_fwd_kernel<KP, VP, float>), dim3(a.B * a.H), dim3(NT), 0, st, a);
    return hipGetLastError();
}

template <int KP, int VP>
static hipError_t bwd_typed(const SeqArgs &a, bool bf16, hipStream_t st) {
    constexpr int NT = (KP / SEQ_KR) * VP;
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

hipError_t launch_seq_bwd(const SeqArgs &a, bool bf16, hipStream_t st) {
    GDN2_SEQ_DISPATCH(bwd_typed)
}

}  // namespace gdn2
