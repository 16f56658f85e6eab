// Chunked channel-wise GDN-2 in f32 (d_k, d_v <= 64, 16-token chunks).
#pragma once

#include "gdn2_seq.h"

namespace gdn2 {

constexpr int FC_C = 16;    // tokens per chunk
constexpr int FC_MAX = 64;  // largest d_k and d_v

inline bool fc_eligible_shape(const gdn2_shape *s) {
    return s->keys <= FC_MAX && s->values <= FC_MAX;
}

// The token-sequential argument block (shapes, views, outputs, gradients)
// plus the chunk path's checkpoint and workspace arrays, each indexed by
// chunk ci = (b * H + h) * nc + c:
//   st     S at the chunk start, [K][V]                 (forward scan -> out, bgrad)
//   tm     T = (I + A)^-1, [16][16]                       (prep -> out, bgrad)
//   dl     the edits delta, [16][V]                       (out -> bprep, bgrad)
//   fw, fk the factored map: W' = T (b . e . k) and Ktil = lam . k, [16][KP] each
//   fu     U = T (w . v), [16][V];  gv  b_15 (the map's diagonal), [KP]
// KP = d_k rounded up to 16: the key axis of the map's factors is padded with
// zeros to whole 16-row MFMA tiles for the scans.
// Backward workspace: ds, the state adjoint at each chunk end, and n, the
// adjoint map's additive term, [K][V] each.
struct FcArgs {
    SeqArgs s;
    int nc;
    int in_bf16;  // q, k, v, dO and dq, dk, dv are bf16 (else f32)
    float *st, *tm, *dl, *fw, *fk, *fu, *gv;
    float *ds, *n;
};

inline int64_t fc_chunks(int64_t B, int64_t T, int64_t H) { return B * H * ((T + FC_C - 1) / FC_C); }
__host__ __device__ inline int fc_kp(int K) { return (K + 15) & ~15; }

inline size_t fc_chunk_floats(int K, int V) {
    return (size_t)K * V + FC_C * FC_C + FC_C * V + 2 * FC_C * fc_kp(K) + FC_C * V + fc_kp(K);
}

inline size_t fc_checkpoint_bytes(int64_t B, int64_t T, int64_t H, int K, int V) {
    return (size_t)fc_chunks(B, T, H) * fc_chunk_floats(K, V) * sizeof(float);
}

inline size_t fc_workspace_bytes(int64_t B, int64_t T, int64_t H, int K, int V) {
    return (size_t)fc_chunks(B, T, H) * 2 * K * V * sizeof(float);
}

inline void fc_bind(FcArgs &a, void *ck, void *ws) {
    const int64_t n = fc_chunks(a.s.B, a.s.T, a.s.H);
    const int K = a.s.K, V = a.s.V;
    float *p = static_cast<float *>(ck);
    a.st = p;
    p += n * K * V;
    a.tm = p;
    p += n * FC_C * FC_C;
    a.dl = p;
    p += n * FC_C * V;
    a.fw = p;
    p += n * FC_C * fc_kp(K);
    a.fk = p;
    p += n * FC_C * fc_kp(K);
    a.fu = p;
    p += n * FC_C * V;
    a.gv = p;
    if (ws) {
        a.ds = static_cast<float *>(ws);
        a.n = a.ds + n * K * V;
    }
}

hipError_t launch_fc_fwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev);
hipError_t launch_fc_bwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev);

}  // namespace gdn2
