// Chunked channel-wise GDN-2 in f32 (d_k, d_v <= 128, 16-token chunks).
#pragma once

#include "gdn2_seq.h"

namespace gdn2 {

constexpr int FC_C = 16;    // tokens per chunk
constexpr int FC_MAX = 128;  // largest d_k and d_v

inline bool fc_eligible_shape(const gdn2_shape *s) {
    return s->keys <= FC_MAX && s->values <= FC_MAX;
}

// The token-sequential argument block (shapes, views, outputs, gradients)
// plus the chunk path's checkpoint and workspace arrays, each indexed by
// chunk ci = (b * H + h) * nc + c:
//   st     S at the chunk start, tile-packed: [VT][KT][4][16][4], element
//          (((vt * KT + tau) * 4 + g) * 16 + n) * 4 + r = S[16 tau + 4 g + r][16 vt + n]
//          (forward scan -> out, bgrad)
//   tm     T = (I + A)^-1, [16][16]                       (prep -> out, bgrad)
//   dl     the edits delta, [16][V]                       (out -> bprep, bgrad)
//   fw, fk the factored map: W' = T (b . e . k) and Ktil = lam . k, [16][KP] each
//   fu     U = T (w . v), lane-packed for the scan: [VT][4][16][4], element
//          ((vt * 4 + g) * 16 + n) * 4 + r = U[4 g + r][16 vt + n]
//   gv     b_15 (the map's diagonal), [KP]
// KP = d_k and VP = d_v rounded up to 16 (VT = VP / 16): the key axis of the
// map's factors is padded with zeros to whole 16-row MFMA tiles for the scans.
// KT = KP / 16.  A scan wave stores its 16 x 16 tile of S as one 16-byte piece
// per lane, its accumulator registers as they are.  Backward workspace: ds, the
// state adjoint at each chunk end, and n, the adjoint map's additive term, both
// tile-packed like st.  st, ds and n are zero outside K x V.  Every array starts
// on a 16-byte boundary.
struct FcArgs {
    SeqArgs s;
    int nc;
    int in_bf16;  // q, k, v, dO and dq, dk, dv are bf16 (else f32)
    float *st, *tm, *dl, *fw, *fk, *fu, *gv;
    float *ds, *n;
};

inline int64_t fc_chunks(int64_t B, int64_t T, int64_t H) { return B * H * ((T + FC_C - 1) / FC_C); }
__host__ __device__ inline int fc_kp(int K) { return (K + 15) & ~15; }
inline size_t fc_pad4(size_t x) { return (x + 3) & ~(size_t)3; }

// The checkpoint's arrays in order, in floats, for n chunks.
inline void fc_checkpoint_parts(int64_t n, int K, int V, size_t part[7]) {
    const size_t KP = fc_kp(K), VP = fc_kp(V);
    part[0] = n * KP * VP;              // st
    part[1] = fc_pad4(n * FC_C * FC_C); // tm
    part[2] = fc_pad4(n * FC_C * V);    // dl
    part[3] = n * FC_C * KP;            // fw
    part[4] = n * FC_C * KP;            // fk
    part[5] = n * FC_C * VP;            // fu
    part[6] = n * KP;                   // gv
}

inline size_t fc_checkpoint_bytes(int64_t B, int64_t T, int64_t H, int K, int V) {
    size_t part[7], total = 0;
    fc_checkpoint_parts(fc_chunks(B, T, H), K, V, part);
    for (size_t x : part) total += x;
    return total * sizeof(float);
}

inline size_t fc_workspace_bytes(int64_t B, int64_t T, int64_t H, int K, int V) {
    const int64_t n = fc_chunks(B, T, H);
    return 2 * (size_t)n * fc_kp(K) * fc_kp(V) * sizeof(float);
}

inline void fc_bind(FcArgs &a, void *ck, void *ws) {
    const int64_t n = fc_chunks(a.s.B, a.s.T, a.s.H);
    size_t part[7];
    fc_checkpoint_parts(n, a.s.K, a.s.V, part);
    float *p = static_cast<float *>(ck);
    float **dst[7] = {&a.st, &a.tm, &a.dl, &a.fw, &a.fk, &a.fu, &a.gv};
    for (int i = 0; i < 7; ++i) {
        *dst[i] = p;
        p += part[i];
    }
    if (ws) {
        a.ds = static_cast<float *>(ws);
        a.n = a.ds + n * fc_kp(a.s.K) * fc_kp(a.s.V);
    }
}

hipError_t launch_fc_fwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev);
hipError_t launch_fc_bwd(const FcArgs &a, hipStream_t stream, const hipEvent_t *ev);

}  // namespace gdn2
