// Token-sequential GDN-2 kernels (general channel-wise surface, decode).
#pragma once

#include "gdn2_common.h"

namespace gdn2 {

constexpr int SEQ_CT = 16;  // tokens per staging block == checkpoint interval
constexpr int SEQ_KR = 16;  // state rows held by one thread

struct SeqArgs {
    int B, T, H, K, V;
    View q, k, v, alpha, erase, write, valid, reset, initial;
    // Document limits (int32 [batch, time] views, inclusive; end < start marks
    // padding).  When set they replace valid/reset, and the backward follows
    // the reference's doc-limit VJP: the adjoint is cleared at tokens with
    // end == t and passes through resets.
    int doc;
    View doc_start, doc_end;
    // Scalar-gate mode: alpha[i] = exp(g), erase[i] = write[j] = beta, with
    // beta and g read as [batch, time, head] views; gradients dbeta and dg.
    int scalar;
    View beta, g;
    float *dbeta, *dg;
    // forward outputs
    void *out;
    int out_bf16;
    float *final_state, *scores;
    float *ck;  // checkpoints [B*H][nck][KR][NT]; null = not written (decode)
    int nck;
    // backward
    View dout;
    const float *dfinal, *dscores;
    void *dq, *dk, *dv;
    float *dalpha, *derase, *dwrite, *dinitial;
    float *replay;  // [B*H][SEQ_CT][KR][NT]
};

// Padded widths used by the kernels: 32, 64 or 128.
inline int seq_pad(int n) { return n <= 32 ? 32 : (n <= 64 ? 64 : 128); }
inline int64_t seq_threads(int K, int V) { return (int64_t)(seq_pad(K) / SEQ_KR) * seq_pad(V); }
inline int64_t seq_state_floats(int K, int V) { return (int64_t)seq_pad(K) * seq_pad(V); }

hipError_t launch_seq_fwd(const SeqArgs &a, bool in_bf16, hipStream_t stream);
hipError_t launch_seq_bwd(const SeqArgs &a, bool in_bf16, hipStream_t stream);

}  // namespace gdn2
