// Token-sequential GDN-2 kernels (general channel-wise surface, decode).
#pragma once

#include "gdn2_common.h"

namespace gdn2 {

constexpr int SEQ_CT = 16;  // tokens per staging block == checkpoint interval

struct SeqArgs {
    int B, T, H, K, V;
    View q, k, v, alpha, erase, write, valid, reset, initial;
    // Document limits (int32 [batch, time] views, inclusive; end < start marks
    // padding, start == t resets the state).  When set they replace
    // valid/reset; the backward is the exact VJP, as with masks.
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
    // Checkpoint (null = not written, decode), carved by seq_bind_checkpoint:
    //   ck       [B*H][nck][K_pad][V_pad]  state at the start of every block
    //   ck_delta [B*H][nck*SEQ_CT][V_pad]  the edit delta of every token
    //   ck_norm  [B*H][nck*SEQ_CT][2]      |k| and |delta| of every token
    float *ck, *ck_delta, *ck_norm;
    int nck;
    // backward
    View dout;
    const float *dfinal, *dscores;
    void *dq, *dk, *dv;
    float *dalpha, *derase, *dwrite, *dinitial;
    float *replay;  // [B*H][SEQ_CT][K_pad * V_pad], thread-major
};

// Padded widths used by the kernels: 32, 64 or 128.
inline int seq_pad(int n) { return n <= 32 ? 32 : (n <= 64 ? 64 : 128); }
inline int64_t seq_state_floats(int K, int V) { return (int64_t)seq_pad(K) * seq_pad(V); }

inline int64_t seq_checkpoint_floats(int64_t B, int64_t T, int64_t H, int K, int V) {
    const int64_t nck = (T + SEQ_CT - 1) / SEQ_CT, tp = nck * SEQ_CT;
    return B * H * (nck * seq_state_floats(K, V) + tp * seq_pad(V) + tp * 2);
}

inline int64_t seq_workspace_floats(int64_t B, int64_t H, int K, int V) {
    return B * H * SEQ_CT * seq_state_floats(K, V);
}

inline void seq_bind_checkpoint(SeqArgs &a, const void *ck) {
    a.ck = static_cast<float *>(const_cast<void *>(ck));
    if (!ck) {
        a.ck_delta = a.ck_norm = nullptr;
        return;
    }
    const int64_t bh = (int64_t)a.B * a.H, tp = (int64_t)a.nck * SEQ_CT;
    a.ck_delta = a.ck + bh * a.nck * seq_state_floats(a.K, a.V);
    a.ck_norm = a.ck_delta + bh * tp * seq_pad(a.V);
}

hipError_t launch_seq_fwd(const SeqArgs &a, bool in_bf16, hipStream_t stream);
// One token (T == 1, masks only) on a carried state; no checkpoint.
hipError_t launch_seq_decode(const SeqArgs &a, bool in_bf16, hipStream_t stream);
hipError_t launch_seq_bwd(const SeqArgs &a, bool in_bf16, hipStream_t stream);

}  // namespace gdn2
