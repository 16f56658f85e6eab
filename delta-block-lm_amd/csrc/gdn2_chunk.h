// Chunk-WY scalar-gate GDN kernels on MFMA (bf16 inputs, fp32 state).
#pragma once

#include "gdn2_common.h"

namespace gdn2 {

constexpr int CHUNK = 64;   // tokens per chunk (computational chunk)
constexpr int CHUNK_D = 64; // d_k = d_v handled by these kernels

// Per-chunk gate summary written by the prep kernel: chunk-local cumulative
// log decay G, masked beta, validity and reset-segment index of every token.
struct GateBlock {
    float G[CHUNK];
    float beta[CHUNK];
    float val[CHUNK];
    int seg[CHUNK];
};

// Per-chunk private storage handed from the forward to the backward:
//   state, state_lo  S at the chunk start, bf16 hi and lo, transposed (S^T rows)
//   T      (I + A)^-1, bf16 row-major
//   gate   GateBlock
//   delta  the chunk's edits delta[t][v], f32 row-major
// plus the dense state map S_C = A_c S0 + B_c that the scans read: A_c rows and
// A_c^T rows (the adjoint map M), each bf16 hi then lo [64][64], and B_c^T
// [value][key] (f32).
constexpr size_t CK_STATE_BYTES = CHUNK_D * CHUNK_D * sizeof(uint16_t);
constexpr size_t CK_T_BYTES = CHUNK * CHUNK * sizeof(uint16_t);
constexpr size_t CK_GATE_BYTES = sizeof(GateBlock);
constexpr size_t CK_DELTA_BYTES = CHUNK * CHUNK_D * sizeof(float);
constexpr size_t CK_MAP_BYTES = 2 * CHUNK_D * CHUNK_D * sizeof(uint16_t);  // hi and lo
constexpr size_t CK_MAPB_BYTES = CHUNK_D * CHUNK_D * sizeof(float);
constexpr size_t CK_CHUNK_BYTES = 2 * CK_STATE_BYTES + CK_T_BYTES + CK_GATE_BYTES + CK_DELTA_BYTES +
                                  2 * CK_MAP_BYTES + CK_MAPB_BYTES;
// Backward workspace per chunk: dS at the chunk end (bf16 hi and lo,
// transposed) and N^T of the adjoint map (f32).
constexpr size_t WS_CHUNK_BYTES = 2 * CK_STATE_BYTES + CHUNK_D * CHUNK_D * sizeof(float);

struct ChunkArgs {
    int B, T, H, nc;
    // bf16 q/k/v with unit channel stride: element (b,t,h,c) at b*s0 + t*s1 + h*s2 + c
    const uint16_t *q, *k, *v;
    int64_t qs[3], ks[3], vs[3];
    View beta, g, valid, reset, initial;
    // forward outputs
    void *out;
    int out_bf16;
    float *final_state, *scores;
    // checkpoint arrays, each [B*H*nc] per-chunk blocks
    uint16_t *ck_state;
    uint16_t *ck_t;
    GateBlock *ck_gate;
    float *ck_delta;
    // backward
    const uint16_t *dout;
    int64_t ds[3];
    const float *dfinal, *dscores;
    void *dq, *dk, *dv;
    float *dbeta, *dg, *dinitial;
    uint16_t *ws_dstate;  // [B*H*nc] adjoint of the state at each chunk end
    float *ws_n;       // N^T of the adjoint map dS_start = M dS_end + N (f32)
    // Wide path (d_k = d_v = 128, value blocks of 64): per-chunk |k_t|^2 and the
    // value blocks' partial |delta_t|^2 (forward checkpoint).
    float *ck_kk, *ck_ddp;
    // Channel-wise path (16-token chunks): the gates alpha, erase [B,T,H,K] and
    // write [B,T,H,V] (f32 views), the chunk-local cumulative log decay checkpoint,
    // and the per-channel gate gradients.
    View alpha, erase, write;
    struct CwGate *ck_cwg;
    float *ck_lam;
    float *ck_tf;  // T = (I + A)^-1 per 16-token chunk, f32
    float *ck_p;   // P (decay-weighted q.k overlaps, lower, same segment) per chunk, f32
    // Lo parts (x - bf16(x)) of the chunk-start states and the chunk-end state
    // adjoints, kept by the scan when non-null.
    uint16_t *ck_state_lo, *ws_dstate_lo;
    // Document limits (int32 [B,T] views, inclusive) in place of valid/reset:
    // a token is live when end >= start and resets the state when start == t.
    int doc;
    View doc_start, doc_end;
    float *dalpha, *derase, *dwrite;
    // Factored chunk map (the scan of gdn2_chunk_lr.hip): -W'^T [D][C] and
    // Ktil = lam K [C][D] (bf16), U^T [D][C] and the map's diagonal [D] (f32).
    uint16_t *lr_wt, *lr_kt;
    float *lr_u, *lr_gv;
    // Dense chunk map (d = 64 scalar gates): A_c and M = A_c^T rows (bf16 hi
    // then lo), B_c^T (f32).
    uint16_t *map_m, *map_mt;
    float *map_b;
};

// The kernel's ChunkArgs argument, read again from the kernel argument segment;
// only for kernels whose first argument is the ChunkArgs (it sits at offset 0).
// A kernel that walks many chunks calls this at the top of each chunk: behind
// the opaque move the compiler reloads the fields a chunk uses with scalar
// loads, instead of holding every field in SGPRs across the loop, where they
// spill into VGPR lanes.  (In the one-chunk cw_bgrad it measured 3% slower.)
__device__ inline const ChunkArgs &chunk_args_reloaded() {
    typedef const __attribute__((address_space(4))) ChunkArgs KernArgs;
    KernArgs *p = (KernArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const ChunkArgs *)p;
}

inline bool chunk_eligible_shape(const gdn2_shape *s, int chunk) {
    return chunk == CHUNK && s->keys == CHUNK_D && s->values == CHUNK_D;
}

inline int64_t chunk_count(int64_t B, int64_t T, int64_t H) {
    return B * H * ((T + CHUNK - 1) / CHUNK);
}

inline size_t chunk_checkpoint_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)chunk_count(B, T, H) * CK_CHUNK_BYTES;
}

inline size_t chunk_workspace_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)chunk_count(B, T, H) * WS_CHUNK_BYTES;
}

// Carve the checkpoint buffer into its arrays.
inline void chunk_bind_checkpoint(ChunkArgs &a, void *ck) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ck);
    a.ck_state = reinterpret_cast<uint16_t *>(p);
    p += n * CK_STATE_BYTES;
    a.ck_state_lo = reinterpret_cast<uint16_t *>(p);
    p += n * CK_STATE_BYTES;
    a.ck_t = reinterpret_cast<uint16_t *>(p);
    p += n * CK_T_BYTES;
    a.ck_gate = reinterpret_cast<GateBlock *>(p);
    p += n * CK_GATE_BYTES;
    a.ck_delta = reinterpret_cast<float *>(p);
    p += n * CK_DELTA_BYTES;
    a.map_m = reinterpret_cast<uint16_t *>(p);
    p += n * CK_MAP_BYTES;
    a.map_mt = reinterpret_cast<uint16_t *>(p);
    p += n * CK_MAP_BYTES;
    a.map_b = reinterpret_cast<float *>(p);
}

// Carve the backward workspace.
inline void chunk_bind_workspace(ChunkArgs &a, void *ws) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ws);
    a.ws_dstate = reinterpret_cast<uint16_t *>(p);
    p += n * CK_STATE_BYTES;
    a.ws_dstate_lo = reinterpret_cast<uint16_t *>(p);
    p += n * CK_STATE_BYTES;
    a.ws_n = reinterpret_cast<float *>(p);
}

// ---- channel-wise path: per-channel gates, 16-token chunks, d_k = d_v = 64 ------
constexpr int CW_C = 16;  // tokens per chunk
struct CwGate {
    float val[CW_C];
    int seg[CW_C];  // resets at or before the token within the chunk
};

inline bool cw_eligible_shape(const gdn2_shape *s) {
    return s->keys == CHUNK_D && s->values == CHUNK_D;
}

inline int64_t cw_chunk_count(int64_t B, int64_t T, int64_t H) {
    return B * H * ((T + CW_C - 1) / CW_C);
}

// Checkpoint per chunk: S0^T (bf16 hi/lo, 64x64), T and P (f32 16x16), CwGate,
// the cumulative log decay Lambda (f32 16x64), delta (f32 16x64), and the
// factored chunk map: -W'^T and Ktil (bf16 hi and lo, 16x64 each), U^T (f32
// 16x64), b_15 (f32 64).
constexpr size_t CWK_STATE = (size_t)CHUNK_D * CHUNK_D * 2;
constexpr size_t CWK_T = (size_t)CW_C * CW_C * 4;
constexpr size_t CWK_GATE = sizeof(CwGate);
constexpr size_t CWK_LAM = (size_t)CW_C * CHUNK_D * 4;
constexpr size_t CWK_DELTA = (size_t)CW_C * CHUNK_D * 4;
constexpr size_t CWK_LRW = (size_t)CW_C * CHUNK_D * 2 * 2;  // hi and lo
constexpr size_t CWK_LRU = (size_t)CW_C * CHUNK_D * 4;
constexpr size_t CWK_LRG = (size_t)CHUNK_D * 4;
constexpr size_t CWK_MAPN = (size_t)CHUNK_D * CHUNK_D * 4;
constexpr size_t CWK_CHUNK = 2 * CWK_STATE + 2 * CWK_T + CWK_GATE + CWK_LAM + CWK_DELTA + 2 * CWK_LRW +
                             CWK_LRU + CWK_LRG;
constexpr size_t CWW_CHUNK = 2 * CWK_STATE + CWK_MAPN;  // backward: dS^T (bf16 hi/lo), N^T (f32)

inline size_t cw_checkpoint_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)cw_chunk_count(B, T, H) * CWK_CHUNK;
}
inline size_t cw_workspace_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)cw_chunk_count(B, T, H) * CWW_CHUNK;
}

inline void cw_bind_checkpoint(ChunkArgs &a, void *ck) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ck);
    a.ck_state = reinterpret_cast<uint16_t *>(p);
    p += n * CWK_STATE;
    a.ck_state_lo = reinterpret_cast<uint16_t *>(p);
    p += n * CWK_STATE;
    a.ck_tf = reinterpret_cast<float *>(p);
    p += n * CWK_T;
    a.ck_p = reinterpret_cast<float *>(p);
    p += n * CWK_T;
    a.ck_cwg = reinterpret_cast<CwGate *>(p);
    p += n * CWK_GATE;
    a.ck_lam = reinterpret_cast<float *>(p);
    p += n * CWK_LAM;
    a.ck_delta = reinterpret_cast<float *>(p);
    p += n * CWK_DELTA;
    a.lr_wt = reinterpret_cast<uint16_t *>(p);
    p += n * CWK_LRW;
    a.lr_kt = reinterpret_cast<uint16_t *>(p);
    p += n * CWK_LRW;
    a.lr_u = reinterpret_cast<float *>(p);
    p += n * CWK_LRU;
    a.lr_gv = reinterpret_cast<float *>(p);
}

inline void cw_bind_workspace(ChunkArgs &a, void *ws) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ws);
    a.ws_dstate = reinterpret_cast<uint16_t *>(p);
    a.ws_dstate_lo = reinterpret_cast<uint16_t *>(p + n * CWK_STATE);
    a.ws_n = reinterpret_cast<float *>(p + 2 * n * CWK_STATE);
}

// The affine scan over a.nc chunks of per-chunk 64 x 64 maps (gdn2_chunk.hip),
// forward (state) or reverse (adjoint).
hipError_t launch_chunk_scan(const ChunkArgs &a, bool reverse, hipStream_t stream);

hipError_t launch_cw_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);
hipError_t launch_cw_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);

// ---- wide path: d_k = d_v = WIDE_D, value blocks of 64 -------------------------
constexpr int WIDE_D = 128;
constexpr int WIDE_NVB = WIDE_D / 64;

inline bool wide_eligible_shape(const gdn2_shape *s, int chunk) {
    return chunk == CHUNK && s->keys == WIDE_D && s->values == WIDE_D;
}

// Checkpoint per chunk: S0^T (bf16 hi and lo, D x D each), T (bf16 C x C), GateBlock, delta (f32
// C x D), the factored chunk map (-W'^T bf16 C x D; Ktil = lam K as the masked K
// rows, bf16 C x D; U^T f32 C x D; the diagonal f32 D followed by lam f32 C),
// |k|^2 and the value blocks' |delta|^2 (f32 C each).
constexpr size_t WCK_STATE = (size_t)WIDE_D * WIDE_D * 2;
constexpr size_t WCK_T = CK_T_BYTES;
constexpr size_t WCK_GATE = CK_GATE_BYTES;
constexpr size_t WCK_DELTA = (size_t)CHUNK * WIDE_D * 4;
constexpr size_t WCK_LRW = (size_t)CHUNK * WIDE_D * 2;
constexpr size_t WCK_LRK = WCK_LRW;  // K rows (Ktil = lam K)
constexpr size_t WCK_LRU = (size_t)CHUNK * WIDE_D * 4;
constexpr size_t WCK_LRG = (size_t)(WIDE_D + CHUNK) * 4;  // diagonal, then lam
constexpr size_t WCK_MAPN = (size_t)WIDE_D * WIDE_D * 4;
constexpr size_t WCK_NORM = (size_t)CHUNK * (1 + WIDE_NVB) * 4;
constexpr size_t WCK_CHUNK =
    2 * WCK_STATE + WCK_T + WCK_GATE + WCK_DELTA + WCK_LRW + WCK_LRK + WCK_LRU + WCK_LRG + WCK_NORM;
// Backward workspace per chunk: dS^T (bf16 hi and lo) and N^T (f32).
constexpr size_t WWS_CHUNK = 2 * WCK_STATE + WCK_MAPN;

inline size_t wide_checkpoint_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)chunk_count(B, T, H) * WCK_CHUNK;
}

inline size_t wide_workspace_bytes(int64_t B, int64_t T, int64_t H) {
    return (size_t)chunk_count(B, T, H) * WWS_CHUNK;
}

inline void wide_bind_checkpoint(ChunkArgs &a, void *ck) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ck);
    a.ck_state = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_STATE;
    a.ck_state_lo = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_STATE;
    a.ck_t = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_T;
    a.ck_gate = reinterpret_cast<GateBlock *>(p);
    p += n * WCK_GATE;
    a.ck_delta = reinterpret_cast<float *>(p);
    p += n * WCK_DELTA;
    a.lr_wt = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_LRW;
    a.lr_kt = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_LRK;
    a.lr_u = reinterpret_cast<float *>(p);
    p += n * WCK_LRU;
    a.lr_gv = reinterpret_cast<float *>(p);
    p += n * WCK_LRG;
    a.ck_kk = reinterpret_cast<float *>(p);
    a.ck_ddp = a.ck_kk + n * CHUNK;
}

inline void wide_bind_workspace(ChunkArgs &a, void *ws) {
    const int64_t n = (int64_t)a.B * a.H * a.nc;
    char *p = static_cast<char *>(ws);
    a.ws_dstate = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_STATE;
    a.ws_dstate_lo = reinterpret_cast<uint16_t *>(p);
    p += n * WCK_STATE;
    a.ws_n = reinterpret_cast<float *>(p);
}

hipError_t launch_wide_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);
hipError_t launch_wide_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);

// Factored affine scan (gdn2_chunk_lr.hip) over chunks of one (batch, head):
//   forward  X_next = diag(gv) X + Ktil^T (U - W' X),   X0 = initial state
//   reverse  X_prev = diag(gv) X + N - W'^T (Ktil X),   X0 = final-state adjoint
// with X before each step to ckpt[c] (X^T, bf16 hi and, when ckpt_lo is set, lo).
struct LrScanArgs {
    int nc, B, H, vd;      // chunks per head, batch, heads, state columns
    const uint16_t *wt;    // -W'^T per chunk [kd][ct] bf16 (kd x ct = 64 x 16: hi, then lo)
    const uint16_t *kt;    // per chunk: kd = 128, K [ct][kd] bf16 (Ktil = lam K);
                           // kd = 64, Ktil [ct][kd] bf16 hi, then lo
    const float *u;        // U^T per chunk [vd][ct] f32 (forward)
    const float *n;        // N^T per chunk [vd][kd] f32 (reverse)
    const float *gv;       // per chunk: the map's diagonal [kd] f32; kd = 128: then lam [ct]
    uint16_t *ckpt, *ckpt_lo;  // X^T per chunk [vd][kd] bf16
    View x0;               // [B,H,kd,vd] strided (data may be null: zero)
    float *xout;           // [B,H,kd,vd] dense (may be null)
    int reverse;
};
// kd x ct in {128 x 64, 64 x 16}; hipErrorInvalidValue for other shapes.
hipError_t launch_lr_scan(const LrScanArgs &p, int kd, int ct, hipStream_t stream);

// Compute units of the current device (queried once per device); sizes the
// grids of the kernels that walk several chunks per workgroup.
int device_cus();

hipError_t launch_chunk_fwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);
hipError_t launch_chunk_bwd(const ChunkArgs &a, hipStream_t stream, const hipEvent_t *ev);

}  // namespace gdn2
