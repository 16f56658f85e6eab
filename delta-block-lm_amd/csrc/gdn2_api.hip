// C ABI of libgdn2_amd.so: argument validation and kernel dispatch.
//
// Every entry point validates its whole argument list before it launches
// anything, mirroring the reference's fail-fast asserts
// (crates/kernels/src/gdn_training.rs:286-342, :356-390; chunk.rs:110-124):
// an unsupported shape, dtype or buffer size is an error, never a fallback.
#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "gdn2_chunk.h"
#include "gdn2_chunk_f32.h"
#include "gdn2_seq.h"
#include "gdn2_status.h"

namespace gdn2 {

namespace {
thread_local std::string g_error;
}

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int ok() {
    g_error.clear();
    return GDN2_OK;
}

const char *last_error() { return g_error.c_str(); }

int check_view(const gdn2_view *v, const char *name, int dtype, bool data_may_be_null) {
    if (!v) return fail(GDN2_ERR_ARGUMENT, "%s: view is null", name);
    if (!v->data && !data_may_be_null) return fail(GDN2_ERR_ARGUMENT, "%s: data is null", name);
    if (v->dtype != GDN2_F32 && v->dtype != GDN2_BF16 && v->dtype != GDN2_I32)
        return fail(GDN2_ERR_DTYPE, "%s: unknown dtype %d", name, v->dtype);
    if (dtype < 0 && v->dtype == GDN2_I32)
        return fail(GDN2_ERR_DTYPE, "%s: dtype must be F32 or BF16", name);
    if (dtype >= 0 && v->dtype != dtype)
        return fail(GDN2_ERR_DTYPE, "%s: dtype must be %s", name,
                    dtype == GDN2_F32 ? "F32" : (dtype == GDN2_BF16 ? "BF16" : "I32"));
    for (int d = 0; d < 4; ++d)
        if (v->stride[d] < 0) return fail(GDN2_ERR_ARGUMENT, "%s: negative stride", name);
    return GDN2_OK;
}

int launch_status(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(GDN2_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

}  // namespace gdn2

using namespace gdn2;

namespace {

// Stage timing (gdn2_stage_timing): six stages, an event pair each; the
// forward records pairs 0-2, the backward pairs 3-5.  A measurement hook for
// benchmarks only: the events and flags below are process-wide (not thread
// safe), and no event is recorded on a stream that is being captured, so a
// graph never holds them.
constexpr int kStages = 6;
const char *const kStageNames[kStages] = {"chunk_prep", "state_scan", "chunk_out",
                                          "chunk_bprep", "adjoint_scan", "chunk_bgrad"};
hipEvent_t g_stage_ev[2 * kStages];
bool g_stage_ready = false;  // events created
bool g_stage_on = false;
bool g_stage_ran[kStages];

const hipEvent_t *stage_events(int first_stage, hipStream_t stream) {
    if (!g_stage_on) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return nullptr;
    for (int i = 0; i < 3; ++i) g_stage_ran[first_stage + i] = true;
    return g_stage_ev + 2 * first_stage;
}

int check_shape(const gdn2_shape *s) {
    if (!s) return fail(GDN2_ERR_ARGUMENT, "shape is null");
    if (s->batch <= 0 || s->time <= 0 || s->heads <= 0)
        return fail(GDN2_ERR_SHAPE, "GDN-2 requires nonempty axes (batch=%lld time=%lld heads=%lld)",
                    (long long)s->batch, (long long)s->time, (long long)s->heads);
    if (s->keys < 1 || s->keys > 128 || s->values < 1 || s->values > 128)
        return fail(GDN2_ERR_SHAPE, "key/value widths must be 1..128 (keys=%lld values=%lld)",
                    (long long)s->keys, (long long)s->values);
    if (s->batch * s->heads > INT_MAX || s->time > INT_MAX / 2)
        return fail(GDN2_ERR_SHAPE, "batch*heads or time exceeds the launch limits");
    return GDN2_OK;
}

int check_chunk(int chunk) {
    if (chunk < 1 || chunk > 64) return fail(GDN2_ERR_ARGUMENT, "chunk must be 1..64 (got %d)", chunk);
    return GDN2_OK;
}

int check_out_dtype(int32_t dt) {
    if (dt != GDN2_F32 && dt != GDN2_BF16) return fail(GDN2_ERR_DTYPE, "output dtype must be F32 or BF16");
    return GDN2_OK;
}

size_t seq_checkpoint_bytes(const gdn2_shape *s) {
    return (size_t)seq_checkpoint_floats(s->batch, s->time, s->heads, (int)s->keys,
                                         (int)s->values) * 4;
}

size_t seq_workspace_bytes(const gdn2_shape *s) {
    return (size_t)seq_workspace_floats(s->batch, s->heads, (int)s->keys, (int)s->values) * 4;
}

int check_channel_inputs(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                         const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                         const gdn2_view *write, const gdn2_view *valid, const gdn2_view *reset) {
    GDN2_TRY(check_view(q, "q", -1, false));
    GDN2_TRY(check_view(k, "k", q->dtype, false));
    GDN2_TRY(check_view(v, "v", q->dtype, false));
    GDN2_TRY(check_view(alpha, "alpha", GDN2_F32, false));
    GDN2_TRY(check_view(erase, "erase", GDN2_F32, false));
    GDN2_TRY(check_view(write, "write", GDN2_F32, false));
    GDN2_TRY(check_view(valid, "valid", GDN2_F32, false));
    GDN2_TRY(check_view(reset, "reset", GDN2_F32, false));
    return GDN2_OK;
}

int check_doc_inputs(const gdn2_view *q, const gdn2_view *k, const gdn2_view *v,
                     const gdn2_view *alpha, const gdn2_view *erase, const gdn2_view *write,
                     const gdn2_view *doc_start, const gdn2_view *doc_end) {
    GDN2_TRY(check_view(q, "q", -1, false));
    GDN2_TRY(check_view(k, "k", q->dtype, false));
    GDN2_TRY(check_view(v, "v", q->dtype, false));
    GDN2_TRY(check_view(alpha, "alpha", GDN2_F32, false));
    GDN2_TRY(check_view(erase, "erase", GDN2_F32, false));
    GDN2_TRY(check_view(write, "write", GDN2_F32, false));
    GDN2_TRY(check_view(doc_start, "doc_start", GDN2_I32, false));
    GDN2_TRY(check_view(doc_end, "doc_end", GDN2_I32, false));
    return GDN2_OK;
}

SeqArgs seq_args(const gdn2_shape *s, const gdn2_view *q, const gdn2_view *k, const gdn2_view *v,
                 const gdn2_view *alpha, const gdn2_view *erase, const gdn2_view *write,
                 const gdn2_view *valid, const gdn2_view *reset) {
    SeqArgs a{};
    a.B = (int)s->batch;
    a.T = (int)s->time;
    a.H = (int)s->heads;
    a.K = (int)s->keys;
    a.V = (int)s->values;
    a.q = make_view(q);
    a.k = make_view(k);
    a.v = make_view(v);
    a.alpha = make_view(alpha);
    a.erase = make_view(erase);
    a.write = make_view(write);
    a.valid = make_view(valid);
    a.reset = make_view(reset);
    a.nck = (a.T + SEQ_CT - 1) / SEQ_CT;
    return a;
}

}  // namespace

// Device scratch of gdn_scalar_backward_noalloc: a fixed array in every
// device's copy of the code object, held until the process ends.  Host code
// never uses the array's name as an address: each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static __device__ __align__(256) unsigned char scratch[GDN2_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // per device, null until first use

int noalloc_scratch(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(GDN2_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(GDN2_ERR_ARGUMENT, "device ordinal %d outside 0..%d", dev, kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(GDN2_ERR_LAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GDN2_OK;
}
}  // namespace

static int scalar_backward_impl(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                                const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                                const gdn2_view *g, const gdn2_view *valid,
                                const gdn2_view *reset, const void *checkpoint,
                                size_t checkpoint_bytes, const gdn2_view *d_output,
                                const float *d_final_state, const float *d_scores, void *dq,
                                void *dk, void *dv, float *dbeta, float *dg, float *d_initial,
                                void *workspace, size_t workspace_bytes, void *stream);

// The chunk kernels take bf16 q/k/v with unit channel stride and 16-byte
// aligned token rows (every stride a multiple of 8 elements).
static bool rows_aligned(const gdn2_view *v) {
    return v->stride[3] == 1 && ((uintptr_t)v->data & 15) == 0 && v->stride[0] % 8 == 0 &&
           v->stride[1] % 8 == 0 && v->stride[2] % 8 == 0;
}

// The channel-wise op runs the 16-token chunk-WY MFMA kernels
// (gdn2_chunk_cw.hip) for bf16 q/k/v with d_k = d_v = 64 and aligned rows,
// whatever the chunk argument (the chunking changes no result).  Forward and backward apply the
// same rule, so the checkpoint format always matches.
static bool use_cw_path(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                        const gdn2_view *v) {
    return cw_eligible_shape(shape) && q->dtype == GDN2_BF16 && rows_aligned(q) &&
           rows_aligned(k) && rows_aligned(v);
}

// Otherwise f32 or bf16 q/k/v of any width (d_k, d_v <= 128) run the f32 chunk
// kernels (gdn2_chunk_f32.hip; any element strides; bf16 inputs are read as
// their exact f32 values and the gradients written back as bf16), again
// whatever the chunk argument.
static bool use_fc_path(const gdn2_shape *shape, const gdn2_view *q) {
    return fc_eligible_shape(shape) && (q->dtype == GDN2_F32 || q->dtype == GDN2_BF16);
}

// The checkpoint and workspace sizes do not depend on the dtype: each is the
// largest that any kernel family eligible for the shape needs.
static size_t training_checkpoint_bytes(const gdn2_shape *s) {
    const size_t c = cw_eligible_shape(s) ? cw_checkpoint_bytes(s->batch, s->time, s->heads) : 0;
    const size_t f = fc_eligible_shape(s) ? fc_checkpoint_bytes(s->batch, s->time, s->heads,
                                                                (int)s->keys, (int)s->values)
                                          : 0;
    const size_t q = seq_checkpoint_bytes(s);
    return std::max(c, std::max(f, q));
}

static size_t training_workspace_bytes(const gdn2_shape *s) {
    const size_t c = cw_eligible_shape(s) ? cw_workspace_bytes(s->batch, s->time, s->heads) : 0;
    const size_t f = fc_eligible_shape(s) ? fc_workspace_bytes(s->batch, s->time, s->heads,
                                                               (int)s->keys, (int)s->values)
                                          : 0;
    const size_t q = seq_workspace_bytes(s);
    return std::max(c, std::max(f, q));
}

// The f32 chunk path's argument block over the token-sequential one.
static FcArgs fc_args(const SeqArgs &s, const gdn2_view *q, void *checkpoint, void *workspace) {
    FcArgs f{};
    f.s = s;
    f.in_bf16 = q->dtype == GDN2_BF16;
    f.nc = (s.T + FC_C - 1) / FC_C;
    fc_bind(f, checkpoint, workspace);
    return f;
}

static ChunkArgs cw_args(const gdn2_shape *s, const gdn2_view *q, const gdn2_view *k,
                         const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                         const gdn2_view *write, const gdn2_view *valid, const gdn2_view *reset) {
    ChunkArgs a{};
    a.B = (int)s->batch;
    a.T = (int)s->time;
    a.H = (int)s->heads;
    a.nc = (a.T + CW_C - 1) / CW_C;
    a.q = (const uint16_t *)q->data;
    a.k = (const uint16_t *)k->data;
    a.v = (const uint16_t *)v->data;
    for (int d = 0; d < 3; ++d) {
        a.qs[d] = q->stride[d];
        a.ks[d] = k->stride[d];
        a.vs[d] = v->stride[d];
    }
    a.alpha = make_view(alpha);
    a.erase = make_view(erase);
    a.write = make_view(write);
    a.valid = make_view(valid);
    a.reset = make_view(reset);
    return a;
}

extern "C" {

int gdn2_abi_version(void) { return 101; }

const char *gdn2_last_error(void) { return gdn2::last_error(); }

size_t gdn2_training_checkpoint_bytes(const gdn2_shape *shape, int chunk) {
    if (check_shape(shape) || check_chunk(chunk)) return 0;
    return training_checkpoint_bytes(shape);  // large enough for either kernel family
}

size_t gdn2_training_workspace_bytes(const gdn2_shape *shape, int chunk) {
    if (check_shape(shape) || check_chunk(chunk)) return 0;
    return training_workspace_bytes(shape);
}

int gdn2_training_scan(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                       const gdn2_view *k, const gdn2_view *v, const gdn2_view *alpha,
                       const gdn2_view *erase, const gdn2_view *write, const gdn2_view *valid,
                       const gdn2_view *reset, const gdn2_view *initial, void *output,
                       int32_t output_dtype, float *final_state, float *scores, void *checkpoint,
                       size_t checkpoint_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_chunk(chunk));
    GDN2_TRY(check_channel_inputs(shape, q, k, v, alpha, erase, write, valid, reset));
    GDN2_TRY(check_view(initial, "initial", GDN2_F32, true));
    GDN2_TRY(check_out_dtype(output_dtype));
    if (!output || !final_state || !scores)
        return fail(GDN2_ERR_ARGUMENT, "output, final_state and scores must be non-null");
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if ((uintptr_t)checkpoint & 15) return fail(GDN2_ERR_ARGUMENT, "checkpoint must be 16-byte aligned");
    if (checkpoint_bytes < training_checkpoint_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    training_checkpoint_bytes(shape), checkpoint_bytes);
    if (use_cw_path(shape, q, k, v)) {
        ChunkArgs c = cw_args(shape, q, k, v, alpha, erase, write, valid, reset);
        c.initial = make_view(initial);
        c.out = output;
        c.out_bf16 = output_dtype == GDN2_BF16;
        c.final_state = final_state;
        c.scores = scores;
        cw_bind_checkpoint(c, checkpoint);
        const hipEvent_t *ev = stage_events(0, (hipStream_t)stream);
        return launch_status(launch_cw_fwd(c, (hipStream_t)stream, ev), "gdn2_training_scan");
    }
    SeqArgs a = seq_args(shape, q, k, v, alpha, erase, write, valid, reset);
    a.initial = make_view(initial);
    a.out = output;
    a.out_bf16 = output_dtype == GDN2_BF16;
    a.final_state = final_state;
    a.scores = scores;
    if (use_fc_path(shape, q)) {
        const FcArgs f = fc_args(a, q, checkpoint, nullptr);
        const hipEvent_t *ev = stage_events(0, (hipStream_t)stream);
        return launch_status(launch_fc_fwd(f, (hipStream_t)stream, ev), "gdn2_training_scan");
    }
    seq_bind_checkpoint(a, checkpoint);
    return launch_status(launch_seq_fwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn2_training_scan");
}

int gdn2_training_backward(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                           const gdn2_view *k, const gdn2_view *v, const gdn2_view *alpha,
                           const gdn2_view *erase, const gdn2_view *write,
                           const gdn2_view *valid, const gdn2_view *reset,
                           const void *checkpoint, size_t checkpoint_bytes,
                           const gdn2_view *d_output, const float *d_final_state,
                           const float *d_scores, void *dq, void *dk, void *dv, float *dalpha,
                           float *derase, float *dwrite, float *d_initial, void *workspace,
                           size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_chunk(chunk));
    GDN2_TRY(check_channel_inputs(shape, q, k, v, alpha, erase, write, valid, reset));
    if (d_output) GDN2_TRY(check_view(d_output, "d_output", q->dtype, true));
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if ((uintptr_t)checkpoint & 15) return fail(GDN2_ERR_ARGUMENT, "checkpoint must be 16-byte aligned");
    if (checkpoint_bytes < training_checkpoint_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    training_checkpoint_bytes(shape), checkpoint_bytes);
    if (!workspace) return fail(GDN2_ERR_ARGUMENT, "workspace is null");
    if ((uintptr_t)workspace & 15) return fail(GDN2_ERR_ARGUMENT, "workspace must be 16-byte aligned");
    if (workspace_bytes < training_workspace_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    training_workspace_bytes(shape), workspace_bytes);
    if (use_cw_path(shape, q, k, v)) {
        if (d_output && d_output->data && !rows_aligned(d_output))
            return fail(GDN2_ERR_ARGUMENT,
                        "d_output needs unit channel stride and 16-byte aligned rows on the "
                        "chunked path (bf16, d_k = d_v = 64)");
        ChunkArgs c = cw_args(shape, q, k, v, alpha, erase, write, valid, reset);
        cw_bind_checkpoint(c, const_cast<void *>(checkpoint));
        cw_bind_workspace(c, workspace);
        if (d_output && d_output->data) {
            c.dout = (const uint16_t *)d_output->data;
            for (int d = 0; d < 3; ++d) c.ds[d] = d_output->stride[d];
        }
        c.dfinal = d_final_state;
        c.dscores = d_scores;
        c.dq = dq;
        c.dk = dk;
        c.dv = dv;
        c.dalpha = dalpha;
        c.derase = derase;
        c.dwrite = dwrite;
        c.dinitial = d_initial;
        const hipEvent_t *ev = stage_events(3, (hipStream_t)stream);
        return launch_status(launch_cw_bwd(c, (hipStream_t)stream, ev), "gdn2_training_backward");
    }
    SeqArgs a = seq_args(shape, q, k, v, alpha, erase, write, valid, reset);
    if (d_output) a.dout = make_view(d_output);
    a.dfinal = d_final_state;
    a.dscores = d_scores;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.dalpha = dalpha;
    a.derase = derase;
    a.dwrite = dwrite;
    a.dinitial = d_initial;
    if (use_fc_path(shape, q)) {
        const FcArgs f = fc_args(a, q, const_cast<void *>(checkpoint), workspace);
        const hipEvent_t *ev = stage_events(3, (hipStream_t)stream);
        return launch_status(launch_fc_bwd(f, (hipStream_t)stream, ev), "gdn2_training_backward");
    }
    seq_bind_checkpoint(a, checkpoint);
    a.replay = (float *)workspace;
    return launch_status(launch_seq_bwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn2_training_backward");
}

size_t gdn2_scan_checkpoint_bytes(const gdn2_shape *shape) {
    if (check_shape(shape)) return 0;
    return training_checkpoint_bytes(shape);
}

size_t gdn2_scan_workspace_bytes(const gdn2_shape *shape) {
    if (check_shape(shape)) return 0;
    return training_workspace_bytes(shape);
}

int gdn2_scan(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k, const gdn2_view *v,
              const gdn2_view *alpha, const gdn2_view *erase, const gdn2_view *write,
              const gdn2_view *doc_start, const gdn2_view *doc_end, void *output,
              int32_t output_dtype, void *checkpoint, size_t checkpoint_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_doc_inputs(q, k, v, alpha, erase, write, doc_start, doc_end));
    GDN2_TRY(check_out_dtype(output_dtype));
    if (!output) return fail(GDN2_ERR_ARGUMENT, "output is null");
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if ((uintptr_t)checkpoint & 15) return fail(GDN2_ERR_ARGUMENT, "checkpoint must be 16-byte aligned");
    if (checkpoint_bytes < training_checkpoint_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    training_checkpoint_bytes(shape), checkpoint_bytes);
    if (use_cw_path(shape, q, k, v)) {
        ChunkArgs c = cw_args(shape, q, k, v, alpha, erase, write, nullptr, nullptr);
        c.doc = 1;
        c.doc_start = make_view(doc_start);
        c.doc_end = make_view(doc_end);
        c.out = output;
        c.out_bf16 = output_dtype == GDN2_BF16;
        cw_bind_checkpoint(c, checkpoint);
        const hipEvent_t *ev = stage_events(0, (hipStream_t)stream);
        return launch_status(launch_cw_fwd(c, (hipStream_t)stream, ev), "gdn2_scan");
    }
    SeqArgs a = seq_args(shape, q, k, v, alpha, erase, write, nullptr, nullptr);
    a.doc = 1;
    a.doc_start = make_view(doc_start);
    a.doc_end = make_view(doc_end);
    a.out = output;
    a.out_bf16 = output_dtype == GDN2_BF16;
    if (use_fc_path(shape, q)) {
        const FcArgs f = fc_args(a, q, checkpoint, nullptr);
        const hipEvent_t *ev = stage_events(0, (hipStream_t)stream);
        return launch_status(launch_fc_fwd(f, (hipStream_t)stream, ev), "gdn2_scan");
    }
    seq_bind_checkpoint(a, checkpoint);
    return launch_status(launch_seq_fwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn2_scan");
}

int gdn2_backward(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                  const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                  const gdn2_view *write, const gdn2_view *doc_start, const gdn2_view *doc_end,
                  const void *checkpoint, size_t checkpoint_bytes, const gdn2_view *d_output,
                  void *dq, void *dk, void *dv, float *dalpha, float *derase, float *dwrite,
                  void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_doc_inputs(q, k, v, alpha, erase, write, doc_start, doc_end));
    if (d_output) GDN2_TRY(check_view(d_output, "d_output", q->dtype, true));
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if ((uintptr_t)checkpoint & 15) return fail(GDN2_ERR_ARGUMENT, "checkpoint must be 16-byte aligned");
    if (checkpoint_bytes < training_checkpoint_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    training_checkpoint_bytes(shape), checkpoint_bytes);
    if (!workspace) return fail(GDN2_ERR_ARGUMENT, "workspace is null");
    if ((uintptr_t)workspace & 15) return fail(GDN2_ERR_ARGUMENT, "workspace must be 16-byte aligned");
    if (workspace_bytes < training_workspace_bytes(shape))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    training_workspace_bytes(shape), workspace_bytes);
    if (use_cw_path(shape, q, k, v)) {
        if (d_output && d_output->data && !rows_aligned(d_output))
            return fail(GDN2_ERR_ARGUMENT,
                        "d_output needs unit channel stride and 16-byte aligned rows on the "
                        "chunked path (bf16, d_k = d_v = 64)");
        ChunkArgs c = cw_args(shape, q, k, v, alpha, erase, write, nullptr, nullptr);
        c.doc = 1;
        c.doc_start = make_view(doc_start);
        c.doc_end = make_view(doc_end);
        cw_bind_checkpoint(c, const_cast<void *>(checkpoint));
        cw_bind_workspace(c, workspace);
        if (d_output && d_output->data) {
            c.dout = (const uint16_t *)d_output->data;
            for (int d = 0; d < 3; ++d) c.ds[d] = d_output->stride[d];
        }
        c.dq = dq;
        c.dk = dk;
        c.dv = dv;
        c.dalpha = dalpha;
        c.derase = derase;
        c.dwrite = dwrite;
        const hipEvent_t *ev = stage_events(3, (hipStream_t)stream);
        return launch_status(launch_cw_bwd(c, (hipStream_t)stream, ev), "gdn2_backward");
    }
    SeqArgs a = seq_args(shape, q, k, v, alpha, erase, write, nullptr, nullptr);
    a.doc = 1;
    a.doc_start = make_view(doc_start);
    a.doc_end = make_view(doc_end);
    if (d_output) a.dout = make_view(d_output);
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.dalpha = dalpha;
    a.derase = derase;
    a.dwrite = dwrite;
    if (use_fc_path(shape, q)) {
        const FcArgs f = fc_args(a, q, const_cast<void *>(checkpoint), workspace);
        const hipEvent_t *ev = stage_events(3, (hipStream_t)stream);
        return launch_status(launch_fc_bwd(f, (hipStream_t)stream, ev), "gdn2_backward");
    }
    seq_bind_checkpoint(a, checkpoint);
    a.replay = (float *)workspace;
    return launch_status(launch_seq_bwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn2_backward");
}

size_t gdn_scalar_checkpoint_bytes(const gdn2_shape *shape, int chunk) {
    if (check_shape(shape) || check_chunk(chunk)) return 0;
    // Large enough for whichever kernel family the call will select.
    size_t c = 0;
    if (chunk_eligible_shape(shape, chunk))
        c = chunk_checkpoint_bytes(shape->batch, shape->time, shape->heads);
    else if (wide_eligible_shape(shape, chunk))
        c = wide_checkpoint_bytes(shape->batch, shape->time, shape->heads);
    const size_t q = seq_checkpoint_bytes(shape);
    return c > q ? c : q;
}

size_t gdn_scalar_workspace_bytes(const gdn2_shape *shape, int chunk) {
    if (check_shape(shape) || check_chunk(chunk)) return 0;
    size_t c = 0;
    if (chunk_eligible_shape(shape, chunk))
        c = chunk_workspace_bytes(shape->batch, shape->time, shape->heads);
    else if (wide_eligible_shape(shape, chunk))
        c = wide_workspace_bytes(shape->batch, shape->time, shape->heads);
    const size_t q = seq_workspace_bytes(shape);
    return c > q ? c : q;
}

// The chunk-WY MFMA kernels take bf16 q/k/v with d_k = d_v = 64 (gdn2_chunk.hip)
// or 128 (gdn2_chunk_wide.hip), chunk 64, unit channel stride and 16-byte
// aligned token rows; everything else runs the token-sequential kernels.
// Forward and backward apply the same rule, so the checkpoint format always
// matches.

static bool use_chunk_path(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                           const gdn2_view *k, const gdn2_view *v) {
    return (chunk_eligible_shape(shape, chunk) || wide_eligible_shape(shape, chunk)) &&
           q->dtype == GDN2_BF16 && rows_aligned(q) && rows_aligned(k) && rows_aligned(v);
}

static ChunkArgs chunk_args(const gdn2_shape *s, const gdn2_view *q, const gdn2_view *k,
                            const gdn2_view *v, const gdn2_view *beta, const gdn2_view *g,
                            const gdn2_view *valid, const gdn2_view *reset) {
    ChunkArgs a{};
    a.B = (int)s->batch;
    a.T = (int)s->time;
    a.H = (int)s->heads;
    a.nc = (a.T + CHUNK - 1) / CHUNK;
    a.q = (const uint16_t *)q->data;
    a.k = (const uint16_t *)k->data;
    a.v = (const uint16_t *)v->data;
    for (int d = 0; d < 3; ++d) {
        a.qs[d] = q->stride[d];
        a.ks[d] = k->stride[d];
        a.vs[d] = v->stride[d];
    }
    a.beta = make_view(beta);
    a.g = make_view(g);
    a.valid = make_view(valid);
    a.reset = make_view(reset);
    return a;
}

static int check_scalar_inputs(const gdn2_view *q, const gdn2_view *k, const gdn2_view *v,
                               const gdn2_view *beta, const gdn2_view *g,
                               const gdn2_view *valid, const gdn2_view *reset) {
    GDN2_TRY(check_view(q, "q", -1, false));
    GDN2_TRY(check_view(k, "k", q->dtype, false));
    GDN2_TRY(check_view(v, "v", q->dtype, false));
    GDN2_TRY(check_view(beta, "beta", GDN2_F32, false));
    GDN2_TRY(check_view(g, "g", GDN2_F32, false));
    GDN2_TRY(check_view(valid, "valid", GDN2_F32, false));
    GDN2_TRY(check_view(reset, "reset", GDN2_F32, false));
    return GDN2_OK;
}

int gdn_scalar_scan(const gdn2_shape *shape, int chunk, const gdn2_view *q, const gdn2_view *k,
                    const gdn2_view *v, const gdn2_view *beta, const gdn2_view *g,
                    const gdn2_view *valid, const gdn2_view *reset, const gdn2_view *initial,
                    void *output, int32_t output_dtype, float *final_state, float *scores,
                    void *checkpoint, size_t checkpoint_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_chunk(chunk));
    GDN2_TRY(check_scalar_inputs(q, k, v, beta, g, valid, reset));
    GDN2_TRY(check_view(initial, "initial", GDN2_F32, true));
    GDN2_TRY(check_out_dtype(output_dtype));
    if (!output || !final_state || !scores)
        return fail(GDN2_ERR_ARGUMENT, "output, final_state and scores must be non-null");
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if (checkpoint_bytes < gdn_scalar_checkpoint_bytes(shape, chunk))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    gdn_scalar_checkpoint_bytes(shape, chunk), checkpoint_bytes);
    if (use_chunk_path(shape, chunk, q, k, v)) {
        ChunkArgs c = chunk_args(shape, q, k, v, beta, g, valid, reset);
        c.initial = make_view(initial);
        c.out = output;
        c.out_bf16 = output_dtype == GDN2_BF16;
        c.final_state = final_state;
        c.scores = scores;
        const hipEvent_t *ev = stage_events(0, (hipStream_t)stream);
        if (wide_eligible_shape(shape, chunk)) {
            wide_bind_checkpoint(c, checkpoint);
            return launch_status(launch_wide_fwd(c, (hipStream_t)stream, ev), "gdn_scalar_scan");
        }
        chunk_bind_checkpoint(c, checkpoint);
        return launch_status(launch_chunk_fwd(c, (hipStream_t)stream, ev), "gdn_scalar_scan");
    }
    SeqArgs a = seq_args(shape, q, k, v, beta, beta, beta, valid, reset);
    a.scalar = 1;
    a.beta = make_view(beta);
    a.g = make_view(g);
    a.initial = make_view(initial);
    a.out = output;
    a.out_bf16 = output_dtype == GDN2_BF16;
    a.final_state = final_state;
    a.scores = scores;
    seq_bind_checkpoint(a, checkpoint);
    return launch_status(launch_seq_fwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn_scalar_scan");
}

int gdn_scalar_backward(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                        const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                        const gdn2_view *g, const gdn2_view *valid, const gdn2_view *reset,
                        const void *checkpoint, size_t checkpoint_bytes,
                        const gdn2_view *d_output, const float *d_final_state,
                        const float *d_scores, void *dq, void *dk, void *dv, float *dbeta,
                        float *dg, float *d_initial, void *workspace, size_t workspace_bytes,
                        void *stream) {
    return scalar_backward_impl(shape, chunk, q, k, v, beta, g, valid, reset, checkpoint,
                                checkpoint_bytes, d_output, d_final_state, d_scores, dq, dk, dv,
                                dbeta, dg, d_initial, workspace, workspace_bytes, stream);
}

int gdn_scalar_backward_noalloc(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                                const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                                const gdn2_view *g, const gdn2_view *valid,
                                const gdn2_view *reset, const void *checkpoint,
                                size_t checkpoint_bytes, const gdn2_view *d_output,
                                const float *d_final_state, const float *d_scores, void *dq,
                                void *dk, void *dv, float *dbeta, float *dg, float *d_initial,
                                void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_chunk(chunk));
    const size_t need = gdn_scalar_workspace_bytes(shape, chunk);
    if (need > GDN2_NOALLOC_SCRATCH_BYTES)
        return fail(GDN2_ERR_WORKSPACE,
                    "gdn_scalar_backward_noalloc: this shape needs %zu bytes of scratch, above "
                    "the library's fixed %zu-byte device scratch; call gdn_scalar_backward "
                    "with a workspace instead",
                    need, (size_t)GDN2_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    GDN2_TRY(noalloc_scratch(&ws));
    return scalar_backward_impl(shape, chunk, q, k, v, beta, g, valid, reset, checkpoint,
                                checkpoint_bytes, d_output, d_final_state, d_scores, dq, dk, dv,
                                dbeta, dg, d_initial, ws, GDN2_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"

static int scalar_backward_impl(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                                const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                                const gdn2_view *g, const gdn2_view *valid,
                                const gdn2_view *reset, const void *checkpoint,
                                size_t checkpoint_bytes, const gdn2_view *d_output,
                                const float *d_final_state, const float *d_scores, void *dq,
                                void *dk, void *dv, float *dbeta, float *dg, float *d_initial,
                                void *workspace, size_t workspace_bytes, void *stream) {
    GDN2_TRY(check_shape(shape));
    GDN2_TRY(check_chunk(chunk));
    GDN2_TRY(check_scalar_inputs(q, k, v, beta, g, valid, reset));
    if (d_output) GDN2_TRY(check_view(d_output, "d_output", q->dtype, true));
    if (!checkpoint) return fail(GDN2_ERR_ARGUMENT, "checkpoint is null");
    if (checkpoint_bytes < gdn_scalar_checkpoint_bytes(shape, chunk))
        return fail(GDN2_ERR_WORKSPACE, "checkpoint needs %zu bytes, got %zu",
                    gdn_scalar_checkpoint_bytes(shape, chunk), checkpoint_bytes);
    if (!workspace) return fail(GDN2_ERR_ARGUMENT, "workspace is null");
    if (workspace_bytes < gdn_scalar_workspace_bytes(shape, chunk))
        return fail(GDN2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu",
                    gdn_scalar_workspace_bytes(shape, chunk), workspace_bytes);
    if (use_chunk_path(shape, chunk, q, k, v)) {
        if (d_output && d_output->data && !rows_aligned(d_output))
            return fail(GDN2_ERR_ARGUMENT,
                        "d_output needs unit channel stride and 16-byte aligned rows on the "
                        "chunked path (chunk 64, bf16, d_k = d_v = 64 or 128)");
        ChunkArgs c = chunk_args(shape, q, k, v, beta, g, valid, reset);
        const bool wide = wide_eligible_shape(shape, chunk);
        if (wide) {
            wide_bind_checkpoint(c, const_cast<void *>(checkpoint));
            wide_bind_workspace(c, workspace);
        } else {
            chunk_bind_checkpoint(c, const_cast<void *>(checkpoint));
            chunk_bind_workspace(c, workspace);
        }
        if (d_output && d_output->data) {
            c.dout = (const uint16_t *)d_output->data;
            for (int d = 0; d < 3; ++d) c.ds[d] = d_output->stride[d];
        }
        c.dfinal = d_final_state;
        c.dscores = d_scores;
        c.dq = dq;
        c.dk = dk;
        c.dv = dv;
        c.dbeta = dbeta;
        c.dg = dg;
        c.dinitial = d_initial;
        const hipEvent_t *ev = stage_events(3, (hipStream_t)stream);
        return launch_status(wide ? launch_wide_bwd(c, (hipStream_t)stream, ev)
                                  : launch_chunk_bwd(c, (hipStream_t)stream, ev),
                             "gdn_scalar_backward");
    }
    SeqArgs a = seq_args(shape, q, k, v, beta, beta, beta, valid, reset);
    a.scalar = 1;
    a.beta = make_view(beta);
    a.g = make_view(g);
    seq_bind_checkpoint(a, checkpoint);
    if (d_output) a.dout = make_view(d_output);
    a.dfinal = d_final_state;
    a.dscores = d_scores;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.dbeta = dbeta;
    a.dg = dg;
    a.dinitial = d_initial;
    a.replay = (float *)workspace;
    return launch_status(launch_seq_bwd(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn_scalar_backward");
}

extern "C" {

int gdn2_stage_timing(int enable) {
    if (enable && !g_stage_ready) {
        for (int i = 0; i < 2 * kStages; ++i) {
            const hipError_t e = hipEventCreate(&g_stage_ev[i]);
            if (e != hipSuccess) {
                for (int j = 0; j < i; ++j) (void)hipEventDestroy(g_stage_ev[j]);
                return fail(GDN2_ERR_LAUNCH, "gdn2_stage_timing: hipEventCreate: %s",
                            hipGetErrorString(e));
            }
        }
        g_stage_ready = true;
    }
    for (int i = 0; i < kStages; ++i) g_stage_ran[i] = false;
    g_stage_on = enable != 0;
    return ok();
}

int gdn2_stage_count(void) { return kStages; }

const char *gdn2_stage_name(int stage) {
    return stage >= 0 && stage < kStages ? kStageNames[stage] : nullptr;
}

float gdn2_stage_ms(int stage) {
    if (stage < 0 || stage >= kStages || !g_stage_ready || !g_stage_ran[stage]) return -1.f;
    float ms = -1.f;
    if (hipEventElapsedTime(&ms, g_stage_ev[2 * stage], g_stage_ev[2 * stage + 1]) != hipSuccess)
        return -1.f;
    return ms;
}

int gdn2_decode_step(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                     const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                     const gdn2_view *write, const gdn2_view *valid, const gdn2_view *reset,
                     float *state, void *output, int32_t output_dtype, float *scores,
                     void *stream) {
    GDN2_TRY(check_shape(shape));
    if (shape->time != 1) return fail(GDN2_ERR_SHAPE, "decode step needs time == 1");
    GDN2_TRY(check_view(q, "q", -1, false));
    GDN2_TRY(check_view(k, "k", q->dtype, false));
    GDN2_TRY(check_view(v, "v", q->dtype, false));
    GDN2_TRY(check_view(alpha, "alpha", GDN2_F32, false));
    GDN2_TRY(check_view(erase, "erase", GDN2_F32, false));
    GDN2_TRY(check_view(write, "write", GDN2_F32, false));
    if (valid) GDN2_TRY(check_view(valid, "valid", GDN2_F32, true));
    if (reset) GDN2_TRY(check_view(reset, "reset", GDN2_F32, true));
    GDN2_TRY(check_out_dtype(output_dtype));
    if (!state || !output || !scores)
        return fail(GDN2_ERR_ARGUMENT, "state, output and scores must be non-null");
    SeqArgs a = seq_args(shape, q, k, v, alpha, erase, write, valid, reset);
    if (!valid) a.valid.data = nullptr;
    if (!reset) a.reset.data = nullptr;
    const int64_t K = shape->keys, V = shape->values;
    gdn2_view st{state, GDN2_F32, 0, {shape->heads * K * V, K * V, V, 1}};
    a.initial = make_view(&st);
    a.final_state = state;  // each workgroup reads its slice before writing it
    a.out = output;
    a.out_bf16 = output_dtype == GDN2_BF16;
    a.scores = scores;
    seq_bind_checkpoint(a, nullptr);
    return launch_status(launch_seq_decode(a, q->dtype == GDN2_BF16, (hipStream_t)stream),
                         "gdn2_decode_step");
}

}  // extern "C"
