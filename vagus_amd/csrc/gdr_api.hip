// extern "C" entry points of libvagus_gdr.so (declared in include/vagus_gdr.h).
// Argument checking, status codes, the per-thread error string, and the
// dispatch to the kernel launchers.  Nothing here allocates or synchronises.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/vagus_gdr.h"
#include "gdr_kernels.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return VGDR_OK;
    return fail(VGDR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// checks shared by both scan entry points; returns VGDR_OK or an error code
int check_common(const char *fn, int dtype, int gate_kind, int use_delta, const void *q, const void *k,
                 const void *v, const float *g, const float *beta, const void *o,
                 const int32_t *cu, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                 int64_t n_seqs) {
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
    if (gate_kind < VGDR_GATE_NONE || gate_kind > VGDR_GATE_VECTOR)
        return fail(VGDR_ERR_INVALID, "%s: unknown gate_kind %d", fn, gate_kind);
    if (B < 0 || T < 0 || H <= 0 || n_seqs < 0)
        return fail(VGDR_ERR_INVALID, "%s: bad sizes B=%lld T=%lld H=%lld n_seqs=%lld", fn, (long long)B,
                    (long long)T, (long long)H, (long long)n_seqs);
    if (dk != 64 && dk != 128)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: dk=%lld (supported: 64, 128)", fn, (long long)dk);
    if (cu) {
        if (B != 1) return fail(VGDR_ERR_INVALID, "%s: a packed batch (cu_seqlens) needs B == 1", fn);
    } else if (n_seqs != B) {
        return fail(VGDR_ERR_INVALID, "%s: n_seqs (%lld) must equal B (%lld) for a dense batch", fn,
                    (long long)n_seqs, (long long)B);
    }
    if (B * T > 0 && (!q || !k || !v || !o))
        return fail(VGDR_ERR_INVALID, "%s: q, k, v and o are required", fn);
    if (gate_kind != VGDR_GATE_NONE && B * T > 0 && !g)
        return fail(VGDR_ERR_INVALID, "%s: gate_kind %d needs g", fn, gate_kind);
    if (use_delta && B * T > 0 && !beta) return fail(VGDR_ERR_INVALID, "%s: the delta rule needs beta", fn);
    if (n_seqs > 0x7fffffffLL / H) return fail(VGDR_ERR_INVALID, "%s: too many (sequence, head) pairs", fn);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v))
        return fail(VGDR_ERR_INVALID, "%s: q, k and v must be 16-byte aligned", fn);
    if (gate_kind == VGDR_GATE_VECTOR && !aligned16(g))
        return fail(VGDR_ERR_INVALID, "%s: a per-channel g must be 16-byte aligned", fn);
    return VGDR_OK;
}

// the producer fusions a call asks for, checked against the scan's settings
int check_fusion(const char *fn, const vgdr_fusion *fz, int dtype, int gate_kind, int use_delta, bool chunked,
                 vgdr::Fusion &out) {
    out = vgdr::Fusion{};
    if (!fz) return VGDR_OK;
    const bool any = fz->qk_l2norm || fz->beta_sigmoid || fz->gate_activation;
    if (!any) return VGDR_OK;
    if (chunked && dtype == VGDR_F32)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: producer fusions take 16-bit q, k, v", fn);
    if (chunked && (fz->qk_l2norm || fz->beta_sigmoid) && !use_delta)
        return fail(VGDR_ERR_INVALID, "%s: the fused L2 norm and beta sigmoid need the delta rule", fn);
    if (fz->gate_activation) {
        if (gate_kind != VGDR_GATE_VECTOR)
            return fail(VGDR_ERR_INVALID, "%s: the fused gate activation is for the per-channel gate", fn);
        if (!fz->A_log || !fz->dt_bias)
            return fail(VGDR_ERR_INVALID, "%s: the fused gate activation needs A_log and dt_bias", fn);
        if (fz->gate_dtype != VGDR_F32 && fz->gate_dtype != dtype)
            return fail(VGDR_ERR_INVALID, "%s: gate_dtype must be VGDR_F32 or the dtype of q", fn);
    }
    out.qk_l2norm = fz->qk_l2norm ? 1 : 0;
    out.beta_sigmoid = fz->beta_sigmoid ? 1 : 0;
    out.gate_act = fz->gate_activation ? 1 : 0;
    out.gate_16 = fz->gate_activation && fz->gate_dtype != VGDR_F32 ? 1 : 0;
    out.A_log = fz->A_log;
    out.dt_bias = fz->dt_bias;
    out.lb_set = fz->lower_bound_set ? 1 : 0;
    out.lb = fz->lower_bound;
    return VGDR_OK;
}

// the output epilogue a call asks for; `elems` = 16 / element size (the
// standalone pass reads rows in 16-byte units)
int check_epilogue(const char *fn, const vgdr_epilogue *ep, int dtype, vgdr::Epilogue &out) {
    out = vgdr::Epilogue{};
    if (!ep) return VGDR_OK;
    if (!ep->gate || !ep->gamma) return fail(VGDR_ERR_INVALID, "%s: the epilogue needs gate and gamma", fn);
    if (!aligned16(ep->gate)) return fail(VGDR_ERR_INVALID, "%s: the epilogue gate must be 16-byte aligned", fn);
    if (ep->gamma_dtype != VGDR_F32 && ep->gamma_dtype != dtype)
        return fail(VGDR_ERR_INVALID, "%s: gamma_dtype must be VGDR_F32 or the dtype of o", fn);
    if (!(ep->eps > 0.f)) return fail(VGDR_ERR_INVALID, "%s: the RMSNorm eps must be positive", fn);
    out.gate = ep->gate;
    out.gamma = ep->gamma;
    out.gamma_f32 = ep->gamma_dtype == VGDR_F32 ? 1 : 0;
    out.eps = ep->eps;
    return VGDR_OK;
}

// the short conv a decode call asks for
int check_conv(const char *fn, const vgdr_short_conv *cv, int dtype, vgdr::ShortConv &out) {
    out = vgdr::ShortConv{};
    if (!cv) return VGDR_OK;
    if (cv->kernel_size < 1 || cv->kernel_size > 8)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: short conv kernel_size=%d (supported: 1..8)", fn, cv->kernel_size);
    if (!cv->weight_q || !cv->weight_k || !cv->weight_v || !cv->cache_q || !cv->cache_k || !cv->cache_v)
        return fail(VGDR_ERR_INVALID, "%s: the short conv needs its three weights and three caches", fn);
    if (cv->weight_dtype != VGDR_F32 && cv->weight_dtype != dtype)
        return fail(VGDR_ERR_INVALID, "%s: the conv weight_dtype must be VGDR_F32 or the dtype of q", fn);
    out.wq = cv->weight_q;
    out.wk = cv->weight_k;
    out.wv = cv->weight_v;
    out.cq = cv->cache_q;
    out.ck = cv->cache_k;
    out.cv = cv->cache_v;
    out.K = cv->kernel_size;
    out.w_f32 = cv->weight_dtype == VGDR_F32 ? 1 : 0;
    return VGDR_OK;
}

// chunk length the kernels use: 32 when asked for <= 32, else 64; fp32 always
// uses 32 (its double-buffered 64-token tiles overflow LDS)
int effective_chunk(int dtype, int64_t dk, int chunk_size) {
    (void)dk;
    if (dtype == VGDR_F32) return 32;
    return chunk_size <= 32 ? 32 : 64;
}

struct ChunkWs {
    int64_t slots;        // chunk slots of the prep kernel (an upper bound on chunks)
    int64_t blocks_off;   // byte offset of the per-(chunk, head) TE / A blocks
    int64_t total;        // bytes
};

ChunkWs chunk_layout(int dtype, int gate_kind, int chunk, int64_t B, int64_t T, int64_t H, int64_t dk,
                     int64_t n_seqs, bool varlen) {
    ChunkWs w{};
    if (varlen) {
        w.slots = (B * T + chunk - 1) / chunk + n_seqs;     // each segment adds at most one partial chunk
        w.blocks_off = ((4 * n_seqs + 1) * 4 + 255) / 256 * 256;
    } else {
        w.slots = B * ((T + chunk - 1) / chunk);
        w.blocks_off = 0;
    }
    w.total = w.blocks_off + vgdr::chunk_blocks_bytes(dtype, chunk, w.slots, H, dk, gate_kind == VGDR_GATE_VECTOR);
    if (w.slots == 0) w.total = varlen ? w.blocks_off : 0;
    return w;
}

// workspace of the backward: the forward's (table, blocks), then each chunk's
// entry state and exit-state gradient (dk x dv per (chunk, head) in the element
// type); with the per-channel gate also chunk prep's N (CH x CH fp32 per
// (chunk, head)) and the column phase's sums (grad_vec_work_floats each)
struct BwdWs {
    ChunkWs fwd;
    int64_t hs_off, dhs_off, nbuf_off, gw_off, dpart_off, total;
};
BwdWs bwd_layout(int dtype, int gate_kind, int chunk, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                 int64_t n_seqs, bool varlen) {
    BwdWs w{};
    w.fwd = chunk_layout(dtype, gate_kind, chunk, B, T, H, dk, n_seqs, varlen);
    const int64_t states = w.fwd.slots * H * dk * dv * (dtype == VGDR_F32 ? 4 : 2);
    w.hs_off = (w.fwd.total + 255) / 256 * 256;
    w.dhs_off = w.hs_off + (states + 255) / 256 * 256;
    w.total = states > 0 ? w.dhs_off + states : w.fwd.total;
    w.nbuf_off = w.gw_off = w.dpart_off = w.total;
    if (gate_kind == VGDR_GATE_VECTOR && dtype != VGDR_F32 && states > 0) {
        // plus N, the column phase's sums and (fused gate activation) the per-chunk parameter sums
        const int64_t nb = w.fwd.slots * H * chunk * chunk * 4;
        const int64_t gw = w.fwd.slots * H * vgdr::grad_vec_work_floats(chunk, (int)dk) * 4;
        const int64_t dp = w.fwd.slots * H * (dk + 1) * 4;
        w.nbuf_off = (w.total + 255) / 256 * 256;
        w.gw_off = w.nbuf_off + (nb + 255) / 256 * 256;
        w.dpart_off = w.gw_off + (gw + 255) / 256 * 256;
        w.total = w.dpart_off + dp;
    }
    return w;
}

// the three chunk entry points: validation, workspace layout, then the phases asked for
int chunk_call(const char *fn, int phases, int dtype, int gate_kind, int use_delta, const void *q, const void *k,
               const void *v, const float *g, const float *beta, void *o, const float *initial_state,
               float *final_state, const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B,
               int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size,
               const vgdr_fusion *fusion, hipStream_t stream, const void *w = nullptr, void *bwd_ws = nullptr) {
    g_err[0] = 0;
    // with an explicit write vector, beta is not read
    int rc = check_common(fn, dtype, gate_kind, w ? 0 : use_delta, q, k, v, g, beta, o, cu_seqlens,
                          B, T, H, dk, dv, n_seqs);
    if (rc) return rc;
    if (w) {
        if (dtype == VGDR_F32)
            return fail(VGDR_ERR_UNSUPPORTED, "%s: the chunked explicit write takes 16-bit q, k, v, w", fn);
        if (gate_kind != VGDR_GATE_VECTOR)
            return fail(VGDR_ERR_INVALID, "%s: the chunked explicit write runs with a per-channel g", fn);
        if (!aligned16(w)) return fail(VGDR_ERR_INVALID, "%s: w must be 16-byte aligned", fn);
        if (fusion && fusion->beta_sigmoid)
            return fail(VGDR_ERR_INVALID, "%s: there is no beta to activate with an explicit w", fn);
    }
    vgdr::Fusion fz;
    rc = check_fusion(fn, fusion, dtype, gate_kind, use_delta, true, fz);
    if (rc) return rc;
    if (dv <= 0 || dv % 16)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: dv=%lld (must be a positive multiple of 16)", fn, (long long)dv);
    if (!aligned16(o)) return fail(VGDR_ERR_INVALID, "%s: o must be 16-byte aligned", fn);
    const int chunk = effective_chunk(dtype, dk, chunk_size);
    const ChunkWs ws = chunk_layout(dtype, gate_kind, chunk, B, T, H, dk, n_seqs, cu_seqlens != nullptr);
    // a saving forward runs in the backward's workspace (its prefix is this layout)
    const int64_t need =
        bwd_ws ? bwd_layout(dtype, gate_kind, chunk, B, T, H, dk, dv, n_seqs, cu_seqlens != nullptr).total : ws.total;
    if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
        return fail(VGDR_ERR_INVALID, "%s: workspace needs %lld bytes, 16-byte aligned (got %lld at %p)", fn,
                    (long long)need, (long long)workspace_bytes, workspace);
    if (ws.slots * H > 0x7fffffffLL || (n_seqs * H + 7) / 8 * 8 * ((dv + 31) / 32) > 0x7fffffffLL)
        return fail(VGDR_ERR_INVALID, "%s: grid too large", fn);
    vgdr::ChunkParams p{};
    if (bwd_ws) {
        const BwdWs bw = bwd_layout(dtype, gate_kind, chunk, B, T, H, dk, dv, n_seqs, cu_seqlens != nullptr);
        p.hs = static_cast<char *>(workspace) + bw.hs_off;
        if (gate_kind == VGDR_GATE_VECTOR)
            p.nout = reinterpret_cast<float *>(static_cast<char *>(workspace) + bw.nbuf_off);
    }
    p.geo.cu = cu_seqlens;
    p.geo.T = T;
    p.geo.n_tokens = B * T;
    p.geo.n_seqs = (int)n_seqs;
    p.geo.chunks_per_seq = (int)((T + chunk - 1) / chunk);
    p.q = q; p.k = k; p.v = v;
    p.g = gate_kind == VGDR_GATE_NONE ? nullptr : g;
    p.beta = beta;
    p.o = o;
    p.h0 = initial_state;
    p.ht = final_state;
    p.blocks = static_cast<char *>(workspace) + ws.blocks_off;
    p.H = (int)H;
    p.DV = (int)dv;
    p.n_chunk_slots = (int)ws.slots;
    p.use_delta = use_delta ? 1 : 0;
    p.scale = scale;
    p.fz = fz;
    p.w = w;
    int32_t *table = cu_seqlens ? static_cast<int32_t *>(workspace) : nullptr;
    return hip_status(vgdr::chunk_fwd(dtype, (int)dk, chunk, gate_kind == VGDR_GATE_VECTOR, p, table, phases, stream),
                      fn);
}

}  // namespace

namespace vgdr {
int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}
}  // namespace vgdr

extern "C" {

int vgdr_version(void) { return 100; }

const char *vgdr_last_error(void) { return g_err; }

int64_t vgdr_chunk_workspace_size(int dtype, int gate_kind, int64_t B, int64_t T, int64_t H, int64_t dk,
                                  int64_t n_seqs, int varlen, int chunk_size) {
    if (B < 0 || T < 0 || H <= 0 || n_seqs < 0) return 0;
    const int chunk = effective_chunk(dtype, dk, chunk_size);
    return chunk_layout(dtype, gate_kind, chunk, B, T, H, dk, n_seqs, varlen).total;
}

#define VGDR_CHUNK_ARGS                                                                                    \
    int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v, const float *g,     \
        const float *beta, void *o, const float *initial_state, float *final_state, const int32_t *cu_seqlens, \
        void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,     \
        int64_t n_seqs, float scale, int chunk_size, hipStream_t stream
#define VGDR_CHUNK_ARGS_FUSED                                                                              \
    int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v, const float *g,     \
        const float *beta, void *o, const float *initial_state, float *final_state, const int32_t *cu_seqlens, \
        void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,     \
        int64_t n_seqs, float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream
#define VGDR_CHUNK_PASS_NOFUSION                                                                           \
    dtype, gate_kind, use_delta, q, k, v, g, beta, o, initial_state, final_state, cu_seqlens, workspace,      \
        workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size, nullptr, stream
#define VGDR_CHUNK_PASS_FUSED                                                                              \
    dtype, gate_kind, use_delta, q, k, v, g, beta, o, initial_state, final_state, cu_seqlens, workspace,      \
        workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size, fusion, stream

int vgdr_chunk_fwd(VGDR_CHUNK_ARGS) {
    return chunk_call("vgdr_chunk_fwd", vgdr::CHUNK_PREP | vgdr::CHUNK_STATE, VGDR_CHUNK_PASS_NOFUSION);
}
int vgdr_chunk_prep(VGDR_CHUNK_ARGS) {
    return chunk_call("vgdr_chunk_prep", vgdr::CHUNK_PREP, VGDR_CHUNK_PASS_NOFUSION);
}
int vgdr_chunk_state(VGDR_CHUNK_ARGS) {
    return chunk_call("vgdr_chunk_state", vgdr::CHUNK_STATE, VGDR_CHUNK_PASS_NOFUSION);
}
int vgdr_chunk_fwd_fused(VGDR_CHUNK_ARGS_FUSED) {
    return chunk_call("vgdr_chunk_fwd_fused", vgdr::CHUNK_PREP | vgdr::CHUNK_STATE, VGDR_CHUNK_PASS_FUSED);
}
int vgdr_chunk_prep_fused(VGDR_CHUNK_ARGS_FUSED) {
    return chunk_call("vgdr_chunk_prep_fused", vgdr::CHUNK_PREP, VGDR_CHUNK_PASS_FUSED);
}
int vgdr_chunk_fwd_w(int dtype, const void *q, const void *k, const void *v, const void *w, const float *g, void *o,
                     const float *initial_state, float *final_state, const int32_t *cu_seqlens, void *workspace,
                     int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                     float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream) {
    if (B * T > 0 && !w) {
        g_err[0] = 0;
        return fail(VGDR_ERR_INVALID, "vgdr_chunk_fwd_w: w is required");
    }
    static const char dummy[16] __attribute__((aligned(16))) = {};     // w for an empty call: never read
    return chunk_call("vgdr_chunk_fwd_w", vgdr::CHUNK_PREP | vgdr::CHUNK_STATE, dtype, VGDR_GATE_VECTOR, 1, q, k, v,
                      g, nullptr, o, initial_state, final_state, cu_seqlens, workspace, workspace_bytes, B, T, H, dk,
                      dv, n_seqs, scale, chunk_size, fusion, stream, w ? w : dummy);
}


int64_t vgdr_chunk_bwd_workspace_size(int dtype, int gate_kind, int64_t B, int64_t T, int64_t H, int64_t dk,
                                      int64_t dv, int64_t n_seqs, int varlen, int chunk_size) {
    if (B < 0 || T < 0 || H <= 0 || n_seqs < 0 || dv < 0) return 0;
    const int chunk = effective_chunk(dtype, dk, chunk_size);
    return bwd_layout(dtype, gate_kind, chunk, B, T, H, dk, dv, n_seqs, varlen).total;
}

#define VGDR_BWD_ARGS                                                                                        \
    int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g, const float *beta,   \
        const float *initial_state, const void *grad_o, const float *grad_final_state, void *grad_q,            \
        void *grad_k, void *grad_v, float *grad_g, float *grad_beta, float *grad_initial_state,                 \
        const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H,    \
        int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size, hipStream_t stream
#define VGDR_BWD_ARGS_FUSED                                                                                  \
    int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g, const float *beta,   \
        const float *initial_state, const void *grad_o, const float *grad_final_state, void *grad_q,            \
        void *grad_k, void *grad_v, float *grad_g, float *grad_beta, float *grad_initial_state,                 \
        const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H,    \
        int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size, const vgdr_fusion *fusion,          \
        float *grad_A_log, float *grad_dt_bias, hipStream_t stream
#define VGDR_BWD_PASS                                                                                        \
    dtype, gate_kind, q, k, v, g, beta, initial_state, grad_o, grad_final_state, grad_q, grad_k, grad_v,        \
        grad_g, grad_beta, grad_initial_state, cu_seqlens, workspace, workspace_bytes, B, T, H, dk, dv, n_seqs, \
        scale, chunk_size, stream

namespace {
// the backward entry points; saved: the workspace holds what a saving forward left
// delta: the delta rule (else the plain recurrence: no beta, no grad_beta)
// w: explicit write vectors (the delta rule without beta; grad_w receives their gradient)
int bwd_call(const char *fn, bool saved, bool delta, VGDR_BWD_ARGS, const vgdr_fusion *fusion, float *grad_A_log,
             float *grad_dt_bias, const void *w = nullptr, void *grad_w = nullptr) {
    g_err[0] = 0;
    int rc = check_common(fn, dtype, gate_kind, delta && !w ? 1 : 0, q, k, v, g, beta, grad_o, cu_seqlens, B, T, H,
                          dk, dv, n_seqs);
    if (rc) return rc;
    if (!delta || w) beta = grad_beta = nullptr;
    if (w) {
        if (dtype == VGDR_F32 || gate_kind != VGDR_GATE_VECTOR)
            return fail(VGDR_ERR_UNSUPPORTED, "%s: the chunked explicit write takes 16-bit q, k, v, w and a "
                        "per-channel g", fn);
        if (!aligned16(w)) return fail(VGDR_ERR_INVALID, "%s: w must be 16-byte aligned", fn);
        if (B * T > 0 && !grad_w) return fail(VGDR_ERR_INVALID, "%s: grad_w is required", fn);
        if (grad_w == w) return fail(VGDR_ERR_INVALID, "%s: the gradients must not alias the inputs", fn);
    }
    vgdr::Fusion fz;
    rc = check_fusion(fn, fusion, dtype, gate_kind, delta ? 1 : 0, true, fz);
    if (rc) return rc;
    if (fz.qk_l2norm)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: the fused L2 norm has no backward here: pass normalised q, k", fn);
    if (fz.gate_act && B * T > 0 && (!grad_A_log || !grad_dt_bias || !grad_g))
        return fail(VGDR_ERR_INVALID, "%s: the fused gate activation needs grad_g, grad_A_log and grad_dt_bias", fn);
    if (dv <= 0 || dv % 16)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: dv=%lld (must be a positive multiple of 16)", fn, (long long)dv);
    if (gate_kind == VGDR_GATE_VECTOR && (dtype == VGDR_F32 || effective_chunk(dtype, dk, chunk_size) != 64))
        return fail(VGDR_ERR_UNSUPPORTED, "%s: the per-channel-gate backward runs 16-bit q, k, v in 64-token chunks",
                    fn);
    if (B * T > 0 && (!grad_q || !grad_k || !grad_v || (delta && !w && !grad_beta)))
        return fail(VGDR_ERR_INVALID, "%s: grad_q, grad_k, grad_v%s are required", fn,
                    delta && !w ? " and grad_beta" : "");
    if (grad_v == v || grad_q == q || grad_k == k)
        return fail(VGDR_ERR_INVALID, "%s: the gradients must not alias the inputs", fn);
    if (!aligned16(grad_o) || !aligned16(grad_v))
        return fail(VGDR_ERR_INVALID, "%s: grad_o and grad_v must be 16-byte aligned", fn);
    const int chunk = effective_chunk(dtype, dk, chunk_size);
    const BwdWs ws = bwd_layout(dtype, gate_kind, chunk, B, T, H, dk, dv, n_seqs, cu_seqlens != nullptr);
    if (ws.total > 0 && (!workspace || workspace_bytes < ws.total || !aligned16(workspace)))
        return fail(VGDR_ERR_INVALID, "%s: workspace needs %lld bytes, 16-byte aligned (got %lld at %p)", fn,
                    (long long)ws.total, (long long)workspace_bytes, workspace);
    if (ws.fwd.slots * H > 0x7fffffffLL || (n_seqs * H + 7) / 8 * 8 * ((dv + 31) / 32) > 0x7fffffffLL)
        return fail(VGDR_ERR_INVALID, "%s: grid too large", fn);
    char *wsb = static_cast<char *>(workspace);
    vgdr::ChunkParams f{};
    f.geo.cu = cu_seqlens;
    f.geo.T = T;
    f.geo.n_tokens = B * T;
    f.geo.n_seqs = (int)n_seqs;
    f.geo.chunks_per_seq = (int)((T + chunk - 1) / chunk);
    f.q = q; f.k = k; f.v = v;
    f.g = gate_kind == VGDR_GATE_NONE ? nullptr : g;
    f.beta = beta;
    f.blocks = wsb + ws.fwd.blocks_off;
    f.H = (int)H;
    f.DV = (int)dv;
    f.n_chunk_slots = (int)ws.fwd.slots;
    f.use_delta = 1;                                          // the delta form's blocks; without the delta
    f.te_identity = delta ? 0 : 1;                            // rule TE = I and GX = 0 make U = V
    f.w = w;
    f.scale = scale;
    f.fz = fz;
    vgdr::ChunkBwdParams p{};
    p.fz = fz;
    p.geo = f.geo;
    p.q = q; p.k = k; p.v = v;
    p.g = f.g;
    p.beta = beta;
    p.dout = grad_o;
    p.h0 = initial_state;
    p.dht = grad_final_state;
    p.dq = grad_q; p.dk = grad_k; p.dv = grad_v;
    p.dg = f.g ? grad_g : nullptr;
    p.dbeta = grad_beta;
    p.dh0 = grad_initial_state;
    p.blocks = f.blocks;
    p.hs = wsb + ws.hs_off;
    p.dhs = wsb + ws.dhs_off;
    p.H = (int)H;
    p.DV = (int)dv;
    p.n_chunk_slots = (int)ws.fwd.slots;
    p.scale = scale;
    p.delta = delta ? 1 : 0;
    p.w = w;
    p.dw = grad_w;
    if (gate_kind == VGDR_GATE_VECTOR) {
        p.nbuf = reinterpret_cast<const float *>(wsb + ws.nbuf_off);
        p.gw = reinterpret_cast<float *>(wsb + ws.gw_off);
        p.dpart = reinterpret_cast<float *>(wsb + ws.dpart_off);
        p.dA_log = grad_A_log;
        p.ddt_bias = grad_dt_bias;
        // the forward run for the entry states writes N and the states where
        // the backward reads them, and no output (ChunkParams::states_only,
        // set by the backward's launcher)
        f.hs = p.hs;
        f.nout = const_cast<float *>(p.nbuf);
        f.h0 = initial_state;
    }
    int32_t *table = cu_seqlens ? reinterpret_cast<int32_t *>(wsb) : nullptr;
    if (f.geo.n_seqs == 0) return VGDR_OK;
    if (saved && dtype == VGDR_F32)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: saved states come from the 16-bit forward kernel", fn);
    return hip_status(vgdr::chunk_bwd(dtype, (int)dk, chunk, gate_kind == VGDR_GATE_VECTOR, f, p, table, saved, stream), fn);
}
}  // namespace

int vgdr_chunk_bwd(VGDR_BWD_ARGS) {
    return bwd_call("vgdr_chunk_bwd", false, true, VGDR_BWD_PASS, nullptr, nullptr, nullptr);
}
int vgdr_chunk_bwd_saved(VGDR_BWD_ARGS) {
    return bwd_call("vgdr_chunk_bwd_saved", true, true, VGDR_BWD_PASS, nullptr, nullptr, nullptr);
}
int vgdr_chunk_bwd_fused(VGDR_BWD_ARGS_FUSED) {
    return bwd_call("vgdr_chunk_bwd_fused", false, true, VGDR_BWD_PASS, fusion, grad_A_log, grad_dt_bias);
}
int vgdr_chunk_bwd_saved_fused(VGDR_BWD_ARGS_FUSED) {
    return bwd_call("vgdr_chunk_bwd_saved_fused", true, true, VGDR_BWD_PASS, fusion, grad_A_log, grad_dt_bias);
}
int vgdr_chunk_bwd_w(int dtype, const void *q, const void *k, const void *v, const void *w, const float *g,
                     const float *initial_state, const void *grad_o, const float *grad_final_state, void *grad_q,
                     void *grad_k, void *grad_v, void *grad_w, float *grad_g, float *grad_initial_state,
                     const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T,
                     int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size,
                     hipStream_t stream) {
    if (B * T > 0 && !w) {
        g_err[0] = 0;
        return fail(VGDR_ERR_INVALID, "vgdr_chunk_bwd_w: w is required");
    }
    static const char dummy[16] __attribute__((aligned(16))) = {};     // w for an empty call: never read
    return bwd_call("vgdr_chunk_bwd_w", false, true, dtype, VGDR_GATE_VECTOR, q, k, v, g, nullptr, initial_state,
                    grad_o, grad_final_state, grad_q, grad_k, grad_v, grad_g, nullptr, grad_initial_state, cu_seqlens,
                    workspace, workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size, stream, nullptr, nullptr,
                    nullptr, w ? w : dummy, grad_w);
}
int vgdr_chunk_bwd_nodelta(int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g,
                           const float *initial_state, const void *grad_o, const float *grad_final_state, void *grad_q,
                           void *grad_k, void *grad_v, float *grad_g, float *grad_initial_state,
                           const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T,
                           int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size,
                           hipStream_t stream) {
    return bwd_call("vgdr_chunk_bwd_nodelta", false, false, dtype, gate_kind, q, k, v, g, nullptr, initial_state,
                    grad_o, grad_final_state, grad_q, grad_k, grad_v, grad_g, nullptr, grad_initial_state, cu_seqlens,
                    workspace, workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size, stream, nullptr, nullptr,
                    nullptr);
}
#undef VGDR_BWD_ARGS
#undef VGDR_BWD_ARGS_FUSED
#undef VGDR_BWD_PASS

}  // extern "C"

namespace {
// Scratch of vgdr_chunk_fwd_noalloc: the chunk workspace (segment table and
// per-(chunk, head) blocks) in a file-scope device array, so that the call
// allocates nothing.  Each GPU holds its own copy for the life of the
// process; host code reaches it only through the address hipGetSymbolAddress
// returns on that device (the array's name is a host-side stand-in).  Its
// contents need no clearing: the prep phase writes every byte the state
// phase reads.  Calls that overlap on one GPU share it and race.
constexpr int64_t kScratchBytes = VGDR_CHUNK_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// the current device's scratch address, looked up once per device with that device current
int scratch_address(const char *fn, void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, fn);
    if (dev < 0 || dev >= kMaxDevices) return fail(VGDR_ERR_UNSUPPORTED, "%s: device %d out of range", fn, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, fn);
        if (!p) return fail(VGDR_ERR_HIP, "%s: no device address for the scratch array", fn);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return VGDR_OK;
}
}  // namespace

extern "C" {

int vgdr_chunk_fwd_noalloc(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                           const float *g, const float *beta, void *o, const float *initial_state,
                           float *final_state, const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t H,
                           int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size,
                           const vgdr_fusion *fusion, hipStream_t stream) {
    const char *fn = "vgdr_chunk_fwd_noalloc";
    g_err[0] = 0;
    if (B >= 0 && T >= 0 && H > 0 && n_seqs >= 0 && B * T > 0) {
        const int chunk = effective_chunk(dtype, dk, chunk_size);
        const int64_t need = chunk_layout(dtype, gate_kind, chunk, B, T, H, dk, n_seqs, cu_seqlens != nullptr).total;
        if (need > kScratchBytes)
            return fail(VGDR_ERR_INVALID, "%s: this call needs %lld bytes of scratch, more than the %lld the "
                        "library holds per GPU (use vgdr_chunk_fwd_fused with a workspace)", fn, (long long)need,
                        (long long)kScratchBytes);
    }
    void *ws = nullptr;
    const int rc = scratch_address(fn, &ws);
    if (rc) return rc;
    return chunk_call(fn, vgdr::CHUNK_PREP | vgdr::CHUNK_STATE, dtype, gate_kind, use_delta, q, k, v, g, beta, o,
                      initial_state, final_state, cu_seqlens, ws, kScratchBytes, B, T, H, dk, dv, n_seqs, scale,
                      chunk_size, fusion, stream);
}

namespace {
int fwd_saving(const char *fn, int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g,
               const float *beta, void *o, const float *initial_state, float *final_state,
               const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H,
               int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size, const vgdr_fusion *fusion,
               hipStream_t stream) {
    if (dtype == VGDR_F32 || (gate_kind == VGDR_GATE_VECTOR && effective_chunk(dtype, dk, chunk_size) != 64)) {
        g_err[0] = 0;
        return fail(VGDR_ERR_UNSUPPORTED, "%s: saving runs the 16-bit kernel (64-token chunks with a per-channel g)",
                    fn);
    }
    if (fusion && fusion->qk_l2norm) {                        // the backward reads q, k as given
        g_err[0] = 0;
        return fail(VGDR_ERR_UNSUPPORTED, "%s: the fused L2 norm has no backward here: pass normalised q, k", fn);
    }
    return chunk_call(fn, vgdr::CHUNK_PREP | vgdr::CHUNK_STATE, dtype, gate_kind, 1, q, k, v, g, beta, o,
                      initial_state, final_state, cu_seqlens, workspace, workspace_bytes, B, T, H, dk, dv, n_seqs,
                      scale, chunk_size, fusion, stream, nullptr, workspace);
}
}  // namespace

int vgdr_chunk_fwd_saving(int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g,
                          const float *beta, void *o, const float *initial_state, float *final_state,
                          const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T,
                          int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale, int chunk_size,
                          hipStream_t stream) {
    return fwd_saving("vgdr_chunk_fwd_saving", dtype, gate_kind, q, k, v, g, beta, o, initial_state, final_state,
                      cu_seqlens, workspace, workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size, nullptr,
                      stream);
}
int vgdr_chunk_fwd_saving_fused(int dtype, int gate_kind, const void *q, const void *k, const void *v,
                                const float *g, const float *beta, void *o, const float *initial_state,
                                float *final_state, const int32_t *cu_seqlens, void *workspace,
                                int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                                int64_t n_seqs, float scale, int chunk_size, const vgdr_fusion *fusion,
                                hipStream_t stream) {
    return fwd_saving("vgdr_chunk_fwd_saving_fused", dtype, gate_kind, q, k, v, g, beta, o, initial_state,
                      final_state, cu_seqlens, workspace, workspace_bytes, B, T, H, dk, dv, n_seqs, scale, chunk_size,
                      fusion, stream);
}

namespace {
struct ScanBwdWs {
    int64_t hs_off, dhs_off, u_off, part_off, total;
    int tw, n_tiles;
};
ScanBwdWs scan_bwd_layout(int64_t n_tokens, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs) {
    ScanBwdWs w{};
    w.tw = 16;
    w.n_tiles = (int)(dv / w.tw);
    auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
    const int64_t slots = vgdr::scan_bwd_ckpt_slots(n_tokens, n_seqs);
    w.hs_off = 0;
    w.dhs_off = up(slots * H * dk * dv * 4);
    w.u_off = w.dhs_off + up(slots * H * dk * dv * 4);
    w.part_off = w.u_off + up(n_tokens * H * dv * 4);
    w.total = w.part_off + up(4 * (int64_t)w.n_tiles * n_tokens * H * dk * 4);
    return w;
}
}  // namespace

int64_t vgdr_scan_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs) {
    if (B < 0 || T < 0 || H <= 0 || n_seqs < 0 || dk <= 0 || dv <= 0) return 0;
    return scan_bwd_layout(B * T, H, dk, dv, n_seqs).total;
}

int vgdr_scan_bwd(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                  const void *w, const float *g, const float *beta, const float *initial_state, const void *grad_o,
                  const float *grad_final_state, void *grad_q, void *grad_k, void *grad_v, void *grad_w,
                  float *grad_g, float *grad_beta, float *grad_initial_state, const int32_t *cu_seqlens,
                  void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk,
                  int64_t dv, int64_t n_seqs, float scale, hipStream_t stream) {
    const char *fn = "vgdr_scan_bwd";
    g_err[0] = 0;
    if (w && !use_delta) return fail(VGDR_ERR_INVALID, "%s: an explicit write vector needs the delta rule", fn);
    const int mode = !use_delta ? 2 : (w ? 1 : 0);
    int rc = check_common(fn, dtype, gate_kind, mode == 0, q, k, v, g, beta, grad_o, cu_seqlens, B, T, H, dk, dv,
                          n_seqs);
    if (rc) return rc;
    if (dv <= 0 || dv % 16)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: dv=%lld (must be a positive multiple of 16)", fn, (long long)dv);
    const bool any = B * T > 0;
    if (any && (!grad_q || !grad_k || !grad_v))
        return fail(VGDR_ERR_INVALID, "%s: grad_q, grad_k and grad_v are required", fn);
    if (any && mode == 1 && !grad_w) return fail(VGDR_ERR_INVALID, "%s: w needs grad_w", fn);
    if (any && mode == 0 && !grad_beta) return fail(VGDR_ERR_INVALID, "%s: the delta rule needs grad_beta", fn);
    if (any && gate_kind != VGDR_GATE_NONE && !grad_g) return fail(VGDR_ERR_INVALID, "%s: a gate needs grad_g", fn);
    if (grad_v == v || grad_q == q || grad_k == k || (w && grad_w == w))
        return fail(VGDR_ERR_INVALID, "%s: the gradients must not alias the inputs", fn);
    if (!aligned16(grad_o) || !aligned16(grad_v) || (w && !aligned16(w)))
        return fail(VGDR_ERR_INVALID, "%s: grad_o, grad_v and w must be 16-byte aligned", fn);
    if (!aligned16(initial_state) || !aligned16(grad_final_state) || !aligned16(grad_initial_state))
        return fail(VGDR_ERR_INVALID, "%s: the state tensors must be 16-byte aligned", fn);
    const ScanBwdWs ws = scan_bwd_layout(B * T, H, dk, dv, n_seqs);
    if (!workspace || workspace_bytes < ws.total || !aligned16(workspace))
        return fail(VGDR_ERR_INVALID, "%s: workspace needs %lld bytes, 16-byte aligned (got %lld at %p)", fn,
                    (long long)ws.total, (long long)workspace_bytes, workspace);
    if (2 * n_seqs * H * ws.n_tiles > 0x7fffffffLL || (B * T * H + 3) / 4 > 0x7fffffffLL ||
        vgdr::scan_bwd_ckpt_slots(B * T, n_seqs) * H * ws.n_tiles > 0x7fffffffLL)
        return fail(VGDR_ERR_INVALID, "%s: grid too large", fn);
    if (n_seqs == 0) return VGDR_OK;
    char *wsb = static_cast<char *>(workspace);
    vgdr::ScanBwdParams p{};
    p.geo.cu = cu_seqlens;
    p.geo.T = T;
    p.geo.n_tokens = B * T;
    p.geo.n_seqs = (int)n_seqs;
    p.q = q; p.k = k; p.v = v; p.w = mode == 1 ? w : nullptr;
    p.g = gate_kind == VGDR_GATE_NONE ? nullptr : g;
    p.beta = mode == 0 ? beta : nullptr;
    p.dout = grad_o;
    p.h0 = initial_state;
    p.dht = grad_final_state;
    p.dq = grad_q; p.dk = grad_k; p.dv = grad_v; p.dw = mode == 1 ? grad_w : nullptr;
    p.dg = gate_kind == VGDR_GATE_NONE ? nullptr : grad_g;
    p.dbeta = mode == 0 ? grad_beta : nullptr;
    p.dh0 = grad_initial_state;
    p.hs = reinterpret_cast<float *>(wsb + ws.hs_off);
    p.dhs = reinterpret_cast<float *>(wsb + ws.dhs_off);
    p.u = reinterpret_cast<float *>(wsb + ws.u_off);
    p.part = reinterpret_cast<float *>(wsb + ws.part_off);
    p.H = (int)H;
    p.DV = (int)dv;
    p.TW = ws.tw;
    p.n_tiles = ws.n_tiles;
    p.gate = gate_kind;
    p.mode = mode;
    p.scale = scale;
    return hip_status(vgdr::scan_bwd(dtype, (int)dk, p, stream), fn);
}

#undef VGDR_CHUNK_ARGS
#undef VGDR_CHUNK_ARGS_FUSED
#undef VGDR_CHUNK_PASS_NOFUSION
#undef VGDR_CHUNK_PASS_FUSED

namespace {

// every token-by-token entry point: validation, then one recurrent_kernel launch
int recurrent_call(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                   const void *w, const float *g, const float *beta, void *o, const float *initial_state,
                   float *final_state, const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t H, int64_t dk,
                   int64_t dv, int64_t n_seqs, float scale, const vgdr_fusion *fusion, const vgdr_short_conv *conv,
                   const vgdr_epilogue *epilogue, hipStream_t stream, int64_t ld_qk = 0, int64_t ld_v = 0,
                   const vgdr_gate_proj *gp = nullptr) {
    g_err[0] = 0;
    // with an explicit write vector, beta is not read; with gate projections
    // (checked by the caller) neither g nor beta is
    int rc = check_common("vgdr_recurrent_fwd", dtype, gate_kind, w ? 0 : use_delta, q, k, v,
                          gp ? gp->neg_exp_a : g, gp ? gp->dt_bias : beta, o, cu_seqlens, B, T, H, dk, dv, n_seqs);
    if (rc) return rc;
    if (w && !use_delta) return fail(VGDR_ERR_INVALID, "vgdr_recurrent_fwd: an explicit write vector needs the delta rule");
    vgdr::Fusion fz;
    rc = check_fusion("vgdr_recurrent_fwd", fusion, dtype, gate_kind, use_delta, false, fz);
    if (rc) return rc;
    vgdr::Epilogue ep;
    rc = check_epilogue("vgdr_recurrent_fwd", epilogue, dtype, ep);
    if (rc) return rc;
    vgdr::ShortConv cv;
    rc = check_conv("vgdr_recurrent_fwd", conv, dtype, cv);
    if (rc) return rc;
    if (dv == 256) {
        // the layer's one-token decode step only: a state, the four-tap conv with
        // 16-byte aligned weights, one token per sequence, no packed offsets
        const bool ok = conv && cv.K == 4 && T == 1 && !cu_seqlens && initial_state && !w &&
                        aligned16(cv.wq) && aligned16(cv.wk) && aligned16(cv.wv);
        if (!ok)
            return fail(VGDR_ERR_UNSUPPORTED,
                        "vgdr_recurrent_fwd: dv=256 runs the one-token decode step with the four-tap short conv "
                        "(T=1, no cu_seqlens, a state, 16-byte aligned conv weights) only");
    } else if (dv != 64 && dv != 128) {
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_recurrent_fwd: dv=%lld (supported: 64, 128; 256 for the decode step "
                    "with the short conv)", (long long)dv);
    }
    if (!aligned16(initial_state) || !aligned16(final_state))
        return fail(VGDR_ERR_INVALID, "vgdr_recurrent_fwd: states must be 16-byte aligned");
    vgdr::RecParams p{};
    p.q = q; p.k = k; p.v = v;
    p.g = gate_kind == VGDR_GATE_NONE ? nullptr : g;
    p.beta = beta;
    p.o = o;
    p.h0 = initial_state;
    p.ht = final_state;
    p.cu = cu_seqlens;
    p.T = T;
    p.n_tokens = B * T;
    p.H = (int)H;
    p.n_seqs = (int)n_seqs;
    p.use_delta = use_delta ? 1 : 0;
    p.scale = scale;
    p.fz = fz;
    p.ep = ep;
    p.cv = cv;
    p.w = w;
    p.ld_qk = ld_qk;
    p.ld_v = ld_v;
    if (gp) {
        p.g = nullptr;
        p.beta = nullptr;
        p.gp = vgdr::GateProj{gp->x, gp->w, gp->neg_exp_a, gp->dt_bias, (int)gp->dim};
    }
    return hip_status(vgdr::recurrent_fwd(dtype, (int)dk, (int)dv, gate_kind == VGDR_GATE_VECTOR, p, stream),
                      "vgdr_recurrent_fwd launch");
}

}  // namespace

int vgdr_decode_step(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                     const float *g, const float *beta, void *o, const float *initial_state, float *final_state,
                     const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                     int64_t n_seqs, float scale, const vgdr_fusion *fusion, const vgdr_short_conv *conv,
                     const vgdr_epilogue *epilogue, hipStream_t stream) {
    return recurrent_call(dtype, gate_kind, use_delta, q, k, v, nullptr, g, beta, o, initial_state, final_state,
                          cu_seqlens, B, T, H, dk, dv, n_seqs, scale, fusion, conv, epilogue, stream);
}

int vgdr_decode_step_strided(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                             const float *g, const float *beta, void *o, const float *initial_state,
                             float *final_state, int64_t B, int64_t H, int64_t dk, int64_t dv, int64_t ld_qk,
                             int64_t ld_v, float scale, const vgdr_fusion *fusion, const vgdr_short_conv *conv,
                             const vgdr_epilogue *epilogue, const vgdr_gate_proj *gate_proj, hipStream_t stream) {
    // the strides reach only the one-token decode kernel: it needs a state and the
    // four-tap conv with 16-byte aligned weights (any other call would run the
    // token walk, which reads dense rows)
    g_err[0] = 0;
    if (ld_qk < H * dk || ld_v < H * dv)
        return fail(VGDR_ERR_INVALID, "vgdr_decode_step_strided: row strides (%lld, %lld) below H*dk = %lld, "
                    "H*dv = %lld", (long long)ld_qk, (long long)ld_v, (long long)(H * dk), (long long)(H * dv));
    if (!conv || conv->kernel_size != 4 || !aligned16(conv->weight_q) || !aligned16(conv->weight_k) ||
        !aligned16(conv->weight_v) || !initial_state)
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_decode_step_strided: strided rows need the four-tap short conv "
                    "with 16-byte aligned weights and an initial state");
    if (gate_proj) {
        const int64_t ve = dtype == VGDR_F32 ? 4 : 8, nt = dv > 128 ? 512 : 256;
        if (gate_kind != VGDR_GATE_SCALAR)
            return fail(VGDR_ERR_UNSUPPORTED, "vgdr_decode_step_strided: gate projections are for the scalar gate");
        if (!gate_proj->x || !gate_proj->w || !gate_proj->neg_exp_a || !gate_proj->dt_bias ||
            !aligned16(gate_proj->x) || !aligned16(gate_proj->w))
            return fail(VGDR_ERR_INVALID, "vgdr_decode_step_strided: gate projections need x, w (16-byte aligned), "
                        "neg_exp_a and dt_bias");
        if (gate_proj->dim <= 0 || gate_proj->dim % ve || gate_proj->dim > 2 * nt * ve)
            return fail(VGDR_ERR_UNSUPPORTED, "vgdr_decode_step_strided: gate projection dim=%lld (a multiple of "
                        "%lld up to %lld)", (long long)gate_proj->dim, (long long)ve, (long long)(2 * nt * ve));
    }
    return recurrent_call(dtype, gate_kind, use_delta, q, k, v, nullptr, g, beta, o, initial_state, final_state,
                          nullptr, B, 1, H, dk, dv, B, scale, fusion, conv, epilogue, stream, ld_qk, ld_v, gate_proj);
}

int vgdr_recurrent_fwd_w(int dtype, int gate_kind, const void *q, const void *k, const void *v, const void *w,
                         const float *g, void *o, const float *initial_state, float *final_state,
                         const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                         int64_t n_seqs, float scale, const vgdr_fusion *fusion, hipStream_t stream) {
    if (B * T > 0 && !w) {
        g_err[0] = 0;
        return fail(VGDR_ERR_INVALID, "vgdr_recurrent_fwd_w: w is required");
    }
    if (fusion && fusion->beta_sigmoid) {
        g_err[0] = 0;
        return fail(VGDR_ERR_INVALID, "vgdr_recurrent_fwd_w: there is no beta to activate with an explicit w");
    }
    static const char dummy = 0;           // w for an empty call: never read
    return recurrent_call(dtype, gate_kind, 1, q, k, v, w ? w : &dummy, g, nullptr, o, initial_state, final_state,
                          cu_seqlens, B, T, H, dk, dv, n_seqs, scale, fusion, nullptr, nullptr, stream);
}

int vgdr_recurrent_fwd_epilogue(int dtype, int gate_kind, int use_delta, const void *q, const void *k,
                                const void *v, const float *g, const float *beta, void *o,
                                const float *initial_state, float *final_state, const int32_t *cu_seqlens,
                                int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale,
                                const vgdr_fusion *fusion, const vgdr_epilogue *epilogue, hipStream_t stream) {
    return vgdr_decode_step(dtype, gate_kind, use_delta, q, k, v, g, beta, o, initial_state, final_state,
                            cu_seqlens, B, T, H, dk, dv, n_seqs, scale, fusion, nullptr, epilogue, stream);
}

int vgdr_recurrent_fwd_fused(int dtype, int gate_kind, int use_delta, const void *q, const void *k,
                             const void *v, const float *g, const float *beta, void *o,
                             const float *initial_state, float *final_state, const int32_t *cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs, float scale,
                             const vgdr_fusion *fusion, hipStream_t stream) {
    return vgdr_decode_step(dtype, gate_kind, use_delta, q, k, v, g, beta, o, initial_state, final_state,
                            cu_seqlens, B, T, H, dk, dv, n_seqs, scale, fusion, nullptr, nullptr, stream);
}

int vgdr_norm_gate(int dtype, const void *o, const vgdr_epilogue *epilogue, void *out, int64_t n_rows, int64_t dv,
                   hipStream_t stream) {
    g_err[0] = 0;
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: unknown dtype %d", dtype);
    if (!epilogue) return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: the epilogue is required");
    vgdr::Epilogue ep;
    int rc = check_epilogue("vgdr_norm_gate", epilogue, dtype, ep);
    if (rc) return rc;
    if (n_rows < 0) return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: n_rows=%lld", (long long)n_rows);
    const int64_t ve = dtype == VGDR_F32 ? 4 : 8, lpr = dv / ve;
    if (dv <= 0 || dv % ve || lpr > 64 || (lpr & (lpr - 1)))
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_norm_gate: dv=%lld (supported: %lld x a power of two, at most %lld)",
                    (long long)dv, (long long)ve, (long long)(64 * ve));
    if (n_rows == 0) return VGDR_OK;
    if (!o || !out) return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: o and out are required");
    if (!aligned16(o) || !aligned16(out) || !aligned16(ep.gamma))
        return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: o, out and gamma must be 16-byte aligned");
    if (n_rows > (int64_t)0xffffffffLL * 256 / lpr) return fail(VGDR_ERR_INVALID, "vgdr_norm_gate: too many rows");
    return hip_status(vgdr::norm_gate(dtype, o, ep, out, n_rows, (int)dv, stream), "vgdr_norm_gate launch");
}

int vgdr_rms_norm(int dtype, const void *x, const void *residual, void *x_out, const void *gamma, void *y,
                  int64_t rows, int64_t dim, float eps, hipStream_t stream) {
    g_err[0] = 0;
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: unknown dtype %d", dtype);
    const int64_t ve = dtype == VGDR_F32 ? 4 : 8;
    if (rows < 0) return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: rows=%lld", (long long)rows);
    if (dim <= 0 || dim % ve || dim / ve > 2048)
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_rms_norm: dim=%lld (supported: a multiple of %lld, at most %lld)",
                    (long long)dim, (long long)ve, (long long)(2048 * ve));
    if (!(eps >= 0.f)) return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: eps must be >= 0");
    if (rows == 0) return VGDR_OK;
    if (rows > 0x7fffffffLL) return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: too many rows");
    if (!x || !gamma || !y) return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: x, gamma and y are required");
    if (!aligned16(x) || !aligned16(gamma) || !aligned16(y) || (residual && !aligned16(residual)) ||
        (x_out && !aligned16(x_out)))
        return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: every tensor must be 16-byte aligned");
    if (y == x || (residual && y == residual) || (x_out && y == x_out))
        return fail(VGDR_ERR_INVALID, "vgdr_rms_norm: y must not alias x, residual or x_out");
    return hip_status(vgdr::rms_norm(dtype, x, residual, x_out, gamma, y, rows, (int)dim, eps, stream),
                      "vgdr_rms_norm launch");
}

int vgdr_scalar_gates(int dtype, const void *x, const void *w_ab, const float *neg_exp_a, const float *dt_bias,
                      float *g, float *beta, int64_t rows, int64_t dim, int64_t H, hipStream_t stream) {
    g_err[0] = 0;
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "vgdr_scalar_gates: unknown dtype %d", dtype);
    const int64_t ve = dtype == VGDR_F32 ? 4 : 8;
    if (rows < 0 || H <= 0 || H > 4096)
        return fail(VGDR_ERR_INVALID, "vgdr_scalar_gates: rows=%lld H=%lld", (long long)rows, (long long)H);
    if (dim <= 0 || dim % ve || dim > 0x7fffffffLL)
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_scalar_gates: dim=%lld (a multiple of %lld)", (long long)dim,
                    (long long)ve);
    if (rows == 0) return VGDR_OK;
    if (rows > 0x7fffffffLL) return fail(VGDR_ERR_INVALID, "vgdr_scalar_gates: too many rows");
    if (!x || !w_ab || !neg_exp_a || !dt_bias || !g)
        return fail(VGDR_ERR_INVALID, "vgdr_scalar_gates: x, w_ab, neg_exp_a, dt_bias and g are required");
    if (!aligned16(x) || !aligned16(w_ab)) return fail(VGDR_ERR_INVALID, "vgdr_scalar_gates: x and w_ab must be 16-byte aligned");
    return hip_status(vgdr::scalar_gates(dtype, x, w_ab, neg_exp_a, dt_bias, g, beta, rows, (int)dim, (int)H,
                                         beta != nullptr, stream),
                      "vgdr_scalar_gates launch");
}

int vgdr_swiglu(int dtype, const void *x, void *y, int64_t rows, int64_t hidden, hipStream_t stream) {
    g_err[0] = 0;
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "vgdr_swiglu: unknown dtype %d", dtype);
    const int64_t ve = dtype == VGDR_F32 ? 4 : 8;
    if (rows < 0) return fail(VGDR_ERR_INVALID, "vgdr_swiglu: rows=%lld", (long long)rows);
    if (hidden <= 0 || hidden % ve || hidden > 0x3fffffffLL)
        return fail(VGDR_ERR_UNSUPPORTED, "vgdr_swiglu: hidden=%lld (a multiple of %lld)", (long long)hidden,
                    (long long)ve);
    if (rows == 0) return VGDR_OK;
    if (!x || !y) return fail(VGDR_ERR_INVALID, "vgdr_swiglu: x and y are required");
    if (!aligned16(x) || !aligned16(y)) return fail(VGDR_ERR_INVALID, "vgdr_swiglu: x and y must be 16-byte aligned");
    if (x == y) return fail(VGDR_ERR_INVALID, "vgdr_swiglu: y must not alias x");
    if (rows * (hidden / ve) > (int64_t)0xffffffffLL * 256)
        return fail(VGDR_ERR_INVALID, "vgdr_swiglu: too many rows");
    return hip_status(vgdr::swiglu(dtype, x, y, rows, (int)hidden, stream), "vgdr_swiglu launch");
}

int vgdr_recurrent_fwd(int dtype, int gate_kind, int use_delta, const void *q, const void *k, const void *v,
                       const float *g, const float *beta, void *o, const float *initial_state,
                       float *final_state, const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t H,
                       int64_t dk, int64_t dv, int64_t n_seqs, float scale, hipStream_t stream) {
    return vgdr_recurrent_fwd_fused(dtype, gate_kind, use_delta, q, k, v, g, beta, o, initial_state, final_state,
                                    cu_seqlens, B, T, H, dk, dv, n_seqs, scale, nullptr, stream);
}

int vgdr_causal_conv1d(int dtype, const void *x, const void *weight, int weight_dtype, const void *initial_state,
                       void *y, void *final_state, const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t D,
                       int64_t n_seqs, int kernel_size, int activation, hipStream_t stream) {
    g_err[0] = 0;
    const char *fn = "vgdr_causal_conv1d";
    if (dtype != VGDR_F32 && dtype != VGDR_BF16 && dtype != VGDR_F16)
        return fail(VGDR_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
    if (weight_dtype != VGDR_F32 && weight_dtype != dtype)
        return fail(VGDR_ERR_INVALID, "%s: weight_dtype must be VGDR_F32 or dtype", fn);
    if (kernel_size < 1 || kernel_size > 8)
        return fail(VGDR_ERR_UNSUPPORTED, "%s: kernel_size=%d (supported: 1..8)", fn, kernel_size);
    if (activation != 0 && activation != 1) return fail(VGDR_ERR_INVALID, "%s: activation %d (0 none, 1 silu)", fn, activation);
    if (B < 0 || T < 0 || D <= 0 || n_seqs < 0 || n_seqs > 0x7fffffffLL)
        return fail(VGDR_ERR_INVALID, "%s: bad sizes", fn);
    const int64_t ve = dtype == VGDR_F32 ? 4 : 8;
    if (D % ve) return fail(VGDR_ERR_UNSUPPORTED, "%s: D=%lld (must be a multiple of %lld)", fn, (long long)D, (long long)ve);
    if (cu_seqlens) {
        if (B != 1) return fail(VGDR_ERR_INVALID, "%s: a packed batch (cu_seqlens) needs B == 1", fn);
    } else if (n_seqs != B) {
        return fail(VGDR_ERR_INVALID, "%s: n_seqs must equal B for a dense batch", fn);
    }
    if (B * T > 0 && (!x || !weight || !y)) return fail(VGDR_ERR_INVALID, "%s: x, weight and y are required", fn);
    if (!aligned16(x) || !aligned16(y) || !aligned16(initial_state) || !aligned16(final_state))
        return fail(VGDR_ERR_INVALID, "%s: x, y and the caches must be 16-byte aligned", fn);
    if (B * T > 0 && x == y) return fail(VGDR_ERR_INVALID, "%s: y must not alias x (outputs read earlier inputs)", fn);
    if (n_seqs > 0 && !weight) return fail(VGDR_ERR_INVALID, "%s: weight is required", fn);
    vgdr::ConvParams p{};
    p.x = x;
    p.w = weight;
    p.state_in = initial_state;
    p.y = y;
    p.state_out = final_state;
    p.cu = cu_seqlens;
    p.T = T;
    p.n_tokens = B * T;
    p.D = D;
    p.n_seqs = (int)n_seqs;
    p.K = kernel_size;
    p.w_f32 = weight_dtype == VGDR_F32 ? 1 : 0;
    p.silu = activation;
    if (p.n_tokens == 0 && (!final_state || n_seqs == 0)) return VGDR_OK;
    return hip_status(vgdr::causal_conv(dtype, p, stream), "vgdr_causal_conv1d launch");
}

int64_t vgdr_varlen_workspace_size(int64_t n_seqs) {
    return n_seqs < 0 ? 0 : (4 * n_seqs + 1) * (int64_t)sizeof(int32_t);
}

int vgdr_varlen_prepare(const int32_t *cu_seqlens, int64_t n_seqs, int64_t n_tokens, int chunk_size,
                        void *workspace, hipStream_t stream) {
    g_err[0] = 0;
    if (n_seqs < 0 || n_seqs > 0x7fffffffLL || n_tokens < 0)
        return fail(VGDR_ERR_INVALID, "vgdr_varlen_prepare: bad sizes");
    if (n_seqs > 0 && (!cu_seqlens || !workspace))
        return fail(VGDR_ERR_INVALID, "vgdr_varlen_prepare: cu_seqlens and workspace are required");
    if (chunk_size <= 0) return fail(VGDR_ERR_INVALID, "vgdr_varlen_prepare: chunk_size must be positive");
    return hip_status(vgdr::varlen_prepare(cu_seqlens, (int)n_seqs, n_tokens, chunk_size,
                                           reinterpret_cast<int32_t *>(workspace), stream),
                      "vgdr_varlen_prepare launch");
}

}  // extern "C"
