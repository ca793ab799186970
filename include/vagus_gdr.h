/*
 * vagus_gdr.h — C ABI of the MI355X (gfx950) gated delta-rule core.
 *
 * Replaces the backend call of the reference's GPU scan path,
 * infra/components/linear_attention.py:474-497 (fla_scan → fla's
 * chunk_gated_delta_rule / chunk_kda / chunk_simple_gla), selected by
 * GatedDeltaNet._pick_impl / _scan (:755-812), and the single-token
 * recurrence it runs for decode (recurrent_scan at L == 1, :945-947).
 *
 * Semantics, per (sequence, head), with state S in R^{dk x dv}
 * (linear_attention.py:8-11, :161-195):
 *     S_t = (I - beta_t k_t k_t^T) Diag(a_t) S_{t-1} + beta_t k_t v_t^T
 *     o_t = scale * S_t^T q_t,          a_t = exp(g_t)
 * use_delta = 0 drops the erase term: S_t = Diag(a_t) S_{t-1} + k_t v_t^T.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (hipMalloc'd or torch tensors); all
 *     tensors are dense row-major (contiguous).  Inputs are read-only.
 *   - Token layout: q, k  [n_tokens, H, dk];  v, o  [n_tokens, H, dv];
 *     g  [n_tokens, H] (gate_kind 1) or [n_tokens, H, dk] (gate_kind 2), fp32;
 *     beta [n_tokens, H] fp32.  n_tokens = B * T for a dense batch.
 *   - Sequences: with cu_seqlens == NULL the batch is dense, B sequences of
 *     T tokens (sequence b owns tokens [b*T, (b+1)*T)).  Otherwise
 *     cu_seqlens is a device int32 array of n_seqs + 1 offsets into a packed
 *     stream of n_tokens = T tokens (B must be 1).  The caller guarantees
 *     cu[0] = 0, cu[n] <= cu[n+1] and cu[n_seqs] = T (the Python layer checks
 *     it on the host); the kernels do not read the table back.  Each segment
 *     is clamped to [0, T], so a malformed table cannot address memory
 *     outside the tensors, but overlapping segments race on o and tokens no
 *     segment covers are left unwritten.
 *   - States: initial_state / final_state are fp32 [n_seqs, H, dk, dv]
 *     (n_seqs = B for a dense batch), either may be NULL (zeros / not
 *     written).  They may alias (in-place update).
 *   - dtype is the element type of q, k, v and o.
 *   - Every call is asynchronous on `stream`, allocates nothing and never
 *     synchronises.  Calls are reentrant.  Return 0 on success; on failure a
 *     VGDR_ERR_* code and a message readable with vgdr_last_error() (a
 *     per-thread string).
 */
#ifndef VAGUS_GDR_H
#define VAGUS_GDR_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vgdr_status {
    VGDR_OK = 0,
    VGDR_ERR_INVALID = 1,      /* misuse: bad shape / pointer / flag (reference: AssertionError)  */
    VGDR_ERR_UNSUPPORTED = 2,  /* valid but not implemented (reference: NotImplementedError)      */
    VGDR_ERR_HIP = 3           /* the HIP runtime reported an error (reference: RuntimeError)      */
};

enum vgdr_dtype { VGDR_F32 = 0, VGDR_BF16 = 1, VGDR_F16 = 2 };

enum vgdr_gate {
    VGDR_GATE_NONE = 0,        /* a_t = 1 (g ignored, may be NULL)      — DeltaNet               */
    VGDR_GATE_SCALAR = 1,      /* g [n_tokens, H]: one decay per head   — Gated DeltaNet (GDN)   */
    VGDR_GATE_VECTOR = 2       /* g [n_tokens, H, dk]: per key channel  — Kimi Delta Attn (KDA)  */
};

/*
 * Producer fusions: elementwise work on the scan's operands that a caller
 * would otherwise do in separate passes, applied where the kernels read those
 * operands.  These are the flags the reference hands to its fla call,
 * linear_attention.py:457-497 (use_qk_l2norm_in_kernel,
 * use_beta_sigmoid_in_kernel, use_gate_in_kernel with A_log / dt_bias and
 * safe_gate / lower_bound), with the reference's own activations
 * (:703-706, :719-736).  A NULL vgdr_fusion pointer means none.
 */
typedef struct vgdr_fusion {
    int qk_l2norm;          /* q, k un-normalised: x rsqrt(sum_c x_c^2 + 1e-6) per (token, head), rounded
                               to q's type (the chunked scan: needs use_delta, as fla) */
    int beta_sigmoid;       /* beta holds logits: sigmoid(beta) (the chunked scan: needs use_delta) */
    int gate_activation;    /* gate_kind 2 only: g holds the pre-activation f [n_tokens, H, dk] and
                               g = lower_bound_set ? lower_bound * sigmoid(exp(A_log[h]) (f + dt_bias[h dk + c]))
                                                   : -exp(A_log[h]) softplus(f + dt_bias[h dk + c]) */
    int gate_dtype;         /* element type of f: VGDR_F32, or the dtype of q */
    const float *A_log;     /* [H] fp32 */
    const float *dt_bias;   /* [H * dk] fp32 */
    int lower_bound_set;
    float lower_bound;
} vgdr_fusion;

/*
 * Output epilogue of the layer: per (token, head), RMSNorm of o over dv with
 * weight gamma, times SiLU of the output gate (linear_attention.py:814-825,
 * norm_layer.py:15-24; fla's rms_norm_gated with activation 'swish', :820-823):
 *     out = x rsqrt(mean_c x_c^2 + eps) gamma * gate sigmoid(gate),   x = o rounded to dtype
 * computed in fp32 and rounded once to dtype.
 */
typedef struct vgdr_epilogue {
    const void *gate;       /* [n_tokens, H, dv] in dtype (the W_g x projection), 16-byte aligned */
    const void *gamma;      /* [dv] RMSNorm weight */
    int gamma_dtype;        /* VGDR_F32 or dtype */
    float eps;              /* > 0 */
} vgdr_epilogue;

/*
 * The layer's short causal convolution + SiLU on the q, k, v projections
 * (ShortConv, opt.py:15-93, applied at linear_attention.py:741-745), with the
 * decode-time conv cache (:929-941): channel c of token t is
 *     SiLU( sum_j w[c][j] x[t - K + 1 + j][c] ),
 * the inputs before a sequence's first token taken from its cache, which holds
 * the sequence's last K inputs and is advanced in place.  The convolution's and
 * the SiLU's results are rounded to dtype, as the module computes them.
 */
typedef struct vgdr_short_conv {
    const void *weight_q;   /* [H * dk, K]: nn.Conv1d's (D, 1, K) weight, squeezed */
    const void *weight_k;   /* [H * dk, K] */
    const void *weight_v;   /* [H * dv, K] */
    void *cache_q;          /* [n_seqs, K, H * dk] in dtype (the module's qp_cache) */
    void *cache_k;          /* [n_seqs, K, H * dk] */
    void *cache_v;          /* [n_seqs, K, H * dv] */
    int kernel_size;        /* K, 1..8 */
    int weight_dtype;       /* VGDR_F32 or dtype */
} vgdr_short_conv;

/* Library version (major * 10000 + minor * 100 + patch). */
int vgdr_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *vgdr_last_error(void);

/*
 * Chunkwise prefill.  Replaces fla's chunk_gated_delta_rule (gate_kind 0/1,
 * use_delta 1), chunk_kda (gate_kind 2) and chunk_simple_gla (use_delta 0)
 * as called at linear_attention.py:474-497, with the reference's WY chunk
 * semantics (chunk_scan :237-309, chunk_scan_vec :312-425).
 *
 * chunk_size is accepted for interface parity: values <= 32 select 32-token
 * chunks, larger ones 64 (fp32 always uses 32); the result is
 * chunk-size invariant up to rounding.  Supported: dk in {64, 128}, dv a
 * positive multiple of 16.
 *
 * The caller provides `workspace` (16-byte aligned device memory of at least
 * vgdr_chunk_workspace_size(...) bytes for the same dtype, gate_kind, sizes
 * and chunk_size; contents irrelevant): it holds the per-chunk intermediate
 * products and, for a packed batch, the segment table (see
 * vgdr_varlen_prepare).  Calls sharing one workspace must not overlap.
 */
int64_t vgdr_chunk_workspace_size(int dtype, int gate_kind, int64_t B, int64_t T, int64_t H, int64_t dk,
                                  int64_t n_seqs, int varlen, int chunk_size);

int vgdr_chunk_fwd(int dtype, int gate_kind, int use_delta,
                   const void *q, const void *k, const void *v,
                   const float *g, const float *beta,
                   void *o, const float *initial_state, float *final_state,
                   const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                   int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                   float scale, int chunk_size, hipStream_t stream);

/*
 * The two phases of vgdr_chunk_fwd as separate calls (same arguments, same
 * checks; no reference counterpart).  vgdr_chunk_prep builds the packed-batch
 * schedule and, for every (chunk, head) in parallel, the state-independent
 * intra-chunk blocks, into `workspace`; it reads q, k, g, beta and cu_seqlens.
 * vgdr_chunk_state then runs the sequential chunk recurrence from that
 * workspace and writes o and final_state.  prep followed by state on one
 * stream (same arguments, workspace untouched in between) equals
 * vgdr_chunk_fwd.  For callers that time or schedule the phases separately.
 */
int vgdr_chunk_prep(int dtype, int gate_kind, int use_delta,
                    const void *q, const void *k, const void *v,
                    const float *g, const float *beta,
                    void *o, const float *initial_state, float *final_state,
                    const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                    int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                    float scale, int chunk_size, hipStream_t stream);
int vgdr_chunk_state(int dtype, int gate_kind, int use_delta,
                     const void *q, const void *k, const void *v,
                     const float *g, const float *beta,
                     void *o, const float *initial_state, float *final_state,
                     const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                     int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                     float scale, int chunk_size, hipStream_t stream);

/*
 * vgdr_chunk_fwd / vgdr_chunk_prep with producer fusions (vgdr_fusion above;
 * 16-bit dtypes).  The state phase reads only what the prep phase wrote, so
 * vgdr_chunk_state is the same for fused and unfused calls.  Replaces the
 * fla call at linear_attention.py:474-497 with its *_in_kernel flags set.
 */
int vgdr_chunk_fwd_fused(int dtype, int gate_kind, int use_delta,
                         const void *q, const void *k, const void *v,
                         const float *g, const float *beta,
                         void *o, const float *initial_state, float *final_state,
                         const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                         int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                         float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream);
int vgdr_chunk_prep_fused(int dtype, int gate_kind, int use_delta,
                          const void *q, const void *k, const void *v,
                          const float *g, const float *beta,
                          void *o, const float *initial_state, float *final_state,
                          const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                          int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                          float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream);

/*
 * vgdr_chunk_fwd_fused without a workspace argument and without allocating
 * (no reference counterpart: for callers that cannot allocate device memory,
 * such as code under HIP graph capture or a serving loop that forbids
 * hipMalloc).  The chunk workspace lives in a file-scope device array,
 * VGDR_CHUNK_SCRATCH_BYTES long, which exists on every GPU where the library's
 * code object is loaded (its first kernel launch of any entry point there)
 * until the end of the process: every process using the library holds it on
 * each GPU it runs on, whether or not it calls this entry point.  A call whose vgdr_chunk_workspace_size exceeds it
 * returns VGDR_ERR_INVALID (use vgdr_chunk_fwd_fused with a workspace).
 * Calls that overlap on one GPU (two streams, two threads) share that array
 * and race; serialise them.  Otherwise the arguments, checks and results are
 * those of vgdr_chunk_fwd_fused (fusion may be NULL).
 */
#define VGDR_CHUNK_SCRATCH_BYTES (64LL << 20)
int vgdr_chunk_fwd_noalloc(int dtype, int gate_kind, int use_delta,
                           const void *q, const void *k, const void *v,
                           const float *g, const float *beta,
                           void *o, const float *initial_state, float *final_state,
                           const int32_t *cu_seqlens,
                           int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                           float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream);

/*
 * vgdr_chunk_fwd with an explicit write vector w [n_tokens, H, dk] (16-bit,
 * 16-byte aligned) in place of beta_t k_t: the asymmetric delta rule of
 * chunk_scan_vec(..., w=w) (linear_attention.py:312-425, :340-353,
 * :389-396), on the per-channel-gate path: g [n_tokens, H, dk] fp32 log-decay
 * (zeros for none).  No beta.  The workspace is vgdr_chunk_workspace_size's
 * for gate_kind 2.  fusion: the q, k L2 norm and the KDA gate activation.
 */
int vgdr_chunk_fwd_w(int dtype, const void *q, const void *k, const void *v, const void *w,
                     const float *g, void *o, const float *initial_state, float *final_state,
                     const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                     int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                     float scale, int chunk_size, const vgdr_fusion *fusion, hipStream_t stream);

/*
 * Backward of the chunked scan, scalar gate (gate_kind 1), per-channel gate
 * (2, 16-bit dtypes, 64-token chunks) or none (0), delta rule: the gradients
 * the reference's training takes through chunk_scan and chunk_scan_vec
 * (linear_attention.py:237-309, :312-425, autograd) or fla's
 * chunk_gated_delta_rule / chunk_kda backward (the calls at :487-491 and
 * :474-479 with grads enabled).  Inputs as the forward call had them (q, k
 * already normalised; beta in [0, 1]; g the log-decay, [n_tokens, H] or
 * [n_tokens, H, dk]; initial_state nullable), plus grad_o [n_tokens, H, dv]
 * in dtype and grad_final_state [n_seqs, H, dk, dv] fp32 (nullable: zero).
 * Outputs: grad_q, grad_k [n_tokens, H, dk], grad_v [n_tokens, H, dv] in
 * dtype; grad_g fp32 shaped as g (unused and nullable without a gate);
 * grad_beta [n_tokens, H] fp32; grad_initial_state [n_seqs, H, dk, dv] fp32
 * (nullable: not computed).
 * The gradients must not alias the inputs; grad_o and grad_v are 16-byte
 * aligned (q, k, v as in vgdr_chunk_fwd).  workspace:
 * vgdr_chunk_bwd_workspace_size(...) bytes, 16-byte aligned; it holds the
 * chunk blocks (rebuilt from q, k, g, beta), each chunk's entry state and the
 * gradient of its exit state.  Same dk, dv, chunk_size and packed-batch
 * rules as vgdr_chunk_fwd.
 */
int64_t vgdr_chunk_bwd_workspace_size(int dtype, int gate_kind, int64_t B, int64_t T, int64_t H, int64_t dk,
                                      int64_t dv, int64_t n_seqs, int varlen, int chunk_size);
int vgdr_chunk_bwd(int dtype, int gate_kind,
                   const void *q, const void *k, const void *v, const float *g, const float *beta,
                   const float *initial_state, const void *grad_o, const float *grad_final_state,
                   void *grad_q, void *grad_k, void *grad_v, float *grad_g, float *grad_beta,
                   float *grad_initial_state,
                   const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                   int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                   float scale, int chunk_size, hipStream_t stream);

/*
 * The same pair with the forward's intermediates kept instead of recomputed
 * (no reference counterpart as an entry point; fla's disable_recompute,
 * linear_attention.py:463-471, is the same trade of memory for time).
 * vgdr_chunk_fwd_saving is vgdr_chunk_fwd (16-bit dtypes, any gate_kind,
 * 64-token chunks with the per-channel gate, delta rule, no fusion) run in
 * the backward's workspace
 * (vgdr_chunk_bwd_workspace_size bytes, same dv): besides o and final_state it
 * leaves there the packed-batch schedule, the chunk blocks and every chunk's
 * entry state.  vgdr_chunk_bwd_saved, called with the same inputs and that
 * workspace untouched in between, is vgdr_chunk_bwd without rebuilding them
 * (it skips the chunk prep and the forward re-walk).
 */
int vgdr_chunk_fwd_saving(int dtype, int gate_kind, const void *q, const void *k, const void *v,
                          const float *g, const float *beta, void *o, const float *initial_state,
                          float *final_state, const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                          int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                          float scale, int chunk_size, hipStream_t stream);
int vgdr_chunk_bwd_saved(int dtype, int gate_kind,
                         const void *q, const void *k, const void *v, const float *g, const float *beta,
                         const float *initial_state, const void *grad_o, const float *grad_final_state,
                         void *grad_q, void *grad_k, void *grad_v, float *grad_g, float *grad_beta,
                         float *grad_initial_state,
                         const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                         int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                         float scale, int chunk_size, hipStream_t stream);

/*
 * Backward of the chunked scan without the delta rule (the plain gated
 * recurrence S_t = g_t S_{t-1} + k_t v_t^T: chunk_simple_gla, and
 * chunk_scan_vec / chunk_scan with delta=False, linear_attention.py:237-309,
 * :312-425, autograd): vgdr_chunk_bwd's arguments and workspace
 * (vgdr_chunk_bwd_workspace_size) without beta and grad_beta.  gate_kind 0 and
 * 1 at every dtype, 2 with 16-bit q, k, v in 64-token chunks.  The delta-form
 * kernels run it: chunk prep writes TE = I and zeroes the K decay factor, so
 * U = V.
 */
int vgdr_chunk_bwd_nodelta(int dtype, int gate_kind, const void *q, const void *k, const void *v, const float *g,
                           const float *initial_state, const void *grad_o, const float *grad_final_state,
                           void *grad_q, void *grad_k, void *grad_v, float *grad_g, float *grad_initial_state,
                           const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                           int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                           float scale, int chunk_size, hipStream_t stream);

/*
 * Backward of the chunked scan with explicit write vectors (vgdr_chunk_fwd_w's
 * recurrence, chunk_scan_vec(..., w=) with grads, linear_attention.py:312-425,
 * :340-353, :389-396): vgdr_chunk_bwd's arguments for gate_kind 2 with w in
 * place of beta, grad_w [n_tokens, H, dk] (dtype, 16-byte aligned like w) in
 * place of grad_beta; 16-bit q, k, v, w, 64-token chunks.  The workspace is
 * vgdr_chunk_bwd_workspace_size's for gate_kind 2.
 */
int vgdr_chunk_bwd_w(int dtype, const void *q, const void *k, const void *v, const void *w, const float *g,
                     const float *initial_state, const void *grad_o, const float *grad_final_state,
                     void *grad_q, void *grad_k, void *grad_v, void *grad_w, float *grad_g,
                     float *grad_initial_state, const int32_t *cu_seqlens, void *workspace,
                     int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                     int64_t n_seqs, float scale, int chunk_size, hipStream_t stream);

/*
 * The training pair with the producer fusions the backward can take through
 * (no reference counterpart as entry points: fla's chunk_kda /
 * chunk_gated_delta_rule with use_beta_sigmoid_in_kernel and
 * use_gate_in_kernel differentiate through them, linear_attention.py:474-479,
 * :487-491).  fusion as in vgdr_chunk_fwd_fused, with qk_l2norm 0 (q, k arrive
 * normalised): beta_sigmoid: beta holds logits and grad_beta receives their
 * gradient; gate_activation (gate_kind 2): g holds the pre-activation f
 * [n_tokens, H, dk] (gate_dtype fp32 or dtype), grad_g receives df (fp32,
 * [n_tokens, H, dk]), grad_A_log [H] and grad_dt_bias [H * dk] (fp32,
 * overwritten) receive the gradients of the activation's parameters, summed
 * over every token in a fixed order (no atomics).  A NULL fusion is the
 * unfused call.  The saving forward and the saved backward take the same
 * fusion.
 */
int vgdr_chunk_fwd_saving_fused(int dtype, int gate_kind, const void *q, const void *k, const void *v,
                                const float *g, const float *beta, void *o, const float *initial_state,
                                float *final_state, const int32_t *cu_seqlens, void *workspace,
                                int64_t workspace_bytes, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv,
                                int64_t n_seqs, float scale, int chunk_size, const vgdr_fusion *fusion,
                                hipStream_t stream);
int vgdr_chunk_bwd_fused(int dtype, int gate_kind,
                         const void *q, const void *k, const void *v, const float *g, const float *beta,
                         const float *initial_state, const void *grad_o, const float *grad_final_state,
                         void *grad_q, void *grad_k, void *grad_v, float *grad_g, float *grad_beta,
                         float *grad_initial_state,
                         const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                         int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                         float scale, int chunk_size, const vgdr_fusion *fusion, float *grad_A_log,
                         float *grad_dt_bias, hipStream_t stream);
int vgdr_chunk_bwd_saved_fused(int dtype, int gate_kind,
                               const void *q, const void *k, const void *v, const float *g, const float *beta,
                               const float *initial_state, const void *grad_o, const float *grad_final_state,
                               void *grad_q, void *grad_k, void *grad_v, float *grad_g, float *grad_beta,
                               float *grad_initial_state,
                               const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                               int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                               float scale, int chunk_size, const vgdr_fusion *fusion, float *grad_A_log,
                               float *grad_dt_bias, hipStream_t stream);

/*
 * Backward of every scan form: the per-channel (KDA) gate, the explicit write
 * vector w (the asymmetric delta rule) and the plain recurrence without the
 * delta rule, besides the scalar gate and no gate.  Replaces the autograd of
 * chunk_scan_vec (linear_attention.py:312-425, the KDA and w path) and of
 * recurrent_scan / chunk_scan for use_delta = 0 (:161-195, :237-309).
 * Inputs as vgdr_recurrent_fwd_w (w != NULL) or vgdr_recurrent_fwd; beta is
 * read only for the delta rule without w.  Gradients: grad_q, grad_k, grad_v
 * (and grad_w with w) in dtype; grad_g (the gate's shape, gate_kind != 0),
 * grad_beta (delta rule without w) and grad_initial_state (may be NULL) in
 * fp32.  grad_final_state may be NULL (zero).  dk in {64, 128}; dv a positive
 * multiple of 16.  Workspace: vgdr_scan_bwd_workspace_size(...) bytes,
 * 16-byte aligned (state and state-gradient checkpoints every 8 tokens in
 * fp32, u_t per token, per-column-tile partial sums).
 */
int64_t vgdr_scan_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs);
int vgdr_scan_bwd(int dtype, int gate_kind, int use_delta,
                  const void *q, const void *k, const void *v, const void *w,
                  const float *g, const float *beta, const float *initial_state,
                  const void *grad_o, const float *grad_final_state,
                  void *grad_q, void *grad_k, void *grad_v, void *grad_w,
                  float *grad_g, float *grad_beta, float *grad_initial_state,
                  const int32_t *cu_seqlens, void *workspace, int64_t workspace_bytes,
                  int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                  float scale, hipStream_t stream);

/*
 * Token-by-token recurrence.  The decode step is T = 1 with
 * initial_state == final_state (in place), replacing recurrent_scan at
 * linear_attention.py:945-947 and the state.copy_ at :950.  Any T works (the
 * reference's fused_recurrent semantics).  dk in {64, 128}, dv in {64, 128}.
 */
int vgdr_recurrent_fwd(int dtype, int gate_kind, int use_delta,
                       const void *q, const void *k, const void *v,
                       const float *g, const float *beta,
                       void *o, const float *initial_state, float *final_state,
                       const int32_t *cu_seqlens,
                       int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                       float scale, hipStream_t stream);

/* vgdr_recurrent_fwd with producer fusions (vgdr_fusion; any dtype).  No
 * reference counterpart (the reference normalises and activates in torch
 * before recurrent_scan, linear_attention.py:698-753); a decode step that
 * takes raw projections. */
int vgdr_recurrent_fwd_fused(int dtype, int gate_kind, int use_delta,
                             const void *q, const void *k, const void *v,
                             const float *g, const float *beta,
                             void *o, const float *initial_state, float *final_state,
                             const int32_t *cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                             float scale, const vgdr_fusion *fusion, hipStream_t stream);

/* vgdr_recurrent_fwd_fused whose o receives the layer's output epilogue
 * (vgdr_epilogue; NULL = plain o) instead of the raw scan output: the decode
 * step of GatedDeltaNet.decode_step through _output, up to W_o
 * (linear_attention.py:945-952 and :814-825), in one kernel.  The workgroup of
 * a (sequence, head) holds the whole dv row, so the norm needs no extra pass. */
int vgdr_recurrent_fwd_epilogue(int dtype, int gate_kind, int use_delta,
                                const void *q, const void *k, const void *v,
                                const float *g, const float *beta,
                                void *o, const float *initial_state, float *final_state,
                                const int32_t *cu_seqlens,
                                int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                                float scale, const vgdr_fusion *fusion, const vgdr_epilogue *epilogue,
                                hipStream_t stream);

/* vgdr_recurrent_fwd with an explicit write vector w [n_tokens, H, dk] (dtype)
 * in place of beta_t k_t: the asymmetric delta rule
 *     S_t = Diag(a_t) S_{t-1} + w_t (v_t - k_t^T Diag(a_t) S_{t-1})^T
 * of recurrent_scan(..., w=w) (linear_attention.py:161-170, :185-188; the
 * write a Kalman gain produces, KalmanDeltaNet).  No beta; fusion as in
 * vgdr_recurrent_fwd_fused (the q, k L2 norm, the KDA gate activation). */
int vgdr_recurrent_fwd_w(int dtype, int gate_kind,
                         const void *q, const void *k, const void *v, const void *w,
                         const float *g, void *o, const float *initial_state, float *final_state,
                         const int32_t *cu_seqlens,
                         int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                         float scale, const vgdr_fusion *fusion, hipStream_t stream);

/* The decode step of GatedDeltaNet.decode_step from the projections to the
 * input of W_o (linear_attention.py:918-952 with _heads :737-747 and _output
 * :814-825), in one kernel per call: with `conv` (NULL = none), q, k, v are
 * the raw projections qp, kp, vp [n_tokens, H, d] and go through the short
 * conv + SiLU (advancing its caches), then the producer fusions (the q, k L2
 * norm, beta sigmoid, KDA gate activation), the recurrence from
 * initial_state, and with `epilogue` the RMSNorm x SiLU(gate) output.
 * dk, dv in {64, 128}; dv = 256 (dk 128 / dv 256 heads) for one token per
 * sequence (T = 1, cu_seqlens NULL) from an initial_state with the four-tap
 * conv and 16-byte aligned conv weights, else VGDR_ERR_UNSUPPORTED. */
int vgdr_decode_step(int dtype, int gate_kind, int use_delta,
                     const void *q, const void *k, const void *v,
                     const float *g, const float *beta,
                     void *o, const float *initial_state, float *final_state,
                     const int32_t *cu_seqlens,
                     int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv, int64_t n_seqs,
                     float scale, const vgdr_fusion *fusion, const vgdr_short_conv *conv,
                     const vgdr_epilogue *epilogue, hipStream_t stream);

/* The scalar gate and beta of a one-token decode step formed inside the
 * decode kernel from the layer's input row (GatedDeltaNet._gates,
 * linear_attention.py:719-721 and :734-735): p_a = W_a x and p_b = W_b x
 * rounded to dtype (nn.Linear's outputs), g = neg_exp_a * softplus(p_a +
 * dt_bias) and beta = p_b (logits; vgdr_fusion.beta_sigmoid activates them).
 * x [B, dim] and w [H, dim] (W_a), followed by [H, dim] (W_b) with the delta
 * rule, are in dtype with 16-byte aligned rows; dim a multiple of 16 bytes,
 * at most 4096 elements for 16-bit dtypes and dv <= 128 (twice that at
 * dv = 256, half for fp32). */
typedef struct vgdr_gate_proj {
    const void *x;
    const void *w;
    const float *neg_exp_a;  /* [H]: -exp(A_log) */
    const float *dt_bias;    /* [H] */
    int64_t dim;
} vgdr_gate_proj;

/* vgdr_decode_step (GatedDeltaNet.decode_step, linear_attention.py:918-952)
 * for one token per sequence (T = 1, n_seqs = B, no cu_seqlens) whose inputs
 * are rows of a wider buffer: token b's q, k are at
 * q + b * ld_qk, k + b * ld_qk and its v and epilogue gate at v + b * ld_v,
 * gate + b * ld_v (elements; each row's H * d block dense).  The layer's four
 * projections from one GEMM over their concatenated weights are read in place
 * this way, with no copy into separate tensors (the reference's projections
 * are separate nn.Linear outputs, :929 and :816, so it has no such form).  Needs `conv`
 * with K = 4 and 16-byte aligned weights and an initial_state
 * (VGDR_ERR_UNSUPPORTED otherwise); ld_qk >= H * dk, ld_v >= H * dv
 * (VGDR_ERR_INVALID otherwise).  With gate_proj (scalar gate only) the kernel
 * forms g and beta itself and the g and beta arguments are not read: the
 * layer's separate gate kernel is then not launched. */
int vgdr_decode_step_strided(int dtype, int gate_kind, int use_delta,
                             const void *q, const void *k, const void *v,
                             const float *g, const float *beta,
                             void *o, const float *initial_state, float *final_state,
                             int64_t B, int64_t H, int64_t dk, int64_t dv, int64_t ld_qk, int64_t ld_v,
                             float scale, const vgdr_fusion *fusion, const vgdr_short_conv *conv,
                             const vgdr_epilogue *epilogue, const vgdr_gate_proj *gate_proj,
                             hipStream_t stream);

/* The short conv + SiLU (vgdr_short_conv's semantics) over a whole call's
 * tokens, for prefill: y[t] from x[t - K + 1 .. t] of the same sequence.
 * Replaces the module's ShortConv (opt.py:15-100; fla's causal_conv1d as the
 * reference calls it, :73-77) and, with caches, the cached conv of a
 * multi-token decode_step (:929-941).  x, y [n_tokens, D] (the q, k or v
 * projection, D = H * d); weight [D, K] (fp32 or dtype); initial_state /
 * final_state: [n_seqs, K, D] conv caches in dtype, NULL = zeros / not
 * written, and may alias.  activation: 0 none, 1 SiLU.  The convolution's and
 * the SiLU's results are rounded to dtype.  Sequences as in the scans
 * (dense B x T, or packed with cu_seqlens and B = 1). */
int vgdr_causal_conv1d(int dtype, const void *x, const void *weight, int weight_dtype,
                       const void *initial_state, void *y, void *final_state,
                       const int32_t *cu_seqlens, int64_t B, int64_t T, int64_t D, int64_t n_seqs,
                       int kernel_size, int activation, hipStream_t stream);

/* The output epilogue as one pass over n_rows rows of dv elements (a row per
 * (token, head)): out = epilogue(o, gate).  Replaces rms_norm_gated / the
 * RMSNorm x SiLU expression at linear_attention.py:820-825 after a chunked
 * prefill (the chunk kernels split dv across workgroups).  out may equal o.
 * dv = 8 x a power of two up to 512 (16-bit), 4 x a power of two up to 256
 * (fp32); o, out and gamma 16-byte aligned. */
int vgdr_norm_gate(int dtype, const void *o, const vgdr_epilogue *epilogue, void *out, int64_t n_rows,
                   int64_t dv, hipStream_t stream);

/* The pre-norm blocks' RMSNorm (infra/components/norm_layer.py:15-23) over rows
 * rows of dim elements, with the residual add in front of it that the blocks
 * make before each norm (infra/components/block.py:57-59, :85-87):
 *     h = x + residual   (rounded to dtype; h = x when residual is NULL)
 *     y = dtype(dtype(h * rsqrt(mean(h^2) + eps)) * gamma)
 * and h is written to x_out unless x_out is NULL.  x, residual, x_out, y:
 * [rows, dim]; gamma: [dim]; all in dtype and 16-byte aligned.  x_out may be x
 * or residual (the residual stream updated in place); y must differ from x,
 * residual and x_out.  dim a multiple of 16 / sizeof(dtype), at most 2048
 * such units (16,384 elements of a 16-bit type). */
int vgdr_rms_norm(int dtype, const void *x, const void *residual, void *x_out, const void *gamma, void *y,
                  int64_t rows, int64_t dim, float eps, hipStream_t stream);

/* The scalar gate and the beta logits of the LM's one-token decode step
 * (GatedDeltaNet._gates, linear_attention.py:719-721 and :734-735), from the
 * layer input x [rows, dim] and the projection weights stacked as
 * w_ab = [W_a; W_b] ([2H, dim], or W_a alone [H, dim] without beta), all in
 * dtype:
 *     p    = dtype(w_ab x)                       (nn.Linear's output)
 *     g    = neg_exp_a * softplus(p[:H] + dt_bias)    -> g [rows, H], fp32
 *     beta = p[H:]                                     -> beta [rows, H], fp32
 * neg_exp_a = -exp(A_log) and dt_bias in fp32, [H].  beta NULL = no W_b rows.
 * x and w_ab 16-byte aligned; dim a multiple of 16 / sizeof(dtype); H <= 4096. */
int vgdr_scalar_gates(int dtype, const void *x, const void *w_ab, const float *neg_exp_a, const float *dt_bias,
                      float *g, float *beta, int64_t rows, int64_t dim, int64_t H, hipStream_t stream);

/* The FFN's SwiGLU (infra/components/ffn.py:48-50): y = dtype(dtype(SiLU(a)) * b)
 * for each row x = [a | b] of 2 * hidden elements, y [rows, hidden], in dtype
 * (fp32, bf16, fp16), 16-byte aligned; hidden a multiple of 16 / sizeof(dtype).
 * y must not alias x. */
int vgdr_swiglu(int dtype, const void *x, void *y, int64_t rows, int64_t hidden, hipStream_t stream);

/*
 * Packed-batch schedule.  No reference counterpart (the reference has no
 * cu_seqlens, see infra/inference/generator.py:19-22); fla builds the same
 * integer tables for its varlen kernels.  Writes into `workspace`
 * (vgdr_varlen_workspace_size(n_seqs) bytes, int32 fields in this order):
 *     lens[n_seqs], chunks[n_seqs], chunk_offsets[n_seqs + 1], order[n_seqs]
 * lens = cu[n+1] - cu[n] (clamped into [0, n_tokens]), chunks =
 * ceil(lens / chunk_size), chunk_offsets = exclusive prefix sum of chunks,
 * order = segments sorted longest first, ties by index.
 */
int64_t vgdr_varlen_workspace_size(int64_t n_seqs);
int vgdr_varlen_prepare(const int32_t *cu_seqlens, int64_t n_seqs, int64_t n_tokens,
                        int chunk_size, void *workspace, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VAGUS_GDR_H */
