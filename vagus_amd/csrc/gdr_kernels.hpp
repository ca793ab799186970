// Kernel parameter blocks and launcher declarations shared by the C ABI
// (gdr_api.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vgdr {

// Sequence geometry shared by the chunk kernels: a dense batch (cu == NULL,
// n_seqs sequences of T tokens) or a packed one indexed by cu (clamped).
struct SeqGeom {
    const int32_t *cu;            // [n_seqs + 1] or NULL
    const int32_t *chunk_offs;    // [n_seqs + 1] first global chunk of each sequence (packed only)
    const int32_t *order;         // schedule position -> sequence, or NULL (identity)
    int64_t T;                    // tokens per sequence (dense)
    int64_t n_tokens;             // total tokens
    int n_seqs;
    int chunks_per_seq;           // dense: ceil(T / CH)
};

// Producer fusions (the flags of the reference's fla call): work a caller
// would otherwise do in elementwise passes over q, k, g and beta before the scan.
struct Fusion {
    int qk_l2norm;                // q, k un-normalised: x rsqrt(sum x^2 + 1e-6) per (token, head)
    int beta_sigmoid;             // beta holds logits
    int gate_act;                 // per-channel gate: g holds the pre-activation f
    int gate_16;                  // f is in q's 16-bit type (else fp32)
    const float *A_log;           // [H]
    const float *dt_bias;         // [H * dk]
    int lb_set;                   // g = lb sigmoid(exp(A_log) (f + dt_bias)), else -exp(A_log) softplus(f + dt_bias)
    float lb;
};

// Output epilogue of the layer (linear_attention.py:814-825): per (token,
// head), RMSNorm over dv with weight gamma, times SiLU of the output gate:
//     out = x rsqrt(mean_c x_c^2 + eps) gamma * gate sigmoid(gate),  x = o in q's type
// computed in fp32 and rounded once.
struct Epilogue {
    const void *gate;             // [n_tokens, H, dv] in the element type; NULL = no epilogue
    const void *gamma;            // [dv], fp32 (gamma_f32) or the element type
    int gamma_f32;
    float eps;
};

// The layer's short causal convolution + SiLU on the q, k, v projections
// (opt.py:15-93, linear_attention.py:741-745), for the token-by-token kernel:
// channel c of token t is SiLU(sum_j w[c][j] x[t - K + 1 + j][c]), where inputs
// before the sequence's first token come from its conv cache (the last K
// inputs of the previous call, linear_attention.py:929-941), which the kernel
// then advances in place.
struct ShortConv {
    const void *wq, *wk, *wv;     // [H * dk, K], [H * dk, K], [H * dv, K]: fp32 (w_f32) or the element type
    void *cq, *ck, *cv;           // [n_seqs, K, H * dk | H * dv] in the element type
    int K;                        // 1..8; 0 = inputs arrive convolved and activated
    int w_f32;
};

// The short conv over a whole call (prefill): x, y [n_tokens, D]; w [D, K];
// conv caches [n_seqs, K, D] (state_in may be NULL = zeros, state_out NULL =
// not written; they may alias).
struct ConvParams {
    const void *x;
    const void *w;
    const void *state_in;
    void *y;
    void *state_out;
    const int32_t *cu;            // [n_seqs + 1] or NULL (dense: n_seqs sequences of T tokens)
    int64_t T, n_tokens, D;
    int n_seqs, K, w_f32, silu;
};

struct ChunkParams {
    SeqGeom geo;
    const void *q, *k, *v;        // [n_tokens, H, dk|dv] in the element type
    const float *g;               // [n_tokens, H] or [n_tokens, H, dk]; NULL = no gate
    const float *beta;            // [n_tokens, H]; unused without the delta rule
    void *o;                      // [n_tokens, H, dv]
    const float *h0;              // [n_seqs, H, dk, dv] or NULL
    float *ht;                    // [n_seqs, H, dk, dv] or NULL
    void *blocks;                 // per (chunk, head): TE and A tiles, fragment order
    int H, DV;
    int n_tiles;                  // dv tiles per (sequence, head)
    int n_chunk_slots;            // chunk-prep grid size / H (upper bound of chunks)
    int use_delta;
    float scale;
    Fusion fz;
    const void *w;                // [n_tokens, H, dk] write vectors in place of beta k (per-channel gate), or NULL
    void *hs;                     // [chunk slots, H, dv, dk] entry states for the backward (16-bit), or NULL
    float *nout;                  // per-channel gate: [chunk slots, H, CH, CH] N = strict_lower(gated K K^T)
                                  // for the backward (chunk prep writes the lower tiles), or NULL
    int te_identity;              // (with use_delta) the recurrence without the delta rule, U = V, in the
                                  // delta form's blocks: TE = I and GX = 0 (per-channel gate: a zero K*G
                                  // tile); beta is not read.  For the chunked backward of that recurrence.
    int states_only;              // (with hs, 16-bit) the state kernel stores the entry states and computes
                                  // no outputs (o is not written): the backward's entry-state walk
};

// Backward of the chunked scan (scalar gate, per-channel gate or none, delta
// rule).  q, k are the normalised inputs the forward scanned; the gradients
// come back in the element type (dq, dk, dv) or fp32 (dg, dbeta, dh0).
struct ChunkBwdParams {
    SeqGeom geo;
    const void *q, *k, *v;        // [n_tokens, H, dk|dv] in the element type
    const float *g;               // [n_tokens, H] or [n_tokens, H, dk] (per-channel); NULL = no gate
    const float *beta;            // [n_tokens, H]
    const void *dout;             // [n_tokens, H, dv] gradient of o
    const float *h0;              // [n_seqs, H, dk, dv] or NULL
    const float *dht;             // [n_seqs, H, dk, dv] gradient of the final state, or NULL
    void *dq, *dk, *dv;           // [n_tokens, H, dk|dv]
    float *dg;                    // [n_tokens, H] or [n_tokens, H, dk] (NULL without a gate)
    float *dbeta;                 // [n_tokens, H]
    float *dh0;                   // [n_seqs, H, dk, dv] or NULL
    const void *blocks;           // chunk_prep's per-(chunk, head) blocks
    void *hs;                     // [chunk slots, H, dv, dk] each chunk's entry state (element type, transposed)
    void *dhs;                    // [chunk slots, H, dv, dk] gradient of each chunk's exit state (same)
    const float *nbuf;            // per-channel gate: chunk prep's N (ChunkParams::nout)
    float *gw;                    // per-channel gate: [chunk slots, H, grad_vec_work_floats] the column phase's sums
    Fusion fz;                    // beta_sigmoid: beta holds logits, dbeta is their gradient; gate_act
                                  // (per-channel gate): g holds the pre-activation f, dg is df
    float *dpart;                 // gate_act: [chunk slots, H, dk + 1] per-chunk sums of ddt_bias, then dA_log
    float *dA_log, *ddt_bias;     // gate_act: [H], [H * dk]
    int delta;                    // 0: the recurrence without the delta rule (blocks from
                                  // ChunkParams::te_identity; beta and dbeta NULL)
    const void *w;                // per-channel gate: [n_tokens, H, dk] explicit write vectors in place of
    void *dw;                     // beta k (chunk prep's WR blocks; beta and dbeta NULL), and their gradient
    int H, DV;
    int n_tiles;                  // dv tiles of the walk kernels (set by the launcher)
    int n_chunk_slots;
    float scale;
};

// Backward of the token recurrence (any gate; write vector beta k, an explicit
// w, or none without the delta rule).  Gradients come back in the element type
// (dq, dk, dv, dw) or fp32 (dg, dbeta, dh0).
struct ScanBwdParams {
    SeqGeom geo;                  // cu / T / n_tokens / n_seqs (chunk fields unused)
    const void *q, *k, *v, *w;    // [n_tokens, H, dk|dv]; w NULL unless mode 1
    const float *g;               // [n_tokens, H] (gate 1) or [n_tokens, H, dk] (gate 2) or NULL
    const float *beta;            // [n_tokens, H] (mode 0)
    const void *dout;             // [n_tokens, H, dv]
    const float *h0, *dht;        // [n_seqs, H, dk, dv] or NULL
    void *dq, *dk, *dv, *dw;      // dw: mode 1 only
    float *dg, *dbeta, *dh0;      // dg: gate != 0; dbeta: mode 0; dh0 may be NULL
    float *hs;                    // [ckpt slots, H, n_tiles, dk * TW] state at each block's entry
    float *dhs;                   // same layout: gradient of the state at each block's exit
    float *u;                     // [n_tokens, H, dv] u_t of every token (delta rule)
    float *part;                  // [4, n_tiles, n_tokens, H, dk] per-tile sums over columns
    int H, DV;
    int TW;                       // columns per workgroup (4 per wave)
    int n_tiles;                  // DV / TW
    int gate;                     // 0 none, 1 scalar, 2 per key channel
    int mode;                     // 0: x = beta k; 1: x = w; 2: no delta rule (x = k, u = v)
    float scale;
};

// The scalar gate and the beta logits of a one-token decode step formed in the
// decode kernel from the layer's input row (GatedDeltaNet._gates,
// linear_attention.py:719-721, :734-735): p = W_a x and W_b x rounded to the
// element type (nn.Linear's output), g = neg_a softplus(p + dt_bias), beta = the
// rounded W_b x (logits).  x NULL: g and beta come in as tensors.
struct GateProj {
    const void *x;                // [n_tokens, dim] in the element type, 16-byte aligned rows
    const void *w;                // [H, dim] W_a, then [H, dim] W_b (delta rule), 16-byte aligned rows
    const float *neg_a;           // [H]: -exp(A_log)
    const float *dt_bias;         // [H]
    int dim;                      // a multiple of 8
};

struct RecParams {
    const void *q, *k, *v;
    const float *g;
    const float *beta;
    void *o;
    const float *h0;
    float *ht;
    const int32_t *cu;
    int64_t T;
    int64_t n_tokens;
    int H, n_seqs;
    int use_delta;
    float scale;
    Fusion fz;
    Epilogue ep;                  // applied to o before it is stored
    ShortConv cv;                 // applied to q, k, v where they are read
    const void *w;                // [n_tokens, H, dk] write vectors in place of beta k, or NULL
    // the one-token decode step's token row strides, in elements: q and k (ld_qk)
    // and v and the epilogue gate (ld_v); 0 for dense rows (H dk, H dv).  Rows of
    // one fused projection output [n_tokens, 4 H d] are read in place this way
    int64_t ld_qk, ld_v;
    GateProj gp;                  // the decode kernel's own gate projections (scalar gate), or x NULL
};

// dtype: 0 fp32, 1 bf16, 2 fp16.  gate_vector: per-channel (KDA) decay.
// phases: CHUNK_PREP runs the packed-batch schedule (if packed) and the
// chunk-prep kernel; CHUNK_STATE runs the chunk-state kernel, which reads what
// the prep phase left in the workspace.  Both are launched on `stream`.
enum { CHUNK_PREP = 1, CHUNK_STATE = 2 };
hipError_t chunk_fwd(int dtype, int dk, int chunk, int gate_vector, ChunkParams p, int32_t *table, int phases,
                     hipStream_t stream);
int64_t chunk_blocks_bytes(int dtype, int chunk, int64_t chunk_slots, int64_t H, int64_t dk, int gate_vector);

// The backward: chunk prep (with `fwd`, the same call's forward parameters,
// writing the blocks p.blocks points at), then the walks and the per-chunk
// gradients.  table: the packed-batch schedule (as chunk_fwd).  saved: a
// forward with ChunkParams::hs = p.hs already left the schedule, the blocks
// and the entry states in the workspace; the prep and the entry walk are skipped.
hipError_t chunk_bwd(int dtype, int dk, int chunk, int gate_vector, const ChunkParams &fwd, ChunkBwdParams p,
                     int32_t *table, bool saved, hipStream_t stream);

// the per-channel-gate backward's per-(chunk, head) work area (fp32 elements):
// dO S^T, dX S^T, U dS'^T (CH x DK each), dO U^T and dU X^T (CH x CH each,
// lower tiles), and per key channel the sum over columns of S * dS' (DK)
constexpr int64_t grad_vec_work_floats(int chunk, int dk) {
    return 3 * (int64_t)chunk * dk + 2 * (int64_t)chunk * chunk + dk;
}

// the token-recurrence backward: the forward and backward walks per (sequence,
// head, column tile), the per-block gradients, then the per-(token, head)
// finish; slots: checkpoint slots the workspace must hold
hipError_t scan_bwd(int dtype, int dk, const ScanBwdParams &p, hipStream_t stream);
int64_t scan_bwd_ckpt_slots(int64_t n_tokens, int64_t n_seqs);

hipError_t recurrent_fwd(int dtype, int dk, int dv, int gate_vector, const RecParams &p,
                         hipStream_t stream);

// The epilogue as its own pass: out[r, :] from o[r, :] and gate[r, :] for
// n_rows rows of dv elements (out may alias o).  dv / (16 / sizeof(E)) must be
// a power of two <= 64.
hipError_t norm_gate(int dtype, const void *o, const Epilogue &ep, void *out, int64_t n_rows, int dv,
                     hipStream_t stream);

// The blocks' RMSNorm with an optional residual add first (res, x_out may be
// null): x_out = x + res, y = RMSNorm(x + res) * gamma over rows of dim
// elements.  dim / (16 / sizeof(E)) <= 2048.
hipError_t rms_norm(int dtype, const void *x, const void *res, void *x_out, const void *gamma, void *y, int64_t rows,
                    int dim, float eps, hipStream_t stream);

// The LM decode step's scalar gate and beta logits from x [rows, dim] and the
// stacked projection weight [W_a; W_b] ([2H or H, dim]): g [rows, H] (fp32),
// beta [rows, H] (fp32, with_beta).  dim % (16 / sizeof(E)) == 0.
hipError_t scalar_gates(int dtype, const void *x, const void *w, const float *neg_a, const float *dt_bias, float *g,
                        float *beta, int64_t rows, int dim, int H, bool with_beta, hipStream_t stream);

// SiLU(x[:, :h]) * x[:, h:] over rows of 2h elements; h % (16 / sizeof(E)) == 0.
hipError_t swiglu(int dtype, const void *x, void *y, int64_t rows, int hidden, hipStream_t stream);

hipError_t causal_conv(int dtype, const ConvParams &p, hipStream_t stream);

hipError_t varlen_prepare(const int32_t *cu, int n_seqs, int64_t n_tokens, int chunk,
                          int32_t *ws, hipStream_t stream);

int device_cu_count();

}  // namespace vgdr
