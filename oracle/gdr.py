"""CPU restatement of the gated delta-rule scans — the oracle (test infrastructure).

This module restates, in plain torch on the CPU, the algorithm of the
reference's hot path ``infra/components/linear_attention.py``.  It is the
checker for the HIP kernels in ``vagus_amd`` and the timed CPU baseline of
``bench.py``; nothing in the product imports it.

Per head, with state S in R^{dk x dv}, log-decay g_t <= 0 (a_t = exp(g_t),
a scalar for GDN or a per-key-channel vector for KDA) and write strength
beta_t (linear_attention.py:8-11):

    S_t = (I - beta_t k_t k_t^T) Diag(a_t) S_{t-1} + beta_t k_t v_t^T
    o_t = scale * S_t^T q_t

Functions and the reference lines they follow:

    recurrent       linear_attention.py:161-195   the definition (with the asymmetric write w)
    recurrent_grads linear_attention.py:237-425   gradients of the scans (autograd of the fp64 recurrence)
    chunk_scalar    linear_attention.py:237-309   WY chunk form, scalar / no gate
    chunk_vector    linear_attention.py:312-425   WY chunk form, per-channel gate (and w)
    chunk           linear_attention.py:251-252   dispatch on g.dim()
    varlen          (no reference counterpart)    per-segment loop over cu_seqlens
    chunk_table     (no reference counterpart)    integer chunk / schedule table
    chunk_scan_flops linear_attention.py:128-143  FLOPs per token per head
    l2norm          linear_attention.py:703-706   the q, k producer (fused by the kernels' qk_l2norm)
    gate_activation linear_attention.py:722-734   per-channel gate from its pre-activation
    beta_sigmoid    linear_attention.py:735-736   beta from its logits
    norm_gate       linear_attention.py:814-825   output epilogue RMSNorm(o) * SiLU(gate)
                    norm_layer.py:15-24           (fused by the kernels' vgdr_epilogue)
    short_conv      opt.py:15-100                 causal depthwise conv + SiLU, decode cache
                    linear_attention.py:929-941   (fused by the decode kernel's vgdr_short_conv)
    decode_step     linear_attention.py:929-947   conv, L2 norm, recurrence of one decode call

Layouts follow the reference (linear_attention.py:146-154): q, k (B, L, H, dk),
v (B, L, H, dv), g (B, L, H) or (B, L, H, dk), beta (B, L, H), S0 (B, H, dk, dv).
Computation is fp64 when q is fp64, else fp32 (linear_attention.py:157-158);
o is returned in q.dtype and S in the compute dtype.

How each function is pinned (tests/test_oracle.py): ``recurrent_grads``
against central finite differences of ``recurrent`` (torch.autograd.gradcheck
in fp64) and against reverse-mode through the independent chunk form
``chunk_scalar``; ``recurrent`` against
closed forms (causal linear attention, pure decay, one-token write, the
delta-rule overwrite identity) and against an independent dense-matrix
statement of the update above; the chunk forms against ``recurrent`` at
1e-12 in fp64, chunk-size / padding invariance and the scalar == constant
vector-gate reduction; ``varlen`` by segment isolation; ``chunk_table`` by
brute-force enumeration; ``chunk_scan_flops`` by the reference's known answers;
the producers by their defining properties (unit norms and scale invariance,
softplus / sigmoid identities and limits, the bounded gate's range);
``norm_gate`` against torch's own ``F.rms_norm`` x ``F.silu`` in fp64, a
constant row's closed form and scale invariance; ``short_conv`` against
torch's ``F.conv1d`` on the left-padded transpose (nn.Conv1d, the module's
'conv1d' path), a unit impulse returning the reversed kernel, and streaming
(token-by-token calls threading the cache equal one call).
"""
from __future__ import annotations

import math

import numpy as np
import torch


def compute_dtype(x: torch.Tensor) -> torch.dtype:
    """fp64 stays fp64 (the exactness oracle), everything else runs in fp32
    (linear_attention.py:157-158)."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


# ---------------------------------------------------------------------------
# the definition
# ---------------------------------------------------------------------------

def recurrent(q, k, v, g, beta, S0=None, *, scale: float, delta: bool = True, w=None):
    """Token-by-token recurrence (linear_attention.py:161-195).

    Per step: decay the key rows of S (scalar or per channel), read what S
    returns for k_t, write beta_t k_t (v_t - k_t^T S)^T (or k_t v_t^T without
    the delta rule), then read out o_t = scale q_t^T S *after* the write.
    w (B, L, H, dk): explicit write vectors in place of beta_t k_t, the
    asymmetric delta rule S <- S + w_t (v_t - k_t^T S)^T (:164-170, :185-188).
    L == 0 returns an empty o and S0 unchanged (as a copy in compute dtype).
    """
    assert w is None or delta, 'an explicit write vector needs the delta rule'
    B, L, H, dk = q.shape
    dv = v.shape[-1]
    ct = compute_dtype(q)
    qs = q.to(ct) * scale
    kc, vc = k.to(ct), v.to(ct)
    S = torch.zeros(B, H, dk, dv, dtype=ct) if S0 is None else S0.to(ct).clone()
    o = torch.zeros(B, L, H, dv, dtype=ct)
    for t in range(L):
        if g is not None:
            a = g[:, t].to(ct).exp()
            if a.dim() == 2:                       # (B, H): one decay per head
                S = S * a[:, :, None, None]
            else:                                  # (B, H, dk): per key row
                S = S * a[:, :, :, None]
        kt, vt = kc[:, t], vc[:, t]                # (B, H, dk), (B, H, dv)
        if delta:
            read = torch.matmul(kt.unsqueeze(-2), S).squeeze(-2)          # k_t^T S  (B, H, dv)
            wt = kt * beta[:, t].to(ct).unsqueeze(-1) if w is None else w[:, t].to(ct)
            S = S + wt.unsqueeze(-1) * (vt - read).unsqueeze(-2)
        else:
            S = S + kt.unsqueeze(-1) * vt.unsqueeze(-2)
        o[:, t] = torch.matmul(qs[:, t].unsqueeze(-2), S).squeeze(-2)
    return o.to(q.dtype), S


def recurrent_grads(q, k, v, g, beta, S0, do, dST=None, *, scale: float, delta: bool = True, w=None):
    """Gradients of ``recurrent``'s (o, final S) under the cotangents do (and
    dST, the final state's; None = zero), by reverse-mode differentiation of
    the fp64 recurrence: the gradients the reference's training takes through
    chunk_scan / chunk_scan_vec's autograd (linear_attention.py:237-309,
    :312-425), which computes the same function.  Returns (dq, dk, dv, dg,
    dbeta, dS0) in fp64, with dw appended when an explicit write w is given
    (beta is then unused and its gradient zero); None for absent inputs."""
    leaves = [None if x is None else x.detach().double().requires_grad_(True) for x in (q, k, v, g, beta, S0, w)]
    o, S = recurrent(*leaves[:6], scale=scale, delta=delta, w=leaves[6])
    outs, cots = [o], [do.double()]
    if dST is not None:
        outs.append(S)
        cots.append(dST.double())
    pairs = [(y, c) for y, c in zip(outs, cots) if y.requires_grad]      # an empty o has no graph
    inputs = [x for x in leaves if x is not None]
    if pairs:
        grads = iter(torch.autograd.grad([y for y, _ in pairs], inputs, [c for _, c in pairs], allow_unused=True))
    else:
        grads = iter([None] * len(inputs))
    res = []
    for x in leaves:
        if x is None:
            res.append(None)
        else:
            gx = next(grads)
            res.append(torch.zeros_like(x) if gx is None else gx)
    return tuple(res) if w is not None else tuple(res[:6])


# ---------------------------------------------------------------------------
# chunk forms
# ---------------------------------------------------------------------------

def _pad_tokens(x, pad):
    """Append `pad` zero tokens along dim 1."""
    if pad == 0 or x is None:
        return x
    shape = list(x.shape)
    shape[1] = pad
    return torch.cat([x, x.new_zeros(shape)], dim=1)


def _blocks(x, N, C):
    """(B, N*C, H, ...) -> (B, H, N, C, ...)."""
    B, _, H = x.shape[:3]
    rest = x.shape[3:]
    y = x.reshape(B, N, C, H, *rest)
    perm = (0, 3, 1, 2) + tuple(range(4, 4 + len(rest)))
    return y.permute(*perm)


def chunk_scalar(q, k, v, g, beta, S0=None, *, scale: float, delta: bool = True,
                 chunk_size: int = 64):
    """WY chunk form for a scalar (or absent) gate (linear_attention.py:237-309).

    Within a chunk with entry state S, gamma = in-chunk cumsum of g,
    D_ij = exp(gamma_i - gamma_j) on i >= j (masked before the exp), and
        W   = (I + Bm)^-1 diag(beta) K,         Bm_ij = beta_i k_i.k_j  (j < i)
        U   = (I + Bm*D)^-1 diag(beta) V
        U~  = U - diag(G) W S
        o   = diag(G) Q S + (Q K^T * D) U~
        S' <- G_C S + K^T diag(G_C / G_j) U~
    Without the delta rule W = 0 and U = V.  Padding tokens (q = k = v = 0,
    g = 0, beta = 0) are inert and the output is cut back to L.  A 4-D g is a
    per-channel gate and goes to chunk_vector (linear_attention.py:251-252).
    """
    if g is not None and g.dim() == 4:
        return chunk_vector(q, k, v, g, beta, S0, scale=scale, delta=delta,
                            chunk_size=chunk_size)
    B, L, H, dk = q.shape
    dv = v.shape[-1]
    C = chunk_size
    ct = compute_dtype(q)
    pad = (-L) % C
    N = (L + pad) // C
    qs = _blocks(_pad_tokens(q.to(ct) * scale, pad), N, C)                 # (B, H, N, C, dk)
    kc = _blocks(_pad_tokens(k.to(ct), pad), N, C)
    vc = _blocks(_pad_tokens(v.to(ct), pad), N, C)
    if g is None:
        gam = torch.zeros(B, H, N, C, dtype=ct)
    else:
        gam = _blocks(_pad_tokens(g.to(ct), pad), N, C).cumsum(-1)         # log G_i
    if delta:
        bt = _blocks(_pad_tokens(beta.to(ct), pad), N, C)                  # (B, H, N, C)
    lower = torch.ones(C, C, dtype=torch.bool).tril()
    strict = lower.tril(-1)
    eye = torch.eye(C, dtype=ct)
    S = torch.zeros(B, H, dk, dv, dtype=ct) if S0 is None else S0.to(ct).clone()
    out = []
    for n in range(N):
        Qn, Kn, Vn, gm = qs[:, :, n], kc[:, :, n], vc[:, :, n], gam[:, :, n]
        diff = gm.unsqueeze(-1) - gm.unsqueeze(-2)                        # gamma_i - gamma_j
        D = torch.where(lower, diff, torch.full_like(diff, -math.inf)).exp()
        Gi = gm.exp().unsqueeze(-1)                                       # G_i     (B, H, C, 1)
        Gtail = (gm[..., -1:] - gm).exp().unsqueeze(-1)                   # G_C/G_j (B, H, C, 1)
        Aqk = torch.matmul(Qn, Kn.transpose(-1, -2)) * D
        if delta:
            bn = bt[:, :, n].unsqueeze(-1)                                # (B, H, C, 1)
            Bm = bn * torch.matmul(Kn, Kn.transpose(-1, -2)) * strict
            W = torch.linalg.solve_triangular(eye + Bm, bn * Kn, upper=False, unitriangular=True)
            U = torch.linalg.solve_triangular(eye + Bm * D, bn * Vn, upper=False, unitriangular=True)
            Ut = U - Gi * torch.matmul(W, S)
        else:
            Ut = Vn
        out.append(Gi * torch.matmul(Qn, S) + torch.matmul(Aqk, Ut))
        S = gm[..., -1].exp()[..., None, None] * S + torch.matmul(Kn.transpose(-1, -2), Gtail * Ut)
    o = torch.stack(out, dim=2) if N else torch.zeros(B, H, 0, C, dv, dtype=ct)
    o = o.permute(0, 2, 3, 1, 4).reshape(B, N * C, H, dv)[:, :L]
    return o.to(q.dtype), S


def chunk_vector(q, k, v, g, beta, S0=None, *, scale: float, delta: bool = True,
                 chunk_size: int = 64, w=None):
    """WY chunk form for a per-channel gate g (B, L, H, dk) (linear_attention.py:312-425).

    Every inner product becomes a gated one,
        <x_i, y_j>_g = sum_c x_i[c] y_j[c] exp(gamma_i[c] - gamma_j[c])   (i >= j),
    whose exponents are <= 0, and per chunk
        (I + M) W = diag(beta) (K * G),  (I + M) U = diag(beta) V,   M_ij = beta_i <k_i, k_j>_g (j < i)
        U~  = U - W S
        o   = (Q * G) S + A U~,          A_ij = <q_i, k_j>_g (j <= i)
        S' <- G_C (.) S + (K * G_C / G_j)^T U~     (G_C scales the key rows of S)
    Without the delta rule U~ = V.  The pairwise exponent tensor is built one
    chunk at a time.

    w (B, L, H, dk): explicit write vectors (the asymmetric delta rule,
    :340-353, :389-396): k stays in the reading slot and w takes the writing
    slot, M_ij = <k_i, w_j>_g (j < i), (I + M) W = K * G, (I + M) U = V,
    A_ij = <q_i, w_j>_g, and the state update writes with W * G_C / G_j.
    """
    assert w is None or delta, 'an explicit write vector needs the delta rule'
    B, L, H, dk = q.shape
    dv = v.shape[-1]
    C = chunk_size
    ct = compute_dtype(q)
    pad = (-L) % C
    N = (L + pad) // C
    qs = _blocks(_pad_tokens(q.to(ct) * scale, pad), N, C)                 # (B, H, N, C, dk)
    kc = _blocks(_pad_tokens(k.to(ct), pad), N, C)
    vc = _blocks(_pad_tokens(v.to(ct), pad), N, C)
    gam = _blocks(_pad_tokens(g.to(ct), pad), N, C).cumsum(3)              # (B, H, N, C, dk)
    if delta and w is None:
        bt = _blocks(_pad_tokens(beta.to(ct), pad), N, C)
    wc = None if w is None else _blocks(_pad_tokens(w.to(ct), pad), N, C)
    lower = torch.ones(C, C, dtype=torch.bool).tril()
    strict = lower.tril(-1)
    eye = torch.eye(C, dtype=ct)
    S = torch.zeros(B, H, dk, dv, dtype=ct) if S0 is None else S0.to(ct).clone()
    out = []
    for n in range(N):
        Qn, Kn, Vn, gm = qs[:, :, n], kc[:, :, n], vc[:, :, n], gam[:, :, n]
        diff = gm.unsqueeze(3) - gm.unsqueeze(2)                          # (B, H, C, C, dk)
        E = torch.where(lower[None, None, :, :, None], diff,
                        torch.full_like(diff, -math.inf)).exp()
        G = gm.exp()                                                      # (B, H, C, dk)
        Gtail = (gm[:, :, -1:, :] - gm).exp()                             # G_C / G_j

        def gated(x, y):
            return torch.einsum('bhic,bhijc,bhjc->bhij', x, E, y)

        Wr = Kn if wc is None else wc[:, :, n]                             # the writing slot
        A = gated(Qn, Wr)
        if wc is not None:
            M = gated(Kn, Wr) * strict
            W = torch.linalg.solve_triangular(eye + M, Kn * G, upper=False, unitriangular=True)
            U = torch.linalg.solve_triangular(eye + M, Vn, upper=False, unitriangular=True)
            Ut = U - torch.matmul(W, S)
        elif delta:
            bn = bt[:, :, n].unsqueeze(-1)
            M = bn * gated(Kn, Kn) * strict
            W = torch.linalg.solve_triangular(eye + M, bn * (Kn * G), upper=False, unitriangular=True)
            U = torch.linalg.solve_triangular(eye + M, bn * Vn, upper=False, unitriangular=True)
            Ut = U - torch.matmul(W, S)
        else:
            Ut = Vn
        out.append(torch.matmul(Qn * G, S) + torch.matmul(A, Ut))
        S = G[:, :, -1, :, None] * S + torch.matmul((Wr * Gtail).transpose(-1, -2), Ut)
    o = torch.stack(out, dim=2) if N else torch.zeros(B, H, 0, C, dv, dtype=ct)
    o = o.permute(0, 2, 3, 1, 4).reshape(B, N * C, H, dv)[:, :L]
    return o.to(q.dtype), S


def chunk(q, k, v, g, beta, S0=None, *, scale: float, delta: bool = True, chunk_size: int = 64):
    """Dispatch on the gate's rank, as chunk_scan does (linear_attention.py:251-252)."""
    fn = chunk_vector if (g is not None and g.dim() == 4) else chunk_scalar
    return fn(q, k, v, g, beta, S0, scale=scale, delta=delta, chunk_size=chunk_size)


# ---------------------------------------------------------------------------
# packed variable-length batches
# ---------------------------------------------------------------------------

def varlen(fn, q, k, v, g, beta, S0, cu_seqlens, **kw):
    """Run `fn` (recurrent / chunk) on each segment [cu[n], cu[n+1]) of a packed
    (1, T, H, d) stream with its own entry state S0[n] (or zeros).  Returns the
    packed o (1, T, H, dv) and the stacked final states (N, H, dk, dv).  A
    per-token keyword (w) is cut per segment like q."""
    cu = [int(x) for x in torch.as_tensor(cu_seqlens).tolist()]
    w = kw.pop('w', None)
    assert q.shape[0] == 1, 'packed varlen input has batch 1'
    N = len(cu) - 1
    ct = compute_dtype(q)
    dk, dv, H = q.shape[-1], v.shape[-1], q.shape[2]
    outs, states = [], []
    for n in range(N):
        s, e = cu[n], cu[n + 1]
        sl = slice(s, e)
        s0 = None if S0 is None else S0[n:n + 1]
        gn = None if g is None else g[:, sl]
        bn = None if beta is None else beta[:, sl]
        if e > s:
            extra = {} if w is None else {'w': w[:, sl]}
            o, S = fn(q[:, sl], k[:, sl], v[:, sl], gn, bn, s0, **kw, **extra)
        else:
            o = q.new_zeros(1, 0, H, dv)
            S = torch.zeros(1, H, dk, dv, dtype=ct) if s0 is None else s0.to(ct).clone()
        outs.append(o)
        states.append(S)
    o = torch.cat(outs, dim=1) if outs else q.new_zeros(1, 0, H, dv)
    return o, torch.cat(states, dim=0)


def chunk_table(cu_seqlens, chunk_size: int):
    """Integer schedule table of a packed batch, computed on the host.

    Returns a dict of int32 numpy arrays:
        lens[n]          = cu[n+1] - cu[n]
        chunks[n]        = ceil(lens[n] / chunk_size)
        chunk_offsets[n] = sum_{m<n} chunks[m]          (length N+1, last = total)
        order[p]         = segments sorted by length, longest first, ties by index
    """
    cu = np.asarray(torch.as_tensor(cu_seqlens).cpu().numpy(), dtype=np.int64)
    lens = cu[1:] - cu[:-1]
    chunks = (lens + chunk_size - 1) // chunk_size
    offs = np.zeros(len(lens) + 1, dtype=np.int64)
    offs[1:] = np.cumsum(chunks)
    order = np.array(sorted(range(len(lens)), key=lambda n: (-lens[n], n)), dtype=np.int64)
    return {'lens': lens.astype(np.int32), 'chunks': chunks.astype(np.int32),
            'chunk_offsets': offs.astype(np.int32), 'order': order.astype(np.int32)}


# ---------------------------------------------------------------------------
# accounting
# ---------------------------------------------------------------------------

def chunk_scan_flops(dk: int, dv: int, chunk: int, delta: bool) -> float:
    """Matmul FLOPs per token per head, forward + backward (x3), of the chunked
    algorithm (linear_attention.py:128-143): state terms (6 or 4) dk dv plus the
    intra-chunk terms 2C (3dk + 2dv) with the delta rule, 2C (dk + dv) without."""
    state = (6 if delta else 4) * dk * dv
    intra = 2 * chunk * ((3 * dk + 2 * dv) if delta else (dk + dv))
    return 3.0 * (state + intra)


# ---------------------------------------------------------------------------
# the producers the kernels can fuse (vgdr_fusion)
# ---------------------------------------------------------------------------

def _hi(x):
    """At least fp32 (linear_attention.py:700-702)."""
    return x.to(torch.promote_types(x.dtype, torch.float32))


def l2norm(x, eps: float = 1e-6):
    """x rsqrt(sum over the last dim of x^2 + eps), computed in at least fp32 and
    returned in x's dtype (linear_attention.py:703-706)."""
    h = _hi(x)
    return (h * torch.rsqrt(h.pow(2).sum(-1, keepdim=True) + eps)).to(x.dtype)


def gate_activation(f, A_log, dt_bias, lower_bound=None):
    """Per-channel log-decay from the pre-activation f (B, L, H, dk), with A_log
    (H,) and dt_bias (H * dk,) (linear_attention.py:722-734):
    -exp(A_log) softplus(f + dt_bias), or lower_bound * sigmoid(exp(A_log)
    (f + dt_bias)) when lower_bound is given.  fp32 (at least)."""
    H, dk = f.shape[-2], f.shape[-1]
    z = _hi(f) + _hi(dt_bias).reshape(H, dk)
    a = _hi(A_log).exp()[:, None]
    if lower_bound is not None:
        return lower_bound * torch.sigmoid(a * z)
    return -a * torch.nn.functional.softplus(z)


def beta_sigmoid(b):
    """beta from its logits (linear_attention.py:735-736)."""
    return torch.sigmoid(_hi(b))


# ---------------------------------------------------------------------------
# the output epilogue the kernels can fuse (vgdr_epilogue)
# ---------------------------------------------------------------------------

def norm_gate(o, gate, gamma, eps: float = 1e-6):
    """The layer's output epilogue before W_o (linear_attention.py:825):
    RMSNorm(o.to(gate.dtype)) * SiLU(gate), RMSNorm per norm_layer.py:15-24:
    statistics in at least fp32, the normalised row cast back to the input
    dtype, then scaled by gamma.  Shapes (..., dv); gamma (dv,)."""
    x = o.to(gate.dtype)
    h = _hi(x)
    y = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * gamma
    return y * torch.nn.functional.silu(gate)


# ---------------------------------------------------------------------------
# the decode step's producers (vgdr_short_conv, vgdr_decode_step)
# ---------------------------------------------------------------------------

def short_conv(x, weight, cache=None, activation: str | None = 'silu'):
    """Depthwise causal 1-D conv over the sequence (ShortConv, opt.py:15-93):
    y[t][c] = sum_j w[c][j] x[t - K + 1 + j][c], with the inputs before t = 0
    taken from `cache` (B, K, D), the previous call's last K inputs
    (linear_attention.py:929-941), or zero.  x (B, L, D); weight (D, 1, K) or
    (D, K).  The sum runs in at least fp32 and is returned in x's dtype, then
    SiLU in that dtype (opt.py:96-100).  Returns (y, new cache = the last K
    inputs of cache ++ x)."""
    B, L, D = x.shape
    K = weight.shape[-1]
    w = _hi(weight.reshape(D, K))
    prev = torch.zeros(B, K, D, dtype=x.dtype) if cache is None else cache.to(x.dtype)
    xs = torch.cat([prev, x], 1)
    h = _hi(xs)
    y = sum(w[:, j] * h[:, 1 + j:1 + j + L] for j in range(K))
    y = y.to(x.dtype)
    if activation is not None:
        y = torch.nn.functional.silu(y)
    return y, xs[:, -K:].clone()


def decode_step(qp, kp, vp, g, beta, S0, conv_weights, conv_cache, *, scale: float, delta: bool = True,
                l2norm_qk: bool = True):
    """GatedDeltaNet.decode_step's data path up to _output (linear_attention.py:
    929-947): short conv + SiLU of the projections (advancing the caches),
    per-head view, q, k L2 norm, then the recurrence from S0.  qp, kp
    (B, L, H*dk), vp (B, L, H*dv); returns (o, S, (new caches))."""
    B, L = qp.shape[0], qp.shape[1]
    H, dk, dv = S0.shape[1], S0.shape[2], S0.shape[3]
    (q, cq), (k, ck), (v, cv) = (short_conv(x, w, c) for x, w, c in zip((qp, kp, vp), conv_weights, conv_cache))
    q, k, v = q.view(B, L, H, dk), k.view(B, L, H, dk), v.view(B, L, H, dv)
    if l2norm_qk:
        q, k = l2norm(q), l2norm(k)
    o, S = recurrent(q, k, v, g, beta, S0, scale=scale, delta=delta)
    return o, S, (cq, ck, cv)
