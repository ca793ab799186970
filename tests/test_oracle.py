"""Pin the CPU oracle before trusting it (CPU only).

The reference holds no golden vectors for this path; its tests are
relational (tests/test_linear_attention.py:30-85).  The oracle is pinned by
  * closed forms that a plausible mistake breaks: causal linear attention,
    pure decay, a one-token write, and the delta-rule overwrite identity
    (with beta = 1, a = 1 and unit k, reading k right after writing (k, v)
    returns v exactly, whatever the state held — a sign error in the erase
    term, a misplaced beta or an o-before-update ordering all fail it);
  * an independent dense-matrix statement of the update
    S_t = (I - b k k^T) Diag(a) S_{t-1} + b k v^T (linear_attention.py:8-11);
  * the reference's own relational checks: chunk == recurrent at 1e-12 in
    fp64 across gate x delta x chunk, the fp32 dtype contract at 1e-4, the
    scalar == channel-constant vector gate reduction, L = 0 and S0 = None;
  * chunk-size and padding invariance, varlen segment isolation, the integer
    chunk table by brute force, and the FLOP formula's known answers.
"""
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr

GATES = ('none', 'scalar', 'vector')
FLAGS = list(itertools.product(GATES, [True, False]))


def inputs(B=2, L=37, H=3, dk=8, dv=12, dtype=torch.float64, seed=0, gate='scalar', s0=0.3):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=dtype)
    q = r(B, L, H, dk)
    k = F.normalize(r(B, L, H, dk), dim=-1)
    v = r(B, L, H, dv)
    gshape = (B, L, H, dk) if gate == 'vector' else (B, L, H)
    g = F.logsigmoid(r(*gshape) + 2.0)
    if gate == 'none':
        g = None
    beta = torch.sigmoid(r(B, L, H))
    S0 = s0 * r(B, H, dk, dv)
    return q, k, v, g, beta, S0


# --- closed forms ---------------------------------------------------------

def test_no_gate_no_delta_is_causal_linear_attention():
    q, k, v, _, beta, S0 = inputs(L=23)
    o, S = gdr.recurrent(q, k, v, None, beta, S0, scale=0.7, delta=False)
    # o = scale (tril(Q K^T) V + Q S0) per (b, h);  S = S0 + K^T V
    Q, K, V = (t.permute(0, 2, 1, 3) for t in (q, k, v))
    ref = 0.7 * (torch.tril(Q @ K.transpose(-1, -2)) @ V + Q @ S0)
    assert torch.allclose(o.permute(0, 2, 1, 3), ref, atol=1e-12)
    assert torch.allclose(S, S0 + K.transpose(-1, -2) @ V, atol=1e-12)


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_zero_write_is_pure_decay(gate):
    q, k, v, g, beta, S0 = inputs(L=11, gate=gate)
    o, S = gdr.recurrent(q, k, v, g, torch.zeros_like(beta), S0, scale=0.5, delta=True)
    gam = g.cumsum(1)                                             # (B, L, H[, dk])
    if gate == 'scalar':
        St = gam.exp()[..., None, None] * S0[:, None]             # (B, L, H, dk, dv)
    else:
        St = gam.exp()[..., None] * S0[:, None]
    assert torch.allclose(S, St[:, -1], atol=1e-12)
    ref = 0.5 * torch.einsum('blhk,blhkv->blhv', q, St)
    assert torch.allclose(o, ref, atol=1e-12)


def test_single_token_write():
    q, k, v, g, beta, _ = inputs(L=1)
    o, S = gdr.recurrent(q, k, v, g, beta, None, scale=0.25, delta=True)
    b = beta[:, 0]
    assert torch.allclose(S, b[..., None, None] * k[:, 0, :, :, None] * v[:, 0, :, None, :], atol=1e-14)
    qk = (q[:, 0] * k[:, 0]).sum(-1)
    assert torch.allclose(o[:, 0], 0.25 * (b * qk)[..., None] * v[:, 0], atol=1e-14)


def test_delta_rule_overwrite_identity():
    """beta = 1, a = 1, |k| = 1: k^T S_t = v_t after the write, for any S."""
    q, k, v, _, beta, S0 = inputs(L=9, s0=1.0)
    o, _ = gdr.recurrent(k, k, v, torch.zeros_like(beta), torch.ones_like(beta), S0,
                         scale=1.0, delta=True)
    assert torch.allclose(o, v, atol=1e-12)


@pytest.mark.parametrize('gate,delta', FLAGS)
def test_recurrent_matches_dense_matrix_statement(gate, delta):
    q, k, v, g, beta, S0 = inputs(B=1, L=7, H=2, dk=5, dv=4, gate=gate)
    o, S = gdr.recurrent(q, k, v, g, beta, S0, scale=0.3, delta=delta)
    qn, kn, vn, bn, Sn = (t.numpy() for t in (q, k, v, beta, S0))
    gn = None if g is None else g.numpy()
    for h in range(2):
        St = Sn[0, h].copy()
        for t in range(7):
            if gn is None:
                a = np.ones(5)
            elif gn.ndim == 3:
                a = np.full(5, np.exp(gn[0, t, h]))
            else:
                a = np.exp(gn[0, t, h])
            kt = kn[0, t, h][:, None]
            vt = vn[0, t, h][None, :]
            if delta:
                bt = bn[0, t, h]
                St = (np.eye(5) - bt * kt @ kt.T) @ np.diag(a) @ St + bt * kt @ vt
            else:
                St = np.diag(a) @ St + kt @ vt
            assert np.allclose(o[0, t, h].numpy(), 0.3 * St.T @ qn[0, t, h], atol=1e-12)
        assert np.allclose(S[0, h].numpy(), St, atol=1e-12)


# --- the reference's relational checks on the chunk forms -------------------

@pytest.mark.parametrize('gate,delta', FLAGS)
@pytest.mark.parametrize('chunk', [8, 16, 64])
def test_chunk_matches_recurrent(gate, delta, chunk):
    q, k, v, g, beta, S0 = inputs(gate=gate)
    kw = dict(scale=0.5, delta=delta)
    o_r, S_r = gdr.recurrent(q, k, v, g, beta, S0, **kw)
    o_c, S_c = gdr.chunk(q, k, v, g, beta, S0, chunk_size=chunk, **kw)
    assert torch.allclose(o_c, o_r, atol=1e-12, rtol=1e-12)
    assert torch.allclose(S_c, S_r, atol=1e-12, rtol=1e-12)
    f = lambda t: None if t is None else t.float()
    o32, S32 = gdr.chunk(f(q), f(k), f(v), f(g), f(beta), f(S0), chunk_size=chunk, **kw)
    assert o32.dtype == torch.float32 and S32.dtype == torch.float32
    assert torch.allclose(o32.double(), o_r, atol=1e-4, rtol=1e-4)
    assert torch.allclose(S32.double(), S_r, atol=1e-4, rtol=1e-4)


def test_vector_gate_reduces_to_scalar():
    q, k, v, g, beta, S0 = inputs(L=21)
    gv = g[..., None].expand(*g.shape, q.shape[-1]).contiguous()
    for delta in (True, False):
        o_s, S_s = gdr.chunk_scalar(q, k, v, g, beta, S0, scale=0.5, delta=delta, chunk_size=8)
        o_v, S_v = gdr.chunk_vector(q, k, v, gv, beta, S0, scale=0.5, delta=delta, chunk_size=8)
        assert torch.allclose(o_s, o_v, atol=1e-12) and torch.allclose(S_s, S_v, atol=1e-12)
    o_d, _ = gdr.chunk_scalar(q, k, v, gv, beta, S0, scale=0.5, delta=True, chunk_size=8)
    assert torch.equal(o_d, gdr.chunk_vector(q, k, v, gv, beta, S0, scale=0.5, delta=True,
                                             chunk_size=8)[0])


def test_empty_and_no_initial_state():
    q, k, v, g, beta, _ = inputs(L=5)
    o1, S1 = gdr.recurrent(q, k, v, g, beta, None, scale=1.0, delta=True)
    o2, S2 = gdr.chunk(q, k, v, g, beta, None, scale=1.0, delta=True, chunk_size=4)
    assert torch.allclose(o1, o2) and torch.allclose(S1, S2)
    o0, S0 = gdr.recurrent(q[:, :0], k[:, :0], v[:, :0], g[:, :0], beta[:, :0], S1,
                           scale=1.0, delta=True)
    assert o0.shape[1] == 0 and torch.equal(S0, S1)


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_chunk_size_and_padding_invariance(gate):
    q, k, v, g, beta, S0 = inputs(L=70, gate=gate)
    ref = gdr.chunk(q, k, v, g, beta, S0, scale=0.4, chunk_size=64)
    for C in (16, 32, 128):
        o, S = gdr.chunk(q, k, v, g, beta, S0, scale=0.4, chunk_size=C)
        assert torch.allclose(o, ref[0], atol=1e-12) and torch.allclose(S, ref[1], atol=1e-12)


def test_strong_decay_stays_finite():
    """A chunk whose decay spans hundreds of nats must not overflow (the
    mask-before-exp rule, linear_attention.py:279-281, :379-382)."""
    q, k, v, g, beta, S0 = inputs(L=64, gate='vector')
    g = g - 8.0                                          # exp(+512) if formed naively
    o_r, S_r = gdr.recurrent(q, k, v, g, beta, S0, scale=0.5)
    o_c, S_c = gdr.chunk(q, k, v, g, beta, S0, scale=0.5, chunk_size=64)
    assert torch.isfinite(o_c).all() and torch.allclose(o_c, o_r, atol=1e-12)
    assert torch.allclose(S_c, S_r, atol=1e-12)


# --- varlen ----------------------------------------------------------------

@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_varlen_segments_are_isolated(gate):
    lens = [5, 0, 17, 64, 1, 33]
    T = sum(lens)
    q, k, v, g, beta, _ = inputs(B=1, L=T, gate=gate)
    S0 = 0.2 * torch.randn(len(lens), 3, 8, 12, dtype=torch.float64)
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32)
    o, S = gdr.varlen(gdr.chunk, q, k, v, g, beta, S0, cu, scale=0.5, chunk_size=16)
    o_r, S_r = gdr.varlen(gdr.recurrent, q, k, v, g, beta, S0, cu, scale=0.5)
    assert torch.allclose(o, o_r, atol=1e-12) and torch.allclose(S, S_r, atol=1e-12)
    for n, (s, e) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        gn = g[:, s:e]
        o1, S1 = gdr.recurrent(q[:, s:e], k[:, s:e], v[:, s:e], gn, beta[:, s:e], S0[n:n + 1], scale=0.5)
        assert torch.equal(o_r[:, s:e], o1) and torch.equal(S_r[n:n + 1], S1)
    # perturbing one segment leaves every other segment bit-identical
    v2 = v.clone()
    v2[:, cu[2]:cu[3]] += 1.0
    o2, S2 = gdr.varlen(gdr.recurrent, q, k, v2, g, beta, S0, cu, scale=0.5)
    keep = torch.ones(T, dtype=torch.bool)
    keep[cu[2]:cu[3]] = False
    assert torch.equal(o2[:, keep], o_r[:, keep])
    assert torch.equal(torch.cat([S2[:2], S2[3:]]), torch.cat([S_r[:2], S_r[3:]]))
    assert not torch.equal(S2[2], S_r[2])


def test_chunk_table_brute_force():
    rng = np.random.default_rng(0)
    for trial in range(20):
        lens = rng.integers(0, 300, size=rng.integers(1, 40)).tolist()
        cu = np.cumsum([0] + lens)
        for C in (16, 32, 64):
            t = gdr.chunk_table(torch.tensor(cu, dtype=torch.int32), C)
            chunks = []                                   # enumerate chunk by chunk
            for n, L in enumerate(lens):
                s = 0
                while s < L:
                    chunks.append((n, s))
                    s += C
            assert t['chunk_offsets'][-1] == len(chunks)
            for n in range(len(lens)):
                got = [c for c in chunks if c[0] == n]
                assert t['chunks'][n] == len(got)
                assert t['chunk_offsets'][n] == chunks.index(got[0]) if got else True
            assert list(t['lens']) == lens
            # longest first, ties by index: a permutation, lengths non-increasing
            order = list(t['order'])
            assert sorted(order) == list(range(len(lens)))
            ls = [lens[i] for i in order]
            assert all(a >= b for a, b in zip(ls, ls[1:]))
            for a, b in zip(order, order[1:]):
                if lens[a] == lens[b]:
                    assert a < b


def test_flop_formula_known_answers():
    # the reference's known answers (test_gdn_lm.py:98-102)
    assert gdr.chunk_scan_flops(16, 32, 8, True) == 3 * (6 * 16 * 32 + 2 * 8 * (3 * 16 + 2 * 32))
    assert gdr.chunk_scan_flops(16, 32, 8, False) == 3 * (4 * 16 * 32 + 2 * 8 * (16 + 32))
    # the forward third at the benchmark shapes
    assert gdr.chunk_scan_flops(128, 128, 64, True) / 3 == 180224
    assert gdr.chunk_scan_flops(64, 64, 64, True) / 3 == 65536


# ---------------------------------------------------------------------------
# the backward (recurrent_grads)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize('gate', ['none', 'scalar'])
def test_recurrent_grads_match_finite_differences(gate):
    """Reverse-mode through the recurrence equals central differences of the
    forward (gradcheck, fp64) for every input, with an initial state and a
    cotangent on the final state: a dropped term in any gradient fails."""
    q, k, v, g, beta, S0 = inputs(B=1, L=6, H=1, dk=3, dv=2, seed=11, gate=gate)
    gen = torch.Generator().manual_seed(12)
    do = torch.randn(1, 6, 1, 2, generator=gen, dtype=torch.float64)
    dST = torch.randn(1, 1, 3, 2, generator=gen, dtype=torch.float64)
    dq, dk_, dv_, dg, db, dS0 = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=0.7)

    def loss(*xs):
        qq, kk, vv, bb, ss = xs[:5]
        gg = xs[5] if gate != 'none' else None
        o, S = gdr.recurrent(qq, kk, vv, gg, bb, ss, scale=0.7)
        return (o * do).sum() + (S * dST).sum()

    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, beta, S0) + ((g,) if gate != 'none' else ())]
    assert torch.autograd.gradcheck(loss, leaves, eps=1e-6, atol=1e-7, rtol=1e-6)
    # and the function's own gradients are those of that loss
    ref = torch.autograd.grad(loss(*leaves), leaves)
    mine = (dq, dk_, dv_, db, dS0) + ((dg,) if gate != 'none' else ())
    for a, b in zip(mine, ref):
        assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize('gate', ['none', 'scalar'])
def test_recurrent_grads_match_chunk_form_gradients(gate):
    """The same gradients through the independent WY chunk form (triangular
    solves, decay masks), partial last chunk included."""
    q, k, v, g, beta, S0 = inputs(B=2, L=37, H=2, dk=8, dv=12, seed=13, gate=gate)
    gen = torch.Generator().manual_seed(14)
    do = torch.randn(2, 37, 2, 12, generator=gen, dtype=torch.float64)
    dST = torch.randn(2, 2, 8, 12, generator=gen, dtype=torch.float64)
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=0.5)
    leaves = [None if x is None else x.clone().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = gdr.chunk_scalar(*leaves, scale=0.5, chunk_size=16)
    got = torch.autograd.grad([o, S], [x for x in leaves if x is not None], [do, dST])
    for a, b in zip([x for x in ref if x is not None], got):
        assert torch.allclose(a, b, rtol=1e-9, atol=1e-10)


@pytest.mark.parametrize('mode', ['vector', 'vector_w', 'vector_nodelta', 'scalar_w', 'none_nodelta'])
def test_recurrent_grads_other_forms_match_finite_differences(mode):
    """gradcheck of the per-channel gate, the explicit write w and the plain
    (no delta rule) recurrence, each with an initial state and a final-state
    cotangent; dw must be the gradient of w and dbeta zero when w replaces
    beta k."""
    gate = mode.split('_')[0]
    delta = not mode.endswith('nodelta')
    q, k, v, g, beta, S0 = inputs(B=1, L=6, H=1, dk=3, dv=2, seed=21, gate=gate)
    gen = torch.Generator().manual_seed(22)
    w = 0.5 * torch.randn(1, 6, 1, 3, generator=gen, dtype=torch.float64) if mode.endswith('_w') else None
    do = torch.randn(1, 6, 1, 2, generator=gen, dtype=torch.float64)
    dST = torch.randn(1, 1, 3, 2, generator=gen, dtype=torch.float64)
    got = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=0.7, delta=delta, w=w)
    names = ['q', 'k', 'v', 'g', 'beta', 'S0', 'w']
    vals = dict(zip(names, (q, k, v, g, beta, S0, w)))
    live = [n for n in names if vals[n] is not None and not (n == 'beta' and (w is not None or not delta))]

    def loss(*xs):
        d = dict(vals, **dict(zip(live, xs)))
        o, S = gdr.recurrent(d['q'], d['k'], d['v'], d['g'], d['beta'], d['S0'], scale=0.7, delta=delta, w=d['w'])
        return (o * do).sum() + (S * dST).sum()

    leaves = [vals[n].clone().requires_grad_(True) for n in live]
    assert torch.autograd.gradcheck(loss, leaves, eps=1e-6, atol=1e-7, rtol=1e-6)
    ref = dict(zip(live, torch.autograd.grad(loss(*leaves), leaves)))
    mine = dict(zip(names, got))
    for n in live:
        assert torch.allclose(mine[n], ref[n], rtol=1e-12, atol=1e-12), n
    if w is not None or not delta:
        assert mine['beta'] is None or float(mine['beta'].abs().max()) == 0.0


@pytest.mark.parametrize('with_w', [False, True])
def test_recurrent_grads_match_vector_chunk_form_gradients(with_w):
    """Per-channel gate: the same gradients through the independent gated
    chunk form (gated inner products, triangular solves), partial last chunk
    and the explicit write included."""
    q, k, v, g, beta, S0 = inputs(B=2, L=37, H=2, dk=8, dv=12, seed=23, gate='vector')
    gen = torch.Generator().manual_seed(24)
    w = 0.3 * torch.randn(2, 37, 2, 8, generator=gen, dtype=torch.float64) if with_w else None
    do = torch.randn(2, 37, 2, 12, generator=gen, dtype=torch.float64)
    dST = torch.randn(2, 2, 8, 12, generator=gen, dtype=torch.float64)
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=0.5, w=w)
    leaves = [None if x is None else x.clone().requires_grad_(True) for x in (q, k, v, g, beta, S0, w)]
    o, S = gdr.chunk_vector(*leaves[:6], scale=0.5, chunk_size=16, w=leaves[6])
    live = [i for i, x in enumerate(leaves) if x is not None and not (i == 4 and with_w)]
    got = torch.autograd.grad([o, S], [leaves[i] for i in live], [do, dST])
    for i, b in zip(live, got):
        assert torch.allclose(ref[i], b, rtol=1e-9, atol=1e-10), i
