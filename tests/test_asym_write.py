"""The asymmetric delta rule: an explicit write vector w_t in place of
beta_t k_t (linear_attention.py:161-195 and :312-425 with w=; the write a
Kalman gain produces, kalman_delta.py).

CPU: the oracle's w path pinned by the agreement of its two independent
forms (token recurrence and WY chunk form) at 1e-12 in fp64 for several chunk
sizes, by w = beta k reducing to the symmetric rule through the other
(symmetric) chunk branch, and by the one-token closed form.
GPU: the HIP decode kernel and the chunked path with w against the fp64
oracle at the 16-bit bar rel_l2 <= 2e-2 (fp32: 1e-5), dense and packed.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr

TOL = 2e-2


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def _inputs(B, L, H, dk, dv, seed, gate='vector', dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, L, H, dk, generator=g, dtype=torch.float64), dim=-1)
    k = F.normalize(torch.randn(B, L, H, dk, generator=g, dtype=torch.float64), dim=-1)
    v = torch.randn(B, L, H, dv, generator=g, dtype=torch.float64)
    # a write of the delta rule's size: direction free, norm in (0, 1) like beta_t k_t (a Kalman gain's
    # scale); norms well above 1 make I - w k^T expansive and the bf16 comparison meaningless
    w = F.normalize(torch.randn(B, L, H, dk, generator=g, dtype=torch.float64), dim=-1) * \
        torch.sigmoid(torch.randn(B, L, H, 1, generator=g, dtype=torch.float64))
    gs = (B, L, H, dk) if gate == 'vector' else (B, L, H)
    gl = None if gate == 'none' else F.logsigmoid(torch.randn(*gs, generator=g, dtype=torch.float64) + 3.0)
    S0 = 0.3 * torch.randn(B, H, dk, dv, generator=g, dtype=torch.float64)
    cast = lambda t: t.to(dtype)
    return cast(q), cast(k), cast(v), cast(w), gl, S0


# --- the oracle (CPU) --------------------------------------------------------

@pytest.mark.parametrize('C', [8, 16, 64])
def test_oracle_w_recurrence_equals_chunk_form(C):
    q, k, v, w, gl, S0 = _inputs(2, 45, 2, 8, 5, seed=C)
    o1, S1 = gdr.recurrent(q, k, v, gl, None, S0, scale=0.3, w=w)
    o2, S2 = gdr.chunk_vector(q, k, v, gl, None, S0, scale=0.3, w=w, chunk_size=C)
    assert torch.allclose(o1, o2, rtol=1e-12, atol=1e-12) and torch.allclose(S1, S2, rtol=1e-12, atol=1e-12)


def test_oracle_w_equal_beta_k_is_the_symmetric_rule():
    q, k, v, _, gl, S0 = _inputs(2, 40, 2, 8, 5, seed=3)
    beta = torch.sigmoid(torch.randn(2, 40, 2, generator=torch.Generator().manual_seed(4), dtype=torch.float64))
    o1, S1 = gdr.chunk_vector(q, k, v, gl, beta, S0, scale=0.3, chunk_size=16)        # symmetric branch
    o2, S2 = gdr.chunk_vector(q, k, v, gl, None, S0, scale=0.3, chunk_size=16, w=k * beta[..., None])
    assert torch.allclose(o1, o2, rtol=1e-12, atol=1e-12) and torch.allclose(S1, S2, rtol=1e-12, atol=1e-12)


def test_oracle_w_one_token_closed_form():
    q, k, v, w, gl, S0 = _inputs(1, 1, 1, 6, 4, seed=5)
    o, S = gdr.recurrent(q, k, v, gl, None, S0, scale=0.5, w=w)
    Sd = gl[0, 0, 0].exp()[:, None] * S0[0, 0]                   # decayed key rows
    want = Sd + torch.outer(w[0, 0, 0], v[0, 0, 0] - k[0, 0, 0] @ Sd)
    assert torch.allclose(S[0, 0], want, rtol=1e-13, atol=1e-13)
    assert torch.allclose(o[0, 0, 0], 0.5 * q[0, 0, 0] @ want, rtol=1e-13, atol=1e-13)


# --- GPU ----------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['vector', 'scalar', 'none'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('dk,dv', [(128, 128), (64, 64)])
def test_recurrent_w_matches_oracle(gate, dtype, dk, dv):
    from vagus_amd import ops
    q, k, v, w, gl, S0 = _inputs(3, 9, 2, dk, dv, seed=dk + dv, gate=gate, dtype=dtype)
    print(f'\n[case] recurrent w gate={gate} dtype={dtype} dk={dk} dv={dv}', flush=True)
    o_ref, S_ref = gdr.recurrent(q.double(), k.double(), v.double(), gl, None, S0, scale=dk ** -0.5, w=w.double())
    dev = lambda t: None if t is None else t.cuda()
    o, S = ops.hip_recurrent(dev(q), dev(k), dev(v), dev(None if gl is None else gl.float()), None, dev(S0.float()),
                             scale=dk ** -0.5, delta=True, w=dev(w))
    tol = 1e-5 if dtype == torch.float32 else TOL
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    print(f'[parity] recurrent w o={eo:.3e} S={es:.3e} (tol {tol:g})', flush=True)
    assert eo <= tol and es <= tol


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['vector', 'scalar', 'none'])
@pytest.mark.parametrize('dk,dv', [(128, 128), (64, 64), (128, 48)])
@pytest.mark.parametrize('T', [64, 200])
def test_chunk_w_matches_oracle(gate, dk, dv, T):
    from vagus_amd import ops
    q, k, v, w, gl, S0 = _inputs(2, T, 2, dk, dv, seed=T + dk + dv, gate=gate, dtype=torch.bfloat16)
    print(f'\n[case] chunk w gate={gate} dk={dk} dv={dv} T={T}', flush=True)
    o_ref, S_ref = gdr.recurrent(q.double(), k.double(), v.double(), gl, None, S0, scale=dk ** -0.5, w=w.double())
    dev = lambda t: None if t is None else t.cuda()
    o, S = ops.chunk_scan_vec(dev(q), dev(k), dev(v), dev(None if gl is None else gl.float()), None,
                              dev(S0.float()), scale=dk ** -0.5, delta=True, w=dev(w))
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    print(f'[parity] chunk w o={eo:.3e} S={es:.3e}', flush=True)
    assert eo <= TOL and es <= TOL


@pytest.mark.gpu
def test_chunk_w_varlen_and_fp32():
    from vagus_amd import ops
    dev = lambda t: None if t is None else t.cuda()
    q, k, v, w, gl, _ = _inputs(1, 150, 2, 128, 64, seed=77, dtype=torch.bfloat16)
    cu = torch.tensor([0, 10, 10, 75, 150], dtype=torch.int32)
    S0 = 0.3 * torch.randn(4, 2, 128, 64, generator=torch.Generator().manual_seed(78), dtype=torch.float64)
    o_ref, S_ref = gdr.varlen(gdr.recurrent, q.double(), k.double(), v.double(), gl, None, S0, cu,
                              scale=128 ** -0.5, w=w.double())
    o, S = ops.chunk_scan_vec(dev(q), dev(k), dev(v), dev(gl.float()), None, dev(S0.float()), scale=128 ** -0.5,
                              delta=True, w=dev(w), cu_seqlens=dev(cu))
    e1o, e1s = _rel(o, o_ref), _rel(S, S_ref)
    # fp32: the same rule token by token
    q, k, v, w, gl, S0 = _inputs(2, 33, 2, 64, 64, seed=79, dtype=torch.float32)
    o_ref, S_ref = gdr.recurrent(q.double(), k.double(), v.double(), gl, None, S0, scale=0.125, w=w.double())
    o, S = ops.chunk_scan_vec(dev(q), dev(k), dev(v), dev(gl.float()), None, dev(S0.float()), scale=0.125,
                              delta=True, w=dev(w))
    e2o, e2s = _rel(o, o_ref), _rel(S, S_ref)
    print(f'\n[parity] chunk w varlen o={e1o:.3e} S={e1s:.3e}; fp32 o={e2o:.3e} S={e2s:.3e}', flush=True)
    assert e1o <= TOL and e1s <= TOL and e2o <= 1e-5 and e2s <= 1e-5
