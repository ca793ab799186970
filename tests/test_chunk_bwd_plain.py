"""Backward of the chunked recurrence without the delta rule (the plain gated
recurrence S_t = g_t S_{t-1} + k_t v_t^T): vgdr_chunk_bwd_nodelta and the
autograd route of ops.chunk_simple_gla / chunk_scan_vec(delta=False), against
the oracle's recurrent_grads(delta=False) (reverse-mode through the fp64
recurrence, pinned in tests/test_oracle.py by finite differences).

The kernels are the delta form's: chunk prep writes TE = I and a zero K decay
factor (a zero K*G tile with the per-channel gate), which makes U = V, and
beta = 0 removes the M terms.  So these tests also pin that reduction.

CPU: the C ABI's argument checks (no launch).
GPU: dq, dk, dv, dg, dS0 at rel_l2 <= 1e-5 (fp32) or 2e-2 (16-bit): the scalar
gate and no gate in fp32 and bf16, the per-channel gate in bf16 and fp16
(also with decays strong enough for the exact diagonal path), a padded head,
a packed batch with empty and one-token segments; at B4 T8192 H8 (bf16, per
channel) against the token-walk backward (vgdr_scan_bwd) on the same inputs.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib, ops


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def test_nodelta_bwd_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, gate=1, q=4096, k=8192, v=12288, g=16384, h0=None, do=24576, dht=None, dq=28672,
                 dk=32768, dv=36864, dg=40960, dh0=None, cu=None, ws=49152, wsb=1 << 40, B=2, T=64, H=2, dk_=64,
                 dv_=64, N=2, chunk=64)
        a.update(over)
        return L.vgdr_chunk_bwd_nodelta(a['dtype'], a['gate'], a['q'], a['k'], a['v'], a['g'], a['h0'], a['do'],
                                        a['dht'], a['dq'], a['dk'], a['dv'], a['dg'], a['dh0'], a['cu'], a['ws'],
                                        a['wsb'], a['B'], a['T'], a['H'], a['dk_'], a['dv_'], a['N'], 0.125,
                                        a['chunk'], None)
    assert call(gate=2, dtype=0) == _lib.VGDR_ERR_UNSUPPORTED        # per-channel: 16-bit
    assert call(gate=2, chunk=32) == _lib.VGDR_ERR_UNSUPPORTED       # per-channel: 64-token chunks
    assert call(dq=None) == _lib.VGDR_ERR_INVALID
    assert call(dv_=40) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(ws=None) == _lib.VGDR_ERR_INVALID
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK


def _inputs(B, T, H, dk, dv, dtype, seed, gate, s0=True, strong=False):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    q = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    k = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    v = r(B, T, H, dv).to(dtype)
    if gate == 'vector':
        g = F.logsigmoid(r(B, T, H, dk) + 3.0)
        if strong:
            fast = torch.rand(dk, generator=gen) < 0.25
            g = torch.where(fast, -2.0 - 6.0 * torch.rand(B, T, H, dk, generator=gen), g)
    elif gate == 'scalar':
        g = F.logsigmoid(r(B, T, H) + 3.0)
    else:
        g = None
    S0 = 0.3 * r(B, H, dk, dv) if s0 else None
    do = r(B, T, H, dv).to(dtype)
    dST = r(B, H, dk, dv)
    return q, k, v, g, S0, do, dST


def _run(q, k, v, g, S0, do, dST, scale, cu=None, chunk=64):
    leaves = [None if x is None else x.cuda().requires_grad_(True) for x in (q, k, v, g, S0)]
    gate = 'none' if g is None else ('vector' if g.dim() == 4 else 'scalar')
    o, S = ops.chunk_scan(leaves[0], leaves[1], leaves[2], leaves[3], None, gate=gate, delta=False, scale=scale,
                          initial_state=leaves[4], output_final_state=True,
                          cu_seqlens=None if cu is None else cu.cuda(), chunk_size=chunk)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    return [None if x is None else x.grad for x in leaves]


NAMES = ('dq', 'dk', 'dv', 'dg', 'dS0')


def _compare(got, ref, tol, case):
    for name, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        err = _rel(a, b)
        print(f'[parity] {case} {name} rel_l2={err:.3e}', flush=True)
        assert err <= tol, f'{name}: {err:.3e} > {tol:g}'


@pytest.mark.gpu
@pytest.mark.parametrize('gate,dtype', [('scalar', torch.float32), ('scalar', torch.bfloat16),
                                        ('none', torch.float32), ('none', torch.bfloat16),
                                        ('vector', torch.bfloat16), ('vector', torch.float16)])
@pytest.mark.parametrize('shape', [(2, 100, 2, 64, 64), (1, 70, 2, 128, 128), (1, 45, 1, 100, 48)])
def test_nodelta_chunk_bwd_matches_oracle(gate, dtype, shape):
    B, T, H, dk, dv = shape
    print(f'\n[case] no-delta chunk bwd gate={gate} dtype={dtype} shape={shape}', flush=True)
    q, k, v, g, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed=T + dk, gate=gate)
    scale = dk ** -0.5
    r = gdr.recurrent_grads(q, k, v, g, None, S0, do, dST, scale=scale, delta=False)
    ref = (r[0], r[1], r[2], r[3], r[5])
    got = _run(q, k, v, g, S0, do, dST, scale)
    _compare(got, ref, 1e-5 if dtype == torch.float32 else 2e-2, f'no-delta {gate} {dtype} {shape}')


@pytest.mark.gpu
def test_nodelta_chunk_bwd_strong_decay_and_varlen():
    cu = torch.tensor([0, 0, 1, 70, 75, 200], dtype=torch.int32)    # empty, one token, multi-chunk, short
    N, T, H, dk, dv = 5, 200, 2, 64, 64
    q, k, v, g, _, do, _ = _inputs(1, T, H, dk, dv, torch.bfloat16, seed=17, gate='vector', strong=True)
    gen = torch.Generator().manual_seed(18)
    S0 = 0.3 * torch.randn(N, H, dk, dv, generator=gen)
    dST = torch.randn(N, H, dk, dv, generator=gen)
    print('\n[case] no-delta chunk bwd varlen, strong per-channel decay', flush=True)
    scale = dk ** -0.5
    parts = [[] for _ in range(6)]
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        sl = lambda x: x[:, a:b]
        r = gdr.recurrent_grads(sl(q), sl(k), sl(v), sl(g), None, S0[n:n + 1], sl(do), dST[n:n + 1],
                                scale=scale, delta=False)
        for i in (0, 1, 2, 3, 5):
            parts[i].append(r[i])
    ref = [torch.cat(parts[i], 1) for i in range(4)] + [torch.cat(parts[5], 0)]
    got = _run(q, k, v, g, S0, do, dST, scale, cu=cu)
    _compare(got, ref, 2e-2, 'no-delta varlen strong')


@pytest.mark.gpu
def test_nodelta_simple_gla_routes_through_the_chunk_backward():
    """chunk_simple_gla with grads, 32-token chunks in bf16 (the chunk
    backward takes every chunk size with the scalar gate)."""
    B, T, H, dk, dv = 2, 77, 2, 64, 128
    q, k, v, g, S0, do, dST = _inputs(B, T, H, dk, dv, torch.bfloat16, seed=29, gate='scalar', s0=False)
    print('\n[case] chunk_simple_gla autograd, chunk 32', flush=True)
    r = gdr.recurrent_grads(q, k, v, g, None, None, do, None, scale=0.2, delta=False)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g)]
    o, _ = ops.chunk_simple_gla(*leaves, scale=0.2, chunk_size=32)
    o.backward(do.cuda())
    _compare([x.grad for x in leaves] + [None], (r[0], r[1], r[2], r[3], None), 2e-2, 'simple_gla chunk 32')


@pytest.mark.gpu
def test_nodelta_chunk_bwd_full_size_matches_token_backward():
    """B4 T8192 H8 dk = dv = 128, bf16, per-channel gate: the chunk backward
    against vgdr_scan_bwd(delta=False) on the same inputs."""
    B, T, H, dk, dv = 4, 8192, 8, 128, 128
    print('\n[case] no-delta chunk bwd full size vs scan_bwd', flush=True)
    g0 = torch.Generator(device='cpu').manual_seed(91)
    r = lambda *s: torch.randn(*s, generator=g0).cuda()
    q = F.normalize(r(B, T, H, dk), dim=-1).bfloat16()
    k = F.normalize(r(B, T, H, dk), dim=-1).bfloat16()
    v = r(B, T, H, dv).bfloat16()
    g = F.logsigmoid(r(B, T, H, dk) + 4.0)
    S0 = 0.1 * r(B, H, dk, dv)
    do, dST = r(B, T, H, dv).bfloat16(), r(B, H, dk, dv)
    scale = dk ** -0.5
    got = ops.chunk_gated_delta_rule_bwd(q, k, v, g, None, S0, do, dST, scale=scale, delta=False)
    ref = ops.scan_bwd(q, k, v, g, None, S0, do, dST, scale=scale, delta=False)
    _compare((got[0], got[1], got[2], got[3], got[5]), (ref[0], ref[1], ref[2], ref[3], ref[5]), 2e-2,
             'no-delta full size vs scan_bwd')
