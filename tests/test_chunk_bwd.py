"""Backward of the chunked delta rule (scalar gate or none): vgdr_chunk_bwd
and the autograd route of ops.chunk_gated_delta_rule, against the oracle's
recurrent_grads (reverse-mode through the fp64 recurrence, pinned in
tests/test_oracle.py by finite differences and by the chunk form's own
gradients).

CPU: the C ABI's argument checks (no launch); CPU tensors fail loudly.
GPU: every gradient (dq, dk, dv, dg, dbeta, dS0) at rel_l2 <= 1e-5 (fp32)
or 2e-2 (bf16; the kernels round intermediates to bf16 as the forward does),
dense with a partial last chunk, a padded head (dk = 100, dv = 48), a packed
batch (empty, one-token and multi-chunk segments), fp16 and 32-token chunks,
no initial state, the fla_scan contract (hip_scan) and the fused producers
(L2 norm and beta sigmoid, differentiated in torch before the kernels).  At
the full 340M shape, where the oracle is too slow, the gradients' directional
derivative against Richardson-extrapolated central differences of the
forward kernel (fp32, relative 1e-3).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib, ops


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def test_chunk_bwd_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, gate=1, q=4096, k=8192, v=12288, g=16384, beta=20480, h0=None, do=24576, dht=None,
                 dq=28672, dk=32768, dv=36864, dg=40960, db=45056, dh0=None, cu=None, ws=49152, wsb=1 << 40,
                 B=2, T=64, H=2, dk_=64, dv_=64, N=2)
        a.update(over)
        return L.vgdr_chunk_bwd(a['dtype'], a['gate'], a['q'], a['k'], a['v'], a['g'], a['beta'], a['h0'], a['do'],
                                a['dht'], a['dq'], a['dk'], a['dv'], a['dg'], a['db'], a['dh0'], a['cu'], a['ws'],
                                a['wsb'], a['B'], a['T'], a['H'], a['dk_'], a['dv_'], a['N'], 0.125, 64, None)
    assert call(gate=2, dtype=0) == _lib.VGDR_ERR_UNSUPPORTED        # the per-channel backward is 16-bit
    assert call(dv_=40) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(dk_=96) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(db=None) == _lib.VGDR_ERR_INVALID
    assert call(dv=12288) == _lib.VGDR_ERR_INVALID                   # grad_v aliasing v
    assert b'alias' in L.vgdr_last_error()
    assert call(do=24578) == _lib.VGDR_ERR_INVALID                  # grad_o alignment
    assert call(ws=None) == _lib.VGDR_ERR_INVALID
    assert call(wsb=16) == _lib.VGDR_ERR_INVALID
    assert call(beta=None) == _lib.VGDR_ERR_INVALID
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK
    # the saving forward and saved backward: 16-bit (64-token chunks with a per-channel gate)
    fwd_saving = lambda dtype, gate: L.vgdr_chunk_fwd_saving(dtype, gate, 4096, 8192, 12288, 16384, 20480, 24576,
                                                             None, None, None, 49152, 1 << 40, 2, 64, 2, 64, 64, 2,
                                                             0.125, 64, None)
    assert fwd_saving(0, 1) == _lib.VGDR_ERR_UNSUPPORTED
    need = L.vgdr_chunk_bwd_workspace_size(1, 1, 2, 64, 2, 64, 64, 2, 0, 64)
    # forward blocks plus two bf16 states per (chunk, head)
    assert need >= 2 * 2 * 2 * 64 * 64 * 2 + L.vgdr_chunk_workspace_size(1, 1, 2, 64, 2, 64, 2, 0, 64)


def test_cpu_tensors_with_grad_fail_loudly():
    q = torch.randn(1, 4, 2, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match='ROCm GPU'):                 # no CPU path, with or without grad
        ops.chunk_gated_delta_rule(q, q, q, torch.zeros(1, 4, 2), torch.ones(1, 4, 2))


def _inputs(B, T, H, dk, dv, dtype, seed, gate=True, s0=True):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    q = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    k = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    v = r(B, T, H, dv).to(dtype)
    g = F.logsigmoid(r(B, T, H) + 3.0) if gate else None
    beta = torch.sigmoid(r(B, T, H))
    S0 = 0.3 * r(B, H, dk, dv) if s0 else None
    do = r(B, T, H, dv).to(dtype)
    dST = r(B, H, dk, dv)
    return q, k, v, g, beta, S0, do, dST


def _device_grads(q, k, v, g, beta, S0, do, dST, scale, cu=None, **kw):
    leaves = [None if x is None else x.cuda().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.chunk_gated_delta_rule(*leaves[:5], scale=scale, initial_state=leaves[5], output_final_state=True,
                                      cu_seqlens=None if cu is None else cu.cuda(), **kw)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    return tuple(None if x is None else x.grad for x in leaves)


NAMES = ('dq', 'dk', 'dv', 'dg', 'dbeta', 'dS0')


def _compare(got, ref, tol, case):
    worst = 0.0
    for name, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        err = _rel(a, b)
        worst = max(worst, err)
        print(f'[parity] {case} {name} rel_l2={err:.3e}', flush=True)
        assert err <= tol, f'{name}: {err:.3e} > {tol:g}'
    return worst


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('gate', [True, False])
@pytest.mark.parametrize('shape', [(2, 100, 2, 64, 64), (1, 70, 2, 128, 128), (1, 45, 1, 100, 48)])
def test_chunk_bwd_matches_oracle(dtype, gate, shape):
    B, T, H, dk, dv = shape
    print(f'\n[case] chunk_bwd dtype={dtype} gate={gate} shape={shape}', flush=True)
    q, k, v, g, beta, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed=T + dk + gate)
    scale = dk ** -0.5
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=scale)
    got = _device_grads(q, k, v, g, beta, S0, do, dST, scale)
    _compare(got, ref, 1e-5 if dtype == torch.float32 else 2e-2, f'{dtype} gate={gate} {shape}')


# packed batches: empty, one-token, two-chunk and short segments; and segments
# of 3, 5, 3 (exactly) and 4 chunks, so that the dS walk's producers, which fill
# each step's slot from one of two register sets loaded two steps ahead, end on
# either set and with one or two loads in flight
VARLEN_CU = [[0, 0, 1, 70, 75, 160], [0, 130, 387, 579, 835]]


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('cu_list', VARLEN_CU)
def test_chunk_bwd_varlen_matches_per_segment_oracle(dtype, cu_list):
    cu = torch.tensor(cu_list, dtype=torch.int32)
    N, T, H, dk, dv = len(cu_list) - 1, cu_list[-1], 2, 64, 64
    q, k, v, g, beta, _, do, _ = _inputs(1, T, H, dk, dv, dtype, seed=3)
    gen = torch.Generator().manual_seed(4)
    S0 = 0.3 * torch.randn(N, H, dk, dv, generator=gen)
    dST = torch.randn(N, H, dk, dv, generator=gen)
    print(f'\n[case] chunk_bwd varlen dtype={dtype} cu={cu_list}', flush=True)
    scale = dk ** -0.5
    parts = [[] for _ in range(6)]
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        sl = lambda x: x[:, a:b]
        r = gdr.recurrent_grads(sl(q), sl(k), sl(v), sl(g), sl(beta), S0[n:n + 1], sl(do), dST[n:n + 1],
                                scale=scale)
        for i in range(6):
            parts[i].append(r[i])
    ref = [torch.cat(parts[i], 1) for i in range(5)] + [torch.cat(parts[5], 0)]
    got = _device_grads(q, k, v, g, beta, S0, do, dST, scale, cu=cu)
    _compare(got, ref, 1e-5 if dtype == torch.float32 else 2e-2, f'varlen {dtype}')


@pytest.mark.gpu
def test_chunk_bwd_with_fused_producers():
    """use_qk_l2norm_in_kernel / use_beta_sigmoid_in_kernel with grads: q, k
    un-normalised and beta logits, differentiated through the producers."""
    B, T, H, dk, dv = 2, 96, 2, 64, 64
    gen = torch.Generator().manual_seed(21)
    r = lambda *s: torch.randn(*s, generator=gen)
    q, k, v = r(B, T, H, dk).bfloat16(), r(B, T, H, dk).bfloat16(), r(B, T, H, dv).bfloat16()
    g = F.logsigmoid(r(B, T, H) + 3.0)
    bl = r(B, T, H)
    do = r(B, T, H, dv).bfloat16()
    print('\n[case] chunk_bwd fused producers', flush=True)
    leaves = [x.double().requires_grad_(True) for x in (q, k, v, g, bl)]
    qn = leaves[0] * torch.rsqrt((leaves[0] ** 2).sum(-1, keepdim=True) + 1e-6)
    kn = leaves[1] * torch.rsqrt((leaves[1] ** 2).sum(-1, keepdim=True) + 1e-6)
    o, _ = gdr.recurrent(qn, kn, leaves[2], leaves[3], torch.sigmoid(leaves[4]), None, scale=dk ** -0.5)
    ref = torch.autograd.grad(o, leaves, do.double())
    dl = [x.cuda().requires_grad_(True) for x in (q, k, v, g, bl)]
    od, _ = ops.chunk_gated_delta_rule(*dl, scale=dk ** -0.5, use_qk_l2norm_in_kernel=True,
                                       use_beta_sigmoid_in_kernel=True)
    od.backward(do.cuda())
    for name, a, b in zip(('dq', 'dk', 'dv', 'dg', 'dbeta_logits'), [x.grad for x in dl], ref):
        err = _rel(a, b)
        print(f'[parity] fused {name} rel_l2={err:.3e}', flush=True)
        assert err <= 2e-2, name


@pytest.mark.gpu
@pytest.mark.parametrize('dtype,chunk', [(torch.float16, 64), (torch.bfloat16, 32), (torch.float16, 32)])
def test_chunk_bwd_fp16_and_32_token_chunks(dtype, chunk):
    """fp16 and the 32-token chunk variants, dk = 64 with dv = 128, no initial
    state and no final-state cotangent (dS0 is then not asked for)."""
    B, T, H, dk, dv = 2, 77, 2, 64, 128
    print(f'\n[case] chunk_bwd dtype={dtype} chunk={chunk}', flush=True)
    q, k, v, g, beta, _, do, _ = _inputs(B, T, H, dk, dv, dtype, seed=31 + chunk, s0=False)
    scale = dk ** -0.5
    ref = gdr.recurrent_grads(q, k, v, g, beta, None, do, None, scale=scale)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta)]
    o, _ = ops.chunk_gated_delta_rule(*leaves, scale=scale, chunk_size=chunk)
    o.backward(do.cuda())
    _compare([x.grad for x in leaves] + [None], ref, 2e-2, f'{dtype} chunk={chunk}')


@pytest.mark.gpu
def test_hip_scan_is_differentiable():
    """hip_scan (the fla_scan contract: o and the final state) with grads, the
    route a training module takes, against the oracle."""
    B, T, H, dk, dv = 1, 90, 2, 128, 64
    print('\n[case] hip_scan backward', flush=True)
    q, k, v, g, beta, S0, do, dST = _inputs(B, T, H, dk, dv, torch.bfloat16, seed=41)
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=dk ** -0.5)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.hip_scan(*leaves, scale=dk ** -0.5, delta=True)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    _compare([x.grad for x in leaves], ref, 2e-2, 'hip_scan')


@pytest.mark.gpu
def test_saved_and_recomputed_backward_agree():
    """Autograd through chunk_gated_delta_rule (16-bit: the saving forward and
    vgdr_chunk_bwd_saved, which read the entry states the forward kernel
    stored) against ops.chunk_gated_delta_rule_bwd (vgdr_chunk_bwd, which
    re-walks the recurrence for them): the same gradients up to the rounding
    of the two state computations (the oracle bar itself is checked above)."""
    B, T, H, dk, dv = 2, 64, 2, 64, 64
    q, k, v, g, beta, S0, do, dST = (None if x is None else x.cuda()
                                     for x in _inputs(B, T, H, dk, dv, torch.bfloat16, seed=51))
    print('\n[case] explicit backward vs autograd', flush=True)
    got = ops.chunk_gated_delta_rule_bwd(q, k, v, g, beta, S0, do, dST, scale=0.125)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.chunk_gated_delta_rule(*leaves[:5], scale=0.125, initial_state=leaves[5], output_final_state=True)
    torch.autograd.backward([o, S], [do, dST])
    for name, a, b in zip(NAMES, got, [x.grad for x in leaves]):
        err = _rel(a, b)
        print(f'[parity] saved vs recomputed {name} rel_l2={err:.3e}', flush=True)
        assert err <= 5e-3, name


@pytest.mark.gpu
def test_chunk_bwd_full_size_directional_derivative():
    """At the 340M shape (B8 T4096 H8 dk=dv=128, fp32), where the fp64 oracle is
    too slow: the backward's directional derivative sum_x <grad_x, delta_x> of
    L = <o, do> + <S_T, dST> equals central differences of the forward kernel
    along delta, for every input (q, k, v, g, beta, S0) at once."""
    B, T, H, dk, dv = 8, 4096, 8, 128, 128
    print('\n[case] chunk_bwd full-size directional derivative', flush=True)
    g0 = torch.Generator(device='cpu').manual_seed(61)
    r = lambda *s: torch.randn(*s, generator=g0).cuda()
    q = F.normalize(r(B, T, H, dk), dim=-1)
    k = F.normalize(r(B, T, H, dk), dim=-1)
    v = r(B, T, H, dv)
    g = F.logsigmoid(r(B, T, H) + 4.0)
    beta = torch.sigmoid(r(B, T, H))
    S0 = 0.1 * r(B, H, dk, dv)
    do, dST = r(B, T, H, dv), r(B, H, dk, dv)
    xs = [q, k, v, g, beta, S0]
    # small directions that keep g <= 0 and beta in (0, 1) under +-eps
    ds = [0.01 * r(*x.shape) for x in xs]
    ds[3] = -0.01 * torch.rand(*g.shape, generator=g0).cuda()
    ds[4] = 0.01 * r(*beta.shape) * beta * (1 - beta)
    scale = dk ** -0.5

    def loss(ys):
        o, S = ops.chunk_gated_delta_rule(*ys[:5], scale=scale, initial_state=ys[5], output_final_state=True)
        return (o.double() * do.double()).sum().item() + (S.double() * dST.double()).sum().item()

    grads = ops.chunk_gated_delta_rule_bwd(q, k, v, g, beta, S0, do, dST, scale=scale)
    ana = sum((gx.double() * d.double()).sum().item() for gx, d in zip(grads, ds))
    def cd(eps):                                               # central difference along the directions
        return (loss([x + eps * d for x, d in zip(xs, ds)]) - loss([x - eps * d for x, d in zip(xs, ds)])) / (2 * eps)

    # Richardson extrapolation of two step sizes cancels the O(eps^2) term (the
    # decays compound over each chunk, so the curvature along g is not small)
    c1, c2 = cd(0.5), cd(0.25)
    fd = (4 * c2 - c1) / 3
    err = abs(ana - fd) / max(abs(fd), 1e-30)
    print(f'[parity] full-size directional derivative: backward {ana:.6e} central differences {c1:.6e} '
          f'(eps 0.5) {c2:.6e} (eps 0.25) extrapolated {fd:.6e} rel {err:.2e}', flush=True)
    assert err <= 1e-3
