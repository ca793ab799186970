"""Backward of every scan form the scalar-gate chunk backward does not take:
vgdr_scan_bwd (per-channel KDA gate, explicit write vector w, the plain
recurrence without the delta rule; the scalar gate and none too) and the
autograd routes of ops.chunk_kda / chunk_simple_gla / chunk_scan_vec / hip_scan
and of the token-by-token hip_recurrent,
against the oracle's recurrent_grads (reverse-mode through the fp64
recurrence, pinned in tests/test_oracle.py by finite differences for every
form and by the per-channel chunk form's own gradients).

CPU: the C ABI's argument checks (no launch) and the workspace size.
GPU: every gradient at rel_l2 <= 1e-5 (fp32; the kernel runs the recurrence
in fp32) or 2e-2 (bf16, fp16 inputs, fp32 arithmetic), dense with sequence
lengths that end inside a checkpoint block, a padded head (dk = 100, dv = 48),
dv = 80 (16-column tiles), a packed batch (empty, one-token and long
segments), no initial state, and the fused producers (L2 norm, beta sigmoid,
the gate activation with and without its lower bound, differentiated in torch
before the kernels).  At the full KDA prefill shape (B4 T8192 H8), where the
oracle is too slow, the gradients' directional derivative against
Richardson-extrapolated central differences of the chunked forward kernel
(fp32, relative 1e-3).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib, ops


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def test_scan_bwd_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, gate=2, delta=1, q=4096, k=8192, v=12288, w=None, g=16384, beta=20480, h0=None,
                 do=24576, dht=None, dq=28672, dk=32768, dv=36864, dw=None, dg=40960, db=45056, dh0=None, cu=None,
                 ws=49152, wsb=1 << 40, B=2, T=64, H=2, dk_=64, dv_=64, N=2)
        a.update(over)
        return L.vgdr_scan_bwd(a['dtype'], a['gate'], a['delta'], a['q'], a['k'], a['v'], a['w'], a['g'],
                               a['beta'], a['h0'], a['do'], a['dht'], a['dq'], a['dk'], a['dv'], a['dw'], a['dg'],
                               a['db'], a['dh0'], a['cu'], a['ws'], a['wsb'], a['B'], a['T'], a['H'], a['dk_'],
                               a['dv_'], a['N'], 0.125, None)
    assert call(w=53248, delta=0) == _lib.VGDR_ERR_INVALID          # w needs the delta rule
    assert call(w=53248) == _lib.VGDR_ERR_INVALID                   # ... and grad_w
    assert b'grad_w' in L.vgdr_last_error()
    assert call(dv_=40) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(dk_=96) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(db=None) == _lib.VGDR_ERR_INVALID                   # beta k writes need grad_beta
    assert call(dg=None) == _lib.VGDR_ERR_INVALID
    assert call(dv=12288) == _lib.VGDR_ERR_INVALID                  # grad_v aliasing v
    assert b'alias' in L.vgdr_last_error()
    assert call(do=24578) == _lib.VGDR_ERR_INVALID                  # grad_o alignment
    assert call(ws=None) == _lib.VGDR_ERR_INVALID
    assert call(wsb=16) == _lib.VGDR_ERR_INVALID
    assert call(beta=None) == _lib.VGDR_ERR_INVALID
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK
    # checkpoints every 8 tokens (fp32 states), u per token, four partials per column tile
    need = L.vgdr_scan_bwd_workspace_size(2, 64, 2, 64, 64, 2)
    assert need >= (128 // 8 + 2) * 2 * 64 * 64 * 4 + 128 * 2 * 64 * 4 + 4 * 2 * 128 * 2 * 64 * 4
    assert L.vgdr_scan_bwd_workspace_size(-1, 64, 2, 64, 64, 2) == 0


def test_cpu_tensors_with_grad_fail_loudly():
    q = torch.randn(1, 4, 2, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match='ROCm GPU'):
        ops.fused_recurrent_gated_delta_rule(q, q, q, torch.zeros(1, 4, 2), torch.ones(1, 4, 2))
    with pytest.raises(RuntimeError, match='ROCm GPU'):
        ops.chunk_kda(q, q, q, torch.zeros(1, 4, 2, 64), torch.ones(1, 4, 2))


def _inputs(B, T, H, dk, dv, dtype, seed, gate, with_w=False, s0=True):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    q = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    k = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    v = r(B, T, H, dv).to(dtype)
    if gate == 'vector':
        g = F.logsigmoid(r(B, T, H, dk) + 3.0)
    elif gate == 'scalar':
        g = F.logsigmoid(r(B, T, H) + 3.0)
    else:
        g = None
    beta = torch.sigmoid(r(B, T, H))
    w = (0.5 * F.normalize(r(B, T, H, dk), dim=-1)).to(dtype) if with_w else None
    S0 = 0.3 * r(B, H, dk, dv) if s0 else None
    do = r(B, T, H, dv).to(dtype)
    dST = r(B, H, dk, dv)
    return q, k, v, g, beta, w, S0, do, dST


NAMES = ('dq', 'dk', 'dv', 'dg', 'dbeta', 'dS0', 'dw')


def _compare(got, ref, tol, case):
    for name, a, b in zip(NAMES, got, ref):
        if b is None or (name == 'dbeta' and a is None):
            continue
        err = _rel(a, b)
        print(f'[parity] {case} {name} rel_l2={err:.3e}', flush=True)
        assert err <= tol, f'{name}: {err:.3e} > {tol:g}'


def _cuda(*xs):
    return [None if x is None else x.cuda() for x in xs]


TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('mode', ['vector', 'vector_w', 'vector_nodelta', 'scalar_nodelta', 'none_nodelta',
                                  'scalar_w', 'scalar', 'none'])
@pytest.mark.parametrize('shape', [(2, 37, 2, 64, 64), (1, 70, 2, 128, 128), (1, 45, 1, 100, 48),
                                   (1, 19, 2, 64, 80)])
def test_scan_bwd_matches_oracle(dtype, mode, shape):
    B, T, H, dk, dv = shape
    gate = mode.split('_')[0]
    delta = not mode.endswith('nodelta')
    with_w = mode.endswith('_w')
    print(f'\n[case] scan_bwd dtype={dtype} mode={mode} shape={shape}', flush=True)
    q, k, v, g, beta, w, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed=T + dk + len(mode), gate=gate,
                                               with_w=with_w)
    scale = dk ** -0.5
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=scale, delta=delta, w=w)
    got = ops.scan_bwd(*_cuda(q, k, v, g, beta, S0, do, dST), scale=scale, delta=delta, w=None if w is None else
                       w.cuda())
    torch.cuda.synchronize()
    assert (got[4] is None) == (not delta or with_w)
    _compare(got, ref, TOL[dtype], f'{mode} {dtype} {shape}')


@pytest.mark.gpu
@pytest.mark.parametrize('mode', ['vector', 'vector_w', 'none_nodelta'])
def test_scan_bwd_varlen(mode):
    """A packed batch: an empty, a one-token, a short and a long segment, each
    with its own entry state and final-state cotangent."""
    gate = mode.split('_')[0]
    delta = not mode.endswith('nodelta')
    with_w = mode.endswith('_w')
    lens = [0, 1, 13, 83]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    q, k, v, g, beta, w, _, do, _ = _inputs(1, T, 2, 128, 64, torch.bfloat16, seed=5, gate=gate, with_w=with_w)
    gen = torch.Generator().manual_seed(6)
    S0 = 0.3 * torch.randn(len(lens), 2, 128, 64, generator=gen)
    dST = torch.randn(len(lens), 2, 128, 64, generator=gen)
    print(f'\n[case] scan_bwd varlen mode={mode} lens={lens}', flush=True)
    got = ops.scan_bwd(*_cuda(q, k, v, g, beta, S0, do, dST), scale=0.1, delta=delta,
                       w=None if w is None else w.cuda(), cu_seqlens=cu.cuda())
    torch.cuda.synchronize()
    refs = [torch.zeros_like(x, dtype=torch.float64) if x is not None else None for x in (q, k, v, g, beta)]
    dS0_ref = torch.zeros(len(lens), 2, 128, 64, dtype=torch.float64)
    dw_ref = torch.zeros_like(q, dtype=torch.float64) if with_w else None
    for n in range(len(lens)):
        a, b = int(cu[n]), int(cu[n + 1])
        sl = lambda x: None if x is None else x[:, a:b]
        r = gdr.recurrent_grads(sl(q), sl(k), sl(v), sl(g), sl(beta), S0[n:n + 1], sl(do), dST[n:n + 1],
                                scale=0.1, delta=delta, w=sl(w))
        for i in range(5):
            if refs[i] is not None and r[i] is not None:
                refs[i][:, a:b] = r[i]
        dS0_ref[n] = r[5][0]
        if with_w:
            dw_ref[:, a:b] = r[6]
    _compare(got, tuple(refs) + (dS0_ref, dw_ref), 2e-2, f'varlen {mode}')


def _autograd(fn, leaves, do, dST):
    dev = [None if x is None else x.cuda().requires_grad_(True) for x in leaves]
    o, S = fn(*dev)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    return [None if x is None else x.grad for x in dev]


@pytest.mark.gpu
@pytest.mark.parametrize('lower_bound', [None, -5.0])
def test_chunk_kda_autograd_with_fused_producers(lower_bound):
    """chunk_kda with q, k un-normalised, beta as logits and the gate as its
    pre-activation: the gradients of every input, A_log and dt_bias included,
    equal those of the oracle's producers followed by its recurrence (with
    grads, 16-bit chunk_kda runs the chunked backward, vgdr_chunk_bwd).
    dA_log and ddt_bias are sums over tokens (and channels) of
    dg * dg/dparam; their error is held to the bar relative to the L2 norm of
    those summands, which is what rounding in dg bounds: with the lower bound
    the sum for A_log is several times smaller than its summands' norm
    (cancellation), and a relative bar on the sum would ask for more than the
    16-bit per-token gradients carry."""
    B, T, H, dk, dv = 1, 50, 2, 64, 64
    gen = torch.Generator().manual_seed(9)
    r = lambda *s: torch.randn(*s, generator=gen)
    q, k, v = r(B, T, H, dk).bfloat16(), r(B, T, H, dk).bfloat16(), r(B, T, H, dv).bfloat16()
    f, bl = r(B, T, H, dk), r(B, T, H)
    A_log, dt_bias = 0.2 * r(H), 0.1 * r(H * dk)
    S0 = 0.3 * r(B, H, dk, dv)
    do, dST = r(B, T, H, dv).bfloat16(), r(B, H, dk, dv)
    print(f'\n[case] chunk_kda autograd fused producers lower_bound={lower_bound}', flush=True)

    def dev_fn(q, k, v, f, bl, S0, A_log, dt_bias):
        return ops.chunk_kda(q, k, v, f, bl, initial_state=S0, output_final_state=True,
                             use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                             use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias,
                             safe_gate=lower_bound is not None, lower_bound=lower_bound)
    got = _autograd(dev_fn, (q, k, v, f, bl, S0, A_log, dt_bias), do, dST)
    leaves = [x.double().requires_grad_(True) for x in (q, k, v, f, bl, S0, A_log, dt_bias)]
    qq, kk = gdr.l2norm(leaves[0]), gdr.l2norm(leaves[1])
    gg = gdr.gate_activation(leaves[3], leaves[6], leaves[7], lower_bound)
    o, S = gdr.recurrent(qq, kk, leaves[2], gg, gdr.beta_sigmoid(leaves[4]), leaves[5], scale=dk ** -0.5)
    ref = torch.autograd.grad([o, S], leaves + [gg], [do.double(), dST.double()])
    dg_ref = ref[-1]
    # the summands of dA_log and ddt_bias: dg times the gate's derivative in
    # that parameter (each gate element depends on one A_log and one dt_bias entry)
    act = lambda a, d: gdr.gate_activation(f.double(), a, d, lower_bound)
    A2, d2 = A_log.double(), dt_bias.double()
    _, wA = torch.func.jvp(lambda a: act(a, d2), (A2,), (torch.ones_like(A2),))
    _, wd = torch.func.jvp(lambda d: act(A2, d), (d2,), (torch.ones_like(d2),))
    norms = {'A_log': (dg_ref * wA).pow(2).sum((0, 1, 3)).sqrt(),
             'dt_bias': (dg_ref * wd).pow(2).sum((0, 1)).sqrt().reshape(-1)}
    for name, a, b in zip(('q', 'k', 'v', 'f', 'beta', 'S0', 'A_log', 'dt_bias'), got, ref[:-1]):
        if name in norms:
            err = ((a.double().cpu() - b).norm() / norms[name].norm()).item()
            print(f'[parity] chunk_kda fused d{name} rel_l2={_rel(a, b):.3e}, over its summands {err:.3e}',
                  flush=True)
        else:
            err = _rel(a, b)
            print(f'[parity] chunk_kda fused d{name} rel_l2={err:.3e}', flush=True)
        assert err <= 2e-2, f'd{name}: {err:.3e}'


@pytest.mark.gpu
def test_chunk_scan_vec_and_simple_gla_autograd():
    """The explicit write vector through chunk_scan_vec and the plain
    recurrence through chunk_simple_gla, differentiated by autograd."""
    B, T, H, dk, dv = 2, 41, 2, 128, 64
    q, k, v, g, beta, w, S0, do, dST = _inputs(B, T, H, dk, dv, torch.bfloat16, seed=31, gate='vector', with_w=True)
    print('\n[case] chunk_scan_vec w autograd', flush=True)
    got = _autograd(lambda q, k, v, g, S0, w: ops.chunk_scan_vec(q, k, v, g, None, S0, scale=0.2, delta=True, w=w),
                    (q, k, v, g, S0, w), do, dST)
    r = gdr.recurrent_grads(q, k, v, g, None, S0, do, dST, scale=0.2, w=w)
    _compare(got[:4] + [None, got[4], got[5]], r, 2e-2, 'chunk_scan_vec w')
    print('\n[case] chunk_simple_gla autograd', flush=True)
    gs = F.logsigmoid(torch.randn(B, T, H) + 3.0)
    got = _autograd(lambda q, k, v, g, S0: ops.chunk_simple_gla(q, k, v, g, scale=0.2, initial_state=S0,
                                                                output_final_state=True),
                    (q, k, v, gs, S0), do, dST)
    r = gdr.recurrent_grads(q, k, v, gs, None, S0, do, dST, scale=0.2, delta=False)
    _compare(got[:4] + [None, got[4]], r, 2e-2, 'chunk_simple_gla')


@pytest.mark.gpu
@pytest.mark.parametrize('mode', ['vector', 'scalar_w', 'none_nodelta'])
def test_recurrent_autograd(mode):
    """The token-by-token calls (hip_recurrent, the contract of recurrent_scan)
    differentiated by autograd through vgdr_scan_bwd."""
    gate = mode.split('_')[0]
    delta = not mode.endswith('nodelta')
    with_w = mode.endswith('_w')
    B, T, H, dk, dv = 1, 29, 2, 64, 64
    q, k, v, g, beta, w, S0, do, dST = _inputs(B, T, H, dk, dv, torch.float32, seed=41, gate=gate, with_w=with_w)
    print(f'\n[case] hip_recurrent autograd mode={mode}', flush=True)
    b = beta if (delta and not with_w) else None

    def fn(q, k, v, g, b, S0, w):
        return ops.hip_recurrent(q, k, v, g, b, S0, scale=0.3, delta=delta, w=w)
    got = _autograd(fn, (q, k, v, g, b, S0, w), do, dST)
    r = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=0.3, delta=delta, w=w)
    _compare(got[:6] + [got[6]], r, 1e-5, f'hip_recurrent {mode}')


@pytest.mark.gpu
def test_scan_bwd_kda_full_size_directional_derivative():
    """At the KDA prefill shape (B4 T8192 H8 dk=dv=128, fp32), where the fp64
    oracle is too slow: the backward's directional derivative
    sum_x <grad_x, delta_x> of L = <o, do> + <S_T, dST> equals central
    differences of the chunked forward kernel along delta, for every input
    (q, k, v, the per-channel g, beta, S0) at once (Richardson-extrapolated,
    relative 1e-3)."""
    B, T, H, dk, dv = 4, 8192, 8, 128, 128
    print('\n[case] scan_bwd KDA full-size directional derivative', flush=True)
    g0 = torch.Generator(device='cpu').manual_seed(71)
    r = lambda *s: torch.randn(*s, generator=g0).cuda()
    q = F.normalize(r(B, T, H, dk), dim=-1)
    k = F.normalize(r(B, T, H, dk), dim=-1)
    v = r(B, T, H, dv)
    g = F.logsigmoid(r(B, T, H, dk) + 4.0)
    beta = torch.sigmoid(r(B, T, H))
    S0 = 0.1 * r(B, H, dk, dv)
    do, dST = r(B, T, H, dv), r(B, H, dk, dv)
    xs = [q, k, v, g, beta, S0]
    ds = [0.01 * r(*x.shape) for x in xs]
    ds[3] = -0.01 * torch.rand(*g.shape, generator=g0).cuda()
    ds[4] = 0.01 * r(*beta.shape) * beta * (1 - beta)
    scale = dk ** -0.5

    def loss(ys):
        o, S = ops.chunk_kda(*ys[:5], scale=scale, initial_state=ys[5], output_final_state=True)
        return (o.double() * do.double()).sum().item() + (S.double() * dST.double()).sum().item()

    grads = ops.scan_bwd(q, k, v, g, beta, S0, do, dST, scale=scale)
    ana = sum((gx.double() * d.double()).sum().item() for gx, d in zip(grads, ds))

    def cd(eps):
        return (loss([x + eps * d for x, d in zip(xs, ds)]) - loss([x - eps * d for x, d in zip(xs, ds)])) / (2 * eps)

    c1, c2 = cd(0.5), cd(0.25)
    fd = (4 * c2 - c1) / 3
    err = abs(ana - fd) / max(abs(fd), 1e-30)
    print(f'[parity] KDA full-size directional derivative: backward {ana:.6e} extrapolated {fd:.6e} rel {err:.2e}',
          flush=True)
    assert err <= 1e-3
