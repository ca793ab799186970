"""Backward of the chunked delta rule with the per-channel (KDA) gate:
vgdr_chunk_bwd / vgdr_chunk_bwd_saved on gate_kind 2 and the autograd route
of ops.chunk_kda, against the oracle's recurrent_grads (reverse-mode through
the fp64 recurrence, pinned in tests/test_oracle.py by finite differences and
by the chunk form's own gradients).

CPU: the C ABI's argument checks for the per-channel gate (no launch).
GPU: every gradient (dq, dk, dv, the per-channel dg, dbeta, dS0) at rel_l2 <=
2e-2 (bf16 / fp16; the kernels round intermediates to 16 bits as the forward
does), dense with a partial last chunk, a padded head (dk = 100, dv = 48), a
packed batch (empty, one-token and multi-chunk segments), no initial state,
decays strong enough that exp(gamma) of a chunk's rows spans many orders of
magnitude (the gated sums then run on the exact per-pair exponentials), and
the saved (vgdr_chunk_fwd_saving) and recomputed backward against each other.
At the KDA prefill shape (B4 T8192 H8 dk = dv = 128, bf16), where the oracle
is too slow: the chunk backward against the token-recurrence backward
(vgdr_scan_bwd, whose fp32 gradients are pinned at that shape by a
directional derivative in tests/test_scan_bwd.py) on the same inputs.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib, ops


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def test_kda_chunk_bwd_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, gate=2, q=4096, k=8192, v=12288, g=16384, beta=20480, h0=None, do=24576, dht=None,
                 dq=28672, dk=32768, dv=36864, dg=40960, db=45056, dh0=None, cu=None, ws=49152, wsb=1 << 40,
                 B=2, T=64, H=2, dk_=64, dv_=64, N=2, chunk=64)
        a.update(over)
        return L.vgdr_chunk_bwd(a['dtype'], a['gate'], a['q'], a['k'], a['v'], a['g'], a['beta'], a['h0'], a['do'],
                                a['dht'], a['dq'], a['dk'], a['dv'], a['dg'], a['db'], a['dh0'], a['cu'], a['ws'],
                                a['wsb'], a['B'], a['T'], a['H'], a['dk_'], a['dv_'], a['N'], 0.125, a['chunk'],
                                None)
    assert call(dtype=0) == _lib.VGDR_ERR_UNSUPPORTED                # fp32: the token-recurrence backward
    assert call(chunk=32) == _lib.VGDR_ERR_UNSUPPORTED               # 64-token chunks only
    assert b'per-channel' in L.vgdr_last_error()
    assert call(ws=None) == _lib.VGDR_ERR_INVALID
    assert call(g=None) == _lib.VGDR_ERR_INVALID
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK
    fwd_saving = lambda dtype, chunk: L.vgdr_chunk_fwd_saving(dtype, 2, 4096, 8192, 12288, 16384, 20480, 24576,
                                                              None, None, None, 49152, 1 << 40, 2, 64, 2, 64, 64, 2,
                                                              0.125, chunk, None)
    assert fwd_saving(0, 64) == _lib.VGDR_ERR_UNSUPPORTED
    assert fwd_saving(1, 32) == _lib.VGDR_ERR_UNSUPPORTED
    # the forward's blocks, two bf16 states, chunk prep's N (64 x 64 fp32) and
    # the column phase's sums (3 x 64 x dk + 2 x 64 x 64 + dk fp32) per (chunk, head)
    B, T, H, dk, dv = 2, 128, 2, 64, 64
    vec = L.vgdr_chunk_bwd_workspace_size(1, 2, B, T, H, dk, dv, B, 0, 64)
    slots = B * T // 64
    per = 2 * dk * dv * 2 + 64 * 64 * 4 + (3 * 64 * dk + 2 * 64 * 64 + dk) * 4
    assert vec >= slots * H * per + L.vgdr_chunk_workspace_size(1, 2, B, T, H, dk, B, 0, 64)


def test_kda_fused_backward_argument_checks():
    """vgdr_chunk_bwd_fused / _saved_fused / vgdr_chunk_fwd_saving_fused:
    the fused L2 norm is refused (q, k arrive normalised), the gate
    activation needs the per-channel gate and its gradient outputs."""
    L = _lib.load()
    A = torch.zeros(2)
    D = torch.zeros(2 * 64)

    def fz(l2=0, beta=0, gate=1):
        return _lib.Fusion(l2, beta, gate, _lib.VGDR_F32, A.data_ptr(), D.data_ptr(), 0, 0.0)

    def call(fusion, gate=2, dA=8192, ddt=12288, saved=False):
        fn = L.vgdr_chunk_bwd_saved_fused if saved else L.vgdr_chunk_bwd_fused
        return fn(1, gate, 4096, 8192, 12288, 16384, 20480, None, 24576, None, 28672, 32768, 36864, 40960, 45056,
                  None, None, 49152, 1 << 40, 2, 64, 2, 64, 64, 2, 0.125, 64, ctypes.byref(fusion), dA, ddt, None)
    assert call(fz(l2=1)) == _lib.VGDR_ERR_UNSUPPORTED
    assert b'L2 norm' in L.vgdr_last_error()
    assert call(fz(l2=1), saved=True) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(fz(), gate=1) == _lib.VGDR_ERR_INVALID                # the activation is per channel
    assert call(fz(), dA=None) == _lib.VGDR_ERR_INVALID
    assert call(fz(), ddt=None) == _lib.VGDR_ERR_INVALID
    f = fz(l2=1)
    assert L.vgdr_chunk_fwd_saving_fused(1, 2, 4096, 8192, 12288, 16384, 20480, 24576, None, None, None, 49152,
                                         1 << 40, 2, 64, 2, 64, 64, 2, 0.125, 64, ctypes.byref(f),
                                         None) == _lib.VGDR_ERR_UNSUPPORTED


def _inputs(B, T, H, dk, dv, dtype, seed, s0=True, strong=False):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    q = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    k = F.normalize(r(B, T, H, dk), dim=-1).to(dtype)
    v = r(B, T, H, dv).to(dtype)
    g = F.logsigmoid(r(B, T, H, dk) + 3.0)
    if strong:
        # a quarter of the channels decay by e^-2 .. e^-8 per token: a chunk's
        # rows then span exp(gamma) down to ~1e-200 on those channels
        fast = torch.rand(dk, generator=gen) < 0.25
        g = torch.where(fast, -2.0 - 6.0 * torch.rand(B, T, H, dk, generator=gen), g)
    beta = torch.sigmoid(r(B, T, H))
    S0 = 0.3 * r(B, H, dk, dv) if s0 else None
    do = r(B, T, H, dv).to(dtype)
    dST = r(B, H, dk, dv)
    return q, k, v, g, beta, S0, do, dST


def _device_grads(q, k, v, g, beta, S0, do, dST, scale, cu=None):
    leaves = [None if x is None else x.cuda().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.chunk_kda(*leaves[:5], scale=scale, initial_state=leaves[5], output_final_state=True,
                         cu_seqlens=None if cu is None else cu.cuda())
    outs, cots = [o, S], [do.cuda(), dST.cuda()]
    torch.autograd.backward(outs, cots)
    return tuple(None if x is None else x.grad for x in leaves)


NAMES = ('dq', 'dk', 'dv', 'dg', 'dbeta', 'dS0')


def _compare(got, ref, tol, case):
    for name, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        err = _rel(a, b)
        print(f'[parity] {case} {name} rel_l2={err:.3e}', flush=True)
        assert err <= tol, f'{name}: {err:.3e} > {tol:g}'


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('shape', [(2, 100, 2, 64, 64), (1, 70, 2, 128, 128), (1, 45, 1, 100, 48)])
@pytest.mark.parametrize('strong', [False, True])
def test_kda_chunk_bwd_matches_oracle(dtype, shape, strong):
    B, T, H, dk, dv = shape
    print(f'\n[case] kda chunk_bwd dtype={dtype} shape={shape} strong={strong}', flush=True)
    q, k, v, g, beta, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed=T + dk + 7 * strong, strong=strong)
    scale = dk ** -0.5
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=scale)
    got = _device_grads(q, k, v, g, beta, S0, do, dST, scale)
    _compare(got, ref, 2e-2, f'kda {dtype} {shape} strong={strong}')


@pytest.mark.gpu
@pytest.mark.parametrize('cu_list', [[0, 0, 1, 70, 75, 200],      # empty, one token, multi-chunk, short
                                     [0, 130, 387, 579, 835]])     # 3, 5, 3 (exactly) and 4 chunks
def test_kda_chunk_bwd_varlen_matches_per_segment_oracle(cu_list):
    cu = torch.tensor(cu_list, dtype=torch.int32)
    N, T, H, dk, dv = len(cu_list) - 1, cu_list[-1], 2, 64, 64
    q, k, v, g, beta, _, do, _ = _inputs(1, T, H, dk, dv, torch.bfloat16, seed=13)
    gen = torch.Generator().manual_seed(14)
    S0 = 0.3 * torch.randn(N, H, dk, dv, generator=gen)
    dST = torch.randn(N, H, dk, dv, generator=gen)
    print(f'\n[case] kda chunk_bwd varlen cu={cu_list}', flush=True)
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
    _compare(got, ref, 2e-2, 'kda varlen')


@pytest.mark.gpu
def test_kda_chunk_bwd_without_initial_state():
    B, T, H, dk, dv = 2, 77, 2, 64, 128
    q, k, v, g, beta, _, do, _ = _inputs(B, T, H, dk, dv, torch.bfloat16, seed=23, s0=False)
    print('\n[case] kda chunk_bwd no initial state, o only', flush=True)
    ref = gdr.recurrent_grads(q, k, v, g, beta, None, do, None, scale=0.2)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta)]
    o, _ = ops.chunk_kda(*leaves, scale=0.2)
    o.backward(do.cuda())
    _compare([x.grad for x in leaves] + [None], ref, 2e-2, 'kda no S0')


@pytest.mark.gpu
def test_kda_saved_and_recomputed_backward_agree():
    """Autograd through chunk_kda (the saving forward and
    vgdr_chunk_bwd_saved, which read the entry states and N the forward
    kernels stored) against ops.chunk_gated_delta_rule_bwd with the same
    per-channel g (vgdr_chunk_bwd, which reruns the forward for them): the same
    gradients up to rounding (the oracle bar itself is checked above)."""
    B, T, H, dk, dv = 2, 128, 2, 128, 64
    q, k, v, g, beta, S0, do, dST = (None if x is None else x.cuda()
                                     for x in _inputs(B, T, H, dk, dv, torch.bfloat16, seed=51))
    print('\n[case] kda explicit backward vs autograd', flush=True)
    got = ops.chunk_gated_delta_rule_bwd(q, k, v, g, beta, S0, do, dST, scale=0.1)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.chunk_kda(*leaves[:5], scale=0.1, initial_state=leaves[5], output_final_state=True)
    torch.autograd.backward([o, S], [do, dST])
    for name, a, b in zip(NAMES, got, [x.grad for x in leaves]):
        err = _rel(a, b)
        print(f'[parity] kda saved vs recomputed {name} rel_l2={err:.3e}', flush=True)
        assert err <= 5e-3, name


@pytest.mark.gpu
def test_kda_chunk_bwd_full_size_matches_token_backward():
    """B4 T8192 H8 dk = dv = 128 in bf16: the chunk backward against
    vgdr_scan_bwd on the same inputs (relative L2 per gradient, the 16-bit bar)."""
    B, T, H, dk, dv = 4, 8192, 8, 128, 128
    print('\n[case] kda chunk_bwd full size vs scan_bwd', flush=True)
    g0 = torch.Generator(device='cpu').manual_seed(81)
    r = lambda *s: torch.randn(*s, generator=g0).cuda()
    q = F.normalize(r(B, T, H, dk), dim=-1).bfloat16()
    k = F.normalize(r(B, T, H, dk), dim=-1).bfloat16()
    v = r(B, T, H, dv).bfloat16()
    g = F.logsigmoid(r(B, T, H, dk) + 4.0)
    beta = torch.sigmoid(r(B, T, H))
    S0 = 0.1 * r(B, H, dk, dv)
    do, dST = r(B, T, H, dv).bfloat16(), r(B, H, dk, dv)
    scale = dk ** -0.5
    got = ops.chunk_gated_delta_rule_bwd(q, k, v, g, beta, S0, do, dST, scale=scale)
    ref = ops.scan_bwd(q, k, v, g, beta, S0, do, dST, scale=scale)
    _compare(got, ref[:6], 2e-2, 'kda full size vs scan_bwd')


@pytest.mark.gpu
@pytest.mark.parametrize('lower_bound', [None, -5.0])
def test_kda_training_keeps_no_fp32_gate_tensor(lower_bound):
    """chunk_kda with the fused L2 norm, beta sigmoid and gate activation under
    autograd: the activation and the sigmoid run inside the kernels, forward
    and backward, and the L2 norm saves its 16-bit input and one float per
    row, so autograd keeps no fp32 (B, T, H, dk) tensor (the reference's
    fused-gate memory saving, linear_attention.py:84-91); the gradients of
    every input and of A_log, dt_bias still match the oracle's (the full check
    at the oracle bar is tests/test_scan_bwd.py's fused-producer test)."""
    B, T, H, dk, dv = 1, 100, 2, 64, 64
    gen = torch.Generator().manual_seed(31)
    r = lambda *s: torch.randn(*s, generator=gen)
    q, k, v = r(B, T, H, dk).bfloat16(), r(B, T, H, dk).bfloat16(), r(B, T, H, dv).bfloat16()
    f, bl = r(B, T, H, dk).bfloat16(), r(B, T, H)
    A_log, dt_bias = 0.2 * r(H), 0.1 * r(H * dk)
    do = r(B, T, H, dv).bfloat16()
    print(f'\n[case] kda training saved tensors lower_bound={lower_bound}', flush=True)
    dev = [x.cuda().requires_grad_(True) for x in (q, k, v, f, bl, A_log, dt_bias)]
    saved = []

    def pack(t):
        saved.append((tuple(t.shape), t.dtype))
        return t
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        o, _ = ops.chunk_kda(*dev[:5], use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                             use_gate_in_kernel=True, A_log=dev[5], dt_bias=dev[6],
                             safe_gate=lower_bound is not None, lower_bound=lower_bound)
    big = [sd for sd in saved if sd[1] == torch.float32 and len(sd[0]) == 4 and sd[0][-1] == dk]
    print(f'[saved] {saved}', flush=True)
    assert not big, big
    o.backward(do.cuda())
    leaves = [x.double().requires_grad_(True) for x in (q, k, v, f, bl, A_log, dt_bias)]
    gg = gdr.gate_activation(leaves[3], leaves[5], leaves[6], lower_bound)
    oo, _ = gdr.recurrent(gdr.l2norm(leaves[0]), gdr.l2norm(leaves[1]), leaves[2], gg,
                          gdr.beta_sigmoid(leaves[4]), None, scale=dk ** -0.5)
    ref = torch.autograd.grad(oo, leaves, do.double())
    # (dA_log, a sum over every token and channel, is held to the bar over its
    # summands in tests/test_scan_bwd.py; here it only has to exist)
    assert dev[5].grad is not None and torch.isfinite(dev[5].grad).all()
    for name, a, b in zip(('q', 'k', 'v', 'f', 'beta', 'dt_bias'), [x.grad for x in dev[:5] + dev[6:]],
                          ref[:5] + ref[6:]):
        err = _rel(a, b)
        print(f'[parity] kda fused training d{name} rel_l2={err:.3e}', flush=True)
        assert err <= 2e-2, f'd{name}: {err:.3e}'


# ---- explicit write vectors (vgdr_chunk_bwd_w) ----------------------------------

def test_write_bwd_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, q=4096, k=8192, v=12288, w=16384, g=20480, h0=None, do=24576, dht=None, dq=28672,
                 dk=32768, dv=36864, dw=40960, dg=45056, dh0=None, cu=None, ws=49152, wsb=1 << 40, B=2, T=64, H=2,
                 dk_=64, dv_=64, N=2, chunk=64)
        a.update(over)
        return L.vgdr_chunk_bwd_w(a['dtype'], a['q'], a['k'], a['v'], a['w'], a['g'], a['h0'], a['do'], a['dht'],
                                  a['dq'], a['dk'], a['dv'], a['dw'], a['dg'], a['dh0'], a['cu'], a['ws'], a['wsb'],
                                  a['B'], a['T'], a['H'], a['dk_'], a['dv_'], a['N'], 0.125, a['chunk'], None)
    assert call(dtype=0) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(chunk=32) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(w=None) == _lib.VGDR_ERR_INVALID
    assert call(w=16392) == _lib.VGDR_ERR_INVALID                   # alignment
    assert call(dw=None) == _lib.VGDR_ERR_INVALID
    assert call(dw=16384) == _lib.VGDR_ERR_INVALID                  # grad_w aliasing w
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK


def _w_inputs(B, T, H, dk, dv, dtype, seed, strong=False):
    q, k, v, g, _, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed, strong=strong)
    gen = torch.Generator().manual_seed(seed + 1000)
    w = (0.5 * F.normalize(torch.randn(B, T, H, dk, generator=gen), dim=-1)).to(dtype)
    return q, k, v, w, g, S0, do, dST


def _w_device_grads(q, k, v, w, g, S0, do, dST, scale, cu=None):
    leaves = [None if x is None else x.cuda().requires_grad_(True) for x in (q, k, v, g, S0, w)]
    o, S = ops.chunk_scan_vec(*leaves[:4], None, leaves[4], scale=scale, delta=True, w=leaves[5],
                              cu_seqlens=None if cu is None else cu.cuda())
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    dq, dk, dv, dg, dS0, dw = (None if x is None else x.grad for x in leaves)
    return dq, dk, dv, dg, dS0, dw


W_NAMES = ('dq', 'dk', 'dv', 'dg', 'dS0', 'dw')


def _w_compare(got, r, tol, case):
    ref = (r[0], r[1], r[2], r[3], r[5], r[6])                 # recurrent_grads with w: dbeta (zero) dropped
    for name, a, b in zip(W_NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        err = _rel(a, b)
        print(f'[parity] {case} {name} rel_l2={err:.3e}', flush=True)
        assert err <= tol, f'{name}: {err:.3e} > {tol:g}'


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('shape', [(2, 100, 2, 64, 64), (1, 70, 2, 128, 128), (1, 45, 1, 100, 48)])
@pytest.mark.parametrize('strong', [False, True])
def test_write_chunk_bwd_matches_oracle(dtype, shape, strong):
    B, T, H, dk, dv = shape
    print(f'\n[case] w chunk_bwd dtype={dtype} shape={shape} strong={strong}', flush=True)
    q, k, v, w, g, S0, do, dST = _w_inputs(B, T, H, dk, dv, dtype, seed=T + dk + 3 * strong, strong=strong)
    scale = dk ** -0.5
    r = gdr.recurrent_grads(q, k, v, g, None, S0, do, dST, scale=scale, w=w)
    got = _w_device_grads(q, k, v, w, g, S0, do, dST, scale)
    _w_compare(got, r, 2e-2, f'w {dtype} {shape} strong={strong}')


@pytest.mark.gpu
def test_write_chunk_bwd_varlen_and_full_size():
    """A packed batch (empty, one-token, multi-chunk segments) against the
    oracle, then B4 T8192 H8 against vgdr_scan_bwd with w on the same inputs."""
    cu = torch.tensor([0, 0, 1, 70, 75, 200], dtype=torch.int32)
    N, T, H, dk, dv = 5, 200, 2, 64, 64
    q, k, v, w, g, _, do, _ = _w_inputs(1, T, H, dk, dv, torch.bfloat16, seed=43)
    gen = torch.Generator().manual_seed(44)
    S0 = 0.3 * torch.randn(N, H, dk, dv, generator=gen)
    dST = torch.randn(N, H, dk, dv, generator=gen)
    print('\n[case] w chunk_bwd varlen', flush=True)
    scale = dk ** -0.5
    parts = [[] for _ in range(7)]
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        sl = lambda x: x[:, a:b]
        r = gdr.recurrent_grads(sl(q), sl(k), sl(v), sl(g), None, S0[n:n + 1], sl(do), dST[n:n + 1],
                                scale=scale, w=sl(w))
        for i in (0, 1, 2, 3, 5, 6):
            parts[i].append(r[i])
    ref = [torch.cat(parts[i], 0 if i == 5 else 1) if parts[i] else None for i in range(7)]
    got = _w_device_grads(q, k, v, w, g, S0, do, dST, scale, cu=cu)
    _w_compare(got, ref, 2e-2, 'w varlen')

    B, T, H, dk, dv = 4, 8192, 8, 128, 128
    print('\n[case] w chunk_bwd full size vs scan_bwd', flush=True)
    g0 = torch.Generator(device='cpu').manual_seed(45)
    rr = lambda *s: torch.randn(*s, generator=g0).cuda()
    q = F.normalize(rr(B, T, H, dk), dim=-1).bfloat16()
    k = F.normalize(rr(B, T, H, dk), dim=-1).bfloat16()
    w = (0.5 * F.normalize(rr(B, T, H, dk), dim=-1)).bfloat16()
    v = rr(B, T, H, dv).bfloat16()
    g = F.logsigmoid(rr(B, T, H, dk) + 4.0)
    S0 = 0.1 * rr(B, H, dk, dv)
    do, dST = rr(B, T, H, dv).bfloat16(), rr(B, H, dk, dv)
    got = ops.chunk_write_bwd(q, k, v, w, g, S0, do, dST, scale=dk ** -0.5)
    ref = ops.scan_bwd(q, k, v, g, None, S0, do, dST, scale=dk ** -0.5, w=w)
    for name, a, b in zip(('dq', 'dk', 'dv', 'dw', 'dg', 'dS0'), got, (ref[0], ref[1], ref[2], ref[6], ref[3], ref[5])):
        err = _rel(a, b)
        print(f'[parity] w full size vs scan_bwd {name} rel_l2={err:.3e}', flush=True)
        assert err <= 2e-2, f'{name}: {err:.3e}'


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('strong', [False, True])
def test_kda_autograd_in_32_token_chunks(dtype, strong):
    """chunk_kda(..., chunk_size=32) under autograd (the reference's HAX1 / HAX2
    training setting, recipe/model/hax1_340M.yaml:94) runs the chunked
    per-channel backward in 64-token chunks (the gradient does not depend on
    the blocking): every gradient against the fp64 recurrence's."""
    B, T, H, dk, dv = 1, 150, 2, 128, 128
    print(f'\n[case] kda autograd chunk_size=32 dtype={dtype} strong={strong}', flush=True)
    q, k, v, g, beta, S0, do, dST = _inputs(B, T, H, dk, dv, dtype, seed=91 + strong, strong=strong)
    scale = dk ** -0.5
    ref = gdr.recurrent_grads(q, k, v, g, beta, S0, do, dST, scale=scale)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, beta, S0)]
    o, S = ops.chunk_kda(*leaves[:5], scale=scale, initial_state=leaves[5], output_final_state=True, chunk_size=32)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    _compare(tuple(x.grad for x in leaves), ref, 2e-2, f'kda C=32 {dtype} strong={strong}')


@pytest.mark.gpu
def test_write_and_plain_autograd_in_32_token_chunks():
    """chunk_scan_vec with explicit write vectors and without the delta rule,
    chunk_size=32, under autograd: the 64-token chunked backwards, against the
    oracle's gradients."""
    B, T, H, dk, dv = 1, 90, 2, 64, 64
    q, k, v, g, beta, S0, do, dST = _inputs(B, T, H, dk, dv, torch.bfloat16, seed=93)
    gen = torch.Generator().manual_seed(94)
    w = (0.5 * F.normalize(torch.randn(B, T, H, dk, generator=gen), dim=-1)).bfloat16()
    print('\n[case] chunk_scan_vec w autograd chunk_size=32', flush=True)
    ref = gdr.recurrent_grads(q, k, v, g, None, S0, do, dST, scale=0.2, w=w)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, S0, w)]
    o, S = ops.chunk_scan_vec(leaves[0], leaves[1], leaves[2], leaves[3], None, leaves[4], scale=0.2, delta=True,
                              chunk_size=32, w=leaves[5])
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    got = tuple(x.grad for x in leaves)
    names = ('dq', 'dk', 'dv', 'dg', 'dS0', 'dw')
    refm = dict(zip(('dq', 'dk', 'dv', 'dg', 'dbeta', 'dS0', 'dw'), ref)) if len(ref) == 7 else None
    assert refm is not None, len(ref)
    for n, a in zip(names, got):
        e = _rel(a, refm[n])
        print(f'[parity] w C=32 {n} rel_l2={e:.3e}', flush=True)
        assert e <= 2e-2, (n, e)
    print('\n[case] chunk_simple_gla-like per-channel, no delta rule, chunk_size=32', flush=True)
    ref = gdr.recurrent_grads(q, k, v, g, None, S0, do, dST, scale=0.2, delta=False)
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, g, S0)]
    o, S = ops.chunk_scan_vec(leaves[0], leaves[1], leaves[2], leaves[3], None, leaves[4], scale=0.2, delta=False,
                              chunk_size=32)
    torch.autograd.backward([o, S], [do.cuda(), dST.cuda()])
    for n, a, r in zip(('dq', 'dk', 'dv', 'dg', 'dS0'), (x.grad for x in leaves),
                       (ref[0], ref[1], ref[2], ref[3], ref[5])):
        e = _rel(a, r)
        print(f'[parity] nodelta C=32 {n} rel_l2={e:.3e}', flush=True)
        assert e <= 2e-2, (n, e)
