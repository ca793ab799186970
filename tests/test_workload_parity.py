"""Parity at the benchmark workloads' full sizes, against the fp64 oracle on
the CPU (the chunk forms, pinned against the fp64 recurrence in
tests/test_oracle.py), with the inputs the benchmark itself draws
(vagus_amd.workloads, seeded, bf16 q/k/v rounded first so the oracle sees the
same values).

    gdn_340m     GDN prefill, B8 T4096 H8 dk=dv=128, S0 = 0.1 N(0,1): all of it
    kda_prefill  KDA prefill, B4 T8192 H8 dk=dv=128, per-channel gate: all of it
    gdn_varlen   32 packed segments of 128..8192 tokens, H16: every segment,
                 plus bit-exact segment isolation and standalone == packed
                 for the longest and the shortest segment at that scale

The wide-tile state kernel (64 state columns per workgroup, four compute
waves) is chosen once (sequences x heads) x ceil(dv / 64) reaches the CU
count; gdn_varlen (512 pairs) runs it, and so do the dense B16 H16 cases
below, for the scalar gate, the per-channel gate and the training forward
that saves each chunk's entry state (autograd), whose gradients are checked
against the recomputing backward and, on a few (sequence, head) slices,
against the oracle's reverse-mode gradients.

Bar: relative L2 error <= 2e-2 for bf16 inputs on outputs and
final states; integer work bit-exact.
"""
import pytest
import torch

from oracle import gdr
from vagus_amd import ops, workloads

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
DEV = 'cuda'


def rel_l2(x, ref):
    x, ref = x.detach().double().cpu(), ref.detach().double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def case(msg):
    print(f'\n[case] {msg}', flush=True)


def report(what, o, S, ref, tol=TOL_BF16):
    eo, es = rel_l2(o, ref[0]), rel_l2(S, ref[1])
    print(f'[parity] {what}: rel_l2 o={eo:.3e} S={es:.3e} (tol {tol:g})', flush=True)
    assert torch.isfinite(o.float()).all() and torch.isfinite(S).all()
    assert eo <= tol, f'{what}: output rel L2 {eo:.3e} > {tol}'
    assert es <= tol, f'{what}: state rel L2 {es:.3e} > {tol}'


def _d(t):
    return None if t is None else t.double()


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _chunk(y, scale, **kw):
    fn = ops.chunk_kda if (y.g is not None and y.g.dim() == 4) else ops.chunk_gated_delta_rule
    return fn(y.q, y.k, y.v, y.g, y.beta, scale=scale, initial_state=y.initial_state, output_final_state=True,
              cu_seqlens=y.cu_seqlens, **kw)


@pytest.fixture(scope='module', autouse=True)
def _threads():
    prev = torch.get_num_threads()
    torch.set_num_threads(min(16, max(1, len(__import__('os').sched_getaffinity(0)))))
    yield
    torch.set_num_threads(prev)


def test_gdn_340m_full_workload():
    case('gdn_340m full: B8 T4096 H8 dk=dv=128 bf16, S0 = 0.1 N')
    x = workloads.workload('gdn_340m')
    scale = 128 ** -0.5
    o, S = _chunk(x.to(DEV), scale)
    torch.cuda.synchronize()
    ref = gdr.chunk_scalar(_d(x.q), _d(x.k), _d(x.v), _d(x.g), _d(x.beta), _d(x.initial_state), scale=scale)
    report('gdn_340m (B8 T4096 H8)', o, S, ref)


def test_kda_prefill_full_workload():
    case('kda_prefill full: B4 T8192 H8 dk=dv=128 bf16, per-channel gate')
    x = workloads.workload('kda_prefill')
    scale = 128 ** -0.5
    o, S = _chunk(x.to(DEV), scale)
    torch.cuda.synchronize()
    for b in range(x.q.shape[0]):                 # one sequence at a time keeps the oracle's memory small
        sl = slice(b, b + 1)
        ref = gdr.chunk_vector(_d(x.q[sl]), _d(x.k[sl]), _d(x.v[sl]), _d(x.g[sl]), _d(x.beta[sl]), None,
                               scale=scale)
        report(f'kda_prefill sequence {b} (T8192 H8)', o[sl], S[sl], ref)


def test_gdn_varlen_full_workload():
    x = workloads.workload('gdn_varlen')
    cu = x.cu_seqlens.tolist()
    lens = [e - s for s, e in zip(cu[:-1], cu[1:])]
    N, H = len(lens), x.q.shape[2]
    case(f'gdn_varlen full: {N} segments, {cu[-1]} tokens, H{H}, lengths {min(lens)}..{max(lens)}')
    assert N * H * 2 >= _cus(), 'this workload runs the wide-tile state kernel'
    scale = 128 ** -0.5
    y = x.to(DEV)
    o, S = _chunk(y, scale)
    torch.cuda.synchronize()
    ref = gdr.varlen(gdr.chunk_scalar, _d(x.q), _d(x.k), _d(x.v), _d(x.g), _d(x.beta), None, x.cu_seqlens,
                     scale=scale)
    report(f'gdn_varlen ({N} segments)', o, S, ref)
    # per segment, so no short segment hides under the long ones
    worst = 0.0
    for n in range(N):
        s, e = cu[n], cu[n + 1]
        worst = max(worst, rel_l2(o[:, s:e], ref[0][:, s:e]), rel_l2(S[n], ref[1][n]))
    print(f'[parity] gdn_varlen worst segment rel_l2 {worst:.3e}', flush=True)
    assert worst <= TOL_BF16

    # segment isolation at this scale: perturb the shortest segment's values
    short, long_ = min(range(N), key=lambda n: lens[n]), max(range(N), key=lambda n: lens[n])
    y2 = x.to(DEV)
    y2.v[:, cu[short]:cu[short + 1]] += 1.0
    o2, S2 = _chunk(y2, scale)
    keep = torch.ones(cu[-1], dtype=torch.bool, device=DEV)
    keep[cu[short]:cu[short + 1]] = False
    assert torch.equal(o[:, keep], o2[:, keep]), 'a perturbed segment changed another segment\'s output'
    others = [n for n in range(N) if n != short]
    assert torch.equal(S[others], S2[others]) and not torch.equal(S[short], S2[short])
    # a segment run alone equals its slot in the packed run, bit for bit
    for n in (short, long_):
        s, e = cu[n], cu[n + 1]
        o1, S1 = ops.chunk_gated_delta_rule(y.q[:, s:e], y.k[:, s:e], y.v[:, s:e], y.g[:, s:e], y.beta[:, s:e],
                                            scale=scale, output_final_state=True)
        assert torch.equal(o1, o[:, s:e]) and torch.equal(S1[0], S[n]), f'segment {n} alone != packed'
    print(f'[parity] gdn_varlen isolation and standalone == packed (segments {short}, {long_}): bit-exact',
          flush=True)


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_wide_tile_variant_dense(gate):
    B, T, H = 16, 130, 16
    case(f'wide-tile state kernel: {gate} gate B{B} T{T} H{H} dk=dv=128 bf16')
    assert B * H * 2 >= _cus()
    x = workloads.make_inputs(B, T, H, 128, 128, gate=gate, dtype=torch.bfloat16, s0_scale=0.2, seed=21)
    scale = 128 ** -0.5
    o, S = _chunk(x.to(DEV), scale)
    fn = gdr.chunk_vector if gate == 'vector' else gdr.chunk_scalar
    ref = fn(_d(x.q), _d(x.k), _d(x.v), _d(x.g), _d(x.beta), _d(x.initial_state), scale=scale)
    report(f'wide tile {gate} B{B} T{T} H{H}', o, S, ref)


def test_wide_tile_variant_training_forward_and_backward():
    """Autograd on bf16 inputs runs the saving forward (entry states kept) in
    its wide-tile form at this size, then the saved-state backward."""
    B, T, H = 16, 130, 16
    case(f'wide-tile saving forward + saved backward: B{B} T{T} H{H} dk=dv=128 bf16')
    x = workloads.make_inputs(B, T, H, 128, 128, gate='scalar', dtype=torch.bfloat16, s0_scale=0.2, seed=22)
    scale = 128 ** -0.5
    y = x.to(DEV)
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    dST = torch.randn(B, H, 128, 128, generator=gen)
    leaves = [t.clone().requires_grad_(True) for t in (y.q, y.k, y.v, y.g, y.beta, y.initial_state)]
    o, S = ops.chunk_gated_delta_rule(*leaves[:5], scale=scale, initial_state=leaves[5], output_final_state=True)
    # the saving forward computes what the inference forward computes
    with torch.no_grad():
        o_inf, S_inf = _chunk(y, scale)
    print(f'[parity] saving forward vs inference forward: o max|diff| '
          f'{(o.detach().float() - o_inf.float()).abs().max().item():.3e}', flush=True)
    assert rel_l2(o, o_inf) <= 1e-3 and rel_l2(S, S_inf) <= 1e-3
    torch.autograd.backward([o, S], [do.to(DEV), dST.to(DEV)])
    got = [t.grad for t in leaves]
    rec = ops.chunk_gated_delta_rule_bwd(y.q, y.k, y.v, y.g, y.beta, y.initial_state, do.to(DEV), dST.to(DEV),
                                         scale=scale)
    names = ('dq', 'dk', 'dv', 'dg', 'dbeta', 'dS0')
    for nm, a, b in zip(names, got, rec):
        e = rel_l2(a, b)
        print(f'[parity] saved backward vs recomputing backward {nm}: rel_l2 {e:.3e}', flush=True)
        assert e <= 1e-2, nm
    # against the oracle's reverse-mode gradients on a few (sequence, head) slices
    for b, h in ((0, 0), (7, 9), (15, 15)):
        sl = lambda t: t[b:b + 1, :, h:h + 1]
        ref = gdr.recurrent_grads(sl(x.q), sl(x.k), sl(x.v), sl(x.g), sl(x.beta), x.initial_state[b:b + 1, h:h + 1],
                                  sl(do), dST[b:b + 1, h:h + 1], scale=scale)
        for nm, a, r in zip(names, got, ref):
            a = a[b:b + 1, h:h + 1] if nm == 'dS0' else sl(a)
            e = rel_l2(a, r)
            print(f'[parity] seq {b} head {h} {nm} vs oracle: rel_l2 {e:.3e}', flush=True)
            assert e <= TOL_BF16, f'{nm} at ({b}, {h})'
