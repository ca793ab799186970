"""The HIP GatedDeltaNet layer (vagus_amd.layer) against the reference
module's interface and the oracle's composition of it.

CPU: the drop-in surface.  Parameter names and shapes are the reference
module's (linear_attention.py:624-679), so its state_dict loads unchanged.
The fusion filters follow :761-781.  The layer refuses CPU tensors and
impl='torch'.

GPU:
  * forward against oracle.model.layer_forward, fp64 on the CPU, with the same
    weights;
  * the reference's relational checks (tests/test_linear_attention.py:98-132):
    decode_step over a prefill block, single tokens and a multi-token block
    reproduces forward; export / load mid-stream is exact; L == 0 is a no-op;
    the layer is causal;
  * ragged packed prefill into cache rows against each sequence alone;
  * the one-token step's regrouped weight copies follow in-place parameter
    changes (bit-equal to a layer rebuilt from the changed state);
  * the explicit-write route (_write returning w) into chunk_scan_vec.
Bars: rel-L2 <= 2e-2 for bf16 modules, <= 1e-4 for fp32 modules (fp32
projections and fp32 kernels against the fp64 oracle).
"""
import itertools

import pytest
import torch

from oracle import gdr
from oracle import model as om
from vagus_amd.layer import GatedDeltaNet, parse_fusions

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def cfg_of(m):
    return dict(head_count=m.head_count, key_head_dim=m.key_head_dim, value_head_dim=m.value_head_dim,
                short_conv_size=m.short_conv_size, gate=m.gate, delta=m.delta, gate_lower_bound=m.gate_lower_bound)


def make(gate='vector', delta=True, conv=4, *, dim=256, H=2, dk=128, dv=128, dtype=torch.float32, device='cpu',
         seed=0, **kw):
    torch.manual_seed(seed)
    m = GatedDeltaNet(dim=dim, head_count=H, key_head_dim=dk, value_head_dim=dv, short_conv_size=conv, gate=gate,
                      delta=delta, gate_rank=16, chunk_size=64, layer_count=4, **kw)
    with torch.no_grad():
        m.o_norm.gamma.uniform_(0.5, 1.5)
        for n in ('conv_q', 'conv_k', 'conv_v'):
            if hasattr(m, n):
                getattr(m, n).conv.weight.normal_(0, 0.5)
        for lin in (m.wq, m.wk, m.wv, m.wg):             # projections of O(1) outputs
            lin.weight.normal_(0, dim ** -0.5)
    return m.to(device=device, dtype=dtype).eval()


# --------------------------------------------------------------------------
# CPU: the interface
# --------------------------------------------------------------------------

def test_parameter_layout_is_the_reference_modules():
    H, dk, dv, dim, K, r = 2, 128, 64, 256, 4, 16
    m = GatedDeltaNet(dim=dim, head_count=H, key_head_dim=dk, value_head_dim=dv, short_conv_size=K,
                      gate='vector', gate_rank=r)
    want = {'wq.weight': (H * dk, dim), 'wk.weight': (H * dk, dim), 'wv.weight': (H * dv, dim),
            'wg.weight': (H * dv, dim), 'wo.weight': (dim, H * dv), 'o_norm.gamma': (dv,),
            'conv_q.conv.weight': (H * dk, 1, K), 'conv_k.conv.weight': (H * dk, 1, K),
            'conv_v.conv.weight': (H * dv, 1, K), 'wa1.weight': (r, dim), 'wa2.weight': (H * dk, r),
            'A_log': (H,), 'dt_bias': (H * dk,), 'wb.weight': (H, dim)}
    assert {k: tuple(v.shape) for k, v in m.state_dict().items()} == want
    s = GatedDeltaNet(dim=dim, head_count=H, key_head_dim=dk, value_head_dim=dv, short_conv_size=None,
                      gate='scalar', delta=False, out_proj=False)
    assert {k: tuple(v.shape) for k, v in s.state_dict().items()} == {
        'wq.weight': (H * dk, dim), 'wk.weight': (H * dk, dim), 'wv.weight': (H * dv, dim),
        'wg.weight': (H * dv, dim), 'o_norm.gamma': (dv,), 'wa.weight': (H, dim), 'A_log': (H,), 'dt_bias': (H,)}
    assert s.gate_projections == [s.wa.weight]
    # the legacy boolean gate spelling (linear_attention.py:594-595)
    assert GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, gate=True).gate == 'scalar'


def test_dt_bias_inverts_each_gate_activation():
    """At f = 0 both gate forms start from the decay -A dt (:650-666)."""
    torch.manual_seed(0)
    m = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, gate='vector', gate_rank=4)
    A = m.A_log.detach().exp()
    g = gdr.gate_activation(torch.zeros(1, 1, 2, 16), m.A_log.detach(), m.dt_bias.detach())
    dt = torch.nn.functional.softplus(m.dt_bias.detach()).view(2, 16)
    assert torch.allclose(g[0, 0], -A[:, None] * dt, atol=1e-6)
    torch.manual_seed(0)
    b = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, gate='vector', gate_rank=4,
                      gate_lower_bound=-5.0)
    gb = gdr.gate_activation(torch.zeros(1, 1, 2, 16), b.A_log.detach(), b.dt_bias.detach(), lower_bound=-5.0)
    assert torch.allclose(gb[0, 0], g[0, 0], rtol=1e-4, atol=1e-7)


def test_fusion_spec_and_filters(monkeypatch):
    assert parse_fusions(True) == frozenset({'conv', 'l2norm', 'gate', 'beta', 'norm_gate'})
    assert parse_fusions(False) == frozenset() and parse_fusions(None) == frozenset()
    assert parse_fusions('scan') == frozenset({'l2norm', 'gate', 'beta'})
    assert parse_fusions(['conv', 'gate']) == frozenset({'conv', 'gate'})
    with pytest.raises(AssertionError):
        parse_fusions('warp')
    monkeypatch.setattr(GatedDeltaNet, '_pick_impl', lambda self, q: 'hip')
    x = torch.zeros(1, dtype=torch.bfloat16)
    kda = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, fused='scan')
    assert kda._active_fusions(x) == frozenset({'l2norm', 'gate', 'beta'})
    gdn = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, gate='scalar', fused='scan')
    assert gdn._active_fusions(x) == frozenset({'l2norm', 'beta'})
    gla = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, delta=False, fused=True)
    assert gla._active_fusions(x) == frozenset({'conv', 'gate', 'norm_gate'})
    assert kda._active_fusions(x.float()) == frozenset()           # fp32: nothing fused (:771-772)


def test_refuses_cpu_tensors_and_the_torch_impl():
    with pytest.raises(NotImplementedError):
        GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16, impl='torch')
    m = GatedDeltaNet(dim=32, head_count=2, key_head_dim=16, value_head_dim=16)
    with pytest.raises(RuntimeError, match='GPU'):
        m(torch.randn(1, 5, 32))
    m.reset_cache(1)
    with pytest.raises(RuntimeError, match='GPU'):
        m.decode_step(torch.randn(1, 1, 32))


# --------------------------------------------------------------------------
# GPU
# --------------------------------------------------------------------------

LAYERS = [('scalar', True, 4, {}), ('vector', True, 4, {}), ('none', True, 4, {}), ('scalar', False, 4, {}),
          ('vector', True, None, {}), ('vector', True, 4, {'gate_lower_bound': -5.0})]


@pytest.mark.gpu
@pytest.mark.parametrize('gate,delta,conv,kw', LAYERS)
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('fused', [False, 'scan'])
def test_forward_matches_oracle(gate, delta, conv, kw, dtype, fused):
    m = make(gate, delta, conv, dtype=dtype, device='cuda', fused=fused, **kw)
    x = torch.randn(2, 70, 256, generator=torch.Generator().manual_seed(1)).to(dtype)
    with torch.no_grad():
        y = m(x.cuda())
    ref = om.layer_forward(m.state_dict(), x.double(), cfg_of(m))
    e = rel(y, ref)
    print(f'[layer] {gate} delta={delta} conv={conv} {kw} {dtype} fused={fused}: rel_l2 {e:.2e}', flush=True)
    assert y.dtype == dtype and y.shape == x.shape
    assert e < TOL[dtype]


@pytest.mark.gpu
@pytest.mark.parametrize('gate,delta,conv', [('scalar', True, 4), ('vector', True, 4), ('none', False, 4),
                                             ('vector', True, None)])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('dk,dv', [(128, 128), (64, 32)])
def test_decode_matches_forward(gate, delta, conv, dtype, dk, dv):
    """The reference's streaming relations (tests/test_linear_attention.py:98-121).
    dk, dv = 128 runs the one-kernel token step; 64, 32 the unfused one."""
    m = make(gate, delta, conv, dtype=dtype, device='cuda', dk=dk, dv=dv)
    x = torch.randn(2, 23, 256, generator=torch.Generator().manual_seed(2)).to(dtype).cuda()
    ref = m(x)
    m.reset_cache(2)
    parts = [m.decode_step(x[:, :9])]
    parts += [m.decode_step(x[:, t:t + 1]) for t in range(9, 14)]
    parts.append(m.decode_step(x[:, 14:]))
    out = torch.cat(parts, dim=1)
    e = rel(out, ref)
    print(f'[layer decode] {gate} delta={delta} conv={conv} {dtype} dk={dk} dv={dv}: rel_l2 {e:.2e}', flush=True)
    assert e < TOL[dtype]
    assert m.cache_len == 23
    # export / load mid-stream: exact
    m.reset_cache(2)
    m.decode_step(x[:, :10])
    snap = m.export_cache()
    a = m.decode_step(x[:, 10:11])
    a2 = m.decode_step(x[:, 11:])
    m.load_cache(snap)
    b = m.decode_step(x[:, 10:11])
    b2 = m.decode_step(x[:, 11:])
    assert torch.equal(a, b) and torch.equal(a2, b2) and m.cache_len == 23
    assert torch.equal(m.decode_step(x[:, :0]), x[:, :0])


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_decode_weight_copies_follow_the_parameters(gate, dtype):
    """The one-token decode step reads regrouped copies of its projection
    weights (and the scalar gate's constants); an in-place change of a
    parameter between steps must reach the next step.  Two identical layers
    step through the same tokens; one has W_q, W_a (or W_a2), A_log and dt_bias
    changed in place after its first step, the other is rebuilt from that
    state: their later outputs and states are equal."""
    import copy
    m = make(gate, True, 4, dtype=dtype, device='cuda')
    x = torch.randn(2, 4, 256, generator=torch.Generator().manual_seed(5)).to(dtype).cuda()
    m.reset_cache(2)
    m.decode_step(x[:, :1])
    with torch.no_grad():
        m.wq.weight.mul_(0.5)
        (m.wa if gate == 'scalar' else m.wa2).weight.add_(0.01)
        m.A_log.add_(0.1)
        m.dt_bias.sub_(0.05)
    fresh = copy.deepcopy(m)
    fresh.__dict__.pop('_decode_w', None)                     # a layer that never cached anything
    for t in range(1, 4):
        a = m.decode_step(x[:, t:t + 1])
        b = fresh.decode_step(x[:, t:t + 1])
        assert torch.equal(a, b), t
    assert torch.equal(m.state, fresh.state)


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_causal(dtype):
    m = make('vector', True, 4, dtype=dtype, device='cuda')
    x = torch.randn(1, 100, 256, generator=torch.Generator().manual_seed(3)).to(dtype).cuda()
    y = m(x)
    x2 = x.clone()
    x2[:, 70:] += torch.randn(1, 30, 256, generator=torch.Generator().manual_seed(4)).to(dtype).cuda()
    y2 = m(x2)
    assert torch.allclose(y[:, :70].float(), y2[:, :70].float(), atol=1e-6, rtol=1e-5)
    assert not torch.allclose(y[:, 70:].float(), y2[:, 70:].float())


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_prefill_packed_matches_each_sequence_alone(gate, dtype):
    """Ragged blocks (one empty, one shorter than the conv and the chunk)
    into rows of a continuing cache: each row's output and final state as
    if the sequence had been decoded alone."""
    m = make(gate, True, 4, dtype=dtype, device='cuda')
    g = torch.Generator().manual_seed(5)
    first = [7, 3, 40, 12]                       # an earlier block per row
    lens = [70, 0, 2, 33]
    xs0 = [torch.randn(1, n, 256, generator=g).to(dtype).cuda() for n in first]
    xs = [torch.randn(1, n, 256, generator=g).to(dtype).cuda() for n in lens]
    # alone: each sequence through decode_step (block, then block)
    alone, states = [], []
    for x0, x in zip(xs0, xs):
        m.reset_cache(1)
        m.decode_step(x0)
        alone.append(m.decode_step(x) if x.shape[1] else x)
        states.append(m.state.clone())
    # packed: the earlier blocks, then the ragged blocks, rows 3, 0, 2, 1
    rows = [3, 0, 2, 1]
    m.reset_cache(4)
    cu0 = torch.tensor([0] + list(torch.tensor([first[r] for r in range(4)]).cumsum(0)), dtype=torch.int32).cuda()
    m.prefill_packed(torch.cat(xs0, 1), cu0)
    order = [rows.index(r) for r in range(4)]    # block n goes to rows[n]; blocks listed by row here
    blocks = [xs[rows[n]] for n in range(4)]
    cu = torch.tensor([0] + list(torch.tensor([b.shape[1] for b in blocks]).cumsum(0)), dtype=torch.int32).cuda()
    y = m.prefill_packed(torch.cat(blocks, 1), cu, rows=rows)
    for n in range(4):
        r = rows[n]
        seg = y[:, int(cu[n]):int(cu[n + 1])]
        if lens[r]:
            assert rel(seg, alone[r]) < TOL[dtype], (n, r)
        assert rel(m.state[r], states[r][0]) < TOL[dtype], (n, r)
    del order


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_explicit_write_routes_to_chunk_scan_vec(dtype):
    """A _write override returning w (KalmanDeltaNet's hook, :783-800) runs
    the per-channel chunk form with w: w = 0.7 beta k must give the
    symmetric rule with beta scaled by 0.7."""
    class Scaled(GatedDeltaNet):
        def _write(self, x, k, g, beta):
            return None, (0.7 * beta[..., None] * k.float()).to(k.dtype)

    torch.manual_seed(0)
    base = make('vector', True, 4, dtype=dtype, device='cuda')
    m = Scaled(dim=256, head_count=2, key_head_dim=128, value_head_dim=128, gate='vector', gate_rank=16,
               layer_count=4).to(device='cuda', dtype=dtype).eval()
    m.load_state_dict(base.state_dict())
    x = torch.randn(2, 70, 256, generator=torch.Generator().manual_seed(6)).to(dtype)
    with torch.no_grad():
        y = m(x.cuda())
    # expected: the oracle's pieces with beta -> 0.7 beta
    sd, c = m.state_dict(), cfg_of(m)
    xd = x.double()
    B, L = xd.shape[:2]
    qp, kp, vp = om._proj(sd, '', xd, torch.float64)
    qp = gdr.short_conv(qp, om._w(sd, 'conv_q.conv.weight', torch.float64))[0]
    kp = gdr.short_conv(kp, om._w(sd, 'conv_k.conv.weight', torch.float64))[0]
    vp = gdr.short_conv(vp, om._w(sd, 'conv_v.conv.weight', torch.float64))[0]
    q, k, v = gdr.l2norm(qp.view(B, L, 2, 128)), gdr.l2norm(kp.view(B, L, 2, 128)), vp.view(B, L, 2, 128)
    g, beta = om._gates(sd, '', xd, c, torch.float64)
    o, _ = gdr.recurrent(q, k, v, g, 0.7 * beta, None, scale=128 ** -0.5)
    ref = om._output(sd, '', o, xd, c, torch.float64)
    e = rel(y, ref)
    print(f'[layer w] {dtype}: rel_l2 {e:.2e}', flush=True)
    assert e < TOL[dtype]


@pytest.mark.gpu
def test_training_forward_differentiates():
    """With grads, the scan runs its HIP backward and the conv and epilogue
    their torch expressions: every parameter receives a gradient, and the
    input gradient matches torch autograd through the oracle composition."""
    m = make('scalar', True, 4, dtype=torch.float32, device='cuda').train()
    x = torch.randn(1, 40, 256, generator=torch.Generator().manual_seed(7)).cuda().requires_grad_(True)
    y = m(x)
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(8)).cuda()
    (y * w).sum().backward()
    for n, p in m.named_parameters():
        assert p.grad is not None and p.grad.abs().sum() > 0, n
    xd = x.detach().double().cpu().requires_grad_(True)
    sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    ref = om.layer_forward(sd, xd, cfg_of(m))
    (ref * w.double().cpu()).sum().backward()
    e = rel(x.grad, xd.grad)
    print(f'[layer grad] dx rel_l2 {e:.2e}', flush=True)
    assert e < 1e-3
