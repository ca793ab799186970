"""The reference's other head shapes on the GPU.  dv = 256 is the shape of
its LAX1 / HAX1 / HAX2 recipes and of its own layer bench
(recipe/model/lax1_340M.yaml:39-41, hax1_340M.yaml:64-66,
bench_linear_attention.py:18-20).  It runs through the chunk kernels as
more dv tiles and through the token kernel as 128-column slices; the layer's
one-token decode step (the conv with its caches, the L2 norm, the gates, the
recurrence and the epilogue) is one kernel at this width too.  Checked against the fp64
oracle at the parity bars (relative L2 1e-5 fp32, 2e-2 bf16).  dk = 256 (the LAX3
recipe, lax3_340M.yaml:83-85) is refused with NotImplementedError: the kernels
hold at most 128 key rows per state strip."""
import pytest
import torch

from oracle import gdr
from oracle import model as om
from vagus_amd import ops, workloads
from vagus_amd.layer import GatedDeltaNet

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-5}


def rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def d(t):
    return None if t is None else t.double()


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_chunk_dv256(gate, dtype):
    x = workloads.make_inputs(2, 130, 2, 128, 256, gate=gate, dtype=dtype, s0_scale=0.1, seed=11)
    ref = gdr.recurrent(d(x.q), d(x.k), d(x.v), d(x.g), d(x.beta), d(x.initial_state), scale=128 ** -0.5)
    y = x.to('cuda')
    fn = ops.chunk_kda if gate == 'vector' else ops.chunk_gated_delta_rule
    o, S = fn(y.q, y.k, y.v, y.g, y.beta, initial_state=y.initial_state, output_final_state=True)
    eo, es = rel(o, ref[0]), rel(S, ref[1])
    print(f'[dv256] chunk {gate} {dtype}: o {eo:.2e} S {es:.2e}', flush=True)
    assert eo < TOL[dtype] and es < TOL[dtype]


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_decode_dv256(dtype):
    x = workloads.make_inputs(8, 1, 4, 128, 256, gate='scalar', dtype=dtype, s0_scale=0.5, seed=12)
    ref = gdr.recurrent(d(x.q), d(x.k), d(x.v), d(x.g), d(x.beta), d(x.initial_state), scale=128 ** -0.5)
    y = x.to('cuda')
    state = y.initial_state.clone()
    o, _ = ops.fused_recurrent_gated_delta_rule(y.q, y.k, y.v, y.g, y.beta, initial_state=state,
                                                inplace_final_state=True)
    eo, es = rel(o, ref[0]), rel(state, ref[1])
    print(f'[dv256] decode {dtype}: o {eo:.2e} S {es:.2e}', flush=True)
    assert eo < TOL[dtype] and es < TOL[dtype]


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_layer_lax1_shape(dtype):
    """LAX1's mixer shape: dim 1024, 4 heads of dk 128 / dv 256, KDA gate."""
    torch.manual_seed(0)
    m = GatedDeltaNet(dim=1024, head_count=4, key_head_dim=128, value_head_dim=256, gate='vector', gate_rank=64,
                      layer_count=4)
    with torch.no_grad():
        m.o_norm.gamma.uniform_(0.5, 1.5)
        for lin in (m.wq, m.wk, m.wv, m.wg):
            lin.weight.normal_(0, 1024 ** -0.5)
    m = m.to(device='cuda', dtype=dtype).eval()
    x = torch.randn(2, 70, 1024, generator=torch.Generator().manual_seed(1)).to(dtype)
    with torch.no_grad():
        y = m(x.cuda())
    cfg = dict(head_count=4, key_head_dim=128, value_head_dim=256, short_conv_size=4, gate='vector', delta=True)
    e = rel(y, om.layer_forward(m.state_dict(), x.double(), cfg))
    m.reset_cache(2)
    parts = [m.decode_step(x[:, :40].cuda())] + [m.decode_step(x[:, t:t + 1].cuda()) for t in range(40, 70)]
    ed = rel(torch.cat(parts, 1), y)
    print(f'[dv256] layer {dtype}: forward {e:.2e} decode vs forward {ed:.2e}', flush=True)
    bar = 2e-2 if dtype == torch.bfloat16 else 1e-4
    assert e < bar and ed < bar


@pytest.mark.gpu
def test_dk256_is_refused():
    x = workloads.make_inputs(1, 16, 2, 256, 128, gate='scalar', dtype=torch.bfloat16, seed=13).to('cuda')
    with pytest.raises(NotImplementedError, match='128'):
        ops.chunk_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta)
    with pytest.raises(NotImplementedError, match='128'):
        ops.fused_recurrent_gated_delta_rule(x.q[:, :1], x.k[:, :1], x.v[:, :1], x.g[:, :1], x.beta[:, :1])


@pytest.mark.gpu
@pytest.mark.parametrize('gate,dtype,epilogue', [('scalar', torch.bfloat16, True), ('vector', torch.bfloat16, True),
                                                 ('scalar', torch.float32, False), ('vector', torch.float32, True)])
def test_fused_decode_step_dv256(gate, dtype, epilogue):
    """The one-kernel decode step at dk 128 / dv 256 (decode_conv_kernel<128,
    256>, 512 threads) against the oracle's decode_step (+ norm_gate)."""
    from test_decode_conv import _run
    _run(gate, dtype, 4, 1, epilogue=epilogue, w_dtype=torch.float32 if dtype == torch.float32 else torch.bfloat16,
         seed=17, B=4, H=2, dk=128, dv=256)


@pytest.mark.gpu
def test_fused_decode_step_dv256_lax1_batch():
    """LAX1's decode at a serving batch: B64 H4 dk 128 / dv 256, the KDA gate
    from its pre-activation inside the kernel as the layer calls it."""
    from test_decode_conv import _decode_inputs, _rel
    B, H, dk, dv, K = 64, 4, 128, 256, 4
    qp, kp, vp, ws, cs, _, beta, S0 = _decode_inputs(B, 1, H, dk, dv, K, 'vector', torch.bfloat16, seed=51,
                                                     w_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(52)
    f = torch.randn(B, 1, H, dk, generator=g)                  # the gate's pre-activation
    A_log = torch.rand(H, generator=g) * 2.0
    dt_bias = 0.5 * torch.randn(H * dk, generator=g)
    og = torch.randn(B, 1, H, dv, generator=g).bfloat16()
    gamma = (torch.rand(dv, generator=g) + 0.5).bfloat16()
    gl = gdr.gate_activation(f.double(), A_log.double(), dt_bias.double().view(H, dk), None)
    o_ref, S_ref, c_ref = gdr.decode_step(qp, kp, vp, gl, beta.double(), S0.double(), ws, cs, scale=dk ** -0.5)
    o_ref = gdr.norm_gate(o_ref.to(torch.bfloat16).double(), og.double(), gamma.double(), 1e-6)
    dev = lambda t: t.cuda()
    S = dev(S0.clone())
    caches = tuple(dev(c.clone()) for c in cs)
    print(f'\n[case] fused decode dv256 B{B} H{H}, KDA gate in the kernel', flush=True)
    o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(f), dev(beta), S, scale=dk ** -0.5,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=caches, gate_in_kernel=True,
                            A_log=dev(A_log), dt_bias=dev(dt_bias), out_gate=dev(og), out_norm_weight=dev(gamma))
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    exact = all(torch.equal(a.cpu(), b) for a, b in zip(caches, c_ref))
    print(f'[parity] fused decode dv256 o={eo:.3e} S={es:.3e} caches exact={exact}', flush=True)
    assert eo <= 2e-2 and es <= 2e-2 and exact


@pytest.mark.gpu
def test_dv256_multi_token_conv_is_refused():
    """Only the one-token step runs at dv = 256 with the fused conv."""
    from test_decode_conv import _decode_inputs
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(2, 3, 2, 128, 256, 4, 'scalar', torch.bfloat16, seed=5)
    dev = lambda t: t.cuda()
    with pytest.raises(NotImplementedError, match='256'):
        ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), dev(S0), scale=0.1,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=tuple(dev(c) for c in cs))
