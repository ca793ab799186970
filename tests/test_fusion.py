"""Producer fusions (vgdr_fusion; the fla flags of linear_attention.py:457-497).

CPU: the oracle's producers pinned by their defining properties.
GPU: the fused kernels against the fp64 oracle fed with the oracle's activated
inputs (q, k L2-normalised and rounded to bf16, beta = sigmoid(logits),
per-channel g = the reference's activation of the pre-activation f), at the
bf16 bar rel_l2 <= 2e-2, and against the unfused kernels on the same activated
inputs; the reference's misuse / unsupported cases map to its exception types.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdr

TOL = 2e-2


# --- the oracle's producers (CPU) ------------------------------------------

def test_l2norm_unit_rows_and_scale_invariance():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 2, 64, generator=gen, dtype=torch.float64)
    y = gdr.l2norm(x)
    assert torch.allclose(y.norm(dim=-1), torch.ones(3, 5, 2, dtype=torch.float64), atol=1e-6)
    assert torch.allclose(gdr.l2norm(7.5 * x), y, atol=1e-9)
    assert gdr.l2norm(torch.zeros(4, 8)).abs().max() == 0            # eps keeps zero rows at zero
    yb = gdr.l2norm(x.to(torch.bfloat16))
    assert yb.dtype == torch.bfloat16                                # rounded back to the input type


def test_gate_activation_identities():
    H, dk = 3, 8
    gen = torch.Generator().manual_seed(2)
    f = torch.randn(2, 4, H, dk, generator=gen, dtype=torch.float64)
    A_log = torch.randn(H, generator=gen, dtype=torch.float64)
    dt = torch.randn(H * dk, generator=gen, dtype=torch.float64)
    g = gdr.gate_activation(f, A_log, dt)
    z = f + dt.view(H, dk)
    # softplus(z) = log(1 + e^z) and the decay is a = exp(g) = (1 + e^z)^(-exp(A_log))
    a = torch.exp(A_log)[:, None]
    assert torch.allclose(torch.exp(g), (1 + torch.exp(z)) ** (-a), rtol=1e-12)
    assert (g <= 0).all()
    # f -> -inf: no decay (g -> 0); a large f: g ~ -exp(A_log) (f + dt)
    big = gdr.gate_activation(torch.full_like(f, 60.0), A_log, dt)
    assert torch.allclose(big, -a * (60.0 + dt.view(H, dk)), rtol=1e-12)
    small = gdr.gate_activation(torch.full_like(f, -60.0), A_log, dt)
    assert small.abs().max() < 1e-20
    # the bounded form: lower_bound * sigmoid(exp(A_log) z), inside (lower_bound, 0); z = 0 gives lb / 2
    lb = -5.0
    gb = gdr.gate_activation(f, A_log, dt, lower_bound=lb)
    assert ((gb > lb) & (gb < 0)).all()
    zero = gdr.gate_activation(-dt.view(1, 1, H, dk).expand_as(f), A_log, dt, lower_bound=lb)
    assert torch.allclose(zero, torch.full_like(f, lb / 2))


def test_beta_sigmoid():
    b = torch.tensor([0.0, 2.0, -3.0], dtype=torch.bfloat16)
    s = gdr.beta_sigmoid(b)
    assert s.dtype == torch.float32
    assert torch.allclose(s, torch.tensor([0.5, 1 / (1 + math.exp(-2.0)), 1 / (1 + math.exp(3.0))]), atol=1e-6)


# --- fused kernels (GPU) -------------------------------------------------------

def _raw_inputs(B, T, H, dk, dv, gate, seed, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    raw = dict(q=(3 * r(B, T, H, dk)).to(dtype), k=(2 * r(B, T, H, dk)).to(dtype), v=r(B, T, H, dv).to(dtype),
               b=r(B, T, H).to(dtype), S0=0.1 * r(B, H, dk, dv))
    if gate == 'vector':
        raw['f'] = (r(B, T, H, dk) - 1.0).to(dtype)
        raw['A_log'] = 0.3 * r(H)
        raw['dt_bias'] = 0.5 * r(H * dk)
    else:
        raw['g'] = F.logsigmoid(r(B, T, H) + 3.0)
    return raw


def _activated(raw, gate, lower_bound=None):
    """The oracle's producers: what the unfused reference path hands the scan."""
    q, k = gdr.l2norm(raw['q']), gdr.l2norm(raw['k'])
    beta = gdr.beta_sigmoid(raw['b'])
    if gate == 'vector':
        g = gdr.gate_activation(raw['f'], raw['A_log'], raw['dt_bias'], lower_bound)
    else:
        g = raw['g']
    return q, k, raw['v'], g, beta, raw['S0']


def _rel(x, ref):
    x, ref = x.detach().double().cpu(), ref.detach().double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('lower_bound', [None, -5.0])
@pytest.mark.parametrize('dk', [64, 128])
def test_chunk_fused_producers_match_oracle(gate, lower_bound, dk):
    from vagus_amd import ops
    if gate == 'scalar' and lower_bound is not None:
        pytest.skip('the bounded activation belongs to the per-channel gate')
    B, T, H, dv = 2, 200, 3, 64
    raw = _raw_inputs(B, T, H, dk, dv, gate, seed=dk + (lower_bound is not None))
    q, k, v, g, beta, S0 = _activated(raw, gate, lower_bound)
    print(f'\n[case] fused chunk gate={gate} lower_bound={lower_bound} dk={dk}', flush=True)
    ref = gdr.recurrent(q.double(), k.double(), v.double(), g.double(), beta.double(), S0.double(),
                        scale=dk ** -0.5)
    dev = lambda t: t.cuda()
    if gate == 'vector':
        o, S = ops.chunk_kda(dev(raw['q']), dev(raw['k']), dev(raw['v']), dev(raw['f']), dev(raw['b']),
                             scale=dk ** -0.5, initial_state=dev(S0), output_final_state=True,
                             use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                             use_gate_in_kernel=True, A_log=dev(raw['A_log']), dt_bias=dev(raw['dt_bias']),
                             safe_gate=lower_bound is not None, lower_bound=lower_bound)
        o2, S2 = ops.chunk_kda(dev(q), dev(k), dev(v), dev(g), dev(beta), scale=dk ** -0.5,
                               initial_state=dev(S0), output_final_state=True)
    else:
        o, S = ops.chunk_gated_delta_rule(dev(raw['q']), dev(raw['k']), dev(raw['v']), dev(raw['g']),
                                          dev(raw['b']), scale=dk ** -0.5, initial_state=dev(S0),
                                          output_final_state=True, use_qk_l2norm_in_kernel=True,
                                          use_beta_sigmoid_in_kernel=True)
        o2, S2 = ops.chunk_gated_delta_rule(dev(q), dev(k), dev(v), dev(g), dev(beta), scale=dk ** -0.5,
                                            initial_state=dev(S0), output_final_state=True)
    eo, es = _rel(o, ref[0]), _rel(S, ref[1])
    print(f'[parity] fused vs oracle o={eo:.3e} S={es:.3e}; fused vs unfused o={_rel(o, o2):.3e} '
          f'S={_rel(S, S2):.3e}', flush=True)
    assert eo <= TOL and es <= TOL
    assert _rel(o, o2) <= TOL and _rel(S, S2) <= TOL


@pytest.mark.gpu
def test_chunk_fused_varlen_and_gate_in_fp32():
    from vagus_amd import ops
    H, dk, dv = 2, 128, 128
    lens = [1, 64, 65, 130, 0, 37]
    T = sum(lens)
    raw = _raw_inputs(1, T, H, dk, dv, 'vector', seed=5)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    S0 = 0.1 * torch.randn(len(lens), H, dk, dv, generator=torch.Generator().manual_seed(6))
    q, k, v, g, beta, _ = _activated(raw, 'vector')
    print('\n[case] fused varlen KDA, fp32 gate pre-activation', flush=True)
    ref = gdr.varlen(gdr.recurrent, q.double(), k.double(), v.double(), g.double(), beta.double(), S0.double(), cu,
                     scale=dk ** -0.5)
    dev = lambda t: t.cuda()
    o, S = ops.chunk_kda(dev(raw['q']), dev(raw['k']), dev(raw['v']), dev(raw['f'].float()), dev(raw['b']),
                         scale=dk ** -0.5, initial_state=dev(S0), output_final_state=True, cu_seqlens=dev(cu),
                         use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True, use_gate_in_kernel=True,
                         A_log=dev(raw['A_log']), dt_bias=dev(raw['dt_bias']))
    eo, es = _rel(o, ref[0]), _rel(S, ref[1])
    print(f'[parity] fused varlen o={eo:.3e} S={es:.3e}', flush=True)
    assert eo <= TOL and es <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_recurrent_fused_producers_match_oracle(gate, dtype):
    from vagus_amd import ops
    B, T, H, dk, dv = 3, 9, 2, 128, 64
    raw = _raw_inputs(B, T, H, dk, dv, gate, seed=11, dtype=dtype)
    q, k, v, g, beta, S0 = _activated(raw, gate)
    print(f'\n[case] fused recurrent gate={gate} dtype={dtype}', flush=True)
    ref = gdr.recurrent(q.double(), k.double(), v.double(), g.double(), beta.double(), S0.double(),
                        scale=dk ** -0.5)
    dev = lambda t: t.cuda()
    if gate == 'vector':
        o, S = ops.fused_recurrent_kda(dev(raw['q']), dev(raw['k']), dev(raw['v']), dev(raw['f']), dev(raw['b']),
                                       scale=dk ** -0.5, initial_state=dev(S0), output_final_state=True,
                                       use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                                       use_gate_in_kernel=True, A_log=dev(raw['A_log']), dt_bias=dev(raw['dt_bias']))
    else:
        o, S = ops.fused_recurrent_gated_delta_rule(dev(raw['q']), dev(raw['k']), dev(raw['v']), dev(raw['g']),
                                                    dev(raw['b']), scale=dk ** -0.5, initial_state=dev(S0),
                                                    output_final_state=True, use_qk_l2norm_in_kernel=True,
                                                    use_beta_sigmoid_in_kernel=True)
    tol = 1e-5 if dtype == torch.float32 else TOL
    eo, es = _rel(o, ref[0]), _rel(S, ref[1])
    print(f'[parity] fused recurrent o={eo:.3e} S={es:.3e} (tol {tol:g})', flush=True)
    assert eo <= tol and es <= tol


@pytest.mark.gpu
def test_fused_misuse_maps_to_reference_exceptions():
    from vagus_amd import ops
    raw = _raw_inputs(1, 8, 1, 64, 64, 'scalar', seed=3)
    dev = lambda t: t.cuda()
    q, k, v, g, b = (dev(raw[n]) for n in ('q', 'k', 'v', 'g', 'b'))
    with pytest.raises(AssertionError):                      # the fused gate is the per-channel gate's
        ops.hip_scan(q, k, v, g, b, None, scale=0.125, delta=True, gate_in_kernel=True,
                     A_log=torch.zeros(1, device='cuda'), dt_bias=torch.zeros(64, device='cuda'))
    with pytest.raises(AssertionError):                      # simple_gla takes no fused l2norm / beta
        ops.hip_scan(q, k, v, g, None, None, scale=0.125, delta=False, l2norm_in_kernel=True)
    with pytest.raises(NotImplementedError):                 # fused producers take 16-bit q, k, v
        ops.chunk_gated_delta_rule(q.float(), k.float(), v.float(), g, b.float(), use_qk_l2norm_in_kernel=True)
