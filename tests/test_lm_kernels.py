"""The LM decode step's two small kernels around the layer kernels:
vgdr_scalar_gates (ops.scalar_gates; the scalar gate and the beta logits,
GatedDeltaNet._gates, linear_attention.py:719-721 and :734-735) and
vgdr_swiglu (ops.swiglu; the FFN's SiLU(x1) x xgate, infra/components/ffn.py:48-50).

CPU: the C ABI's argument checks (no launch).
GPU: against the module's own expressions run on the CPU with the same
weights (vagus_amd.layer.GatedDeltaNet._gates in fp32, and torch's
F.silu(a) * b in the dtype).  fp32: g, beta and the SwiGLU within 1e-5
relative.  16-bit: the projections are rounded to the dtype after a sum whose
order differs from the CPU GEMM's, so beta is within two units in the last
place of the dtype and g (a smooth function of it) within 2e-2 relative; the
SwiGLU within two units in the last place (its two roundings).  The decode
step of the LM runs both (tests/test_model.py, tests/test_lm_workload.py).
"""
import pytest
import torch
import torch.nn.functional as F

from vagus_amd import _lib


def test_scalar_gates_and_swiglu_argument_checks():
    L = _lib.load()

    def gates(**over):
        a = dict(dtype=1, x=4096, w=8192, na=12288, dt=16384, g=20480, b=24576, rows=4, dim=2048, H=16)
        a.update(over)
        return L.vgdr_scalar_gates(a['dtype'], a['x'], a['w'], a['na'], a['dt'], a['g'], a['b'], a['rows'],
                                   a['dim'], a['H'], None)
    assert gates(dtype=9) == _lib.VGDR_ERR_INVALID
    assert gates(dim=2044) == _lib.VGDR_ERR_UNSUPPORTED
    assert gates(H=0) == _lib.VGDR_ERR_INVALID
    assert gates(x=4100) == _lib.VGDR_ERR_INVALID
    assert gates(g=None) == _lib.VGDR_ERR_INVALID
    assert gates(rows=0, x=None, w=None, na=None, dt=None, g=None) == _lib.VGDR_OK

    def swiglu(**over):
        a = dict(dtype=1, x=4096, y=8192, rows=4, h=5632)
        a.update(over)
        return L.vgdr_swiglu(a['dtype'], a['x'], a['y'], a['rows'], a['h'], None)
    assert swiglu(h=5630) == _lib.VGDR_ERR_UNSUPPORTED
    assert swiglu(y=4096) == _lib.VGDR_ERR_INVALID
    assert b'alias' in L.vgdr_last_error()
    assert swiglu(x=None) == _lib.VGDR_ERR_INVALID
    assert swiglu(rows=0, x=None, y=None) == _lib.VGDR_OK


def _two_ulp(y, ref, dtype):
    y, ref = y.float().cpu(), ref.float().cpu()
    a = ref.abs().to(dtype)
    ulp = torch.nextafter(a, torch.full_like(a, float('inf'))).float() - a.float()
    return int(((y - ref).abs() > 2 * ulp).sum())


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('delta', [True, False])
@pytest.mark.parametrize('rows,dim,H', [(64, 2048, 16), (3, 96, 2), (130, 512, 5)])
def test_scalar_gates_match_the_module(dtype, delta, rows, dim, H):
    from vagus_amd import ops
    from vagus_amd.layer import GatedDeltaNet
    torch.manual_seed(rows + H)
    m = GatedDeltaNet(dim=dim, head_count=H, key_head_dim=64, value_head_dim=64, gate='scalar', delta=delta)
    x = torch.randn(rows, 1, dim).to(dtype)
    print(f'\n[case] scalar_gates dtype={dtype} delta={delta} rows={rows} dim={dim} H={H}', flush=True)
    with torch.no_grad():
        m = m.to(dtype)                                      # its projections round to the dtype on the CPU
        g_ref, b_ref = m._gates(x, raw_beta=True)
        w = torch.cat([m.wa.weight] + ([m.wb.weight] if delta else []))
        na = -m.A_log.float().exp()
        g, beta = ops.scalar_gates(x.cuda(), w.cuda(), na.cuda(), m.dt_bias.float().cuda(), with_beta=delta)
    eg = _rel(g, g_ref)
    if dtype == torch.float32:
        eb = _rel(beta, b_ref) if delta else 0.0
        print(f'[parity] scalar_gates g={eg:.2e} beta={eb:.2e}', flush=True)
        assert eg <= 1e-5 and eb <= 1e-5
    else:
        nb = _two_ulp(beta, b_ref, dtype) if delta else 0
        print(f'[parity] scalar_gates g={eg:.2e} beta beyond 2 ulp={nb}', flush=True)
        assert eg <= 2e-2 and nb == 0
    assert (beta is None) == (not delta)


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('rows,h', [(64, 5632), (7, 8), (300, 1000)])
def test_swiglu_matches_the_module(dtype, rows, h):
    from vagus_amd import ops
    g = torch.Generator().manual_seed(rows + h)
    x = (torch.randn(rows, 2 * h, generator=g) * 3).to(dtype)
    a, b = torch.chunk(x, 2, dim=-1)
    ref = F.silu(a) * b                                               # ffn.py:50 in the dtype
    print(f'\n[case] swiglu dtype={dtype} rows={rows} h={h}', flush=True)
    y = ops.swiglu(x.cuda())
    if dtype == torch.float32:
        e = _rel(y, ref)
        print(f'[parity] swiglu rel={e:.2e}', flush=True)
        assert e <= 1e-5
    else:
        n = _two_ulp(y, ref, dtype)
        frac = (y.cpu() != ref).float().mean().item()
        print(f'[parity] swiglu beyond 2 ulp={n} differing={frac:.2%}', flush=True)
        assert n == 0 and frac <= 0.01
