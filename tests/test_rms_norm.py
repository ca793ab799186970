"""The pre-norm blocks' RMSNorm with the residual add in front of it
(vgdr_rms_norm, ops.rms_norm; RMSNorm, infra/components/norm_layer.py:15-23,
and the adds of infra/components/block.py:57-59, :85-87), which the LM's
decode step and packed prefill run once per norm.

CPU: the oracle's rms_norm against torch's F.rms_norm in fp64 (the same
closed form: a dropped mean, a wrong eps or a missing gamma fails it) and the
module's RMSNorm in bf16 (the oracle keeps the module's two roundings); the C
ABI's argument checks (no launch).
GPU: against the oracle on the same inputs.  The residual sum x + residual is
bit-exact (one rounding of the float sum, as torch's add).  The norm: fp32
within 1e-6 relative; 16-bit within two units in the last place of each
element, at most 1% of the elements differing (the mean's summation order
differs from torch's, which moves the fp32 scale by a few ulps and can flip
the first of the expression's two roundings, which gamma then scales).
Row widths cover one to eight 16-byte units per thread and a partial last
pass; the in-place update of the residual stream (out_residual = x).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import model as om
from vagus_amd import _lib


def test_oracle_rms_norm_is_the_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 96, generator=g, dtype=torch.float64) * 3
    gamma = torch.rand(96, generator=g, dtype=torch.float64) + 0.5
    ref = F.rms_norm(x, (96,), weight=gamma, eps=1e-6)
    assert torch.allclose(om.rms_norm(x, gamma, 1e-6), ref, rtol=1e-13, atol=0)
    # a constant row: x / sqrt(x^2 + eps) * gamma
    c = torch.full((1, 96), 2.0, dtype=torch.float64)
    assert torch.allclose(om.rms_norm(c, gamma, 0.25), 2.0 / (4.25 ** 0.5) * gamma, rtol=1e-14)


def test_oracle_rms_norm_matches_the_module_in_bf16():
    from vagus_amd.layer import RMSNorm
    g = torch.Generator().manual_seed(1)
    m = RMSNorm(256).bfloat16()
    with torch.no_grad():
        m.gamma.copy_((torch.rand(256, generator=g) + 0.5).bfloat16())
    x = torch.randn(9, 256, generator=g).bfloat16()
    assert torch.equal(om.rms_norm(x, m.gamma.detach(), m.eps), m(x).detach())


def test_rms_norm_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, x=4096, r=None, xo=None, w=8192, y=12288, rows=4, dim=2048, eps=1e-6)
        a.update(over)
        return L.vgdr_rms_norm(a['dtype'], a['x'], a['r'], a['xo'], a['w'], a['y'], a['rows'], a['dim'], a['eps'],
                               None)
    assert call(dtype=7) == _lib.VGDR_ERR_INVALID
    assert call(dim=2044) == _lib.VGDR_ERR_UNSUPPORTED               # 16-bit rows in 8-element units
    assert call(dim=8 * 2049) == _lib.VGDR_ERR_UNSUPPORTED           # more than 2048 units
    assert call(dtype=0, dim=4 * 2049) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(y=4096) == _lib.VGDR_ERR_INVALID                     # y aliasing x
    assert b'alias' in L.vgdr_last_error()
    assert call(r=16384, xo=12288) == _lib.VGDR_ERR_INVALID          # y aliasing x_out
    assert call(x=4100) == _lib.VGDR_ERR_INVALID                     # alignment
    assert call(w=None) == _lib.VGDR_ERR_INVALID
    assert call(eps=-1.0) == _lib.VGDR_ERR_INVALID
    assert call(rows=0, x=None, w=None, y=None) == _lib.VGDR_OK      # nothing to do


def _ulp_close(y, ref, dtype):
    y, ref = y.float().cpu(), ref.float().cpu()
    if dtype == torch.float32:
        err = ((y - ref).norm() / ref.norm()).item()
        return err <= 1e-6, f'rel_l2={err:.2e}'
    # the spacing of the dtype at each reference value (subnormals included)
    a = ref.abs().to(dtype)
    ulp = (torch.nextafter(a, torch.full_like(a, float('inf'))).float() - a.float())
    bad = (y - ref).abs() > 2 * ulp
    frac = (y != ref).float().mean().item()
    return (not bool(bad.any())) and frac <= 0.01, f'differing={frac:.2%} beyond-2ulp={int(bad.sum())}'


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('rows,dim', [(64, 2048), (3, 64), (1000, 96), (2, 16384 // 2), (5, 2056)])
@pytest.mark.parametrize('residual', [False, True])
def test_rms_norm_matches_oracle(dtype, rows, dim, residual):
    from vagus_amd import ops
    if dtype == torch.float32 and dim * 4 > 16 * 2048:
        pytest.skip('wider than 2048 16-byte units')
    g = torch.Generator().manual_seed(rows + dim)
    x = (torch.randn(rows, dim, generator=g) * 2).to(dtype)
    r = torch.randn(rows, dim, generator=g).to(dtype) if residual else None
    gamma = (torch.rand(dim, generator=g) + 0.5).to(dtype)
    print(f'\n[case] rms_norm dtype={dtype} rows={rows} dim={dim} residual={residual}', flush=True)
    h_ref = (x + r) if residual else x
    ref = om.rms_norm(h_ref, gamma, 1e-6)
    xd = x.cuda()
    if residual:
        y, h = ops.rms_norm(xd, gamma.cuda(), 1e-6, residual=r.cuda())
        assert torch.equal(h.cpu(), h_ref)
        assert torch.equal(xd.cpu(), x)                              # x untouched without out_residual
    else:
        y = ops.rms_norm(xd, gamma.cuda(), 1e-6)
    ok, msg = _ulp_close(y, ref, dtype)
    print(f'[parity] rms_norm {msg}', flush=True)
    assert ok, msg


@pytest.mark.gpu
def test_rms_norm_updates_the_stream_in_place():
    from vagus_amd import ops
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 1, 2048, generator=g).bfloat16()
    d = torch.randn(64, 1, 2048, generator=g).bfloat16()
    gamma = (torch.rand(2048, generator=g) + 0.5).bfloat16()
    xd = x.cuda()
    y, h = ops.rms_norm(xd, gamma.cuda(), 1e-6, residual=d.cuda(), out_residual=xd)
    assert h.data_ptr() == xd.data_ptr()
    assert torch.equal(xd.cpu(), x + d)
    ok, msg = _ulp_close(y, om.rms_norm(x + d, gamma, 1e-6), torch.bfloat16)
    print(f'[parity] rms_norm in place {msg}', flush=True)
    assert ok, msg
