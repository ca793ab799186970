"""The layer's output epilogue RMSNorm(o) * SiLU(gate) (vgdr_epilogue;
linear_attention.py:814-825, norm_layer.py:15-24).

CPU: the oracle's norm_gate pinned against torch's own F.rms_norm x F.silu in
fp64, a constant row's closed form and scale invariance; the C ABI's argument
checks (no launch).
GPU: vgdr_norm_gate (the rms_norm_gated drop-in) and the decode step with the
epilogue fused into its output store, against the oracle at the 16-bit bar
rel_l2 <= 2e-2 (1e-5 for fp32), and the fused decode against the two-pass
form (decode, then vgdr_norm_gate) on the same inputs.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib

TOL = 2e-2


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


# --- the oracle (CPU) --------------------------------------------------------

def test_norm_gate_equals_torch_rms_norm_times_silu():
    g = torch.Generator().manual_seed(0)
    o = torch.randn(3, 5, 2, 128, generator=g, dtype=torch.float64)
    gate = torch.randn(3, 5, 2, 128, generator=g, dtype=torch.float64)
    gamma = torch.rand(128, generator=g, dtype=torch.float64) + 0.5
    ref = F.rms_norm(o, (128,), weight=gamma, eps=1e-6) * F.silu(gate)
    assert torch.allclose(gdr.norm_gate(o, gate, gamma, 1e-6), ref, rtol=1e-12, atol=1e-12)


def test_norm_gate_constant_row_and_scale_invariance():
    dv = 64
    gamma = torch.linspace(0.5, 2.0, dv, dtype=torch.float64)
    gate = torch.full((dv,), 40.0, dtype=torch.float64)          # silu(40) = 40 (1 - 4e-18)
    for c in (-3.0, 0.25, 7.0):
        out = gdr.norm_gate(torch.full((dv,), c, dtype=torch.float64), gate, gamma, 1e-6)
        want = torch.sign(torch.tensor(c)) * gamma * 40.0 / torch.sqrt(torch.tensor(1.0 + 1e-6 / c ** 2,
                                                                                      dtype=torch.float64))
        assert torch.allclose(out, want, rtol=1e-12, atol=0)
    g = torch.Generator().manual_seed(1)
    o = torch.randn(4, dv, generator=g, dtype=torch.float64)
    gt = torch.randn(4, dv, generator=g, dtype=torch.float64)
    a = gdr.norm_gate(o, gt, gamma, 1e-30)
    assert torch.allclose(gdr.norm_gate(37.5 * o, gt, gamma, 1e-30), a, rtol=1e-12, atol=1e-14)


def test_norm_gate_rounds_like_the_module_in_bf16():
    g = torch.Generator().manual_seed(2)
    o = torch.randn(64, 128, generator=g).bfloat16()
    gate = torch.randn(64, 128, generator=g).bfloat16()
    gamma = (torch.rand(128, generator=g) + 0.5).bfloat16()
    out = gdr.norm_gate(o, gate, gamma)
    assert out.dtype == torch.bfloat16
    assert _rel(out, gdr.norm_gate(o.double(), gate.double(), gamma.double())) < 1e-2


# --- C ABI argument checks (no launch) --------------------------------------

def test_epilogue_argument_checks():
    L = _lib.load()
    ok = _lib.Epilogue(gate=4096, gamma=8192, gamma_dtype=_lib.VGDR_BF16, eps=1e-6)
    assert L.vgdr_norm_gate(1, None, ctypes.byref(ok), None, 0, 128, None) == _lib.VGDR_OK   # no rows
    assert L.vgdr_norm_gate(1, None, None, None, 4, 128, None) == _lib.VGDR_ERR_INVALID
    assert L.vgdr_norm_gate(1, 4096, ctypes.byref(ok), 4096, 4, 96, None) == _lib.VGDR_ERR_UNSUPPORTED
    assert b'dv=96' in L.vgdr_last_error()
    assert L.vgdr_norm_gate(1, 4096, ctypes.byref(ok), 4096, 4, 1024, None) == _lib.VGDR_ERR_UNSUPPORTED
    assert L.vgdr_norm_gate(1, 4100, ctypes.byref(ok), 4096, 4, 128, None) == _lib.VGDR_ERR_INVALID
    for bad in (_lib.Epilogue(gate=None, gamma=8192, gamma_dtype=1, eps=1e-6),
                _lib.Epilogue(gate=4104, gamma=8192, gamma_dtype=1, eps=1e-6),       # alignment
                _lib.Epilogue(gate=4096, gamma=8192, gamma_dtype=2, eps=1e-6),       # bf16 o, fp16 gamma
                _lib.Epilogue(gate=4096, gamma=8192, gamma_dtype=1, eps=0.0)):
        assert L.vgdr_norm_gate(1, 4096, ctypes.byref(bad), 4096, 4, 128, None) == _lib.VGDR_ERR_INVALID
    bad = _lib.Epilogue(gate=4096, gamma=8192, gamma_dtype=1, eps=-1.0)
    rc = L.vgdr_recurrent_fwd_epilogue(1, 1, 1, 16, 32, 48, 64, 80, 96, None, None, None,
                                       1, 1, 4, 128, 128, 1, 1.0, None, ctypes.byref(bad), None)
    assert rc == _lib.VGDR_ERR_INVALID and b'eps' in L.vgdr_last_error()


# --- GPU ----------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('dv', [64, 128, 256])
@pytest.mark.parametrize('gamma_f32', [True, False])
def test_rms_norm_gated_matches_oracle(dtype, dv, gamma_f32):
    from vagus_amd import ops
    g = torch.Generator().manual_seed(dv)
    shape = (3, 37, 5, dv)                                  # 555 rows: not a multiple of the rows per wave
    o = (2.0 * torch.randn(*shape, generator=g)).to(dtype)
    gate = torch.randn(*shape, generator=g).to(dtype)
    gamma = (torch.rand(dv, generator=g) + 0.5).to(torch.float32 if gamma_f32 else dtype)
    print(f'\n[case] rms_norm_gated dtype={dtype} dv={dv} gamma_f32={gamma_f32}', flush=True)
    out = ops.rms_norm_gated(o.cuda(), gate.cuda(), gamma.cuda(), None, activation='swish', eps=1e-6)
    ref = gdr.norm_gate(o.double(), gate.double(), gamma.double(), 1e-6)
    tol = 1e-5 if dtype == torch.float32 else TOL
    err = _rel(out, ref)
    print(f'[parity] rms_norm_gated rel={err:.3e} (tol {tol:g})', flush=True)
    assert out.dtype == dtype and out.shape == o.shape
    assert err <= tol
    # the module's own rounding sequence (cast back to the input dtype between steps)
    assert _rel(out, gdr.norm_gate(o, gate, gamma.to(dtype), 1e-6)) <= (1e-5 if dtype == torch.float32 else TOL)


def _decode_inputs(B, T, H, dk, dv, gate, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).to(dtype)
    v = torch.randn(B, T, H, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gshape = (B, T, H, dk) if gate == 'vector' else (B, T, H)
    gl = F.logsigmoid(torch.randn(*gshape, generator=g) + 4.0)
    S0 = 0.1 * torch.randn(B, H, dk, dv, generator=g)
    og = torch.randn(B, T, H, dv, generator=g).to(dtype)
    gamma = (torch.rand(dv, generator=g) + 0.5)
    return q, k, v, gl, beta, S0, og, gamma


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('dv', [64, 128])
@pytest.mark.parametrize('T', [1, 6])
def test_decode_with_fused_epilogue(gate, dtype, dv, T):
    from vagus_amd import ops
    B, H, dk = 5, 3, 128
    q, k, v, gl, beta, S0, og, gamma = _decode_inputs(B, T, H, dk, dv, gate, dtype, seed=T * 7 + dv)
    print(f'\n[case] decode epilogue gate={gate} dtype={dtype} dv={dv} T={T}', flush=True)
    o_ref, S_ref = gdr.recurrent(q.double(), k.double(), v.double(), gl.double(), beta.double(), S0.double(),
                                 scale=dk ** -0.5)
    ref = gdr.norm_gate(o_ref.to(dtype).double(), og.double(), gamma.double(), 1e-6)
    dev = lambda t: t.cuda()
    S = dev(S0.clone())
    out, S_out = ops.hip_recurrent(dev(q), dev(k), dev(v), dev(gl), dev(beta), S, scale=dk ** -0.5, delta=True,
                                   inplace=True, out_gate=dev(og), out_norm_weight=dev(gamma), out_norm_eps=1e-6)
    assert S_out.data_ptr() == S.data_ptr()                       # the state was updated in place
    tol = 1e-5 if dtype == torch.float32 else TOL
    eo, es = _rel(out, ref), _rel(S, S_ref)
    # the two-pass form: the plain decode step, then the standalone epilogue
    o2, _ = ops.hip_recurrent(dev(q), dev(k), dev(v), dev(gl), dev(beta), dev(S0.clone()), scale=dk ** -0.5,
                              delta=True)
    two = ops.rms_norm_gated(o2, dev(og), dev(gamma), eps=1e-6)
    e2 = _rel(out, two)
    print(f'[parity] decode epilogue out={eo:.3e} S={es:.3e} vs two-pass={e2:.3e} (tol {tol:g})', flush=True)
    assert eo <= tol and es <= tol and e2 <= tol


@pytest.mark.gpu
def test_decode_epilogue_varlen_and_wide_dv():
    from vagus_amd import ops
    dev = lambda t: t.cuda()
    # packed segments, fused in the kernel
    q, k, v, gl, beta, _, og, gamma = _decode_inputs(1, 23, 2, 64, 128, 'scalar', torch.bfloat16, seed=5)
    cu = torch.tensor([0, 4, 4, 17, 23], dtype=torch.int32)
    S0 = 0.1 * torch.randn(4, 2, 64, 128, generator=torch.Generator().manual_seed(6))
    o_ref, _ = gdr.varlen(gdr.recurrent, q.double(), k.double(), v.double(), gl.double(), beta.double(),
                          S0.double(), cu, scale=0.125)
    ref = gdr.norm_gate(o_ref.to(torch.bfloat16).double(), og.double(), gamma.double(), 1e-5)
    out, _ = ops.hip_recurrent(dev(q), dev(k), dev(v), dev(gl), dev(beta), dev(S0), scale=0.125, delta=True,
                               cu_seqlens=dev(cu), out_gate=dev(og), out_norm_weight=dev(gamma), out_norm_eps=1e-5)
    e1 = _rel(out, ref)
    # dv = 256: two 128-column kernel calls, then the epilogue as its own pass over the whole row
    q, k, v, gl, beta, S0, og, gamma = _decode_inputs(2, 3, 2, 64, 256, 'vector', torch.bfloat16, seed=8)
    o_ref, _ = gdr.recurrent(q.double(), k.double(), v.double(), gl.double(), beta.double(), S0.double(),
                             scale=0.125)
    ref = gdr.norm_gate(o_ref.to(torch.bfloat16).double(), og.double(), gamma.double(), 1e-6)
    out, _ = ops.hip_recurrent(dev(q), dev(k), dev(v), dev(gl), dev(beta), dev(S0), scale=0.125, delta=True,
                               out_gate=dev(og), out_norm_weight=dev(gamma))
    e2 = _rel(out, ref)
    print(f'\n[parity] decode epilogue varlen={e1:.3e} dv256={e2:.3e}', flush=True)
    assert e1 <= TOL and e2 <= TOL


@pytest.mark.gpu
def test_epilogue_misuse_maps_to_reference_exceptions():
    from vagus_amd import ops
    x = torch.randn(4, 128, device='cuda').bfloat16()
    w = torch.ones(128, device='cuda')
    with pytest.raises(NotImplementedError):                 # only the reference's swish call
        ops.rms_norm_gated(x, x, w, activation='sigmoid')
    with pytest.raises(NotImplementedError):                 # gate in another dtype than o
        ops.rms_norm_gated(x, x.float(), w)
    with pytest.raises(AssertionError):                      # eps must be positive
        ops.rms_norm_gated(x, x, w, eps=0.0)
    with pytest.raises(AssertionError):                      # gamma (dv,) must match the gate's last dim
        ops.rms_norm_gated(x, x, torch.ones(64, device='cuda'))
    with pytest.raises(RuntimeError):                        # CPU tensors: no CPU implementation
        ops.rms_norm_gated(x.cpu(), x.cpu(), w.cpu())
