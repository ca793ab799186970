"""The decode step with the short conv fused (vgdr_decode_step,
vgdr_short_conv; linear_attention.py:918-952, opt.py:15-100).

CPU: the oracle's short_conv pinned against torch's F.conv1d on the
left-padded transpose (nn.Conv1d, the module's 'conv1d' path), a unit
impulse, and streaming (token-by-token calls threading the cache equal one
call); the oracle's decode_step against itself token by token; the C ABI's
argument checks (no launch).
GPU: hip_decode_step against the oracle's decode_step (fp64 recurrence fed
the oracle's producers) at rel_l2 <= 2e-2 for bf16 and 1e-5 for fp32, and the
advanced conv caches bit-exact (they are copies of inputs).
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

def test_short_conv_equals_conv1d_on_left_padded_input():
    g = torch.Generator().manual_seed(0)
    B, L, D, K = 2, 11, 6, 4
    x = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, 1, K, generator=g, dtype=torch.float64)
    y, cache = gdr.short_conv(x, w, None, activation=None)
    ref = F.conv1d(F.pad(x.transpose(1, 2), (K - 1, 0)), w, groups=D).transpose(1, 2)
    assert torch.allclose(y, ref, rtol=1e-12, atol=1e-12)
    assert torch.equal(cache, x[:, -K:])
    ys, _ = gdr.short_conv(x, w, None)
    assert torch.allclose(ys, F.silu(ref), rtol=1e-12, atol=1e-12)


def test_short_conv_impulse_returns_reversed_kernel():
    D, K = 3, 4
    w = torch.arange(1.0, D * K + 1, dtype=torch.float64).reshape(D, K)
    x = torch.zeros(1, 6, D, dtype=torch.float64)
    x[0, 0] = 1.0
    y, _ = gdr.short_conv(x, w, None, activation=None)
    for t in range(K):
        assert torch.equal(y[0, t], w[:, K - 1 - t])
    assert torch.equal(y[0, K:], torch.zeros(6 - K, D, dtype=torch.float64))


@pytest.mark.parametrize('K', [1, 2, 4])
def test_short_conv_streams_through_its_cache(K):
    g = torch.Generator().manual_seed(K)
    B, L, D = 2, 9, 5
    x = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, K, generator=g, dtype=torch.float64)
    c0 = torch.randn(B, K, D, generator=g, dtype=torch.float64)
    y_all, c_all = gdr.short_conv(x, w, c0)
    c, ys = c0, []
    for sl in (slice(0, 1), slice(1, 3), slice(3, 4), slice(4, 9)):      # calls shorter and longer than K
        y, c = gdr.short_conv(x[:, sl], w, c)
        ys.append(y)
    assert torch.allclose(torch.cat(ys, 1), y_all, rtol=1e-12, atol=1e-12)
    assert torch.equal(c, c_all)
    assert torch.equal(c_all, torch.cat([c0, x], 1)[:, -K:])


def _decode_inputs(B, L, H, dk, dv, K, gate, dtype, seed, w_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    qp = torch.randn(B, L, H * dk, generator=g).to(dtype)
    kp = torch.randn(B, L, H * dk, generator=g).to(dtype)
    vp = torch.randn(B, L, H * dv, generator=g).to(dtype)
    ws = tuple((0.5 * torch.randn(d, 1, K, generator=g)).to(w_dtype) for d in (H * dk, H * dk, H * dv))
    cs = tuple(torch.randn(B, K, d, generator=g).to(dtype) for d in (H * dk, H * dk, H * dv))
    beta = torch.sigmoid(torch.randn(B, L, H, generator=g))
    gl = F.logsigmoid(torch.randn(*((B, L, H, dk) if gate == 'vector' else (B, L, H)), generator=g) + 4.0)
    S0 = 0.1 * torch.randn(B, H, dk, dv, generator=g)
    return qp, kp, vp, ws, cs, gl, beta, S0


def test_oracle_decode_step_is_token_by_token_consistent():
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(2, 5, 2, 8, 4, 3, 'scalar', torch.float64, seed=1,
                                                      w_dtype=torch.float64)
    o_all, S_all, c_all = gdr.decode_step(qp, kp, vp, gl, beta.double(), S0.double(), ws, cs, scale=0.3)
    S, c, os_ = S0.double(), cs, []
    for t in range(5):
        o, S, c = gdr.decode_step(qp[:, t:t + 1], kp[:, t:t + 1], vp[:, t:t + 1], gl[:, t:t + 1],
                                  beta[:, t:t + 1].double(), S, ws, c, scale=0.3)
        os_.append(o)
    assert torch.allclose(torch.cat(os_, 1), o_all, rtol=1e-12, atol=1e-12)
    assert torch.allclose(S, S_all, rtol=1e-12, atol=1e-12)
    assert all(torch.equal(a, b) for a, b in zip(c, c_all))


# --- C ABI argument checks (no launch) --------------------------------------

def test_short_conv_argument_checks():
    L = _lib.load()

    def call(sc):
        return L.vgdr_decode_step(1, 1, 1, 16, 32, 48, 64, 80, 96, None, None, None,
                                  1, 1, 4, 128, 128, 1, 1.0, None, ctypes.byref(sc), None, None)
    good = dict(weight_q=256, weight_k=512, weight_v=768, cache_q=1024, cache_k=1280, cache_v=1536,
                kernel_size=4, weight_dtype=_lib.VGDR_F32)
    for k_, v_ in (('kernel_size', 0), ('kernel_size', 9)):
        assert call(_lib.ShortConv(**{**good, k_: v_})) == _lib.VGDR_ERR_UNSUPPORTED
    assert b'kernel_size' in L.vgdr_last_error()
    assert call(_lib.ShortConv(**{**good, 'cache_v': None})) == _lib.VGDR_ERR_INVALID
    assert call(_lib.ShortConv(**{**good, 'weight_dtype': _lib.VGDR_F16})) == _lib.VGDR_ERR_INVALID


def test_strided_decode_step_argument_checks():
    """vgdr_decode_step_strided refuses row strides below a dense row, and a call
    the decode kernel would not run (no conv), before touching a device."""
    L = _lib.load()

    def call(ld_qk, ld_v, sc, gp=None, gate_kind=1, h0=None):
        # q, k, v NULL: were a check below ever to pass, the common check refuses the call
        return L.vgdr_decode_step_strided(1, gate_kind, 1, None, None, None, None, None, None, h0, None,
                                          4, 16, 128, 128, ld_qk, ld_v, 1.0, None, sc, None, gp, None)
    assert call(1024, 8192, None) == _lib.VGDR_ERR_INVALID
    assert b'row strides' in L.vgdr_last_error()
    assert call(8192, 2047, None) == _lib.VGDR_ERR_INVALID
    assert call(8192, 8192, None) == _lib.VGDR_ERR_UNSUPPORTED
    assert b'four-tap' in L.vgdr_last_error()
    sc = _lib.ShortConv(weight_q=None, weight_k=None, weight_v=None, cache_q=None, cache_k=None, cache_v=None,
                        kernel_size=2, weight_dtype=_lib.VGDR_F32)
    assert call(8192, 8192, ctypes.byref(sc)) == _lib.VGDR_ERR_UNSUPPORTED
    # the gate projections: scalar gate only, their pointers, dim a multiple of 8 up to 4096 (bf16, dv 128)
    sc4 = _lib.ShortConv(weight_q=256, weight_k=512, weight_v=768, cache_q=1024, cache_k=1280, cache_v=1536,
                         kernel_size=4, weight_dtype=_lib.VGDR_F32)
    good = dict(x=4096, w=8192, neg_exp_a=12288, dt_bias=16384, dim=2048)
    h0 = 20480
    gp = _lib.GateProj(**good)
    assert call(8192, 8192, ctypes.byref(sc4), ctypes.byref(gp), gate_kind=2, h0=h0) == _lib.VGDR_ERR_UNSUPPORTED
    assert b'scalar gate' in L.vgdr_last_error()
    for k_, v_, err in (('x', None, _lib.VGDR_ERR_INVALID), ('w', 8200, _lib.VGDR_ERR_INVALID),
                        ('dim', 2044, _lib.VGDR_ERR_UNSUPPORTED), ('dim', 4104, _lib.VGDR_ERR_UNSUPPORTED)):
        gp = _lib.GateProj(**{**good, k_: v_})
        assert call(8192, 8192, ctypes.byref(sc4), ctypes.byref(gp), h0=h0) == err, (k_, v_)
    gp = _lib.GateProj(**good)                       # passes its checks, then q, k, v NULL are refused
    assert call(8192, 8192, ctypes.byref(sc4), ctypes.byref(gp), h0=h0) == _lib.VGDR_ERR_INVALID
    assert b'q, k, v and o are required' in L.vgdr_last_error()


# --- GPU ----------------------------------------------------------------------

def _run(gate, dtype, K, L, epilogue, w_dtype, seed, B=4, H=2, dk=128, dv=64):
    from vagus_amd import ops
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(B, L, H, dk, dv, K, gate, dtype, seed, w_dtype)
    g = torch.Generator().manual_seed(seed + 100)
    og = torch.randn(B, L, H, dv, generator=g).to(dtype)
    gamma = torch.rand(dv, generator=g) + 0.5
    print(f'\n[case] decode conv gate={gate} dtype={dtype} K={K} L={L} epilogue={epilogue} w={w_dtype}', flush=True)
    o_ref, S_ref, c_ref = gdr.decode_step(qp, kp, vp, gl.double(), beta.double(), S0.double(), ws, cs,
                                          scale=dk ** -0.5)
    if epilogue:
        o_ref = gdr.norm_gate(o_ref.to(dtype).double(), og.double(), gamma.double(), 1e-6)
    dev = lambda t: t.cuda()
    S = dev(S0.clone())
    caches = tuple(dev(c.clone()) for c in cs)
    o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), S, scale=dk ** -0.5,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=caches,
                            out_gate=dev(og) if epilogue else None, out_norm_weight=dev(gamma) if epilogue else None)
    tol = 1e-5 if dtype == torch.float32 else TOL
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    exact = all(torch.equal(a.cpu(), b) for a, b in zip(caches, c_ref))
    print(f'[parity] decode conv o={eo:.3e} S={es:.3e} caches exact={exact} (tol {tol:g})', flush=True)
    assert eo <= tol and es <= tol and exact


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('L', [1, 3, 6])
@pytest.mark.parametrize('K', [4, 2])
def test_decode_step_conv_matches_oracle(dtype, L, K):
    _run('scalar', dtype, K, L, epilogue=False, w_dtype=torch.float32, seed=L * 10 + K)


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_decode_step_conv_with_epilogue(gate):
    _run(gate, torch.bfloat16, 4, 1, epilogue=True, w_dtype=torch.bfloat16, seed=7)


@pytest.mark.gpu
def test_decode_step_conv_varlen():
    from vagus_amd import ops
    H, dk, dv, K = 2, 64, 128, 4
    cu = torch.tensor([0, 1, 1, 3, 8], dtype=torch.int32)      # lengths 1, 0, 2, 5
    N, T = 4, 8
    qp, kp, vp, ws, _, gl, beta, _ = _decode_inputs(1, T, H, dk, dv, K, 'scalar', torch.bfloat16, seed=21)
    g = torch.Generator().manual_seed(22)
    cs = tuple(torch.randn(N, K, d, generator=g).bfloat16() for d in (H * dk, H * dk, H * dv))
    S0 = 0.1 * torch.randn(N, H, dk, dv, generator=g)
    print('\n[case] decode conv varlen', flush=True)
    os_, Ss, cref = [], [], [[], [], []]
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        o, S, c = gdr.decode_step(qp[:, a:b], kp[:, a:b], vp[:, a:b], gl[:, a:b].double(), beta[:, a:b].double(),
                                  S0[n:n + 1].double(), ws, tuple(x[n:n + 1] for x in cs), scale=dk ** -0.5)
        os_.append(o)
        Ss.append(S)
        for i in range(3):
            cref[i].append(c[i])
    o_ref, S_ref = torch.cat(os_, 1), torch.cat(Ss, 0)
    dev = lambda t: t.cuda()
    S = dev(S0.clone())
    caches = tuple(dev(c.clone()) for c in cs)
    o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), S, scale=dk ** -0.5,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=caches, cu_seqlens=dev(cu))
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    exact = all(torch.equal(a.cpu(), torch.cat(b, 0)) for a, b in zip(caches, cref))
    print(f'[parity] decode conv varlen o={eo:.3e} S={es:.3e} caches exact={exact}', flush=True)
    assert eo <= TOL and es <= TOL and exact


@pytest.mark.gpu
def test_decode_step_conv_misuse():
    from vagus_amd import ops
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(2, 1, 2, 96, 64, 4, 'scalar', torch.bfloat16, seed=3)
    dev = lambda t: t.cuda()
    with pytest.raises(NotImplementedError):                 # dk = 96 would need padding
        ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), dev(S0), scale=0.1,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=tuple(dev(c) for c in cs))
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(2, 1, 2, 64, 64, 4, 'scalar', torch.bfloat16, seed=3)
    with pytest.raises(AssertionError):                      # caches are updated in place: q's dtype
        ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), dev(S0), scale=0.1,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=tuple(dev(c.float()) for c in cs))


@pytest.mark.gpu
def test_decode_step_at_lm_layer_shape():
    """The one-token step exactly as the 1.3B LM's layers call it (B64 H16
    dk=dv=128, K4, bf16 projections and weights, the L2 norm, beta from its
    logits, the scalar gate, the RMSNorm x SiLU(gate) epilogue): decode_conv_kernel<128, 128>
    against the oracle's decode_step + norm_gate in fp64."""
    from vagus_amd import ops
    B, H, dk, dv, K = 64, 16, 128, 128, 4
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(B, 1, H, dk, dv, K, 'scalar', torch.bfloat16, seed=41,
                                                      w_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(42)
    blog = torch.randn(B, 1, H, generator=g)                   # beta logits
    og = torch.randn(B, 1, H, dv, generator=g).bfloat16()
    gamma = (torch.rand(dv, generator=g) + 0.5).bfloat16()
    print(f'\n[case] decode step at the LM layer shape B{B} H{H} dk={dk} dv={dv}', flush=True)
    o_ref, S_ref, c_ref = gdr.decode_step(qp, kp, vp, gl.double(), torch.sigmoid(blog).double(), S0.double(), ws, cs,
                                          scale=dk ** -0.5)
    o_ref = gdr.norm_gate(o_ref.to(torch.bfloat16).double(), og.double(), gamma.double(), 1e-6)
    dev = lambda t: t.cuda()
    S = dev(S0.clone())
    caches = tuple(dev(c.clone()) for c in cs)
    o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), dev(gl), dev(blog), S, scale=dk ** -0.5,
                            conv_weights=tuple(dev(w) for w in ws), conv_cache=caches, l2norm=True,
                            beta_logits=True, out_gate=dev(og), out_norm_weight=dev(gamma))
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    exact = all(torch.equal(a.cpu(), b) for a, b in zip(caches, c_ref))
    print(f'[parity] LM-shape decode step o={eo:.3e} S={es:.3e} caches exact={exact} (tol {TOL:g})', flush=True)
    assert eo <= TOL and es <= TOL and exact


@pytest.mark.gpu
@pytest.mark.parametrize('dk,dv,gate,epilogue', [(128, 128, 'scalar', True), (64, 64, 'scalar', False),
                                                 (128, 256, 'scalar', True), (128, 128, 'vector', True)])
def test_decode_step_reads_projection_rows_in_place(dk, dv, gate, epilogue):
    """q, k, v and the output gate as column blocks of one (B, 1, 2 H dk + 2 H dv)
    projection output, as the layer's concatenated GEMM leaves them: the kernel
    reads the rows in place (vgdr_decode_step_strided) and gives exactly what it
    gives on dense copies of the same values (o, the state and the conv caches
    bit-exact), which is within the tolerance of the oracle's decode step."""
    from vagus_amd import ops
    B, H, K = 16, 4, 4
    qp, kp, vp, ws, cs, gl, beta, S0 = _decode_inputs(B, 1, H, dk, dv, K, gate, torch.bfloat16, seed=51,
                                                      w_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(52)
    og = torch.randn(B, 1, H * dv, generator=g).bfloat16()
    gamma = (torch.rand(dv, generator=g) + 0.5).bfloat16()
    print(f'\n[case] strided decode step dk={dk} dv={dv} gate={gate} epilogue={epilogue}', flush=True)
    dev = lambda t: t.cuda()
    y = dev(torch.cat([qp.reshape(B, 1, -1), kp.reshape(B, 1, -1), vp.reshape(B, 1, -1), og], -1))
    a, b_, c_ = H * dk, 2 * H * dk, 2 * H * dk + H * dv
    views = (y[..., :a], y[..., a:b_], y[..., b_:c_], y[..., c_:])
    assert all(not t.is_contiguous() for t in views)

    def step(q_, k_, v_, og_):
        S = dev(S0.clone())
        caches = tuple(dev(c.clone()) for c in cs)
        o = ops.hip_decode_step(q_, k_, v_, dev(gl), dev(beta), S, scale=dk ** -0.5,
                                conv_weights=tuple(dev(w) for w in ws), conv_cache=caches,
                                out_gate=og_ if epilogue else None, out_norm_weight=dev(gamma) if epilogue else None)
        torch.cuda.synchronize()
        return o, S, caches

    o1, S1, c1 = step(*views)
    o2, S2, c2 = step(*(t.contiguous() for t in views))
    same = torch.equal(o1, o2) and torch.equal(S1, S2) and all(torch.equal(x1, x2) for x1, x2 in zip(c1, c2))
    o_ref, S_ref, _ = gdr.decode_step(qp, kp, vp, gl.double(), beta.double(), S0.double(), ws, cs, scale=dk ** -0.5)
    if epilogue:
        o_ref = gdr.norm_gate(o_ref.to(torch.bfloat16).double(), og.reshape(B, 1, H, dv).double(),
                              gamma.double(), 1e-6)
    eo, es = _rel(o1, o_ref), _rel(S1, S_ref)
    print(f'[parity] strided decode step: equal to dense={same}, o={eo:.3e} S={es:.3e} (tol {TOL:g})', flush=True)
    assert same and eo <= TOL and es <= TOL



@pytest.mark.gpu
@pytest.mark.parametrize('dv,delta', [(128, True), (256, True), (128, False)])
def test_decode_step_forms_the_scalar_gate_in_kernel(dv, delta):
    """gate_proj: the decode kernel forms g = -exp(A_log) softplus(W_a x + dt_bias)
    and the beta logits W_b x from the layer's input row itself (one kernel less
    per layer), as the separate gate kernel does (vgdr_scalar_gates: the same
    roundings; only the order of the fp32 sums over dim differs).  Checked
    against the step fed that kernel's g and beta, and against the oracle."""
    from vagus_amd import ops
    B, H, dk, K, dim = 16, 4, 128, 4, 2048
    qp, kp, vp, ws, cs, _, _, S0 = _decode_inputs(B, 1, H, dk, dv, K, 'scalar', torch.bfloat16, seed=61,
                                                  w_dtype=torch.bfloat16)
    g_ = torch.Generator().manual_seed(62)
    x = torch.randn(B, 1, dim, generator=g_).bfloat16()
    wab = (0.02 * torch.randn((2 if delta else 1) * H, dim, generator=g_)).bfloat16()
    neg_a = -torch.exp(torch.rand(H, generator=g_) * 2.0 - 1.0)
    dt_bias = torch.randn(H, generator=g_) * 0.5
    print(f'\n[case] in-kernel scalar gate dv={dv} delta={delta}', flush=True)
    dev = lambda t: t.cuda()

    def step(gp):
        S = dev(S0.clone())
        caches = tuple(dev(c.clone()) for c in cs)
        if gp:
            g, beta, proj = None, None, (dev(x), dev(wab), dev(neg_a), dev(dt_bias))
        else:
            g, beta = ops.scalar_gates(dev(x), dev(wab), dev(neg_a), dev(dt_bias), with_beta=delta)
            proj = None
        o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), g, beta, S, scale=dk ** -0.5, delta=delta,
                                conv_weights=tuple(dev(w) for w in ws), conv_cache=caches, beta_logits=delta,
                                gate_proj=proj)
        torch.cuda.synchronize()
        return o, S, caches, g, beta

    o1, S1, c1, _, _ = step(True)
    o2, S2, c2, g2, b2 = step(False)
    d_o, d_s = _rel(o1, o2), _rel(S1, S2)
    caches_same = all(torch.equal(a, b) for a, b in zip(c1, c2))
    # the oracle fed the gate kernel's g and beta (that kernel is checked against the module's _gates)
    o_ref, S_ref, _ = gdr.decode_step(qp, kp, vp, g2.cpu().double(),
                                      torch.sigmoid(b2.cpu().double()) if delta else None, S0.double(), ws, cs,
                                      scale=dk ** -0.5, delta=delta)
    eo, es = _rel(o1, o_ref), _rel(S1, S_ref)
    print(f'[parity] in-kernel gate vs gate kernel: o {d_o:.2e} S {d_s:.2e} caches equal={caches_same}; '
          f'vs oracle o {eo:.3e} S {es:.3e} (tol {TOL:g})', flush=True)
    assert d_o <= 1e-3 and d_s <= 1e-3 and caches_same and eo <= TOL and es <= TOL


@pytest.mark.gpu
def test_decode_step_gate_proj_falls_back_beyond_the_kernel_row():
    """A gate projection row longer than the decode kernel holds (dim 8192 > 4096
    at dv = 128) is formed by the gate kernel first: the step then equals the one
    fed that kernel's g and beta exactly."""
    from vagus_amd import ops
    B, H, dk, dv, K, dim = 8, 2, 64, 128, 4, 8192
    qp, kp, vp, ws, cs, _, _, S0 = _decode_inputs(B, 1, H, dk, dv, K, 'scalar', torch.bfloat16, seed=71,
                                                  w_dtype=torch.bfloat16)
    g_ = torch.Generator().manual_seed(72)
    x = torch.randn(B, 1, dim, generator=g_).bfloat16()
    wab = (0.01 * torch.randn(2 * H, dim, generator=g_)).bfloat16()
    neg_a, dt_bias = -torch.rand(H, generator=g_) - 0.5, torch.randn(H, generator=g_) * 0.5
    print('\n[case] gate projections beyond the kernel row (dim 8192)', flush=True)
    dev = lambda t: t.cuda()
    outs = []
    for gp in (True, False):
        S = dev(S0.clone())
        caches = tuple(dev(c.clone()) for c in cs)
        if gp:
            g, beta, proj = None, None, (dev(x), dev(wab), dev(neg_a), dev(dt_bias))
        else:
            g, beta = ops.scalar_gates(dev(x), dev(wab), dev(neg_a), dev(dt_bias))
            proj = None
        o = ops.hip_decode_step(dev(qp), dev(kp), dev(vp), g, beta, S, scale=dk ** -0.5, beta_logits=True,
                                conv_weights=tuple(dev(w) for w in ws), conv_cache=caches, gate_proj=proj)
        outs.append((o, S))
    same = torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    print(f'[parity] fallback equal={same}', flush=True)
    assert same
