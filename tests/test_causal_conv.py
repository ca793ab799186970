"""The prefill short conv + SiLU (vgdr_causal_conv1d; ShortConv, opt.py:15-100;
fla's causal_conv1d as the reference calls it, :73-77).

CPU: the C ABI's argument checks (no launch).  The oracle's short_conv is
pinned in tests/test_decode_conv.py (F.conv1d, impulse, streaming).
GPU: the kernel against the oracle's short_conv: outputs at rel_l2 <= 1e-2
(16-bit; the kernel rounds the conv and the SiLU to the element type as the
module does) or 1e-6 (fp32), advanced caches bit-exact, dense and packed
(empty, one-token and run-crossing segments); and the whole prefill producer
chain on the GPU (conv + SiLU, then the chunked scan with the fused L2 norm)
against the oracle's composition at the 16-bit bar 2e-2.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr
from vagus_amd import _lib


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def test_causal_conv_argument_checks():
    L = _lib.load()

    def call(**over):
        a = dict(dtype=1, x=4096, w=8192, wdt=0, si=None, y=12288, so=None, cu=None, B=2, T=4, D=128, N=2, K=4,
                 act=1)
        a.update(over)
        return L.vgdr_causal_conv1d(a['dtype'], a['x'], a['w'], a['wdt'], a['si'], a['y'], a['so'], a['cu'],
                                    a['B'], a['T'], a['D'], a['N'], a['K'], a['act'], None)
    assert call(K=0) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(K=9) == _lib.VGDR_ERR_UNSUPPORTED
    assert call(D=100) == _lib.VGDR_ERR_UNSUPPORTED                 # 16-bit rows in 8-channel units
    assert call(y=4096) == _lib.VGDR_ERR_INVALID                    # y aliasing x
    assert b'alias' in L.vgdr_last_error()
    assert call(act=2) == _lib.VGDR_ERR_INVALID
    assert call(wdt=2) == _lib.VGDR_ERR_INVALID                     # bf16 x, fp16 weight
    assert call(N=3) == _lib.VGDR_ERR_INVALID                       # dense: N == B
    assert call(x=4100) == _lib.VGDR_ERR_INVALID                    # alignment
    assert call(B=0, N=0, T=0) == _lib.VGDR_OK                      # nothing to do


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('K', [1, 3, 4])
@pytest.mark.parametrize('act', ['silu', None])
@pytest.mark.parametrize('cached', [False, True])
def test_causal_conv_dense_matches_oracle(dtype, K, act, cached):
    from vagus_amd import ops
    g = torch.Generator().manual_seed(K * 7 + cached)
    B, T, D = 3, 37, 192
    x = torch.randn(B, T, D, generator=g).to(dtype)
    w = (0.5 * torch.randn(D, 1, K, generator=g)).to(torch.float32 if K != 3 else dtype)
    cache = torch.randn(B, K, D, generator=g).to(dtype) if cached else None
    print(f'\n[case] causal_conv dense dtype={dtype} K={K} act={act} cached={cached}', flush=True)
    ref, ref_cache = gdr.short_conv(x, w, cache, activation=act)
    c_dev = cache.cuda() if cached else None
    y, fs = ops.causal_conv1d(x.cuda(), w.cuda(), activation=act, conv_cache=c_dev, output_final_state=True)
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    err = _rel(y, ref)
    exact = torch.equal(fs.cpu(), ref_cache)
    print(f'[parity] causal_conv y={err:.3e} cache exact={exact} (tol {tol:g})', flush=True)
    assert err <= tol and exact
    if cached:
        assert fs.data_ptr() == c_dev.data_ptr()


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('B,T,D', [(2, 300, 1040), (1, 1000, 256), (4, 9, 2048)])
def test_causal_conv_workgroup_tiling(dtype, B, T, D):
    """Shapes whose channel units (16 bytes each) fill several 16-unit workgroup
    columns, the last one partly (1040 bf16 = 130 units), and runs of 8 tokens that
    span several workgroup rows with a partial last one; window rows that cross
    workgroups; a sequence shorter than two runs."""
    from vagus_amd import ops
    g = torch.Generator().manual_seed(T + D)
    K = 4
    x = torch.randn(B, T, D, generator=g).to(dtype)
    w = 0.5 * torch.randn(D, 1, K, generator=g)
    cache = torch.randn(B, K, D, generator=g).to(dtype)
    print(f'\n[case] causal_conv tiling dtype={dtype} B={B} T={T} D={D}', flush=True)
    ref, ref_cache = gdr.short_conv(x, w, cache, activation='silu')
    y, fs = ops.causal_conv1d(x.cuda(), w.cuda(), activation='silu', conv_cache=cache.cuda(),
                              output_final_state=True)
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    err = _rel(y, ref)
    exact = torch.equal(fs.cpu(), ref_cache)
    print(f'[parity] causal_conv tiling y={err:.3e} cache exact={exact} (tol {tol:g})', flush=True)
    assert err <= tol and exact


@pytest.mark.gpu
def test_causal_conv_varlen_matches_oracle():
    from vagus_amd import ops
    g = torch.Generator().manual_seed(5)
    cu = torch.tensor([0, 5, 5, 20, 21, 40], dtype=torch.int32)    # empty, one-token and run-crossing segments
    N, T, D, K = 5, 40, 128, 4
    x = torch.randn(1, T, D, generator=g).bfloat16()
    w = 0.5 * torch.randn(D, K, generator=g)
    cache = torch.randn(N, K, D, generator=g).bfloat16()
    ys, cs = [], []
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        y, c = gdr.short_conv(x[:, a:b], w, cache[n:n + 1])
        ys.append(y)
        cs.append(c)
    ref, ref_cache = torch.cat(ys, 1), torch.cat(cs, 0)
    print('\n[case] causal_conv varlen', flush=True)
    c_dev = cache.cuda()
    y, _ = ops.causal_conv1d(x.cuda(), w.cuda(), activation='silu', cu_seqlens=cu.cuda(), conv_cache=c_dev)
    err = _rel(y, ref)
    exact = torch.equal(c_dev.cpu(), ref_cache)
    print(f'[parity] causal_conv varlen y={err:.3e} cache exact={exact}', flush=True)
    assert err <= 1e-2 and exact


@pytest.mark.gpu
def test_prefill_producer_chain_on_gpu():
    """conv + SiLU (causal_conv1d), then the chunked GDN scan with the L2 norm and
    beta sigmoid fused: every producer of linear_attention.py:737-747 on the GPU."""
    from vagus_amd import ops
    g = torch.Generator().manual_seed(9)
    B, T, H, dk, dv, K = 2, 100, 2, 64, 64, 4
    qp = torch.randn(B, T, H * dk, generator=g).bfloat16()
    kp = torch.randn(B, T, H * dk, generator=g).bfloat16()
    vp = torch.randn(B, T, H * dv, generator=g).bfloat16()
    ws = [0.5 * torch.randn(d, 1, K, generator=g) for d in (H * dk, H * dk, H * dv)]
    bl = torch.randn(B, T, H, generator=g)
    gl = F.logsigmoid(torch.randn(B, T, H, generator=g) + 4.0)
    # oracle: the module's producers in torch, then the fp64 recurrence
    q, k, v = (gdr.short_conv(x, w)[0] for x, w in zip((qp, kp, vp), ws))
    q = gdr.l2norm(q.view(B, T, H, dk))
    k = gdr.l2norm(k.view(B, T, H, dk))
    v = v.view(B, T, H, dv)
    o_ref, S_ref = gdr.recurrent(q.double(), k.double(), v.double(), gl.double(), torch.sigmoid(bl).double(),
                                 None, scale=dk ** -0.5)
    print('\n[case] prefill producer chain', flush=True)
    dev = lambda t: t.cuda()
    qc, kc, vc = (ops.causal_conv1d(dev(x), dev(w), activation='silu')[0] for x, w in zip((qp, kp, vp), ws))
    o, S = ops.chunk_gated_delta_rule(qc.view(B, T, H, dk), kc.view(B, T, H, dk), vc.view(B, T, H, dv), dev(gl),
                                      dev(bl), scale=dk ** -0.5, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True)
    eo, es = _rel(o, o_ref), _rel(S, S_ref)
    print(f'[parity] producer chain o={eo:.3e} S={es:.3e}', flush=True)
    assert eo <= 2e-2 and es <= 2e-2
