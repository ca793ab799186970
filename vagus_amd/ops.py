"""Gated delta-rule operators on MI355X: the drop-in for the reference's
fla backend calls (infra/components/linear_attention.py:474-497) and its
single-token recurrence (:161-195 at L == 1, :945-947).

Names, argument meaning and return values follow the calls the reference
makes: ``chunk_gated_delta_rule`` / ``chunk_kda`` / ``chunk_simple_gla``
(fla's chunk kernels) and ``fused_recurrent_*`` (fla's recurrent kernels),
plus ``hip_scan`` with the contract of ``fla_scan`` (:428-498) and
``hip_recurrent`` with the contract of ``recurrent_scan``.  ``cu_seqlens``
adds packed variable-length batches (B = 1, int32/int64 offsets, one entry
and final state per segment).

Layouts: q, k (B, T, H, dk); v (B, T, H, dv); g (B, T, H) scalar log-decay
(GDN) or (B, T, H, dk) per-channel (KDA), fp32 in the kernel; beta (B, T, H);
states (N, H, dk, dv) fp32 with N = B (dense) or the segment count.  o comes
back in q's dtype.

The fla flags use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel and (KDA)
use_gate_in_kernel with A_log / dt_bias / lower_bound move the producers'
elementwise work into the kernels (struct vgdr_fusion): q, k arrive
un-normalised, beta as logits, g as the gate pre-activation (in q's dtype or
fp32).  They need 16-bit q, k, v for the chunked scan, as fla does.  Every call runs the HIP kernels of libvagus_gdr.so on the
current stream; there is no CPU path.  The chunked scans are differentiable:
the delta rule with a scalar gate or none (chunk_gated_delta_rule, hip_scan
with such a g) through vgdr_chunk_bwd, every other form (chunk_kda's
per-channel gate, chunk_simple_gla's plain recurrence, chunk_scan_vec's
explicit write vector w) through vgdr_scan_bwd, and so are the token-by-token
calls (fused_recurrent_*, hip_recurrent) without the short conv or the output
epilogue.  The decode step, the fused epilogue and in-place state updates
raise NotImplementedError for inputs that require grad.
"""
from __future__ import annotations

import ctypes
import weakref

import torch
import torch.nn.functional as F

from . import _lib

_DTYPES = {torch.float32: _lib.VGDR_F32, torch.bfloat16: _lib.VGDR_BF16, torch.float16: _lib.VGDR_F16}
_CHUNK_TILE_DV = 16          # the chunk kernel takes dv in multiples of 16
_REC_DVS = (64, 128)         # the recurrent kernel's column widths
_DEC_DVS = (64, 128, 256)    # the one-token decode step with the short conv (one kernel)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _dk_pad(dk: int) -> int:
    if dk <= 64:
        return 64
    if dk <= 128:
        return 128
    raise NotImplementedError(f'dk={dk}: the kernels take key heads up to 128 wide')


def _pad_to(t, dims: dict):
    """Zero-pad trailing dims of t: {dim_from_end: new_size}.  Zero keys, values,
    queries, log-decays and states are inert in the recurrence, so padding is exact."""
    if t is None:
        return None
    pads = [0, 0] * max(dims) if dims else []
    changed = False
    for d, n in dims.items():
        cur = t.shape[-d]
        if n != cur:
            pads[2 * (d - 1) + 1] = n - cur
            changed = True
    return F.pad(t, pads) if changed else t


def _aligned(t):
    """Contiguous and 16-byte aligned (the kernels use 16-byte vector loads);
    a view that starts mid-vector is copied."""
    if t is None:
        return None
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _check_device(*ts):
    for t in ts:
        if t is not None and t.device.type != 'cuda':
            raise RuntimeError('vagus_amd kernels run on a ROCm GPU; got a tensor on '
                               f'{t.device} (there is no CPU implementation)')


# cu_seqlens tensors already checked: data_ptr -> (weak reference, version, n_tokens)
_CU_CHECKED: dict = {}


def _check_cu(cu_seqlens, n_tokens: int):
    """The packed-batch contract, checked on the host: integer offsets,
    cu[0] == 0, non-decreasing, cu[-1] == n_tokens, inside int32.  The
    kernels only clamp each segment into [0, n_tokens] (memory safety);
    overlapping or uncovered rows would otherwise race on o or be left
    unwritten.  Reads the offsets back (one small device-to-host copy, which
    waits for the stream) once per tensor: a tensor that passed, still alive
    and unmodified (the same object and in-place version), with the same
    token count, is not read again, so the several kernels of one packed
    layer call (conv, scan, epilogue) and the layers of one prefill check
    their shared offsets once.  Inside HIP graph capture no copy may run and
    the caller vouches for the table."""
    assert cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 1, 'cu_seqlens is 1-D with N + 1 entries'
    assert not cu_seqlens.is_floating_point() and cu_seqlens.dtype != torch.bool, \
        'cu_seqlens holds integer offsets'
    if cu_seqlens.is_cuda and torch.cuda.is_current_stream_capturing():
        return
    key = (cu_seqlens.data_ptr(), cu_seqlens.device, cu_seqlens.dtype, cu_seqlens.numel())
    hit = _CU_CHECKED.get(key)
    if hit is not None and hit[0]() is cu_seqlens and hit[1] == cu_seqlens._version and hit[2] == n_tokens:
        return
    cu = cu_seqlens.detach().to('cpu', torch.int64)
    assert int(cu[0]) == 0, f'cu_seqlens[0] must be 0, got {int(cu[0])}'
    assert int(cu[-1]) == n_tokens, f'cu_seqlens[-1] must equal the {n_tokens} packed tokens, got {int(cu[-1])}'
    assert n_tokens < 2 ** 31, f'{n_tokens} packed tokens exceed the int32 offsets'
    if cu.numel() > 1:
        assert bool((cu[1:] >= cu[:-1]).all()), 'cu_seqlens must be non-decreasing'
    if len(_CU_CHECKED) >= 64:
        _CU_CHECKED.clear()
    _CU_CHECKED[key] = (weakref.ref(cu_seqlens), cu_seqlens._version, n_tokens)


def _wants_grad(*ts):
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _check_grad(*ts):
    if _wants_grad(*ts):
        raise NotImplementedError('vagus_amd differentiates the chunked scans (chunk_gated_delta_rule, chunk_kda, '
                                  'chunk_simple_gla, hip_scan, chunk_scan_vec); this call has no backward')


def _gate_activation_rows(f, fz):
    """The per-channel gate from its pre-activation f (B, T, H, dk) in fp32
    (linear_attention.py:722-734): -exp(A_log) softplus(f + dt_bias), or
    lower_bound sigmoid(exp(A_log) (f + dt_bias)); differentiable in torch."""
    H, dk = f.shape[2], f.shape[3]
    x = f.float() + fz.dt_bias.float().reshape(H, dk)
    a = fz.A_log.float().reshape(H, 1).exp()
    if fz.lower_bound is not None:
        return fz.lower_bound * torch.sigmoid(a * x)
    return -a * F.softplus(x)


class _L2NormRows(torch.autograd.Function):
    """y = x r, r = rsqrt(sum x^2 + 1e-6) per (token, head), computed in >= fp32
    and rounded to x's type (linear_attention.py:703-706).  Saves x (its own
    type) and r (one float per row): autograd through the torch expression
    would keep fp32 copies of the whole (B, T, H, dk) row block.
    dx = r dy - r^3 x <x, dy>."""

    @staticmethod
    def forward(ctx, x):
        xf = x if x.dtype == torch.float64 else x.float()
        r = torch.rsqrt((xf * xf).sum(-1, keepdim=True) + 1e-6)
        ctx.save_for_backward(x, r)
        return (xf * r).to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        x, r = ctx.saved_tensors
        xf = x.to(r.dtype)
        dyf = dy.to(r.dtype)
        return (r * dyf - r * r * r * xf * (xf * dyf).sum(-1, keepdim=True)).to(x.dtype)


def _l2norm_rows(x):
    """x rsqrt(sum x^2 + 1e-6) per (token, head) in >= fp32, cast back
    (linear_attention.py:703-706): the q, k producer, differentiable."""
    return _L2NormRows.apply(x)


class _Fusion:
    """The producer fusions of one call (linear_attention.py:457-497 flags)."""

    def __init__(self, *, l2norm=False, beta=False, gate=False, A_log=None, dt_bias=None, lower_bound=None):
        self.l2norm, self.beta, self.gate = bool(l2norm), bool(beta), bool(gate)
        self.A_log, self.dt_bias, self.lower_bound = A_log, dt_bias, lower_bound
        if self.gate:
            assert A_log is not None and dt_bias is not None, 'use_gate_in_kernel needs A_log and dt_bias'
        else:
            assert lower_bound is None, 'lower_bound belongs to the fused gate activation'

    @property
    def any(self):
        return self.l2norm or self.beta or self.gate

    def struct(self, c):
        """(the C struct, tensors it points into) for the padded operands of call c."""
        keep = []
        fz = _lib.Fusion(int(self.l2norm), int(self.beta), int(self.gate), _lib.VGDR_F32, None, None, 0, 0.0)
        if self.gate:
            a_log = self.A_log.detach().float().reshape(c.H).contiguous()
            dt = self.dt_bias.detach().float().reshape(c.H, c.dk)
            dt = _aligned(_pad_to(dt, {1: c.dkp}))
            keep += [a_log, dt]
            fz.A_log, fz.dt_bias = a_log.data_ptr(), dt.data_ptr()
            fz.gate_dtype = _DTYPES[c.g.dtype]
            if self.lower_bound is not None:
                fz.lower_bound_set, fz.lower_bound = 1, float(self.lower_bound)
        return fz, keep


_NO_FUSION = _Fusion()


def _row_stride(t):
    """The token row stride, in elements, of a one-token-per-sequence input t
    (B, 1, H, d) whose (H, d) block is dense and 16-byte aligned, else None."""
    B, T, H, d = t.shape
    if T != 1 or t.stride(3) != 1 or t.stride(2) != d or t.data_ptr() % 16:
        return None
    ld = t.stride(0) if B > 1 else H * d
    return ld if ld >= H * d else None


class _Call:
    """Validated, padded, contiguous operands of one kernel call.  rows: q, k, v
    of a one-token call may stay rows of a wider buffer (ld_qk, ld_v: their token
    row strides; 0 when the operands are dense)."""

    def __init__(self, q, k, v, g, beta, initial_state, cu_seqlens, *, gate: str, delta: bool,
                 dv_to, fusion: _Fusion = _NO_FUSION, rows: bool = False, gate_proj: bool = False):
        _check_device(q, k, v, g, beta, initial_state, cu_seqlens)
        _check_grad(q, k, v, g, beta, initial_state)
        assert q.dim() == 4 and k.shape == q.shape and v.dim() == 4 and v.shape[:3] == q.shape[:3], \
            f'q, k must be (B, T, H, dk) and v (B, T, H, dv); got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}'
        if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
            raise NotImplementedError(f'q, k, v must share one of {list(_DTYPES)}; got '
                                      f'{q.dtype}, {k.dtype}, {v.dtype}')
        B, T, H, dk = q.shape
        dv = v.shape[-1]
        if gate == 'vector':
            assert g is not None and g.shape == (B, T, H, dk), \
                f'a per-channel gate is (B, T, H, dk); got {None if g is None else tuple(g.shape)}'
        elif gate == 'scalar' and not gate_proj:
            assert g is not None and g.shape == (B, T, H), \
                f'a scalar gate is (B, T, H); got {None if g is None else tuple(g.shape)}'
        if delta and not gate_proj:
            assert beta is not None and beta.shape == (B, T, H), 'the delta rule needs beta (B, T, H)'
        if cu_seqlens is not None:
            assert B == 1, f'packed varlen input (cu_seqlens) has batch 1, got {B}'
            _check_cu(cu_seqlens, T)
            N = cu_seqlens.numel() - 1
            cu = cu_seqlens.to(torch.int32).contiguous()
        else:
            N = B
            cu = None
        if initial_state is not None:
            assert initial_state.shape == (N, H, dk, dv), \
                f'initial_state must be {(N, H, dk, dv)}, got {tuple(initial_state.shape)}'
        dkp, dvp = _dk_pad(dk), dv_to(dv)
        self.B, self.T, self.H, self.dk, self.dv, self.N = B, T, H, dk, dv, N
        self.dkp, self.dvp = dkp, dvp
        self.dtype = q.dtype
        self.device = q.device
        self.ld_qk = self.ld_v = 0
        if rows and cu is None and dkp == dk and dvp == dv:
            lq, lk, lv = _row_stride(q), _row_stride(k), _row_stride(v)
            if lq is not None and lq == lk and lv is not None and (lq, lv) != (H * dk, H * dv):
                self.ld_qk, self.ld_v = lq, lv                  # (dense rows keep the dense entry point)
        if self.ld_qk:
            self.q, self.k, self.v = q, k, v
        else:
            self.q = _aligned(_pad_to(q, {1: dkp}))
            self.k = _aligned(_pad_to(k, {1: dkp}))
            self.v = _aligned(_pad_to(v, {1: dvp}))
        if gate == 'none' or (g is None and not gate_proj):
            self.g, self.gate_kind = None, _lib.VGDR_GATE_NONE
        elif gate == 'vector':
            # a fused gate pre-activation stays in q's 16-bit type (no fp32 copy)
            gk = g if (fusion.gate and g.dtype == q.dtype and q.dtype != torch.float32) else g.float()
            self.g, self.gate_kind = _aligned(_pad_to(gk, {1: dkp})), _lib.VGDR_GATE_VECTOR
        elif gate_proj:                                   # the decode kernel forms g and beta itself
            self.g, self.gate_kind = None, _lib.VGDR_GATE_SCALAR
        else:
            self.g, self.gate_kind = g.float().contiguous(), _lib.VGDR_GATE_SCALAR
        self.beta = beta.float().contiguous() if delta and not gate_proj else None
        self.h0 = None if initial_state is None else \
            _aligned(_pad_to(initial_state.float(), {1: dvp, 2: dkp}))
        self.cu = cu
        self.padded = (dkp != dk) or (dvp != dv)

    def new_output(self):
        return torch.empty(self.B, self.T, self.H, self.dvp, dtype=self.dtype, device=self.device)

    def new_state(self):
        return torch.empty(self.N, self.H, self.dkp, self.dvp, dtype=torch.float32, device=self.device)

    def unpad_o(self, o):
        return o[..., :self.dv].contiguous() if self.dvp != self.dv else o

    def unpad_state(self, S):
        if S is None or not self.padded:
            return S
        return S[:, :, :self.dk, :self.dv].contiguous()


def _gate_of(g):
    """The gate form of a log-decay tensor: None, (B, T, H) or (B, T, H, dk)."""
    return 'none' if g is None else ('vector' if g.dim() == 4 else 'scalar')


# The per-channel-gate chunked backward runs 64-token chunks (its gradient
# kernel holds a chunk's gated products in LDS at that size).  The chunk size
# is a blocking choice, not part of the function: a per-channel 16-bit call
# asked for 32-token chunks under autograd runs the forward it saves for the
# backward, and the backward, in 64-token chunks (the reference's HAX1 / HAX2
# recipes train KDA with chunk_size 32, recipe/model/hax1_340M.yaml:94).
_VEC_BWD_CHUNK = 64


def _chunk_bwd_covers(q, g, chunk_size):
    """Whether vgdr_chunk_bwd takes this delta-rule call: a scalar gate or
    none at any dtype, a per-channel gate with 16-bit q, k, v (in 64-token
    chunks whatever chunk_size asks; the token-recurrence backward takes
    fp32 per-channel calls)."""
    return g is None or g.dim() == 3 or q.dtype != torch.float32


def _bwd_chunk(q, g, chunk_size):
    """The chunk size the chunked backward (and a saving forward) runs."""
    return _VEC_BWD_CHUNK if (g is not None and g.dim() == 4 and q.dtype != torch.float32) else chunk_size


def chunk_gated_delta_rule_bwd(q, k, v, g, beta, initial_state, do, dht=None, *, scale=None, cu_seqlens=None,
                               chunk_size=64, saved_workspace=None, fusion: _Fusion = _NO_FUSION, delta=True):
    """Backward of chunk_gated_delta_rule / chunk_kda without autograd
    (vgdr_chunk_bwd): the gradients of (o, final_state) under the cotangents
    do (and dht, None = zero) with respect to q, k, v, g, beta and
    initial_state, for the delta rule with a scalar gate (g (B, T, H)), a
    per-channel gate (g (B, T, H, dk); 16-bit q, k, v, run in 64-token chunks
    whatever chunk_size asks) or none (g None).  q, k as the forward scanned them (normalised), beta in
    [0, 1], g the log-decay.  Returns (dq, dk, dv, dg, dbeta, dh0) in the
    inputs' dtypes; dg is None without a gate and dh0 None without an initial
    state.  The gradients the reference's training takes through chunk_scan /
    chunk_scan_vec (linear_attention.py:237-309, :312-425) or fla's backward.
    saved_workspace: the workspace a saving forward (_chunk_fwd_saving, same
    inputs) filled; the backward then skips rebuilding the chunk blocks and
    the per-chunk entry states.
    fusion: the producer fusions the kernels differentiate through (16-bit;
    no L2 norm): beta as logits (dbeta is their gradient) and, with a
    per-channel g, the gate activation (g is its pre-activation f, dg is df,
    and the tuple gains dA_log and ddt_bias).
    delta=False: the recurrence without the delta rule (chunk_simple_gla,
    chunk_scan_vec(delta=False)) through vgdr_chunk_bwd_nodelta; beta is None
    and so is dbeta."""
    assert not fusion.l2norm, 'the fused L2 norm is differentiated in torch, before the kernels'
    assert delta or (beta is None and not fusion.any and saved_workspace is None), \
        'without the delta rule there is no beta, fusion or saved workspace'
    c = _Call(q, k, v, g, beta, initial_state, cu_seqlens, gate=_gate_of(g), delta=delta,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV, fusion=fusion)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    assert do.shape == (c.B, c.T, c.H, c.dv), f'do must be {(c.B, c.T, c.H, c.dv)}, got {tuple(do.shape)}'
    assert dht is None or dht.shape == (c.N, c.H, c.dk, c.dv), \
        f'dht must be {(c.N, c.H, c.dk, c.dv)}, got {tuple(dht.shape)}'
    _check_device(do, dht)
    dop = _aligned(_pad_to(do.to(c.dtype), {1: c.dvp}))
    dSp = None if dht is None else _aligned(_pad_to(dht.float(), {1: c.dvp, 2: c.dkp}))
    new = lambda *shape, dt=torch.float32: torch.empty(*shape, dtype=dt, device=c.device)
    dq, dk = new(c.B, c.T, c.H, c.dkp, dt=c.dtype), new(c.B, c.T, c.H, c.dkp, dt=c.dtype)
    dv = new(c.B, c.T, c.H, c.dvp, dt=c.dtype)
    vec = c.gate_kind == _lib.VGDR_GATE_VECTOR
    chunk_size = _bwd_chunk(q, g, chunk_size)
    dg = None if g is None else (new(c.B, c.T, c.H, c.dkp) if vec else new(c.B, c.T, c.H))
    db = new(c.B, c.T, c.H) if delta else None
    dS0 = new(c.N, c.H, c.dkp, c.dvp) if initial_state is not None else None
    L = _lib.load()
    dtype = _DTYPES[c.dtype]
    nbytes = L.vgdr_chunk_bwd_workspace_size(dtype, c.gate_kind, c.B, c.T, c.H, c.dkp, c.dvp, c.N,
                                             int(c.cu is not None), int(chunk_size))
    if saved_workspace is not None:
        assert saved_workspace.numel() >= nbytes, 'saved_workspace is smaller than this backward needs'
        ws, saved = saved_workspace, True
    else:
        ws, saved = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device), False
    head = (dtype, c.gate_kind, _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g), _ptr(c.beta), _ptr(c.h0), _ptr(dop),
            _ptr(dSp), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dg), _ptr(db), _ptr(dS0), _ptr(c.cu), _ptr(ws), nbytes,
            c.B, c.T, c.H, c.dkp, c.dvp, c.N, scale, int(chunk_size))
    dA = ddt = None
    with torch.cuda.device(c.device):
        if not delta:
            _lib.check(L.vgdr_chunk_bwd_nodelta(dtype, c.gate_kind, _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
                                                _ptr(c.h0), _ptr(dop), _ptr(dSp), _ptr(dq), _ptr(dk), _ptr(dv),
                                                _ptr(dg), _ptr(dS0), _ptr(c.cu), _ptr(ws), nbytes, c.B, c.T, c.H,
                                                c.dkp, c.dvp, c.N, scale, int(chunk_size), _stream(c.device)))
        elif fusion.any:
            fz, keep = fusion.struct(c)
            if fusion.gate:
                dA, ddt = new(c.H), new(c.H * c.dkp)
            fn = L.vgdr_chunk_bwd_saved_fused if saved else L.vgdr_chunk_bwd_fused
            _lib.check(fn(*head, ctypes.byref(fz), _ptr(dA), _ptr(ddt), _stream(c.device)))
        else:
            fn = L.vgdr_chunk_bwd_saved if saved else L.vgdr_chunk_bwd
            _lib.check(fn(*head, _stream(c.device)))
    if c.dkp != c.dk:
        dq, dk = dq[..., :c.dk], dk[..., :c.dk]
        dg = dg[..., :c.dk] if vec else dg
    if c.dvp != c.dv:
        dv = dv[..., :c.dv]
    if dS0 is not None:
        dS0 = c.unpad_state(dS0).to(initial_state.dtype)
    out = (dq, dk, dv, None if dg is None else dg.to(g.dtype), None if db is None else db.to(beta.dtype), dS0)
    if fusion.gate:
        ddt = ddt.reshape(c.H, c.dkp)[:, :c.dk].reshape(fusion.dt_bias.shape).to(fusion.dt_bias.dtype)
        out += (dA.reshape(fusion.A_log.shape).to(fusion.A_log.dtype), ddt)
    return out


def _chunk_fwd_saving(q, k, v, g, beta, initial_state, *, scale, cu_seqlens, chunk_size,
                      fusion: _Fusion = _NO_FUSION):
    """vgdr_chunk_fwd_saving: the chunked forward (16-bit, any gate, delta
    rule) run in a backward workspace, which keeps the chunk blocks and every
    chunk's entry state for vgdr_chunk_bwd_saved.  fusion: beta logits and
    the gate activation in the kernels (no L2 norm).  Returns (o,
    final_state, workspace)."""
    c = _Call(q, k, v, g, beta, initial_state, cu_seqlens, gate=_gate_of(g), delta=True,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV, fusion=fusion)
    chunk_size = _bwd_chunk(q, g, chunk_size)                  # the backward's blocking
    o, S = c.new_output(), c.new_state()
    L = _lib.load()
    dtype = _DTYPES[c.dtype]
    nbytes = L.vgdr_chunk_bwd_workspace_size(dtype, c.gate_kind, c.B, c.T, c.H, c.dkp, c.dvp, c.N,
                                             int(c.cu is not None), int(chunk_size))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    head = (dtype, c.gate_kind, _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g), _ptr(c.beta), _ptr(o), _ptr(c.h0),
            _ptr(S), _ptr(c.cu), _ptr(ws), nbytes, c.B, c.T, c.H, c.dkp, c.dvp, c.N, float(scale), int(chunk_size))
    with torch.cuda.device(c.device):
        if fusion.any:
            fz, keep = fusion.struct(c)
            _lib.check(L.vgdr_chunk_fwd_saving_fused(*head, ctypes.byref(fz), _stream(c.device)))
        else:
            _lib.check(L.vgdr_chunk_fwd_saving(*head, _stream(c.device)))
    return c.unpad_o(o), c.unpad_state(S), ws


def scan_bwd(q, k, v, g, beta, initial_state, do, dht=None, *, scale=None, delta=True, w=None, cu_seqlens=None):
    """Backward of every scan form without autograd (vgdr_scan_bwd): the
    gradients of (o, final_state) under do (and dht, None = zero) for g None,
    (B, T, H) or (B, T, H, dk), the delta rule with beta_t k_t or an explicit
    write w (B, T, H, dk), or (delta=False) the plain recurrence.  Returns
    (dq, dk, dv, dg, dbeta, dh0), with dw appended when w is given; dg is None
    without a gate, dbeta None unless the delta rule writes beta_t k_t, dh0
    None without an initial state.  The gradients the reference's training
    takes through chunk_scan_vec / chunk_scan / recurrent_scan
    (linear_attention.py:161-425)."""
    gate = _gate_of(g)
    writes_beta = delta and w is None
    c = _Call(q, k, v, g, beta if writes_beta else None, initial_state, cu_seqlens, gate=gate,
              delta=writes_beta, dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    assert do.shape == (c.B, c.T, c.H, c.dv), f'do must be {(c.B, c.T, c.H, c.dv)}, got {tuple(do.shape)}'
    assert dht is None or dht.shape == (c.N, c.H, c.dk, c.dv), \
        f'dht must be {(c.N, c.H, c.dk, c.dv)}, got {tuple(dht.shape)}'
    if w is not None:
        assert delta, 'an explicit write vector needs the delta rule'
        assert w.shape == q.shape, f'w must be {tuple(q.shape)} (B, T, H, dk); got {tuple(w.shape)}'
    _check_device(do, dht, w)
    wk = None if w is None else _aligned(_pad_to(w.to(c.dtype), {1: c.dkp}))
    dop = _aligned(_pad_to(do.to(c.dtype), {1: c.dvp}))
    dSp = None if dht is None else _aligned(_pad_to(dht.float(), {1: c.dvp, 2: c.dkp}))
    new = lambda *shape, dt=torch.float32: torch.empty(*shape, dtype=dt, device=c.device)
    dq, dk = new(c.B, c.T, c.H, c.dkp, dt=c.dtype), new(c.B, c.T, c.H, c.dkp, dt=c.dtype)
    dv = new(c.B, c.T, c.H, c.dvp, dt=c.dtype)
    dw = new(c.B, c.T, c.H, c.dkp, dt=c.dtype) if w is not None else None
    dg = None if gate == 'none' else (new(c.B, c.T, c.H, c.dkp) if gate == 'vector' else new(c.B, c.T, c.H))
    db = new(c.B, c.T, c.H) if writes_beta else None
    dS0 = new(c.N, c.H, c.dkp, c.dvp) if initial_state is not None else None
    L = _lib.load()
    nbytes = L.vgdr_scan_bwd_workspace_size(c.B, c.T, c.H, c.dkp, c.dvp, c.N)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        _lib.check(L.vgdr_scan_bwd(_DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v),
                                   _ptr(wk), _ptr(c.g), _ptr(c.beta), _ptr(c.h0), _ptr(dop), _ptr(dSp), _ptr(dq),
                                   _ptr(dk), _ptr(dv), _ptr(dw), _ptr(dg), _ptr(db), _ptr(dS0), _ptr(c.cu),
                                   _ptr(ws), nbytes, c.B, c.T, c.H, c.dkp, c.dvp, c.N, scale, _stream(c.device)))
    if c.dkp != c.dk:
        dq, dk = dq[..., :c.dk], dk[..., :c.dk]
        dw = None if dw is None else dw[..., :c.dk]
        dg = dg[..., :c.dk] if gate == 'vector' else dg
    if c.dvp != c.dv:
        dv = dv[..., :c.dv]
    if dS0 is not None:
        dS0 = c.unpad_state(dS0).to(initial_state.dtype)
    res = (dq, dk, dv, None if dg is None else dg.to(g.dtype), None if db is None else db.to(beta.dtype), dS0)
    return res + ((dw,) if w is not None else ())


class _ScanRule(torch.autograd.Function):
    """Every form the scalar-gate chunk backward does not take, differentiable:
    the per-channel gate, the plain recurrence (delta=False) and the explicit
    write w.  Forward: the chunked kernels (chunk_scan, or chunk_scan_vec with
    w), or with token=True the token-by-token kernel; backward: vgdr_scan_bwd,
    which rebuilds the states it needs from q, k, v, g, beta (w) and the entry
    state."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, S0, w, scale, cu, chunk_size, delta, token=False):
        if token:
            o, S = _recurrent(q, k, v, g, beta, gate=_gate_of(g), delta=delta, scale=scale, initial_state=S0,
                              output_final_state=True, cu_seqlens=cu, w=w)
        elif w is None:
            o, S = chunk_scan(q, k, v, g, beta, gate=_gate_of(g), delta=delta, scale=scale, initial_state=S0,
                              output_final_state=True, cu_seqlens=cu, chunk_size=chunk_size)
        else:
            o, S = chunk_scan_vec(q, k, v, g, None, S0, scale=scale, delta=True, chunk_size=chunk_size, w=w,
                                  cu_seqlens=cu)
        ctx.save_for_backward(q, k, v, g, beta, S0, w, cu)
        ctx.scale, ctx.delta = scale, delta
        return o, S

    @staticmethod
    def backward(ctx, do, dS):
        q, k, v, g, beta, S0, w, cu = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        r = scan_bwd(q, k, v, g, beta, S0, do, dS, scale=ctx.scale, delta=ctx.delta, w=w, cu_seqlens=cu)
        return r[:6] + (r[6] if w is not None else None, None, None, None, None, None)


class _ChunkDeltaRule(torch.autograd.Function):
    """The chunked delta rule with a scalar gate, a per-channel gate (16-bit,
    64-token chunks) or none, differentiable.
    16-bit inputs: forward vgdr_chunk_fwd_saving, which keeps the chunk blocks
    and the per-chunk entry states in the backward's workspace, and backward
    vgdr_chunk_bwd_saved (fla's disable_recompute trade: about 2 dk dv bytes
    per chunk and head of device memory held from forward to backward for
    skipping two of the backward's kernels).  fp32: forward vgdr_chunk_fwd,
    backward vgdr_chunk_bwd.  q, k arrive normalised.  fusion (16-bit only):
    beta as logits and the per-channel gate as its pre-activation f with
    A_log, dt_bias, both differentiated inside the kernels; otherwise beta in
    [0, 1] and g the log-decay."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, S0, A_log, dt_bias, scale, cu, chunk_size, fusion):
        ctx.ws = None
        chunk_size = _bwd_chunk(q, g, chunk_size)
        if q.dtype != torch.float32:
            o, S, ctx.ws = _chunk_fwd_saving(q, k, v, g, beta, S0, scale=scale, cu_seqlens=cu,
                                             chunk_size=chunk_size, fusion=fusion)
        else:
            assert not fusion.any, 'the kernel fusions take 16-bit q, k, v'
            o, S = chunk_scan(q, k, v, g, beta, gate=_gate_of(g), delta=True,
                              scale=scale, initial_state=S0, output_final_state=True, cu_seqlens=cu,
                              chunk_size=chunk_size)
        ctx.save_for_backward(q, k, v, g, beta, S0, cu, A_log, dt_bias)
        ctx.scale, ctx.chunk_size, ctx.fusion = scale, chunk_size, fusion
        return o, S

    @staticmethod
    def backward(ctx, do, dS):
        q, k, v, g, beta, S0, cu, A_log, dt_bias = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        fz = ctx.fusion
        if fz.gate:                                            # the saved tensors, not the forward's references
            fz = _Fusion(beta=fz.beta, gate=True, A_log=A_log, dt_bias=dt_bias, lower_bound=fz.lower_bound)
        grads = chunk_gated_delta_rule_bwd(q, k, v, g, beta, S0, do, dS, scale=ctx.scale, cu_seqlens=cu,
                                           chunk_size=ctx.chunk_size, saved_workspace=ctx.ws, fusion=fz)
        ctx.ws = None
        dA, ddt = grads[6:] if fz.gate else (None, None)
        return grads[:6] + (dA, ddt, None, None, None, None)


class _ChunkPlain(torch.autograd.Function):
    """The chunked recurrence without the delta rule (chunk_simple_gla,
    chunk_scan_vec / chunk_scan with delta=False), differentiable: forward
    vgdr_chunk_fwd, backward vgdr_chunk_bwd_nodelta (the delta form's
    kernels on blocks with TE = I and no K decay, so U = V; they recompute
    the entry states)."""

    @staticmethod
    def forward(ctx, q, k, v, g, S0, scale, cu, chunk_size):
        o, S = chunk_scan(q, k, v, g, None, gate=_gate_of(g), delta=False, scale=scale, initial_state=S0,
                          output_final_state=True, cu_seqlens=cu, chunk_size=chunk_size)
        ctx.save_for_backward(q, k, v, g, S0, cu)
        ctx.scale, ctx.chunk_size = scale, chunk_size
        return o, S

    @staticmethod
    def backward(ctx, do, dS):
        q, k, v, g, S0, cu = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        dq, dk, dv, dg, _, dS0 = chunk_gated_delta_rule_bwd(q, k, v, g, None, S0, do, dS, scale=ctx.scale,
                                                            cu_seqlens=cu, chunk_size=_bwd_chunk(q, g, ctx.chunk_size),
                                                            delta=False)
        return dq, dk, dv, dg, dS0, None, None, None


def chunk_scan(q, k, v, g, beta, *, gate, delta, scale=None, initial_state=None, output_final_state=False,
               cu_seqlens=None, chunk_size=64, phase_event=None, fusion: _Fusion = _NO_FUSION):
    """Chunkwise prefill, the general form behind chunk_gated_delta_rule,
    chunk_kda and chunk_simple_gla: gate in {'none', 'scalar', 'vector'},
    delta selects the delta rule.  Returns (o, final_state or None).

    phase_event: optional torch.cuda.Event recorded on the current stream
    between the chunk-prep and the chunk-state kernels (the same two launches
    either way), so that a caller can time the two phases separately.
    fusion: the producer fusions (_Fusion).

    With grads enabled and an input that requires grad, the scan runs through
    _ChunkDeltaRule (delta rule: scalar gate or none, or the per-channel gate
    with 16-bit inputs in 64-token chunks), _ChunkPlain (no delta rule, the
    same gate forms) or _ScanRule (every other form).
    The fused L2 norm then runs in torch, differentiably; the beta sigmoid and
    the gate activation stay inside the kernels, forward and backward, on the
    16-bit _ChunkDeltaRule path (no fp32 (B, T, H, dk) gate tensor is made),
    and run in torch elsewhere."""
    if _wants_grad(q, k, v, g, beta, initial_state, fusion.A_log, fusion.dt_bias):
        if fusion.l2norm:
            q, k = _l2norm_rows(q), _l2norm_rows(k)
        scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
        gk = None if gate == 'none' else g
        chunked = delta and _chunk_bwd_covers(q, gk, chunk_size)
        if chunked and q.dtype != torch.float32 and (fusion.beta or fusion.gate):
            # beta sigmoid and the gate activation inside the kernels, forward and backward
            kf = _Fusion(beta=fusion.beta, gate=fusion.gate, A_log=fusion.A_log, dt_bias=fusion.dt_bias,
                         lower_bound=fusion.lower_bound)
            o, S = _ChunkDeltaRule.apply(q, k, v, gk, beta, initial_state, fusion.A_log, fusion.dt_bias, scale,
                                         cu_seqlens, chunk_size, kf)
            return o, (S if output_final_state else None)
        if fusion.beta:
            beta = torch.sigmoid(beta.float())
        if fusion.gate:
            g = _gate_activation_rows(g, fusion)
        gk = None if gate == 'none' else g
        if not delta and _chunk_bwd_covers(q, gk, chunk_size):
            o, S = _ChunkPlain.apply(q, k, v, gk, initial_state, scale, cu_seqlens, chunk_size)
        elif not chunked:
            o, S = _ScanRule.apply(q, k, v, gk, beta if delta else None, initial_state, None, scale, cu_seqlens,
                                   chunk_size, delta)
        else:
            o, S = _ChunkDeltaRule.apply(q, k, v, gk, beta, initial_state, None, None, scale, cu_seqlens, chunk_size,
                                         _NO_FUSION)
        return o, (S if output_final_state else None)
    c = _Call(q, k, v, g, beta, initial_state, cu_seqlens, gate=gate, delta=delta,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV, fusion=fusion)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    o = c.new_output()
    S = c.new_state() if output_final_state else None
    L = _lib.load()
    varlen = c.cu is not None
    nbytes = L.vgdr_chunk_workspace_size(_DTYPES[c.dtype], c.gate_kind, c.B, c.T, c.H, c.dkp, c.N, int(varlen),
                                         int(chunk_size))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        head = (_DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
                _ptr(c.beta), _ptr(o), _ptr(c.h0), _ptr(S), _ptr(c.cu), _ptr(ws), nbytes,
                c.B, c.T, c.H, c.dkp, c.dvp, c.N, scale, int(chunk_size))
        args = head + (_stream(c.device),)
        if fusion.any:
            fz, keep = fusion.struct(c)
            fargs = head + (ctypes.byref(fz), _stream(c.device))
            if phase_event is None:
                _lib.check(L.vgdr_chunk_fwd_fused(*fargs))
            else:
                _lib.check(L.vgdr_chunk_prep_fused(*fargs))
                phase_event.record(torch.cuda.current_stream(c.device))
                _lib.check(L.vgdr_chunk_state(*args))
            del keep
        elif phase_event is None:
            _lib.check(L.vgdr_chunk_fwd(*args))
        else:
            _lib.check(L.vgdr_chunk_prep(*args))
            phase_event.record(torch.cuda.current_stream(c.device))
            _lib.check(L.vgdr_chunk_state(*args))
    return c.unpad_o(o), c.unpad_state(S)


def _kda_fusion(use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias,
                safe_gate, lower_bound) -> _Fusion:
    # safe_gate / lower_bound select the bounded activation lower_bound *
    # sigmoid(exp(A_log) (f + dt_bias)) of the fused gate (the reference passes
    # them only together with use_gate_in_kernel, linear_attention.py:465-471)
    if safe_gate:
        assert lower_bound is not None, 'safe_gate needs lower_bound'
    return _Fusion(l2norm=use_qk_l2norm_in_kernel, beta=use_beta_sigmoid_in_kernel, gate=use_gate_in_kernel,
                   A_log=A_log, dt_bias=dt_bias, lower_bound=lower_bound if use_gate_in_kernel else None)


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, cu_seqlens=None, chunk_size=64,
                           use_qk_l2norm_in_kernel=False, use_beta_sigmoid_in_kernel=False):
    """GDN chunkwise prefill (the call at linear_attention.py:487-491).

    g: (B, T, H) log-decay (None for DeltaNet, a = 1).  Returns (o, final_state),
    final_state None unless output_final_state.  use_qk_l2norm_in_kernel: q, k
    arrive un-normalised; use_beta_sigmoid_in_kernel: beta arrives as logits."""
    fz = _Fusion(l2norm=use_qk_l2norm_in_kernel, beta=use_beta_sigmoid_in_kernel)
    return chunk_scan(q, k, v, g, beta, gate='scalar' if g is not None else 'none', delta=True,
                  scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size, fusion=fz)


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
              cu_seqlens=None, chunk_size=64, use_qk_l2norm_in_kernel=False,
              use_beta_sigmoid_in_kernel=False, use_gate_in_kernel=False, A_log=None, dt_bias=None,
              safe_gate=False, lower_bound=None, disable_recompute=False):
    """KDA chunkwise prefill (the call at linear_attention.py:474-479).

    g: (B, T, H, dk) per-channel log-decay, or with use_gate_in_kernel the gate
    pre-activation f (q's dtype or fp32) with A_log (H,) and dt_bias (H*dk,):
    g = -exp(A_log) softplus(f + dt_bias), or lower_bound * sigmoid(exp(A_log)
    (f + dt_bias)) with lower_bound (linear_attention.py:719-734).
    disable_recompute only concerns a backward pass and is accepted and ignored."""
    fz = _kda_fusion(use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias,
                     safe_gate, lower_bound)
    return chunk_scan(q, k, v, g, beta, gate='vector', delta=True, scale=scale,
                  initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size, fusion=fz)


def chunk_simple_gla(q, k, v, g, scale=None, initial_state=None, output_final_state=False,
                     cu_seqlens=None, chunk_size=64):
    """Gated linear attention without the delta rule (the call at linear_attention.py:495-497):
    S_t = a_t S_{t-1} + k_t v_t^T.  g: (B, T, H) or None."""
    return chunk_scan(q, k, v, g, None, gate='scalar' if g is not None else 'none', delta=False,
                  scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size)


class _Epilogue:
    """The layer's output epilogue (linear_attention.py:814-825): RMSNorm of o
    over dv with weight gamma, times SiLU(gate)."""

    def __init__(self, gate, gamma, eps):
        assert gate is not None and gamma is not None, 'the output epilogue needs the gate and the norm weight'
        assert gamma.dim() == 1 and gate.shape[-1] == gamma.shape[0], \
            f'gamma is (dv,) and gate (..., dv); got {tuple(gamma.shape)}, {tuple(gate.shape)}'
        assert eps > 0, 'the RMSNorm eps must be positive'
        _check_device(gate, gamma)
        self.gate, self.gamma, self.eps = gate, gamma, float(eps)

    def struct(self, dtype, rows: bool = False):
        """(vgdr_epilogue, tensors to keep alive) for o in `dtype`; rows: the gate
        is passed as it is, rows of a wider buffer (the caller checked its stride)."""
        if self.gate.dtype != dtype:
            raise NotImplementedError(f'the epilogue gate must have o\'s dtype {dtype}; got {self.gate.dtype}')
        gate = self.gate if rows else _aligned(self.gate)
        gamma = _aligned(self.gamma if self.gamma.dtype in (torch.float32, dtype) else self.gamma.float())
        ep = _lib.Epilogue(gate=_ptr(gate), gamma=_ptr(gamma), gamma_dtype=_DTYPES[gamma.dtype], eps=self.eps)
        return ep, (gate, gamma)


def _norm_gate(o, ep: _Epilogue):
    """One HIP pass: ep applied to o (..., dv), returned in o's dtype."""
    assert o.shape == ep.gate.shape, f'o {tuple(o.shape)} and gate {tuple(ep.gate.shape)} differ'
    if o.dtype not in _DTYPES:
        raise NotImplementedError(f'o must be one of {list(_DTYPES)}; got {o.dtype}')
    x = _aligned(o)
    out = torch.empty_like(x)
    e, keep = ep.struct(x.dtype)
    dv = x.shape[-1]
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().vgdr_norm_gate(_DTYPES[x.dtype], _ptr(x), ctypes.byref(e), _ptr(out),
                                              x.numel() // max(dv, 1), dv, _stream(x.device)))
    del keep
    return out


def rms_norm_gated(x, g, weight, bias=None, activation='swish', residual=None, prenorm=False,
                   residual_in_fp32=False, eps=1e-6):
    """RMSNorm(x) * weight * SiLU(g) over the last dim in one HIP pass: fla's
    rms_norm_gated as the reference calls it (linear_attention.py:820-823,
    bias None, activation 'swish'), equal to the torch expression at :825
    (norm_layer.py:15-24) up to rounding.  x, g: (..., D) in one dtype;
    weight: (D,) fp32 or x's dtype."""
    if bias is not None or residual is not None or prenorm or activation not in ('swish', 'silu'):
        raise NotImplementedError('rms_norm_gated: only bias=None, residual=None, prenorm=False and the '
                                  'swish / silu activation (the reference\'s call) are implemented')
    _check_grad(x, g, weight)
    return _norm_gate(x, _Epilogue(g, weight, eps))


def rms_norm(x, weight, eps: float = 1e-6, residual=None, out_residual=None):
    """The blocks' RMSNorm (infra/components/norm_layer.py:15-23) in one HIP
    pass over the last dim: dtype(dtype(h rsqrt(mean h^2 + eps)) * weight).
    With `residual`, h = x + residual (rounded to x's dtype: the residual add
    each block makes before its norm, infra/components/block.py:57-59), written
    into `out_residual` (a new tensor by default; x itself updates the stream in
    place) and returned with the norm: (y, h).  Without it h = x and only y is
    returned.  x, residual, weight in one dtype; no autograd."""
    _check_device(x, weight, residual, out_residual)
    _check_grad(x, weight, residual)
    if x.dtype not in _DTYPES:
        raise NotImplementedError(f'x must be one of {list(_DTYPES)}; got {x.dtype}')
    D = x.shape[-1]
    assert weight.shape == (D,) and weight.dtype == x.dtype, \
        f'weight must be ({D},) in {x.dtype}; got {tuple(weight.shape)} {weight.dtype}'
    xs = _aligned(x)
    w = _aligned(weight)
    r = h = None
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype, 'residual must match x'
        r = _aligned(residual)
        if out_residual is None:
            h = torch.empty_like(xs)
        else:
            assert out_residual.shape == x.shape and out_residual.dtype == x.dtype and out_residual.is_contiguous() \
                and out_residual.data_ptr() % 16 == 0, 'out_residual: contiguous, aligned, shaped and typed as x'
            h = out_residual
    y = torch.empty_like(xs)
    rows = xs.numel() // max(D, 1)
    with torch.cuda.device(xs.device):
        _lib.check(_lib.load().vgdr_rms_norm(_DTYPES[xs.dtype], _ptr(xs), _ptr(r), _ptr(h), _ptr(w), _ptr(y), rows,
                                             D, float(eps), _stream(xs.device)))
    return y if residual is None else (y, h)


def scalar_gates(x, w_ab, neg_exp_a, dt_bias, with_beta: bool = True):
    """The scalar gate and the beta logits of a decode token in one HIP pass
    (GatedDeltaNet._gates, linear_attention.py:719-721, :734-735): x (..., dim),
    w_ab = [W_a; W_b] (2H, dim) (W_a (H, dim) without beta), both in one dtype;
    neg_exp_a = -exp(A_log) and dt_bias fp32 (H,).  Returns g = neg_exp_a *
    softplus(W_a x + dt_bias) and beta = W_b x (the logits), fp32 (..., H), the
    projections rounded to x's dtype as nn.Linear returns them; beta is None
    without it.  No autograd."""
    _check_device(x, w_ab, neg_exp_a, dt_bias)
    _check_grad(x, w_ab)
    if x.dtype not in _DTYPES or w_ab.dtype != x.dtype:
        raise NotImplementedError(f'x and w_ab in one of {list(_DTYPES)}; got {x.dtype}, {w_ab.dtype}')
    D = x.shape[-1]
    H = w_ab.shape[0] // (2 if with_beta else 1)
    assert w_ab.shape == ((2 if with_beta else 1) * H, D), f'w_ab must be ({(2 if with_beta else 1)}H, {D})'
    na = neg_exp_a.float().contiguous()
    dtb = dt_bias.float().contiguous()
    assert na.shape == (H,) and dtb.shape == (H,), f'neg_exp_a and dt_bias must be ({H},)'
    xs, w = _aligned(x), _aligned(w_ab)
    g = torch.empty(*x.shape[:-1], H, dtype=torch.float32, device=x.device)
    beta = torch.empty_like(g) if with_beta else None
    with torch.cuda.device(xs.device):
        _lib.check(_lib.load().vgdr_scalar_gates(_DTYPES[xs.dtype], _ptr(xs), _ptr(w), _ptr(na), _ptr(dtb), _ptr(g),
                                                 _ptr(beta), xs.numel() // max(D, 1), D, H, _stream(xs.device)))
    return g, beta


def swiglu(x):
    """SiLU(x1) * xgate for x = [x1 | xgate] over the last dim in one HIP pass
    (the FFN's activation, infra/components/ffn.py:48-50), with the module's
    roundings (SiLU's result in x's dtype, then the product).  No autograd."""
    _check_device(x)
    _check_grad(x)
    if x.dtype not in _DTYPES:
        raise NotImplementedError(f'x must be one of {list(_DTYPES)}; got {x.dtype}')
    h2 = x.shape[-1]
    assert h2 % 2 == 0, 'swiglu needs an even last dim'
    xs = _aligned(x)
    y = torch.empty(*x.shape[:-1], h2 // 2, dtype=x.dtype, device=x.device)
    with torch.cuda.device(xs.device):
        _lib.check(_lib.load().vgdr_swiglu(_DTYPES[xs.dtype], _ptr(xs), _ptr(y), xs.numel() // max(h2, 1), h2 // 2,
                                           _stream(xs.device)))
    return y


class _ShortConv:
    """The q, k, v short conv + SiLU (opt.py:15-93) and its decode caches
    (linear_attention.py:929-941) for one decode call."""

    def __init__(self, weights, caches):
        assert weights is not None and caches is not None and len(weights) == 3 and len(caches) == 3, \
            'the short conv takes (w_q, w_k, w_v) and (qp_cache, kp_cache, vp_cache)'
        _check_device(*weights, *caches)
        self.K = weights[0].shape[-1]
        self.weights = [w.reshape(w.shape[0], self.K) for w in weights]
        for w in self.weights:
            assert w.shape[-1] == self.K, 'the three conv weights share one kernel size'
        self.caches = caches

    def struct(self, c):
        """(vgdr_short_conv, tensors to keep alive) for the validated call c."""
        if c.padded:
            raise NotImplementedError(f'the fused short conv needs dk in {_REC_DVS} and dv in {_DEC_DVS} '
                                      f'(no padding); got dk={c.dk}, dv={c.dv}')
        D = (c.H * c.dk, c.H * c.dk, c.H * c.dv)
        for w, d in zip(self.weights, D):
            assert w.shape == (d, self.K), f'conv weight must be ({d}, {self.K}) or ({d}, 1, {self.K}); got {tuple(w.shape)}'
        for x, d in zip(self.caches, D):
            assert x.shape == (c.N, self.K, d), f'conv cache must be {(c.N, self.K, d)}; got {tuple(x.shape)}'
            assert x.dtype == c.dtype and x.is_contiguous() and x.data_ptr() % 16 == 0, \
                'conv caches are updated in place: contiguous, aligned, in q\'s dtype'
        wdt = torch.float32 if all(w.dtype == torch.float32 for w in self.weights) else c.dtype
        ws = [w.to(wdt).contiguous() for w in self.weights]
        sc = _lib.ShortConv(weight_q=_ptr(ws[0]), weight_k=_ptr(ws[1]), weight_v=_ptr(ws[2]),
                            cache_q=_ptr(self.caches[0]), cache_k=_ptr(self.caches[1]),
                            cache_v=_ptr(self.caches[2]), kernel_size=self.K, weight_dtype=_DTYPES[wdt])
        return sc, ws


def _recurrent(q, k, v, g, beta, *, gate, delta, scale, initial_state, output_final_state,
               cu_seqlens, inplace_final_state=False, fusion: _Fusion = _NO_FUSION, epilogue=None,
               conv: _ShortConv | None = None, w=None, rows: bool = False, gate_proj=None):
    if (conv is None and epilogue is None and not inplace_final_state
            and _wants_grad(q, k, v, g, beta, initial_state, w)):
        # differentiable: the producers in torch, then the kernel with vgdr_scan_bwd as its backward
        if fusion.l2norm:
            q, k = _l2norm_rows(q), _l2norm_rows(k)
        if fusion.beta:
            beta = torch.sigmoid(beta.float())
        if fusion.gate:
            g = _gate_activation_rows(g, fusion)
        scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
        o, S = _ScanRule.apply(q, k, v, None if gate == 'none' else g, beta if (delta and w is None) else None,
                               initial_state, w, scale, cu_seqlens, 64, delta, True)
        return o, (S if output_final_state else None)
    dv = v.shape[-1]
    if w is not None:
        assert delta, 'an explicit write vector needs the delta rule'
        assert w.shape == q.shape, f'w must be {tuple(q.shape)} (B, T, H, dk); got {tuple(w.shape)}'
        if conv is not None or epilogue is not None:
            raise NotImplementedError('the explicit write vector runs without the short conv and the epilogue')
    # dv = 256 runs in one kernel as the layer's one-token decode step (the conv's
    # four taps, T = 1, no packed offsets, a state); other calls at that width
    # take 128-column slices (no conv, the epilogue as its own pass)
    wide_step = (conv is not None and dv == 256 and q.shape[1] == 1 and cu_seqlens is None
                 and initial_state is not None and w is None)
    if conv is not None and ((dv not in _REC_DVS and not wide_step) or q.shape[-1] not in _REC_DVS):
        raise NotImplementedError(f'the fused short conv needs dk in {_REC_DVS} and dv in {_REC_DVS} (or dv = 256 '
                                  f'for a one-token step from a state); got dk={q.shape[-1]}, dv={dv}')
    if epilogue is not None and dv not in _REC_DVS and not wide_step:
        # the fused epilogue needs the kernel's whole, unpadded dv row: apply it as its own pass
        o, S = _recurrent(q, k, v, g, beta, gate=gate, delta=delta, scale=scale, initial_state=initial_state,
                          output_final_state=output_final_state, cu_seqlens=cu_seqlens,
                          inplace_final_state=inplace_final_state, fusion=fusion)
        return _norm_gate(o, epilogue), S
    if dv > max(_REC_DVS) and not wide_step:
        # the recurrence is column-separable: independent 128-wide column blocks
        outs, states = [], []
        want_S = output_final_state or (inplace_final_state and initial_state is not None)
        for c0 in range(0, dv, 128):
            sl = slice(c0, min(dv, c0 + 128))
            s0 = None if initial_state is None else initial_state[..., sl]
            o_, s_ = _recurrent(q, k, v[..., sl], g, beta, gate=gate, delta=delta, scale=scale,
                                initial_state=s0, output_final_state=want_S,
                                cu_seqlens=cu_seqlens, fusion=fusion, w=w)
            outs.append(o_)
            states.append(s_)
        S = torch.cat(states, -1) if want_S else None
        if inplace_final_state and initial_state is not None:
            initial_state.copy_(S)
            S = initial_state
        return torch.cat(outs, -1), S
    # with w the delta rule's strength is in w: no beta is validated or passed
    dvs = _DEC_DVS if wide_step else _REC_DVS
    # rows (the layer's one-token step, the four-tap conv, a state): q, k, v and the
    # epilogue gate may be read in place as rows of one projection output
    one_token = (conv is not None and w is None and cu_seqlens is None and initial_state is not None
                 and conv.K == 4 and q.shape[1] == 1)
    rows = rows and one_token and (epilogue is None or _row_stride(epilogue.gate.reshape(v.shape)) is not None)
    if gate_proj is not None:
        # (x, W_ab, -exp(A_log), dt_bias): the decode kernel forms the scalar gate and
        # beta from x; any other call takes them from the gate kernel first
        x_, w_, na_, db_ = gate_proj
        dim = x_.shape[-1]
        fits = (one_token and gate == 'scalar' and x_.dtype == q.dtype and w_.dtype == q.dtype
                and dim % (16 // q.element_size()) == 0
                and dim <= 2 * (512 if dv > 128 else 256) * (16 // q.element_size()))
        if fits:
            gp_x = _aligned(x_.reshape(-1, dim))
            gp_w = _aligned(w_)
            gp_na, gp_db = na_.float().contiguous(), db_.float().contiguous()
        else:
            g, beta = scalar_gates(x_, w_, na_, db_, with_beta=delta)
            g, beta = g.reshape(q.shape[:3]), (beta.reshape(q.shape[:3]) if delta else None)
            gate_proj = None
    c = _Call(q, k, v, g, None if w is not None else beta, initial_state, cu_seqlens, gate=gate,
              delta=delta and w is None, dv_to=lambda d: next(x for x in dvs if x >= d), fusion=fusion, rows=rows,
              gate_proj=gate_proj is not None)
    if c.ld_qk and epilogue is not None and _row_stride(epilogue.gate.reshape(v.shape)) != c.ld_v:
        c.ld_qk = c.ld_v = 0                               # the gate's rows differ from v's: dense copies
        c.q, c.k, c.v = _aligned(c.q), _aligned(c.k), _aligned(c.v)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    o = c.new_output()
    in_place = (inplace_final_state and initial_state is not None and not c.padded
                and initial_state.dtype == torch.float32 and initial_state.is_contiguous())
    if in_place:
        S = initial_state
        h0 = initial_state
    else:
        S = c.new_state() if (output_final_state or inplace_final_state) else None
        h0 = c.h0
    L = _lib.load()
    with torch.cuda.device(c.device):
        head = (_DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
                _ptr(c.beta), _ptr(o), _ptr(h0), _ptr(S), _ptr(c.cu), c.B, c.T, c.H, c.dkp, c.dvp, c.N, scale)
        if w is not None:
            wk = _aligned(_pad_to(w.to(c.dtype), {1: c.dkp}))
            fz, keep = fusion.struct(c) if fusion.any else (None, None)
            _lib.check(L.vgdr_recurrent_fwd_w(_DTYPES[c.dtype], c.gate_kind, _ptr(c.q), _ptr(c.k), _ptr(c.v),
                                              _ptr(wk), _ptr(c.g), _ptr(o), _ptr(h0), _ptr(S), _ptr(c.cu), c.B, c.T,
                                              c.H, c.dkp, c.dvp, c.N, scale,
                                              None if fz is None else ctypes.byref(fz), _stream(c.device)))
            del keep
        elif conv is not None:
            fz, keep = fusion.struct(c) if fusion.any else (None, None)
            ep, keep_ep = (None, None)
            if epilogue is not None:
                assert epilogue.gate.shape == (c.B, c.T, c.H, c.dv), \
                    f'the epilogue gate must be {(c.B, c.T, c.H, c.dv)}; got {tuple(epilogue.gate.shape)}'
                ep, keep_ep = epilogue.struct(c.dtype, rows=bool(c.ld_qk))
            sc, keep_sc = conv.struct(c)
            fzp, scp, epp = (None if fz is None else ctypes.byref(fz)), ctypes.byref(sc), \
                (None if ep is None else ctypes.byref(ep))
            if c.ld_qk or gate_proj is not None:
                gp = None
                if gate_proj is not None:
                    gp = _lib.GateProj(x=_ptr(gp_x), w=_ptr(gp_w), neg_exp_a=_ptr(gp_na), dt_bias=_ptr(gp_db),
                                       dim=dim)
                _lib.check(L.vgdr_decode_step_strided(
                    _DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
                    _ptr(c.beta), _ptr(o), _ptr(h0), _ptr(S), c.B, c.H, c.dkp, c.dvp, c.ld_qk or c.H * c.dkp,
                    c.ld_v or c.H * c.dvp, scale, fzp, scp, epp, None if gp is None else ctypes.byref(gp),
                    _stream(c.device)))
            else:
                _lib.check(L.vgdr_decode_step(*head, fzp, scp, epp, _stream(c.device)))
            del keep, keep_ep, keep_sc
        elif epilogue is not None:
            assert epilogue.gate.shape == (c.B, c.T, c.H, c.dv), \
                f'the epilogue gate must be {(c.B, c.T, c.H, c.dv)}; got {tuple(epilogue.gate.shape)}'
            fz, keep = fusion.struct(c) if fusion.any else (None, None)
            ep, keep_ep = epilogue.struct(c.dtype)
            _lib.check(L.vgdr_recurrent_fwd_epilogue(*head, None if fz is None else ctypes.byref(fz),
                                                     ctypes.byref(ep), _stream(c.device)))
            del keep, keep_ep
        elif fusion.any:
            fz, keep = fusion.struct(c)
            _lib.check(L.vgdr_recurrent_fwd_fused(*head, ctypes.byref(fz), _stream(c.device)))
            del keep
        else:
            _lib.check(L.vgdr_recurrent_fwd(*head, _stream(c.device)))
    if in_place:
        return c.unpad_o(o), S
    S = c.unpad_state(S)
    if inplace_final_state and initial_state is not None:
        initial_state.copy_(S)
        S = initial_state
    return c.unpad_o(o), S


def fused_recurrent_gated_delta_rule(q, k, v, g=None, beta=None, scale=None, initial_state=None,
                                     output_final_state=False, cu_seqlens=None,
                                     inplace_final_state=False, use_qk_l2norm_in_kernel=False,
                                     use_beta_sigmoid_in_kernel=False):
    """Token-by-token GDN (decode: T = 1).  inplace_final_state writes the new
    state into initial_state (the decode step's state.copy_, linear_attention.py:950).
    The fusion flags are those of chunk_gated_delta_rule."""
    fz = _Fusion(l2norm=use_qk_l2norm_in_kernel, beta=use_beta_sigmoid_in_kernel)
    return _recurrent(q, k, v, g, beta, gate='scalar' if g is not None else 'none', delta=True,
                      scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                      cu_seqlens=cu_seqlens, inplace_final_state=inplace_final_state, fusion=fz)


def fused_recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                        cu_seqlens=None, inplace_final_state=False, use_qk_l2norm_in_kernel=False,
                        use_beta_sigmoid_in_kernel=False, use_gate_in_kernel=False, A_log=None,
                        dt_bias=None, safe_gate=False, lower_bound=None):
    """Token-by-token KDA (per-channel decay g (B, T, H, dk)); the fusion flags
    are those of chunk_kda."""
    fz = _kda_fusion(use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias,
                     safe_gate, lower_bound)
    return _recurrent(q, k, v, g, beta, gate='vector', delta=True, scale=scale,
                      initial_state=initial_state, output_final_state=output_final_state,
                      cu_seqlens=cu_seqlens, inplace_final_state=inplace_final_state, fusion=fz)


def hip_scan(q, k, v, g, beta, S0, *, scale: float, delta: bool, chunk_size: int = 64,
             l2norm_in_kernel: bool = False, gate_in_kernel: bool = False, beta_in_kernel: bool = False,
             A_log=None, dt_bias=None, disable_recompute: bool = False, lower_bound: float | None = None,
             cu_seqlens=None):
    """The contract of fla_scan (linear_attention.py:428-498), flags included:
    chunked scan from entry state S0 (or zeros), always returning (o in
    q.dtype, final S fp32).  g: None, (B, L, H) or (B, L, H, dk) (with
    gate_in_kernel the per-channel pre-activation).  The *_in_kernel flags are
    fused into the kernels; disable_recompute concerns a backward pass only."""
    gate = _gate_of(g)
    if gate_in_kernel:
        assert gate == 'vector', 'the fused gate activation is a KDA (vector-gate) kernel'
    if not delta:
        assert not l2norm_in_kernel and not beta_in_kernel, 'simple_gla takes no fused l2norm / beta'
    fz = _Fusion(l2norm=l2norm_in_kernel, beta=beta_in_kernel, gate=gate_in_kernel, A_log=A_log,
                 dt_bias=dt_bias, lower_bound=lower_bound if gate_in_kernel else None)
    return chunk_scan(q, k, v, g, beta, gate=gate, delta=delta, scale=scale,
                  initial_state=S0, output_final_state=True, cu_seqlens=cu_seqlens,
                  chunk_size=chunk_size, fusion=fz)


def hip_recurrent(q, k, v, g, beta, S0, *, scale: float, delta: bool, cu_seqlens=None,
                  inplace: bool = False, out_gate=None, out_norm_weight=None, out_norm_eps: float = 1e-6, w=None):
    """The contract of recurrent_scan (linear_attention.py:161-195) on the GPU:
    token-by-token from S0, returning (o, S).  inplace=True updates S0 itself.

    With out_gate (B, T, H, dv) (the W_g x projection, o's dtype) and
    out_norm_weight (dv,) (o_norm's gamma), o is returned through the layer's
    output epilogue RMSNorm(o) * SiLU(out_gate) (GatedDeltaNet._output before
    W_o, :814-825), computed by the same kernel: the decode step up to W_o.

    w (B, T, H, dk): explicit write vectors in place of beta_t k_t (the
    asymmetric delta rule, recurrent_scan's w, :161-170); beta is then unused."""
    ep = None
    if out_gate is not None or out_norm_weight is not None:
        ep = _Epilogue(out_gate, out_norm_weight, out_norm_eps)
    return _recurrent(q, k, v, g, beta, gate=_gate_of(g), delta=delta, scale=scale,
                      initial_state=S0, output_final_state=True, cu_seqlens=cu_seqlens,
                      inplace_final_state=inplace, epilogue=ep, w=w)


def hip_decode_step(qp, kp, vp, g, beta, state, *, scale: float, delta: bool = True, conv_weights=None,
                    conv_cache=None, l2norm: bool = True, beta_logits: bool = False, gate_in_kernel: bool = False,
                    A_log=None, dt_bias=None, lower_bound: float | None = None, out_gate=None,
                    out_norm_weight=None, out_norm_eps: float = 1e-6, cu_seqlens=None, gate_proj=None):
    """GatedDeltaNet.decode_step (linear_attention.py:918-952) from the
    projections to the input of W_o, in one kernel.

    qp, kp: (B, L, H*dk) or (B, L, H, dk), vp: (B, L, H*dv) or (B, L, H, dv), the
    raw projections W_q x, W_k x, W_v x.  For one token per sequence they (and
    out_gate) may be column slices of one (B, 1, n) projection output: the kernel
    then reads them in place (vgdr_decode_step_strided) instead of from copies.
    gate_proj (x, W_ab, -exp(A_log), dt_bias), for the scalar gate in place of g
    and beta: x (B, 1, dim) is the layer's input, W_ab [W_a; W_b] (W_a alone
    without the delta rule); the kernel forms g = -exp(A_log) softplus(W_a x +
    dt_bias) and the beta logits W_b x itself (linear_attention.py:719-721,
    :734-735), with nn.Linear's rounding of W_a x and W_b x.  conv_weights (w_q, w_k, w_v): the
    ShortConv weights, (D, 1, K) or (D, K); conv_cache (qp_cache, kp_cache,
    vp_cache): (N, K, D) in q's dtype, advanced in place (:929-941).  The
    kernel applies the conv and SiLU (:741-745), the q, k L2 norm unless
    l2norm=False (:746-747), sigmoid to beta logits with beta_logits, the KDA
    gate activation with gate_in_kernel (g is then the pre-activation), the
    recurrence from `state`, which it updates in place (:945-950), and with
    out_gate / out_norm_weight the RMSNorm x SiLU(gate) epilogue (:814-825).
    Returns o (B, L, H, dv) in q's dtype.  dk, dv in {64, 128}; dv = 256 for
    a one-token step (L = 1, no cu_seqlens) with the four-tap conv."""
    B, L = qp.shape[0], qp.shape[1]
    H = state.shape[1]
    dk, dv = state.shape[2], state.shape[3]
    q = qp.reshape(B, L, H, dk)
    k = kp.reshape(B, L, H, dk)
    v = vp.reshape(B, L, H, dv)
    gate = 'scalar' if gate_proj is not None else _gate_of(g)
    if gate_in_kernel:
        assert gate == 'vector', 'the fused gate activation is a KDA (vector-gate) kernel'
    fz = _Fusion(l2norm=l2norm, beta=beta_logits, gate=gate_in_kernel, A_log=A_log, dt_bias=dt_bias,
                 lower_bound=lower_bound if gate_in_kernel else None)
    ep = None
    if out_gate is not None or out_norm_weight is not None:
        ep = _Epilogue(out_gate.reshape(B, L, H, dv) if out_gate is not None else None, out_norm_weight,
                       out_norm_eps)
    o, _ = _recurrent(q, k, v, g, beta, gate=gate, delta=delta, scale=scale, initial_state=state,
                      output_final_state=True, cu_seqlens=cu_seqlens, inplace_final_state=True, fusion=fz,
                      epilogue=ep, conv=_ShortConv(conv_weights, conv_cache), rows=True, gate_proj=gate_proj)
    return o


def causal_conv1d(x, weight, bias=None, residual=None, initial_state=None, output_final_state=False,
                  activation=None, cu_seqlens=None, conv_cache=None):
    """The short causal depthwise conv over the sequence, with the activation
    (opt.py:15-100): fla's causal_conv1d as the reference calls it
    (opt.py:73-77, ``causal_conv1d(x, w, activation='silu')``), one HIP pass.

    x: (B, T, D) (B = 1 with cu_seqlens); weight: (D, K) or (D, 1, K), K <= 8;
    activation: None, 'silu' or 'swish'.  Returns (y, final_state).
    conv_cache: (N, K, D) in x's dtype, the module's decode cache layout
    (linear_attention.py:929-941): the conv continues from it, and it is
    advanced in place to the last K inputs (the cached conv of a multi-token
    decode_step).  output_final_state without conv_cache returns a new
    (N, K, D) cache; with it, the advanced conv_cache itself.  fla's own
    initial_state layout (N, D, K), bias and residual are not implemented."""
    if bias is not None or residual is not None or initial_state is not None:
        raise NotImplementedError('causal_conv1d: bias, residual and fla-layout initial_state are not '
                                  'implemented (pass the (N, K, D) cache as conv_cache)')
    if activation not in (None, 'silu', 'swish'):
        raise NotImplementedError(f'causal_conv1d: activation {activation!r} (None, silu, swish)')
    _check_device(x, weight, cu_seqlens, conv_cache)
    _check_grad(x, weight)
    assert x.dim() == 3, f'x must be (B, T, D); got {tuple(x.shape)}'
    if x.dtype not in _DTYPES:
        raise NotImplementedError(f'x must be one of {list(_DTYPES)}; got {x.dtype}')
    B, T, D = x.shape
    K = weight.shape[-1]
    w = weight.reshape(D, K)
    w = w.contiguous() if w.dtype in (torch.float32, x.dtype) else w.float().contiguous()
    if cu_seqlens is not None:
        assert B == 1, f'packed varlen input (cu_seqlens) has batch 1, got {B}'
        _check_cu(cu_seqlens, T)
        cu = cu_seqlens.to(torch.int32).contiguous()
        N = cu.numel() - 1
    else:
        cu, N = None, B
    xa = _aligned(x)
    y = torch.empty_like(xa)
    st_in = st_out = None
    if conv_cache is not None:
        assert conv_cache.shape == (N, K, D), f'conv_cache must be {(N, K, D)}; got {tuple(conv_cache.shape)}'
        assert conv_cache.dtype == x.dtype and conv_cache.is_contiguous() and conv_cache.data_ptr() % 16 == 0, \
            'conv_cache is advanced in place: contiguous, aligned, in x\'s dtype'
        st_in = st_out = conv_cache
    elif output_final_state:
        st_out = torch.empty(N, K, D, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().vgdr_causal_conv1d(_DTYPES[x.dtype], _ptr(xa), _ptr(w), _DTYPES[w.dtype], _ptr(st_in),
                                                  _ptr(y), _ptr(st_out), _ptr(cu), B, T, D, N, K,
                                                  0 if activation is None else 1, _stream(x.device)))
    return y, (st_out if output_final_state else None)


def chunk_write_bwd(q, k, v, w, g, initial_state, do, dht=None, *, scale=None, cu_seqlens=None, chunk_size=64):
    """Backward of chunk_scan_vec with explicit write vectors w (B, T, H, dk)
    without autograd (vgdr_chunk_bwd_w; 16-bit q, k, v, w, per-channel g,
    run in 64-token chunks whatever chunk_size asks): the gradients of (o,
    final_state) under do (and dht, None = zero).  Returns (dq, dk, dv, dw,
    dg, dh0), dh0 None without an initial state."""
    c = _Call(q, k, v, g, None, initial_state, cu_seqlens, gate='vector', delta=False,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV)
    chunk_size = _VEC_BWD_CHUNK
    scale = c.dk ** -0.5 if scale is None else float(scale)
    assert w.shape == q.shape, f'w must be {tuple(q.shape)} (B, T, H, dk); got {tuple(w.shape)}'
    assert do.shape == (c.B, c.T, c.H, c.dv), f'do must be {(c.B, c.T, c.H, c.dv)}, got {tuple(do.shape)}'
    _check_device(w, do, dht)
    wk = _aligned(_pad_to(w.to(c.dtype), {1: c.dkp}))
    dop = _aligned(_pad_to(do.to(c.dtype), {1: c.dvp}))
    dSp = None if dht is None else _aligned(_pad_to(dht.float(), {1: c.dvp, 2: c.dkp}))
    new = lambda *shape, dt=torch.float32: torch.empty(*shape, dtype=dt, device=c.device)
    dq, dk, dw = (new(c.B, c.T, c.H, c.dkp, dt=c.dtype) for _ in range(3))
    dv = new(c.B, c.T, c.H, c.dvp, dt=c.dtype)
    dg = new(c.B, c.T, c.H, c.dkp)
    dS0 = new(c.N, c.H, c.dkp, c.dvp) if initial_state is not None else None
    L = _lib.load()
    dtype = _DTYPES[c.dtype]
    nbytes = L.vgdr_chunk_bwd_workspace_size(dtype, _lib.VGDR_GATE_VECTOR, c.B, c.T, c.H, c.dkp, c.dvp, c.N,
                                             int(c.cu is not None), int(chunk_size))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        _lib.check(L.vgdr_chunk_bwd_w(dtype, _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(wk), _ptr(c.g), _ptr(c.h0),
                                      _ptr(dop), _ptr(dSp), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dw), _ptr(dg),
                                      _ptr(dS0), _ptr(c.cu), _ptr(ws), nbytes, c.B, c.T, c.H, c.dkp, c.dvp, c.N,
                                      scale, int(chunk_size), _stream(c.device)))
    if c.dkp != c.dk:
        dq, dk, dw, dg = dq[..., :c.dk], dk[..., :c.dk], dw[..., :c.dk], dg[..., :c.dk]
    if c.dvp != c.dv:
        dv = dv[..., :c.dv]
    if dS0 is not None:
        dS0 = c.unpad_state(dS0).to(initial_state.dtype)
    return dq, dk, dv, dw.to(w.dtype), dg.to(g.dtype), dS0


class _ChunkWrite(torch.autograd.Function):
    """chunk_scan_vec with explicit write vectors, differentiable: forward
    vgdr_chunk_fwd_w, backward vgdr_chunk_bwd_w (the per-channel chunk
    backward on chunk prep's WR blocks, which it rebuilds with the entry
    states, in 64-token chunks).  16-bit q, k, v, w, per-channel g."""

    @staticmethod
    def forward(ctx, q, k, v, g, S0, w, scale, cu, chunk_size):
        o, S = chunk_scan_vec(q, k, v, g, None, S0, scale=scale, delta=True, chunk_size=chunk_size, w=w,
                              cu_seqlens=cu)
        ctx.save_for_backward(q, k, v, g, S0, w, cu)
        ctx.scale, ctx.chunk_size = scale, chunk_size
        return o, S

    @staticmethod
    def backward(ctx, do, dS):
        q, k, v, g, S0, w, cu = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        dq, dk, dv, dw, dg, dS0 = chunk_write_bwd(q, k, v, w, g, S0, do, dS, scale=ctx.scale, cu_seqlens=cu,
                                                  chunk_size=_VEC_BWD_CHUNK)
        return dq, dk, dv, dg, dS0, dw, None, None, None


def chunk_scan_vec(q, k, v, g, beta, S0, *, scale: float, delta: bool, chunk_size: int = 64, w=None,
                   cu_seqlens=None):
    """The reference's chunk_scan_vec (linear_attention.py:312-425) on the GPU,
    including its explicit write vectors: returns (o in q's dtype, final S fp32).

    g: (B, T, H, dk) per-channel log-decay; a (B, T, H) scalar gate or None is
    taken as the same decay on every channel.  w (B, T, H, dk): write vectors
    in place of beta_t k_t (the asymmetric delta rule, :340-353, :389-396;
    beta unused), run chunkwise with 16-bit q, k, v and token by token (the
    same rule, vgdr_recurrent_fwd_w) in fp32.  Without w it is chunk_kda.
    Differentiable when an input requires grad: with w, vgdr_chunk_bwd_w for
    16-bit inputs (in 64-token chunks), vgdr_scan_bwd for fp32."""
    B, T, H, dk = q.shape
    if w is not None and _wants_grad(q, k, v, g, beta, S0, w):
        assert delta, 'an explicit write vector needs the delta rule'
        scale = dk ** -0.5 if scale is None else float(scale)
        if q.dtype == torch.float32:
            return _ScanRule.apply(q, k, v, g, None, S0, w, scale, cu_seqlens, chunk_size, True)
    if g is None:
        g = torch.zeros(B, T, H, dk, dtype=torch.float32, device=q.device)
    elif g.dim() == 3:
        g = g.float().unsqueeze(-1).expand(B, T, H, dk)
    if w is not None and _wants_grad(q, k, v, g, beta, S0, w):
        return _ChunkWrite.apply(q, k, v, g, S0, w, scale, cu_seqlens, chunk_size)
    if w is None:
        return chunk_scan(q, k, v, g, beta, gate='vector', delta=delta, scale=scale, initial_state=S0,
                          output_final_state=True, cu_seqlens=cu_seqlens, chunk_size=chunk_size)
    assert delta, 'an explicit write vector needs the delta rule'
    assert w.shape == q.shape, f'w must be {tuple(q.shape)} (B, T, H, dk); got {tuple(w.shape)}'
    if q.dtype == torch.float32:
        return _recurrent(q, k, v, g, None, gate='vector', delta=True, scale=scale, initial_state=S0,
                          output_final_state=True, cu_seqlens=cu_seqlens, w=w)
    c = _Call(q, k, v, g, None, S0, cu_seqlens, gate='vector', delta=False,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    wk = _aligned(_pad_to(w.to(c.dtype), {1: c.dkp}))
    o = c.new_output()
    S = c.new_state()
    L = _lib.load()
    varlen = c.cu is not None
    nbytes = L.vgdr_chunk_workspace_size(_DTYPES[c.dtype], _lib.VGDR_GATE_VECTOR, c.B, c.T, c.H, c.dkp, c.N,
                                         int(varlen), int(chunk_size))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        _lib.check(L.vgdr_chunk_fwd_w(_DTYPES[c.dtype], _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(wk), _ptr(c.g), _ptr(o),
                                      _ptr(c.h0), _ptr(S), _ptr(c.cu), _ptr(ws), nbytes, c.B, c.T, c.H, c.dkp, c.dvp,
                                      c.N, scale, int(chunk_size), None, _stream(c.device)))
    return c.unpad_o(o), c.unpad_state(S)
