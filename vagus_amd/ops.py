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
back in q's dtype.  Every call runs the HIP kernels of libvagus_gdr.so on the
current stream; there is no CPU path and no autograd (backward is out of
scope: inputs that require grad raise NotImplementedError).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_DTYPES = {torch.float32: _lib.VGDR_F32, torch.bfloat16: _lib.VGDR_BF16, torch.float16: _lib.VGDR_F16}
_CHUNK_TILE_DV = 16          # the chunk kernel takes dv in multiples of 16
_REC_DVS = (64, 128)         # the recurrent kernel's column widths


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


def _check_grad(*ts):
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts):
        raise NotImplementedError('vagus_amd implements the forward pass only (no backward)')


class _Call:
    """Validated, padded, contiguous operands of one kernel call."""

    def __init__(self, q, k, v, g, beta, initial_state, cu_seqlens, *, gate: str, delta: bool,
                 dv_to):
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
        elif gate == 'scalar':
            assert g is not None and g.shape == (B, T, H), \
                f'a scalar gate is (B, T, H); got {None if g is None else tuple(g.shape)}'
        if delta:
            assert beta is not None and beta.shape == (B, T, H), 'the delta rule needs beta (B, T, H)'
        if cu_seqlens is not None:
            assert B == 1, f'packed varlen input (cu_seqlens) has batch 1, got {B}'
            assert cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 1, 'cu_seqlens is 1-D with N + 1 entries'
            assert not cu_seqlens.is_floating_point(), 'cu_seqlens holds integer offsets'
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
        self.q = _aligned(_pad_to(q, {1: dkp}))
        self.k = _aligned(_pad_to(k, {1: dkp}))
        self.v = _aligned(_pad_to(v, {1: dvp}))
        if gate == 'none' or g is None:
            self.g, self.gate_kind = None, _lib.VGDR_GATE_NONE
        elif gate == 'vector':
            self.g, self.gate_kind = _aligned(_pad_to(g.float(), {1: dkp})), _lib.VGDR_GATE_VECTOR
        else:
            self.g, self.gate_kind = g.float().contiguous(), _lib.VGDR_GATE_SCALAR
        self.beta = beta.float().contiguous() if delta else None
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


def chunk_scan(q, k, v, g, beta, *, gate, delta, scale=None, initial_state=None, output_final_state=False,
               cu_seqlens=None, chunk_size=64, phase_event=None):
    """Chunkwise prefill, the general form behind chunk_gated_delta_rule,
    chunk_kda and chunk_simple_gla: gate in {'none', 'scalar', 'vector'},
    delta selects the delta rule.  Returns (o, final_state or None).

    phase_event: optional torch.cuda.Event recorded on the current stream
    between the chunk-prep and the chunk-state kernels (the same two launches
    either way), so that a caller can time the two phases separately."""
    c = _Call(q, k, v, g, beta, initial_state, cu_seqlens, gate=gate, delta=delta,
              dv_to=lambda d: -(-d // _CHUNK_TILE_DV) * _CHUNK_TILE_DV)
    scale = c.dk ** -0.5 if scale is None else float(scale)
    o = c.new_output()
    S = c.new_state() if output_final_state else None
    L = _lib.load()
    varlen = c.cu is not None
    nbytes = L.vgdr_chunk_workspace_size(_DTYPES[c.dtype], c.gate_kind, c.B, c.T, c.H, c.dkp, c.N, int(varlen),
                                         int(chunk_size))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        args = (_DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
                _ptr(c.beta), _ptr(o), _ptr(c.h0), _ptr(S), _ptr(c.cu), _ptr(ws), nbytes,
                c.B, c.T, c.H, c.dkp, c.dvp, c.N, scale, int(chunk_size), _stream(c.device))
        if phase_event is None:
            _lib.check(L.vgdr_chunk_fwd(*args))
        else:
            _lib.check(L.vgdr_chunk_prep(*args))
            phase_event.record(torch.cuda.current_stream(c.device))
            _lib.check(L.vgdr_chunk_state(*args))
    return c.unpad_o(o), c.unpad_state(S)


def _unsupported(**flags):
    on = [k for k, v in flags.items() if v]
    if on:
        raise NotImplementedError(f'vagus_amd does not implement {on} yet (pass the activated '
                                  'inputs, as the unfused reference path does)')


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, cu_seqlens=None, chunk_size=64,
                           use_qk_l2norm_in_kernel=False, use_beta_sigmoid_in_kernel=False):
    """GDN chunkwise prefill (the call at linear_attention.py:487-491).

    g: (B, T, H) log-decay (None for DeltaNet, a = 1).  Returns (o, final_state),
    final_state None unless output_final_state."""
    _unsupported(use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                 use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel)
    return chunk_scan(q, k, v, g, beta, gate='scalar' if g is not None else 'none', delta=True,
                  scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size)


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
              cu_seqlens=None, chunk_size=64, use_qk_l2norm_in_kernel=False,
              use_beta_sigmoid_in_kernel=False, use_gate_in_kernel=False, A_log=None, dt_bias=None,
              safe_gate=False, lower_bound=None, disable_recompute=False):
    """KDA chunkwise prefill (the call at linear_attention.py:474-479).

    g: (B, T, H, dk) per-channel log-decay.  disable_recompute only concerns a
    backward pass and is accepted and ignored; safe_gate / lower_bound belong to
    the fused gate activation."""
    _unsupported(use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                 use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel,
                 use_gate_in_kernel=use_gate_in_kernel, safe_gate=safe_gate)
    return chunk_scan(q, k, v, g, beta, gate='vector', delta=True, scale=scale,
                  initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size)


def chunk_simple_gla(q, k, v, g, scale=None, initial_state=None, output_final_state=False,
                     cu_seqlens=None, chunk_size=64):
    """Gated linear attention without the delta rule (the call at linear_attention.py:495-497):
    S_t = a_t S_{t-1} + k_t v_t^T.  g: (B, T, H) or None."""
    return chunk_scan(q, k, v, g, None, gate='scalar' if g is not None else 'none', delta=False,
                  scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                  cu_seqlens=cu_seqlens, chunk_size=chunk_size)


def _recurrent(q, k, v, g, beta, *, gate, delta, scale, initial_state, output_final_state,
               cu_seqlens, inplace_final_state=False):
    dv = v.shape[-1]
    if dv > max(_REC_DVS):
        # the recurrence is column-separable: independent 128-wide column blocks
        outs, states = [], []
        for c0 in range(0, dv, 128):
            sl = slice(c0, min(dv, c0 + 128))
            s0 = None if initial_state is None else initial_state[..., sl]
            o_, s_ = _recurrent(q, k, v[..., sl], g, beta, gate=gate, delta=delta, scale=scale,
                                initial_state=s0, output_final_state=output_final_state,
                                cu_seqlens=cu_seqlens)
            outs.append(o_)
            states.append(s_)
        S = torch.cat(states, -1) if output_final_state else None
        if inplace_final_state and initial_state is not None:
            initial_state.copy_(S)
            S = initial_state
        return torch.cat(outs, -1), S
    c = _Call(q, k, v, g, beta, initial_state, cu_seqlens, gate=gate, delta=delta,
              dv_to=lambda d: next(x for x in _REC_DVS if x >= d))
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
        _lib.check(L.vgdr_recurrent_fwd(
            _DTYPES[c.dtype], c.gate_kind, int(delta), _ptr(c.q), _ptr(c.k), _ptr(c.v), _ptr(c.g),
            _ptr(c.beta), _ptr(o), _ptr(h0), _ptr(S), _ptr(c.cu), c.B, c.T, c.H, c.dkp, c.dvp, c.N,
            scale, _stream(c.device)))
    if in_place:
        return c.unpad_o(o), S
    S = c.unpad_state(S)
    if inplace_final_state and initial_state is not None:
        initial_state.copy_(S)
        S = initial_state
    return c.unpad_o(o), S


def fused_recurrent_gated_delta_rule(q, k, v, g=None, beta=None, scale=None, initial_state=None,
                                     output_final_state=False, cu_seqlens=None,
                                     inplace_final_state=False):
    """Token-by-token GDN (decode: T = 1).  inplace_final_state writes the new
    state into initial_state (the decode step's state.copy_, linear_attention.py:950)."""
    return _recurrent(q, k, v, g, beta, gate='scalar' if g is not None else 'none', delta=True,
                      scale=scale, initial_state=initial_state, output_final_state=output_final_state,
                      cu_seqlens=cu_seqlens, inplace_final_state=inplace_final_state)


def fused_recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                        cu_seqlens=None, inplace_final_state=False):
    """Token-by-token KDA (per-channel decay g (B, T, H, dk))."""
    return _recurrent(q, k, v, g, beta, gate='vector', delta=True, scale=scale,
                      initial_state=initial_state, output_final_state=output_final_state,
                      cu_seqlens=cu_seqlens, inplace_final_state=inplace_final_state)


def _gate_of(g) -> str:
    if g is None:
        return 'none'
    return 'vector' if g.dim() == 4 else 'scalar'


def hip_scan(q, k, v, g, beta, S0, *, scale: float, delta: bool, chunk_size: int = 64,
             cu_seqlens=None):
    """The contract of fla_scan (linear_attention.py:428-498): chunked scan from
    entry state S0 (or zeros), always returning (o in q.dtype, final S fp32).
    g: None, (B, L, H) or (B, L, H, dk)."""
    return chunk_scan(q, k, v, g, beta, gate=_gate_of(g), delta=delta, scale=scale,
                  initial_state=S0, output_final_state=True, cu_seqlens=cu_seqlens,
                  chunk_size=chunk_size)


def hip_recurrent(q, k, v, g, beta, S0, *, scale: float, delta: bool, cu_seqlens=None,
                  inplace: bool = False):
    """The contract of recurrent_scan (linear_attention.py:161-195) on the GPU:
    token-by-token from S0, returning (o, S).  inplace=True updates S0 itself."""
    return _recurrent(q, k, v, g, beta, gate=_gate_of(g), delta=delta, scale=scale,
                      initial_state=S0, output_final_state=True, cu_seqlens=cu_seqlens,
                      inplace_final_state=inplace)
