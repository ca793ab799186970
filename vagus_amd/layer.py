"""The gated delta-rule layer over the HIP kernels: a drop-in for the
reference's ``GatedDeltaNet`` module (infra/components/linear_attention.py:
531-952) and the two modules it is built from, ``ShortConv``
(infra/components/opt.py:15-100) and ``RMSNorm``
(infra/components/norm_layer.py:4-24).

Same constructor arguments, same parameter names, shapes and initial
distributions, so a state_dict of the reference module loads unchanged; the
same stateless ``forward`` and streaming ``reset_cache`` / ``load_cache`` /
``export_cache`` / ``decode_step`` with the module's cache format
(:888-952).  The routing keeps the reference's three decisions
(:755-812):

* ``_pick_impl``: the reference picks fla for CUDA half-precision tensors and
  its torch chunk form otherwise.  Here the HIP kernels are the only
  implementation (fp32, bf16 and fp16 on the GPU); ``impl`` 'auto', 'hip' and
  'fla' (the kernels stand where fla's did) select them, and a CPU tensor or
  ``impl='torch'`` raises.
* ``_active_fusions``: the configured fusions minus those the scan cannot
  take (no beta or L2 norm without the delta rule, the gate activation only
  for the per-channel gate).  'l2norm', 'gate' and 'beta' go into the scan
  kernels as fla's flags do.  The short conv and the RMSNorm x SiLU output
  epilogue always run as their HIP kernels ('conv' and 'norm_gate' are
  accepted and change nothing).
* ``_scan``: an explicit write vector w goes to the per-channel chunk form
  with w (chunk_scan_vec, :792-800); everything else to the chunked scan.

Streaming: a one-token ``decode_step`` is one kernel from the projections to
the input of W_o (short conv with its cache, L2 norm, beta sigmoid, gate,
recurrence updating the state in place, epilogue); a longer block runs the
conv continuing from the cache and the chunked scan from the state.
``prefill_packed`` pushes ragged sequences, packed with cu_seqlens, into cache
rows: the continuous batching the reference's Generator cannot do
(generator.py:19-22).

Projections (W_q, W_k, W_v, W_g, W_o, the gate and beta maps) are torch
GEMMs, and the scalar gate's softplus is torch elementwise work on the GPU, as
in the reference.  Training: the scans differentiate through their HIP
backward kernels; the short conv and the output epilogue have none, so when
autograd needs their gradients they run as the reference's torch
expressions on the GPU (inference always runs the kernels).
"""
from __future__ import annotations

import math

import torch
from torch import nn
from torch.nn import functional as F

from . import ops

GATES = ('none', 'scalar', 'vector')
FUSIONS = ('conv', 'l2norm', 'gate', 'beta', 'norm_gate')
_ALIASES = {'scan': ('l2norm', 'gate', 'beta'), 'all': FUSIONS}
IMPLS = ('auto', 'hip', 'fla', 'torch')
CONV_IMPLS = ('conv1d', 'shift', 'fla')


def _autograd(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def parse_fusions(spec) -> frozenset:
    """`fused=` as the reference accepts it (linear_attention.py:95-112): True
    (all), False / None (none), or a subset ('gate', 'conv,gate', 'scan' =
    l2norm, gate, beta, or a list)."""
    if spec is True:
        return frozenset(FUSIONS)
    if not spec:
        return frozenset()
    names = [s.strip() for s in spec.split(',')] if isinstance(spec, str) else list(spec)
    out: set[str] = set()
    for n in names:
        if n:
            out.update(_ALIASES.get(n, (n,)))
    bad = out - set(FUSIONS)
    assert not bad, f'unknown fusion {sorted(bad)}; pick from {FUSIONS} or {sorted(_ALIASES)}'
    return frozenset(out)


class RMSNorm(nn.Module):
    """x rsqrt(mean x^2 + eps) in at least fp32, cast back, times gamma
    (norm_layer.py:15-24)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        assert dim > 0 and eps > 0
        self.eps = eps
        self.dim = dim
        self.gamma = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        h = x.to(torch.promote_types(x.dtype, torch.float32))
        h = h * torch.rsqrt(h.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return h.to(x.dtype) * self.gamma


class ShortConv(nn.Module):
    """Depthwise causal conv over the sequence with its activation
    (opt.py:15-100), as one HIP pass (vgdr_causal_conv1d).  The parameter is
    the reference's nn.Conv1d weight (D, 1, K); `impl` is accepted for
    interface parity (all three of the reference's paths compute this)."""

    def __init__(self, dim: int, kernel: int, impl: str = 'conv1d'):
        super().__init__()
        assert dim > 0 and kernel > 0
        assert impl in CONV_IMPLS, f'{impl!r} not in {CONV_IMPLS}'
        self.kernel = kernel
        self.impl = impl
        self.conv = nn.Conv1d(dim, dim, kernel, groups=dim, bias=False)

    def forward(self, x, activation: str | None = None, *, cu_seqlens=None, conv_cache=None):
        """x (B, L, D) -> (B, L, D), causal.  conv_cache (N, K, D): continue
        from it and advance it in place (a multi-token decode block)."""
        if _autograd(x, self.conv.weight) and cu_seqlens is None and conv_cache is None:
            # the reference's 'conv1d' path (opt.py:78-80), for its gradients
            y = self.conv(F.pad(x.transpose(1, 2), (self.kernel - 1, 0))).transpose(1, 2)
            return F.silu(y) if activation is not None else y
        y, _ = ops.causal_conv1d(x, self.conv.weight, activation=activation, cu_seqlens=cu_seqlens,
                                 conv_cache=conv_cache)
        return y


class GatedDeltaNet(nn.Module):
    """Gated delta-rule linear attention (GDN: gate='scalar'; KDA:
    gate='vector'; DeltaNet: gate='none'; simple GLA: delta=False) on the HIP
    kernels.  Arguments as the reference's (linear_attention.py:570-592);
    `impl` also takes 'hip'."""

    def __init__(
            self,
            dim: int,
            head_count: int,
            key_head_dim: int,
            value_head_dim: int,
            short_conv_size: int | None = 4,
            gate: str | bool = 'vector',
            delta: bool = True,
            gate_rank: int = 64,
            chunk_size: int = 64,
            impl: str = 'auto',
            fused: bool | str | list = False,
            conv_impl: str = 'conv1d',
            disable_recompute: bool = False,
            gate_lower_bound: float | None = None,
            *,
            init_std: float = 0.02,
            layer_count: int | None = None,
            A_init_range: tuple[float, float] = (1.0, 16.0),
            dt_init_range: tuple[float, float] = (1e-3, 1e-1),
            out_proj: bool = True,
    ):
        super().__init__()
        if isinstance(gate, bool):                     # legacy spelling: True = scalar (GDN)
            gate = 'scalar' if gate else 'none'
        assert gate in GATES, gate
        assert dim > 0 and head_count > 0 and key_head_dim > 0 and value_head_dim > 0
        assert impl in IMPLS, impl
        if impl == 'torch':
            raise NotImplementedError("impl='torch' is the reference's CPU chunk form; this layer runs "
                                      "the HIP kernels only (impl 'auto', 'hip' or 'fla')")
        assert gate_lower_bound is None or gate == 'vector', \
            'the bounded decay is a KDA (vector-gate) parameterisation'
        assert gate_lower_bound is None or -5 <= gate_lower_bound < 0, \
            f'gate_lower_bound must be in [-5, 0), got {gate_lower_bound}'
        assert chunk_size in (32, 64), f'chunk_size must be 32 or 64 (the kernels\' tiles); got {chunk_size}'

        self.dim = dim
        self.head_count = head_count
        self.key_head_dim = key_head_dim
        self.value_head_dim = value_head_dim
        self.short_conv_size = short_conv_size
        self.gate = gate
        self.delta = delta
        self.gate_rank = gate_rank
        self.chunk_size = chunk_size
        self.impl = impl
        self.fusions = parse_fusions(fused)
        self.disable_recompute = disable_recompute
        self.gate_lower_bound = gate_lower_bound
        self.scale = key_head_dim ** -0.5
        self.out_proj = out_proj
        self.out_width = head_count * value_head_dim

        H, dk, dv = head_count, key_head_dim, value_head_dim
        self.wq = nn.Linear(dim, H * dk, bias=False)
        self.wk = nn.Linear(dim, H * dk, bias=False)
        self.wv = nn.Linear(dim, H * dv, bias=False)
        self.wg = nn.Linear(dim, H * dv, bias=False)          # output gate
        if out_proj:
            self.wo = nn.Linear(H * dv, dim, bias=False)
        self.o_norm = RMSNorm(dv)                             # per head, gamma shared

        if short_conv_size is not None:
            self.conv_q = ShortConv(H * dk, short_conv_size, impl=conv_impl)
            self.conv_k = ShortConv(H * dk, short_conv_size, impl=conv_impl)
            self.conv_v = ShortConv(H * dv, short_conv_size, impl=conv_impl)

        if gate != 'none':
            n_dt = H * dk if gate == 'vector' else H
            if gate == 'vector':
                self.wa1 = nn.Linear(dim, gate_rank, bias=False)
                self.wa2 = nn.Linear(gate_rank, H * dk, bias=False)
            else:
                self.wa = nn.Linear(dim, H, bias=False)
            A = torch.empty(H).uniform_(*A_init_range)
            self.A_log = nn.Parameter(A.log())
            lo, hi = math.log(dt_init_range[0]), math.log(dt_init_range[1])
            dt = torch.exp(torch.rand(n_dt) * (hi - lo) + lo).clamp(min=1e-4)
            # dt_bias makes the gate's own activation return -dt at f = 0
            # (:650-666): the softplus inverse, or for the bounded gate the
            # logit that matches the softplus form's decay A dt there
            if gate_lower_bound is None:
                bias = dt + torch.log(-torch.expm1(-dt))
            else:
                a = A.repeat_interleave(dk)
                p = (a * dt / -gate_lower_bound).clamp(1e-6, 1 - 1e-6)
                bias = torch.logit(p) / a
            self.dt_bias = nn.Parameter(bias)
        if delta:
            self.wb = nn.Linear(dim, H, bias=False)

        for lin in (self.wq, self.wk, self.wv, self.wg):
            nn.init.normal_(lin.weight, std=init_std)
        for name in ('wa', 'wa1', 'wa2', 'wb'):
            if hasattr(self, name):
                nn.init.normal_(getattr(self, name).weight, std=init_std)
        if out_proj:
            wo_std = init_std / math.sqrt(2 * layer_count) if layer_count else init_std
            nn.init.normal_(self.wo.weight, std=wo_std)

        # recurrent state (fp32) and conv tails; allocated by reset_cache
        self.cache_len = 0
        self.register_buffer('state', torch.zeros(0, 0, 0, 0), persistent=False)
        if short_conv_size is not None:
            self.register_buffer('qp_cache', torch.zeros(0, short_conv_size, H * dk), persistent=False)
            self.register_buffer('kp_cache', torch.zeros(0, short_conv_size, H * dk), persistent=False)
            self.register_buffer('vp_cache', torch.zeros(0, short_conv_size, H * dv), persistent=False)

    # --- pieces ---------------------------------------------------------

    @property
    def gate_projections(self) -> list[nn.Parameter]:
        """The gate / beta matrices (linear_attention.py:686-691)."""
        return [getattr(self, n).weight for n in ('wa', 'wa1', 'wa2', 'wb') if hasattr(self, n)]

    def _pick_impl(self, q) -> str:
        """'hip' for a GPU tensor in fp32, bf16 or fp16 (:755-759); there is no
        other implementation."""
        if not q.is_cuda:
            raise RuntimeError('GatedDeltaNet (vagus_amd): the HIP kernels need GPU tensors; '
                               f'got a {q.device} tensor')
        if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise NotImplementedError(f'GatedDeltaNet (vagus_amd): {q.dtype} (fp32, bf16, fp16)')
        return 'hip'

    def _active_fusions(self, qp) -> frozenset:
        """The configured fusions this call runs (:761-781): none for fp32
        projections (the kernels take the fused producers with 16-bit inputs,
        the dtypes of the reference's fla path; its fp32 path fuses nothing
        either); without the delta rule no beta and no fused L2 norm; the gate
        activation only for the per-channel gate."""
        self._pick_impl(qp)
        if qp.dtype == torch.float32:
            return frozenset()
        on = self.fusions
        if not self.delta:
            on = on - {'l2norm', 'beta'}
        if self.gate != 'vector':
            on = on - {'gate'}
        return on

    def _gates(self, x, *, raw_gate: bool = False, raw_beta: bool = False):
        """(g, beta): log-decay (fp32) and write strength (fp32), or with
        raw_gate / raw_beta the kernel's inputs (the per-channel pre-activation
        (B, L, H, dk) and beta logits, in x's dtype) (:708-739)."""
        g = beta = None
        H, dk = self.head_count, self.key_head_dim
        if self.gate == 'scalar':
            assert not raw_gate, 'the fused gate activation is KDA-only (vector gate)'
            g = -self.A_log.float().exp() * F.softplus(self.wa(x).float() + self.dt_bias.float())
        elif self.gate == 'vector':
            B, L = x.shape[0], x.shape[1]
            f = self.wa2(self.wa1(x))
            if raw_gate:
                g = f.view(B, L, H, dk)
            elif self.gate_lower_bound is not None:
                f = (f.float() + self.dt_bias.float()).view(B, L, H, dk)
                g = self.gate_lower_bound * torch.sigmoid(self.A_log.float().exp()[:, None] * f)
            else:
                f = f.float() + self.dt_bias.float()
                g = -self.A_log.float().exp()[:, None] * F.softplus(f).view(B, L, H, dk)
        if self.delta and hasattr(self, 'wb'):
            beta = self.wb(x) if raw_beta else torch.sigmoid(self.wb(x).float())
        return g, beta

    @staticmethod
    def _l2norm(x, eps: float = 1e-6):
        h = x.to(torch.promote_types(x.dtype, torch.float32))
        return (h * torch.rsqrt(h.pow(2).sum(-1, keepdim=True) + eps)).to(x.dtype)

    def _heads(self, qp, kp, vp, *, l2norm: bool = True, cu_seqlens=None):
        """conv -> SiLU -> per-head view, and (unless the kernel will do it)
        the L2 norm on q and k (:741-753)."""
        B, L = qp.shape[0], qp.shape[1]
        H, dk, dv = self.head_count, self.key_head_dim, self.value_head_dim
        if self.short_conv_size is not None:
            qp = self.conv_q(qp, 'silu', cu_seqlens=cu_seqlens)
            kp = self.conv_k(kp, 'silu', cu_seqlens=cu_seqlens)
            vp = self.conv_v(vp, 'silu', cu_seqlens=cu_seqlens)
        else:
            qp, kp, vp = F.silu(qp), F.silu(kp), F.silu(vp)
        q, k, v = qp.view(B, L, H, dk), kp.view(B, L, H, dk), vp.view(B, L, H, dv)
        if l2norm:
            q, k = self._l2norm(q), self._l2norm(k)
        return q, k, v

    def _write(self, x, k, g, beta):
        """(beta, w): the delta rule's write for this block.  The family's own
        write is beta_t k_t, so w is None (:783-790); a subclass may return an
        explicit asymmetric w."""
        return beta, None

    def _scan(self, q, k, v, g, beta, S0, *, fusions=frozenset(), w=None, cu_seqlens=None):
        """(o, S): the chunked scan from S0 (:792-812)."""
        if w is not None:
            assert self.delta, 'an explicit write vector needs the delta rule'
            assert g is not None and g.dim() == 4, 'the asymmetric chunk form is implemented for the vector gate'
            return ops.chunk_scan_vec(q, k, v, g, None, S0, scale=self.scale, delta=True,
                                      chunk_size=self.chunk_size, w=w, cu_seqlens=cu_seqlens)
        self._pick_impl(q)
        return ops.hip_scan(q, k, v, g, beta, S0, scale=self.scale, delta=self.delta,
                            chunk_size=self.chunk_size,
                            l2norm_in_kernel='l2norm' in fusions,
                            gate_in_kernel='gate' in fusions,
                            beta_in_kernel='beta' in fusions,
                            A_log=self.A_log if self.gate != 'none' else None,
                            dt_bias=self.dt_bias if self.gate != 'none' else None,
                            disable_recompute=self.disable_recompute,
                            lower_bound=self.gate_lower_bound, cu_seqlens=cu_seqlens)

    def _output(self, o, x):
        """RMSNorm(o) x SiLU(W_g x) per head, then W_o (:814-825): one HIP pass
        for the epilogue."""
        B, L = x.shape[0], x.shape[1]
        gate = self.wg(x).view(B, L, self.head_count, self.value_head_dim)
        if _autograd(o, gate, self.o_norm.gamma):
            o = (self.o_norm(o.to(gate.dtype)) * F.silu(gate)).reshape(B, L, -1)        # :825
        else:
            o = ops.rms_norm_gated(o.to(gate.dtype), gate, self.o_norm.gamma, eps=self.o_norm.eps).reshape(B, L, -1)
        return self.wo(o) if self.out_proj else o

    # --- training / stateless --------------------------------------------

    def forward(self, x, is_causal: bool = True):
        assert is_causal, 'linear attention is causal by construction'
        qp, kp, vp = self.wq(x), self.wk(x), self.wv(x)
        on = self._active_fusions(qp)
        q, k, v = self._heads(qp, kp, vp, l2norm='l2norm' not in on)
        g, beta = self._gates(x, raw_gate='gate' in on, raw_beta='beta' in on)
        beta, w = self._write(x, k, g, beta)
        o, _ = self._scan(q, k, v, g, beta, None, fusions=on, w=w)
        return self._output(o, x)

    # --- streaming ---------------------------------------------------------

    def reset_cache(self, batch_size: int, max_cache_len: int | None = None):
        """A zero state and zero conv tails for batch_size streams
        (:888-899); max_cache_len is accepted for interface parity.  Buffers
        of the right shape are zeroed in place, so a decode step recorded in a
        HIP graph stays valid across resets."""
        p = next(self.parameters())
        device, dtype = p.device, p.dtype
        H, dk, dv = self.head_count, self.key_head_dim, self.value_head_dim
        self.cache_len = 0

        def fresh(buf, shape, dt):
            if buf.shape == shape and buf.dtype == dt and buf.device == device:
                return buf.zero_()
            return torch.zeros(shape, device=device, dtype=dt)

        self.state = fresh(self.state, (batch_size, H, dk, dv), torch.float32)
        if self.short_conv_size is not None:
            K = self.short_conv_size
            self.qp_cache = fresh(self.qp_cache, (batch_size, K, H * dk), dtype)
            self.kp_cache = fresh(self.kp_cache, (batch_size, K, H * dk), dtype)
            self.vp_cache = fresh(self.vp_cache, (batch_size, K, H * dv), dtype)

    def load_cache(self, cache: dict, max_cache_len: int | None = None):
        self.reset_cache(cache['state'].shape[0], max_cache_len)
        self.cache_len = int(cache['cache_len'])
        self.state.copy_(cache['state'])
        if self.short_conv_size is not None:
            self.qp_cache.copy_(cache['qp_cache'])
            self.kp_cache.copy_(cache['kp_cache'])
            self.vp_cache.copy_(cache['vp_cache'])

    def export_cache(self) -> dict:
        cache = {'state': self.state.clone(), 'cache_len': self.cache_len}
        if self.short_conv_size is not None:
            cache.update(qp_cache=self.qp_cache.clone(), kp_cache=self.kp_cache.clone(),
                         vp_cache=self.vp_cache.clone())
        return cache

    def _conv_weights(self):
        return (self.conv_q.conv.weight, self.conv_k.conv.weight, self.conv_v.conv.weight)

    def _caches(self):
        return (self.qp_cache, self.kp_cache, self.vp_cache)

    def _decode_kernel_fits(self) -> bool:
        # dv = 256 (the reference's dk 128 / dv 256 heads) runs the one-kernel step
        # with the usual four conv taps
        return (self.short_conv_size is not None and self.key_head_dim in (64, 128)
                and (self.value_head_dim in (64, 128) or (self.value_head_dim == 256 and self.short_conv_size == 4)))

    def _decode_weights(self):
        """The one-token decode step's projection weights regrouped, rebuilt
        whenever a parameter changed (its storage or version): W_q, W_k, W_v
        and W_g concatenated into one (4 H*dv, dim) weight, so that one GEMM
        replaces four skinny ones (when H*dk == H*dv); for the
        scalar gate [W_a; W_b] as one (2H, dim) weight (W_a alone without the
        delta rule) and the gate's constants -exp(A_log) and dt_bias in fp32.
        The copies hold one more set of these weights (4 dim H dv + 2 H dim
        elements per layer)."""
        ps = [self.wq.weight, self.wk.weight, self.wv.weight, self.wg.weight]
        scalar = self.gate == 'scalar'
        if scalar:
            ps += [self.wa.weight, self.A_log, self.dt_bias]
        if self.delta:
            ps.append(self.wb.weight)
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in ps)
        c = self.__dict__.get('_decode_w')
        if c is None or c[0] != key:
            same = len({p.shape for p in ps[:4]}) == 1
            w4 = torch.cat(ps[:4]).contiguous() if same else None
            wab = gconst = None
            if scalar:
                wab = torch.cat([self.wa.weight] + ([self.wb.weight] if self.delta else [])).contiguous()
                gconst = (-self.A_log.float().exp(), self.dt_bias.float())
            c = (key, w4, wab, gconst)
            self.__dict__['_decode_w'] = c
        return c[1:]

    def _decode_inputs(self, x):
        """(qp, kp, vp, out_gate, g, beta, gate_proj) for the one-token decode
        kernel: the projections of x (B, 1, dim), the log-decay in fp32 (or the
        KDA gate's pre-activation) and the beta logits, with the regrouped
        weights of _decode_weights.  With the scalar gate, g and beta are None
        and gate_proj = (x, [W_a; W_b], -exp(A_log), dt_bias): the decode
        kernel forms them itself.  The values are those of the separate
        projections and of _gates(raw_gate=vector, raw_beta=delta) up to the
        GEMMs' summation order."""
        B, L = x.shape[0], x.shape[1]
        w4, wab, gconst = self._decode_weights()
        if w4 is not None:
            # one GEMM over the concatenated weights; for one token the decode
            # kernel reads the four column blocks of its rows in place, otherwise
            # one copy makes them four contiguous (B*L, H*dv) blocks
            y = F.linear(x.reshape(B * L, -1), w4)
            n = y.shape[-1] // 4
            if L == 1:
                qp, kp, vp, og = (y[:, i * n:(i + 1) * n].view(B, L, n) for i in range(4))
            else:
                y = y.view(B * L, 4, -1).transpose(0, 1).contiguous()
                qp, kp, vp, og = (y[i].view(B, L, -1) for i in range(4))
        else:
            qp, kp, vp, og = self.wq(x), self.wk(x), self.wv(x), self.wg(x)
        if wab is None:
            g, beta = self._gates(x, raw_gate=self.gate == 'vector', raw_beta=self.delta)
            return qp, kp, vp, og, g, beta, None
        return qp, kp, vp, og, None, None, (x, wab, *gconst)

    @torch.no_grad()
    def decode_step(self, x):
        """Consume the next block (B, L, dim), advancing the state (:918-952).
        L == 1 is one kernel (conv with its cache, L2 norm, beta sigmoid, gate,
        recurrence in place, epilogue); a longer block runs the conv from the
        cache and the chunked scan from the state."""
        B, L = x.shape[0], x.shape[1]
        assert self.state.shape[0] > 0, 'No state allocated. Call reset_cache or load_cache first.'
        assert B == self.state.shape[0], 'Batch size does not match the state. Reset or load cache first.'
        if L == 0:
            return x
        self._pick_impl(x)
        H, dk, dv = self.head_count, self.key_head_dim, self.value_head_dim
        if L == 1 and type(self)._write is GatedDeltaNet._write and self._decode_kernel_fits():
            vec = self.gate == 'vector'
            qp, kp, vp, og, g, beta, gp = self._decode_inputs(x)
            o = ops.hip_decode_step(qp, kp, vp, g, beta, self.state, scale=self.scale, delta=self.delta,
                                    gate_proj=gp,
                                    conv_weights=self._conv_weights(), conv_cache=self._caches(), l2norm=True,
                                    beta_logits=self.delta, gate_in_kernel=vec,
                                    A_log=self.A_log if vec else None, dt_bias=self.dt_bias if vec else None,
                                    lower_bound=self.gate_lower_bound, out_gate=og,
                                    out_norm_weight=self.o_norm.gamma, out_norm_eps=self.o_norm.eps)
            self.cache_len += L
            o = o.reshape(B, L, H * dv)
            return self.wo(o) if self.out_proj else o
        qp, kp, vp = self.wq(x), self.wk(x), self.wv(x)
        if self.short_conv_size is not None:
            qp = self.conv_q(qp, 'silu', conv_cache=self.qp_cache)
            kp = self.conv_k(kp, 'silu', conv_cache=self.kp_cache)
            vp = self.conv_v(vp, 'silu', conv_cache=self.vp_cache)
        else:
            qp, kp, vp = F.silu(qp), F.silu(kp), F.silu(vp)
        q, k, v = self._l2norm(qp.view(B, L, H, dk)), self._l2norm(kp.view(B, L, H, dk)), vp.view(B, L, H, dv)
        g, beta = self._gates(x)
        beta, w = self._write(x, k, g, beta)
        if L == 1:
            o, _ = ops.hip_recurrent(q, k, v, g, beta, self.state, scale=self.scale, delta=self.delta,
                                     inplace=True, w=w)
        else:
            o, S = self._scan(q, k, v, g, beta, self.state, w=w)
            self.state.copy_(S)
        self.cache_len += L
        return self._output(o, x)

    @torch.no_grad()
    def prefill_packed(self, x, cu_seqlens, *, rows=None):
        """Push ragged blocks, packed as x (1, T, dim) with cu_seqlens (N + 1),
        into cache rows: block n continues the stream of row rows[n] (default:
        row n) from its state and conv tail, which it advances.  Returns the
        layer output (1, T, dim).  The reference's Generator has no such call:
        its decode_step takes equal-length rows only (generator.py:19-22)."""
        assert x.shape[0] == 1, 'prefill_packed takes a packed batch (1, T, dim)'
        N = cu_seqlens.numel() - 1
        rows = list(range(N)) if rows is None else list(rows)
        assert len(rows) == N, f'{N} blocks for {len(rows)} rows'
        assert self.state.shape[0] > 0, 'No state allocated. Call reset_cache or load_cache first.'
        T = x.shape[1]
        H, dk, dv = self.head_count, self.key_head_dim, self.value_head_dim
        qp, kp, vp = self.wq(x), self.wk(x), self.wv(x)
        on = self._active_fusions(qp)
        whole = rows == list(range(self.state.shape[0]))
        idx = None if whole else torch.as_tensor(rows, dtype=torch.long, device=x.device)
        if self.short_conv_size is not None:
            caches = self._caches() if whole else tuple(c.index_select(0, idx) for c in self._caches())
            qp = self.conv_q(qp, 'silu', cu_seqlens=cu_seqlens, conv_cache=caches[0])
            kp = self.conv_k(kp, 'silu', cu_seqlens=cu_seqlens, conv_cache=caches[1])
            vp = self.conv_v(vp, 'silu', cu_seqlens=cu_seqlens, conv_cache=caches[2])
            if not whole:
                for c, cw in zip(self._caches(), caches):
                    c.index_copy_(0, idx, cw)
        else:
            qp, kp, vp = F.silu(qp), F.silu(kp), F.silu(vp)
        q, k, v = qp.view(1, T, H, dk), kp.view(1, T, H, dk), vp.view(1, T, H, dv)
        if 'l2norm' not in on:
            q, k = self._l2norm(q), self._l2norm(k)
        g, beta = self._gates(x, raw_gate='gate' in on, raw_beta='beta' in on)
        beta, w = self._write(x, k, g, beta)
        S0 = self.state if whole else self.state.index_select(0, idx)
        o, S = self._scan(q, k, v, g, beta, S0, fusions=on, w=w, cu_seqlens=cu_seqlens)
        if whole:
            self.state.copy_(S)
        else:
            self.state.index_copy_(0, idx, S)
        return self._output(o, x)
