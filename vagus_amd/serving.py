"""Continuous batching of ragged sequences over the HIP kernels, for one
gated delta-rule layer at a time (the callers either side of the hot path:
the reference's Generator and its cache API, infra/inference/generator.py
and linear_attention.py:888-916).

The reference decodes only equal-length rows (generator.py:19-22: no
attention mask, so ragged prompts cannot be left-padded).  A recurrent layer
needs no mask: each sequence is its own state.  This module keeps those
states in a pool of slots and runs

* ``prefill``: any set of new or continuing sequences, ragged, in one packed
  call (cu_seqlens) per kernel: the short conv continuing from each slot's
  conv cache, then the chunked scan from each slot's state;
* ``decode``: one token for every active slot in one kernel
  (vgdr_decode_step), updating states and conv caches in place.

Slots are rows of the pool's tensors, in the module's cache format:
``state`` (slots, H, dk, dv) fp32 and the conv caches ``qp_cache``,
``kp_cache``, ``vp_cache`` (slots, K, H*d) in the compute dtype
(linear_attention.py:911-916).  ``export`` / ``load`` move one slot in and
out as the module's export_cache / load_cache do.

``DecodeGraph`` records a multi-layer decode step into a HIP graph (static
buffers in, static buffers out) for a serving loop to replay.  The slots'
token counts (``length``) are host bookkeeping: eager calls advance them,
graph replays do not.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops


@dataclass
class LayerShape:
    H: int
    dk: int
    dv: int
    conv: int | None = 4          # short conv width K (None: q, k, v arrive activated)
    gate: str = 'scalar'          # 'none' | 'scalar' | 'vector'
    delta: bool = True

    @property
    def scale(self) -> float:
        return self.dk ** -0.5


class LayerCache:
    """The state and conv caches of one layer for `slots` sequence slots."""

    def __init__(self, shape: LayerShape, slots: int, *, conv_weights=None, dtype=torch.bfloat16, device='cuda'):
        """conv_weights: the layer's ShortConv weights (w_q, w_k, w_v), each (D, 1, K) or (D, K)."""
        self.shape, self.slots, self.dtype = shape, slots, dtype
        assert not shape.conv or conv_weights is not None, 'a layer with a short conv needs its weights'
        self.conv_weights = conv_weights
        H, dk, dv = shape.H, shape.dk, shape.dv
        self.state = torch.zeros(slots, H, dk, dv, dtype=torch.float32, device=device)
        if shape.conv:
            K = shape.conv
            self.qp_cache = torch.zeros(slots, K, H * dk, dtype=dtype, device=device)
            self.kp_cache = torch.zeros(slots, K, H * dk, dtype=dtype, device=device)
            self.vp_cache = torch.zeros(slots, K, H * dv, dtype=dtype, device=device)
        self.length = [0] * slots              # tokens consumed per slot (the module's cache_len)

    @property
    def caches(self):
        return (self.qp_cache, self.kp_cache, self.vp_cache)

    def reset(self, slots) -> None:
        """Empty the given slots (a new sequence starts from zero state)."""
        idx = torch.as_tensor(list(slots), dtype=torch.long, device=self.state.device)
        self.state.index_fill_(0, idx, 0.0)
        if self.shape.conv:
            for c in self.caches:
                c.index_fill_(0, idx, 0)
        for s in slots:
            self.length[s] = 0

    def export(self, slot: int) -> dict:
        """One slot's cache, cloned (linear_attention.py:905-910)."""
        d = {'state': self.state[slot].clone(), 'cache_len': self.length[slot]}
        if self.shape.conv:
            d.update(qp_cache=self.qp_cache[slot].clone(), kp_cache=self.kp_cache[slot].clone(),
                     vp_cache=self.vp_cache[slot].clone())
        return d

    def load(self, slot: int, d: dict) -> None:
        """Install an exported cache into a slot (linear_attention.py:897-904)."""
        self.state[slot].copy_(d['state'])
        self.length[slot] = int(d['cache_len'])
        if self.shape.conv:
            self.qp_cache[slot].copy_(d['qp_cache'])
            self.kp_cache[slot].copy_(d['kp_cache'])
            self.vp_cache[slot].copy_(d['vp_cache'])


def _rows(t, idx, contiguous_all):
    return t if contiguous_all else t.index_select(0, idx)


def _scatter(dst, idx, src, contiguous_all):
    if not contiguous_all:
        dst.index_copy_(0, idx, src)


def prefill(cache: LayerCache, slots, qp, kp, vp, g, beta, cu_seqlens, *, l2norm: bool = True,
            beta_logits: bool = False, out_gate=None, out_norm_weight=None, out_norm_eps: float = 1e-6):
    """Push ragged token blocks into `slots` (one packed call per kernel).

    qp, kp (1, T, H*dk), vp (1, T, H*dv): the raw projections of all blocks,
    packed; cu_seqlens (len(slots) + 1): block n goes to slots[n], continuing
    from that slot's state and conv caches.  g, beta as the scans take them
    (packed, batch 1); beta_logits: beta holds logits.  Returns o (1, T, H, dv),
    through the output epilogue when out_gate / out_norm_weight are given."""
    sh = cache.shape
    B, T = qp.shape[0], qp.shape[1]
    assert B == 1 and cu_seqlens.numel() == len(slots) + 1, 'prefill takes a packed batch: (1, T, D), N + 1 offsets'
    dev = cache.state.device
    idx = torch.as_tensor(list(slots), dtype=torch.long, device=dev)
    whole = list(slots) == list(range(cache.slots))
    H, dk, dv = sh.H, sh.dk, sh.dv
    if sh.conv:
        cq, ck, cv = (_rows(c, idx, whole) for c in cache.caches)
        w = cache.conv_weights
        q, _ = ops.causal_conv1d(qp, w[0], activation='silu', cu_seqlens=cu_seqlens, conv_cache=cq)
        k, _ = ops.causal_conv1d(kp, w[1], activation='silu', cu_seqlens=cu_seqlens, conv_cache=ck)
        v, _ = ops.causal_conv1d(vp, w[2], activation='silu', cu_seqlens=cu_seqlens, conv_cache=cv)
        for c, cw in zip(cache.caches, (cq, ck, cv)):
            _scatter(c, idx, cw, whole)
    else:
        q, k, v = qp, kp, vp
    q, k, v = q.view(1, T, H, dk), k.view(1, T, H, dk), v.view(1, T, H, dv)
    S0 = _rows(cache.state, idx, whole)
    if sh.gate == 'vector':
        o, S = ops.chunk_kda(q, k, v, g, beta, scale=sh.scale, initial_state=S0, output_final_state=True,
                             cu_seqlens=cu_seqlens, use_qk_l2norm_in_kernel=l2norm,
                             use_beta_sigmoid_in_kernel=beta_logits)
    elif sh.delta:
        o, S = ops.chunk_gated_delta_rule(q, k, v, g if sh.gate == 'scalar' else None, beta, scale=sh.scale,
                                          initial_state=S0, output_final_state=True, cu_seqlens=cu_seqlens,
                                          use_qk_l2norm_in_kernel=l2norm, use_beta_sigmoid_in_kernel=beta_logits)
    else:
        o, S = ops.chunk_simple_gla(q, k, v, g if sh.gate == 'scalar' else None, scale=sh.scale, initial_state=S0,
                                    output_final_state=True, cu_seqlens=cu_seqlens)
    if whole:
        cache.state.copy_(S)
    else:
        cache.state.index_copy_(0, idx, S)
    lens = (cu_seqlens[1:] - cu_seqlens[:-1]).tolist()
    for s, n in zip(slots, lens):
        cache.length[s] += int(n)
    if out_gate is not None or out_norm_weight is not None:
        o = ops.rms_norm_gated(o, out_gate.view(1, T, H, dv), out_norm_weight, eps=out_norm_eps)
    return o


def decode(cache: LayerCache, slots, qp, kp, vp, g, beta, *, l2norm: bool = True, beta_logits: bool = False,
           out_gate=None, out_norm_weight=None, out_norm_eps: float = 1e-6):
    """One token for each of `slots` (row n of the inputs goes to slots[n]),
    in one kernel: conv + SiLU with the cache advanced, L2 norm, recurrence,
    epilogue.  qp, kp (N, 1, H*dk), vp (N, 1, H*dv).  When `slots` is every
    slot in order, the pool is updated in place with no gather."""
    sh = cache.shape
    assert sh.conv, 'decode drives the fused step of a layer with a short conv'
    dev = cache.state.device
    whole = list(slots) == list(range(cache.slots))
    idx = None if whole else torch.as_tensor(list(slots), dtype=torch.long, device=dev)
    state = cache.state if whole else cache.state.index_select(0, idx)
    caches = cache.caches if whole else tuple(c.index_select(0, idx) for c in cache.caches)
    o = ops.hip_decode_step(qp, kp, vp, g, beta, state, scale=sh.scale, delta=sh.delta,
                            conv_weights=cache.conv_weights, conv_cache=caches, l2norm=l2norm,
                            beta_logits=beta_logits, out_gate=out_gate, out_norm_weight=out_norm_weight,
                            out_norm_eps=out_norm_eps)
    if not whole:
        cache.state.index_copy_(0, idx, state)
        for c, cw in zip(cache.caches, caches):
            c.index_copy_(0, idx, cw)
    for s in slots:
        cache.length[s] += qp.shape[1]
    return o


class DecodeGraph:
    """A decode step over several layers recorded once into a HIP graph.

    `step` is a callable that reads the static tensors it closes over (the
    inputs a serving loop refills before each replay, and the layer caches,
    which every replay advances in place) and returns its outputs.  Recording
    executes nothing, so the caches are not advanced by it; the tensors
    `step` returns during the recording live in the graph's memory pool and
    receive each replay's outputs (``outputs``).  Run `step` once eagerly
    before recording (that step loads the kernels), as its first real
    decode step.  The kernels issue no memset, so the recorded graph holds
    kernel launches only."""

    def __init__(self, step):
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = step()

    def replay(self):
        self.graph.replay()
        return self.outputs
