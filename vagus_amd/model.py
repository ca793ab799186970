"""The GDN language model and its generation driver over the HIP layer: the
callers on the hot path's decode side (the reference's GDNLM,
infra/models/gdn_lm.py, its Block and FFN, infra/components/block.py and
ffn.py, and the Generator / greedy sampling, infra/inference/generator.py
and sampling.py).

``GDNLM`` keeps the reference's constructor arguments, parameter names and
shapes for the all-linear layout (layer_pattern 'gdn', write 'delta'):
embedding -> [RMSNorm -> GatedDeltaNet -> residual, RMSNorm -> SwiGLU FFN
-> residual] x layers -> RMSNorm -> head tied to the embedding
(gdn_lm.py:188-195, block.py:54-91).  Softmax and parallel layers and the
Kalman writes are not implemented here and raise NotImplementedError.

``RaggedGenerator`` serves a batch of prompts of any lengths, one stream per
cache row: the prompts go through every layer as one packed call per kernel
(cu_seqlens), then each decode step feeds one token per stream through all
layers, each layer one fused kernel, with the whole step (embedding, the
layers, the head and the greedy pick) recorded once into a HIP graph and
replayed.  Its stream convention is the reference Generator's
(generator.py:8-17): prefill consumes all but the last token of each prompt,
which becomes the pending token; a decode step feeds the pending tokens,
takes the logits' argmax (sampling.py:30-35 at temperature 0) and makes it
pending.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import ops
from .layer import GatedDeltaNet, RMSNorm


def _add_norm(norm: RMSNorm, x, delta=None, *, inplace: bool = False):
    """(x + delta, norm(x + delta)) -- the residual add a pre-norm block makes
    before each norm (block.py:57-59) and the norm -- as one HIP pass
    (ops.rms_norm) for GPU tensors; x + delta lands in x itself with inplace.
    Without delta: (x, norm(x)).  Other devices and shapes take the module's
    expression."""
    D = x.shape[-1]
    ve = 16 // x.element_size() if x.dtype in (torch.bfloat16, torch.float16, torch.float32) else 0
    if x.is_cuda and ve and norm.gamma.dtype == x.dtype and D % ve == 0 and D // ve <= 2048:
        if delta is None:
            return x, ops.rms_norm(x, norm.gamma, norm.eps)
        in_place = inplace and x.is_contiguous() and x.data_ptr() % 16 == 0
        y, h = ops.rms_norm(x, norm.gamma, norm.eps, residual=delta, out_residual=x if in_place else None)
        return h, y
    if delta is not None:
        x = x.add_(delta) if inplace else x + delta
    return x, norm(x)


def _ffn(ffn: 'FFN', h):
    """The FFN with its SwiGLU as one HIP pass (ops.swiglu) for GPU tensors
    without autograd; the module's expression otherwise."""
    if (h.is_cuda and not torch.is_grad_enabled() and h.dtype in (torch.bfloat16, torch.float16, torch.float32)
            and ffn.hidden_dim % (16 // h.element_size()) == 0):
        return ffn.l2(ops.swiglu(ffn.l1(h)))
    return ffn(h)


class FFN(nn.Module):
    """SwiGLU: l1 to 2 x hidden, SiLU(first half) x second half, l2 back
    (ffn.py:7-48)."""

    def __init__(self, dim: int, hidden_dim: int, init_std: float = 0.02, layer_count: int | None = None):
        super().__init__()
        assert dim > 0 and hidden_dim > 0
        self.dim, self.hidden_dim = dim, hidden_dim
        self.l1 = nn.Linear(dim, 2 * hidden_dim, bias=False)
        self.silu = nn.SiLU()
        self.l2 = nn.Linear(hidden_dim, dim, bias=False)
        nn.init.normal_(self.l1.weight, std=init_std)
        nn.init.normal_(self.l2.weight, std=init_std / math.sqrt(2 * layer_count) if layer_count else init_std)

    def forward(self, x):
        x1, xgate = torch.chunk(self.l1(x), 2, dim=-1)
        return self.l2(self.silu(x1) * xgate)


class Block(nn.Module):
    """Pre-norm residual block around the mixer and the FFN (block.py:19-91);
    the mixer is kept under `att`."""

    def __init__(self, dim: int, ffn_hidden_dim: int | None = None, rmsnorm_eps: float = 1e-6, *,
                 mixer: GatedDeltaNet, layer_count: int | None):
        super().__init__()
        ffn_hidden_dim = ffn_hidden_dim or math.ceil(int(8 * dim / 3) / 256) * 256
        self.rmsnorm1 = RMSNorm(dim, rmsnorm_eps)
        self.att = mixer
        self.rmsnorm2 = RMSNorm(dim, rmsnorm_eps)
        self.ffn = FFN(dim=dim, hidden_dim=ffn_hidden_dim, init_std=0.02, layer_count=layer_count)

    def forward(self, x, is_causal: bool = True):
        x = x + self.att(self.rmsnorm1(x), is_causal)
        return x + self.ffn(self.rmsnorm2(x))

    def reset_cache(self, batch_size: int, max_cache_len: int | None = None):
        self.att.reset_cache(batch_size, max_cache_len)

    def load_cache(self, cache: dict, max_cache_len: int | None = None):
        self.att.load_cache(cache['att'], max_cache_len=max_cache_len)

    def export_cache(self) -> dict:
        return {'att': self.att.export_cache()}

    @torch.no_grad()
    def decode_step(self, x):
        _, h = _add_norm(self.rmsnorm1, x)
        x, h = _add_norm(self.rmsnorm2, x, self.att.decode_step(h))
        return x + _ffn(self.ffn, h)

    @torch.no_grad()
    def prefill_packed(self, x, cu_seqlens, rows=None):
        _, h = _add_norm(self.rmsnorm1, x)
        x, h = _add_norm(self.rmsnorm2, x, self.att.prefill_packed(h, cu_seqlens, rows=rows))
        return x + _ffn(self.ffn, h)

    def _stream(self, x, delta, step):
        """One block over the residual stream x with the previous block's
        pending FFN output `delta` folded into this block's first norm:
        returns (x, this block's FFN output).  x is updated in place."""
        x, h = _add_norm(self.rmsnorm1, x, delta, inplace=True)
        x, h = _add_norm(self.rmsnorm2, x, step(h), inplace=True)
        return x, _ffn(self.ffn, h)


class GDNLM(nn.Module):
    """The reference's GDNLM (gdn_lm.py:20-195) for the all-GDN layout."""

    def __init__(self,
                 vocab_size: int,
                 dim: int,
                 layer_count: int,
                 head_count: int,
                 key_head_dim: int,
                 value_head_dim: int,
                 ffn_hidden_dim: int | None = None,
                 short_conv_size: int | None = 4,
                 gate: str | bool = 'vector',
                 delta: bool = True,
                 gate_rank: int = 64,
                 chunk_size: int = 64,
                 la_impl: str = 'auto',
                 la_fused: bool | str | list = False,
                 la_conv_impl: str = 'conv1d',
                 la_disable_recompute: bool = False,
                 gate_lower_bound: float | None = None,
                 write: str = 'delta',
                 kalman_args: dict | None = None,
                 A_init_range: tuple[float, float] = (1.0, 16.0),
                 dt_init_range: tuple[float, float] = (1e-3, 1e-1),
                 layer_pattern: str = 'gdn',
                 layer_kinds: list[str] | None = None,
                 softmax_head_dim: int = 64,
                 softmax_rope: bool = True,
                 softmax_out_gate: bool = False,
                 parallel_width: int | None = None,
                 context_len: int = 2048,
                 rope_base: float = 10000,
                 rmsnorm_eps: float = 1e-6,
                 tie_embedding: bool = True,
                 gate_proj_optimizer: str = 'adamw'):
        super().__init__()
        assert gate_proj_optimizer in ('adamw', 'muon')
        kinds = [k.strip() for k in layer_kinds] if layer_kinds is not None else \
            [[t.strip() for t in layer_pattern.split(',')][i % len(layer_pattern.split(','))] for i in range(layer_count)]
        assert len(kinds) == layer_count, f'layer_kinds has {len(kinds)} entries for layer_count {layer_count}'
        if any(k != 'gdn' for k in kinds):
            raise NotImplementedError('vagus_amd builds the gated delta-rule layers only (layer kind \'gdn\'); '
                                      f'got {sorted(set(kinds))}')
        if write != 'delta':
            raise NotImplementedError(f'write {write!r}: the Kalman writes are not built here (write=\'delta\')')
        self.config = dict(vocab_size=vocab_size, dim=dim, layer_count=layer_count, head_count=head_count,
                           key_head_dim=key_head_dim, value_head_dim=value_head_dim, ffn_hidden_dim=ffn_hidden_dim,
                           short_conv_size=short_conv_size, gate=gate, delta=delta, gate_rank=gate_rank,
                           chunk_size=chunk_size, la_impl=la_impl, la_fused=la_fused, la_conv_impl=la_conv_impl,
                           la_disable_recompute=la_disable_recompute, gate_lower_bound=gate_lower_bound,
                           write=write, kalman_args=kalman_args, A_init_range=tuple(A_init_range),
                           dt_init_range=tuple(dt_init_range), layer_pattern=layer_pattern, layer_kinds=layer_kinds,
                           softmax_head_dim=softmax_head_dim, softmax_rope=softmax_rope,
                           softmax_out_gate=softmax_out_gate, parallel_width=parallel_width,
                           context_len=context_len, rope_base=rope_base, rmsnorm_eps=rmsnorm_eps,
                           tie_embedding=tie_embedding, gate_proj_optimizer=gate_proj_optimizer)
        self.kinds = kinds
        self.embedding = nn.Embedding(vocab_size, dim)

        def linear() -> GatedDeltaNet:
            return GatedDeltaNet(dim=dim, head_count=head_count, key_head_dim=key_head_dim,
                                 value_head_dim=value_head_dim, short_conv_size=short_conv_size, gate=gate,
                                 delta=delta, gate_rank=gate_rank, chunk_size=chunk_size, impl=la_impl,
                                 fused=la_fused, conv_impl=la_conv_impl, disable_recompute=la_disable_recompute,
                                 gate_lower_bound=gate_lower_bound, A_init_range=tuple(A_init_range),
                                 dt_init_range=tuple(dt_init_range), init_std=0.02, layer_count=layer_count)

        self.blocks = nn.ModuleList([Block(dim=dim, ffn_hidden_dim=ffn_hidden_dim, rmsnorm_eps=rmsnorm_eps,
                                           mixer=linear(), layer_count=layer_count) for _ in kinds])
        self.rms_head = RMSNorm(dim, rmsnorm_eps)
        self.head = nn.Linear(dim, vocab_size, bias=False)
        nn.init.normal_(self.embedding.weight, std=0.02)
        if tie_embedding:
            self.head.weight = self.embedding.weight
        else:
            nn.init.normal_(self.head.weight, std=0.02)

    @classmethod
    def from_config(cls, config: dict) -> 'GDNLM':
        return cls(**config)

    def forward(self, tokens, is_causal: bool = True, return_hidden: bool = False):
        x = self.embedding(tokens)
        for blk in self.blocks:
            x = blk(x, is_causal)
        x = self.rms_head(x)
        return x if return_hidden else self.head(x)

    # streaming inference (gdn_lm.py:254-266)

    @property
    def max_stream_len(self) -> int | None:
        return None                                   # fixed-size state: no positional limit

    def reset_cache(self, batch_size: int, max_cache_len: int | None = None):
        for blk in self.blocks:
            blk.reset_cache(batch_size, max_cache_len)

    def load_cache(self, cache: dict, max_cache_len: int | None = None):
        for blk, c in zip(self.blocks, cache['blocks'], strict=True):
            blk.load_cache(c, max_cache_len=max_cache_len)

    def export_cache(self) -> dict:
        return {'blocks': [blk.export_cache() for blk in self.blocks]}

    @torch.no_grad()
    def decode_step(self, tokens, return_logits: bool = True):
        """Consume tokens (B, L) into the streams; logits (B, L, vocab) or None."""
        x = self.embedding(tokens)
        delta = None
        for blk in self.blocks:
            x, delta = blk._stream(x, delta, blk.att.decode_step)
        if not return_logits:
            return None
        return self.head(_add_norm(self.rms_head, x, delta, inplace=True)[1])

    @torch.no_grad()
    def prefill_packed(self, tokens, cu_seqlens, *, rows=None, last_logits: bool = True):
        """Consume ragged token blocks, packed as tokens (T,) or (1, T) with
        cu_seqlens (N + 1), into cache rows (default: block n -> row n).
        Returns the logits (N, vocab) at each block's last token, or None."""
        x = self.embedding(tokens.reshape(1, -1))
        delta = None
        for blk in self.blocks:
            x, delta = blk._stream(x, delta, lambda h, blk=blk: blk.att.prefill_packed(h, cu_seqlens, rows=rows))
        if not last_logits:
            return None
        last = (cu_seqlens[1:] - 1).long()
        x = x[0].index_select(0, last) + delta[0].index_select(0, last)
        return self.head(_add_norm(self.rms_head, x)[1])


class RaggedGenerator:
    """Greedy generation for a batch of ragged prompts over a GDNLM on the
    GPU: one stream per cache row, packed prefill, graph-replayed decode."""

    def __init__(self, model: GDNLM):
        self.model = model
        self.device = next(model.parameters()).device
        self.batch_size = 0
        self.pending: torch.Tensor | None = None
        self.fed_len: list[int] = []
        self._graph = None
        self._graph_key = None

    def reset(self, batch_size: int) -> None:
        """batch_size empty streams.  The caches are zeroed in place when the
        batch size is unchanged, and the recorded decode step is kept."""
        self.model.reset_cache(batch_size)
        if self.pending is None or batch_size != self.batch_size:
            self.pending = torch.zeros(batch_size, dtype=torch.int64, device=self.device)
            self._graph = None
        else:
            self.pending.zero_()
        self.batch_size = batch_size
        self.fed_len = [0] * batch_size

    @torch.no_grad()
    def prefill(self, prompts) -> None:
        """prompts: a list of 1-D int token tensors (each of length >= 1), or
        (packed ids (T,), cu_seqlens (N + 1,)).  Starts one fresh stream per
        prompt: everything but each prompt's last token is consumed, in one
        packed call per kernel; the last tokens become pending."""
        if isinstance(prompts, tuple):
            ids, cu = prompts
            ids = ids.to(self.device, torch.int64)
            cu = cu.to(self.device, torch.int32)
            lens = (cu[1:] - cu[:-1]).tolist()
        else:
            lens = [int(p.numel()) for p in prompts]
            ids = torch.cat([p.reshape(-1) for p in prompts]).to(self.device, torch.int64)
            cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32,
                              device=self.device)
        assert min(lens) >= 1, 'every prompt needs at least one token'
        N = len(lens)
        self.reset(N)
        last = (cu[1:] - 1).long()
        self.pending.copy_(ids.index_select(0, last))
        keep = torch.ones(ids.numel(), dtype=torch.bool, device=self.device)
        keep[last] = False
        body = ids[keep]
        cu_body = cu - torch.arange(N + 1, dtype=torch.int32, device=self.device)
        if body.numel():
            self.model.prefill_packed(body, cu_body, last_logits=False)
        self.fed_len = [n - 1 for n in lens]

    def _step(self):
        logits = self.model.decode_step(self.pending[:, None], return_logits=True)
        nxt = logits[:, -1].float().argmax(dim=-1)
        self.pending.copy_(nxt)
        return nxt

    def _fingerprint(self) -> tuple:
        """What a recorded decode step holds by address: every parameter
        (storage and version: load_state_dict, an optimizer step or .to()
        change one of them), each layer's state and conv-cache buffers, and
        the regrouped decode weights.  A replay is valid only while this is
        unchanged."""
        key = [(p.data_ptr(), p._version) for p in self.model.parameters()]
        for blk in self.model.blocks:
            att = blk.att
            key += [(t.data_ptr(), t.dtype) for t in (att.state,) + (att._caches() if att.short_conv_size else ())]
            c = att.__dict__.get('_decode_w')
            key.append(None if c is None else tuple(None if t is None else t.data_ptr()
                                                    for t in (c[1], c[2]) + (c[3] or ())))
        return tuple(key)

    @torch.no_grad()
    def generate(self, steps: int, *, graph: bool = True) -> torch.Tensor:
        """`steps` greedy decode steps for every stream: (N, steps) int64.
        With graph=True the first step ever taken runs eagerly and is then
        recorded into a HIP graph (recording executes nothing); every later
        step, in this call or a later one, replays it, until a parameter or a
        cache buffer it holds changes (then the next step runs eagerly and
        is recorded again).  Replays read and advance the caches and the
        pending tokens in place; the layers' host-side cache_len counters are
        not advanced by them (fed_len here is)."""
        assert self.pending is not None and self.batch_size > 0, 'prefill first'
        out = torch.empty(self.batch_size, steps, dtype=torch.int64, device=self.device)
        for i in range(steps):
            if graph and self._graph is not None and self._graph_key != self._fingerprint():
                self._graph = None                    # a captured tensor moved or changed: record again
            if graph and self._graph is not None:
                self._graph.replay()
                out[:, i].copy_(self.pending)
            else:
                out[:, i].copy_(self._step())
                if graph and self._graph is None:
                    # recording runs no kernel: the layers' cache_len must not count it
                    lens = [blk.att.cache_len for blk in self.model.blocks]
                    self._graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(self._graph):
                        self._step()
                    for blk, n in zip(self.model.blocks, lens):
                        blk.att.cache_len = n
                    self._graph_key = self._fingerprint()
            self.fed_len = [n + 1 for n in self.fed_len]
        return out
