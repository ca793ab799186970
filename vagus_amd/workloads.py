"""Seeded synthetic inputs for the gated delta-rule benchmark workloads.

The shapes and distributions are the benchmark's:

    gdn_cpu     GDN, fp32, B=2 T=256 H=4 dk=dv=64, chunk 64, zero entry state
    gdn_340m    GDN layer prefill, bf16 q/k/v, B=8 T=4096 H=8 dk=dv=128,
                entry state 0.1 * N(0, 1)
    kda_prefill KDA prefill, bf16, B=4 T=8192 H=8 dk=dv=128, per-channel
                gate (B, T, H, dk), zero entry state, final states returned
    gdn_varlen  packed GDN prefill, bf16, 32 segments with lengths uniform in
                [128, 8192], H=16 dk=dv=128, zero entry states
    gdn_lm_1p3b greedy generation with the 1.3B-shape GDN language model
                (24 layers, hidden 2048, H=16 dk=dv=128, vocab 32000, scalar
                gate, bf16 weights, random init; la_fused=True, the module's
                option that runs the q, k L2 norm and the beta sigmoid inside
                the scan kernels): 64 prompts with token ids
                uniform over the vocabulary and lengths uniform in [64, 2048],
                ragged prefill, then 256 decode steps (lm_workload)

Distributions (all from one torch.Generator seeded with the workload's seed,
drawn in the order below): q, k ~ N(0, 1) then L2-normalised per head;
v ~ N(0, 1); beta = sigmoid(N(0, 1)) per (token, head); log-decay
g = logsigmoid(N(0, 1) + 4) per (token, head) or per (token, head, channel);
optional entry state scale * N(0, 1).  bf16 workloads round q, k, v to bf16;
g, beta and the states stay fp32.  Generation happens on `device` (CPU by
default, so an oracle and the GPU see the same values after a copy).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

WORKLOADS = {
    'gdn_cpu': dict(B=2, T=256, H=4, dk=64, dv=64, gate='scalar', dtype=torch.float32,
                    s0_scale=None, seed=0),
    'gdn_340m': dict(B=8, T=4096, H=8, dk=128, dv=128, gate='scalar', dtype=torch.bfloat16,
                     s0_scale=0.1, seed=1),
    'kda_prefill': dict(B=4, T=8192, H=8, dk=128, dv=128, gate='vector', dtype=torch.bfloat16,
                        s0_scale=None, seed=2),
    'gdn_varlen': dict(n_seqs=32, len_lo=128, len_hi=8192, H=16, dk=128, dv=128, gate='scalar',
                       dtype=torch.bfloat16, s0_scale=None, seed=3),
}


LM_WORKLOADS = {
    'gdn_lm_1p3b': dict(model=dict(vocab_size=32000, dim=2048, layer_count=24, head_count=16, key_head_dim=128,
                                   value_head_dim=128, gate='scalar', short_conv_size=4, chunk_size=64,
                                   la_fused=True),
                        dtype=torch.bfloat16, n_prompts=64, len_lo=64, len_hi=2048, new_tokens=256, seed=4),
}


@dataclass
class ScanInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor | None
    beta: torch.Tensor
    initial_state: torch.Tensor | None
    cu_seqlens: torch.Tensor | None = None

    def to(self, device) -> 'ScanInputs':
        mv = lambda t: None if t is None else t.to(device)
        return ScanInputs(mv(self.q), mv(self.k), mv(self.v), mv(self.g), mv(self.beta),
                          mv(self.initial_state), mv(self.cu_seqlens))

    @property
    def tokens(self) -> int:
        return self.q.shape[0] * self.q.shape[1]


def make_inputs(B: int, T: int, H: int, dk: int, dv: int, *, gate: str = 'scalar',
                dtype=torch.bfloat16, s0_scale: float | None = None, seed: int = 0,
                n_states: int | None = None, g_shift: float = 4.0,
                device='cpu') -> ScanInputs:
    """Draw one batch (see the module docstring for the distributions).

    gate: 'scalar' (g of shape (B, T, H)), 'vector' (B, T, H, dk) or 'none'.
    n_states: number of entry states (defaults to B; packed varlen input uses
    the segment count)."""
    gen = torch.Generator(device).manual_seed(seed)
    kw = dict(generator=gen, device=device, dtype=torch.float32)
    q = F.normalize(torch.randn(B, T, H, dk, **kw), dim=-1)
    k = F.normalize(torch.randn(B, T, H, dk, **kw), dim=-1)
    v = torch.randn(B, T, H, dv, **kw)
    beta = torch.sigmoid(torch.randn(B, T, H, **kw))
    if gate == 'vector':
        g = F.logsigmoid(torch.randn(B, T, H, dk, **kw) + g_shift)
    elif gate == 'scalar':
        g = F.logsigmoid(torch.randn(B, T, H, **kw) + g_shift)
    else:
        g = None
    ns = B if n_states is None else n_states
    S0 = None if s0_scale is None else s0_scale * torch.randn(ns, H, dk, dv, **kw)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    return ScanInputs(q, k, v, g, beta, S0)


def varlen_lengths(n_seqs: int, lo: int, hi: int, seed: int) -> list[int]:
    """Segment lengths uniform in [lo, hi] (inclusive) from `seed`."""
    gen = torch.Generator('cpu').manual_seed(seed)
    return torch.randint(lo, hi + 1, (n_seqs,), generator=gen).tolist()


def cu_from_lengths(lengths, device='cpu') -> torch.Tensor:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    return torch.tensor(cu, dtype=torch.int32, device=device)


def make_varlen_inputs(lengths, H: int, dk: int, dv: int, *, gate: str = 'scalar',
                       dtype=torch.bfloat16, s0_scale: float | None = None, seed: int = 0,
                       device='cpu') -> ScanInputs:
    """One packed (1, sum(lengths), H, d) stream indexed by int32 cu_seqlens."""
    T = int(sum(lengths))
    x = make_inputs(1, T, H, dk, dv, gate=gate, dtype=dtype, s0_scale=s0_scale, seed=seed,
                    n_states=len(lengths), device=device)
    x.cu_seqlens = cu_from_lengths(lengths, device=device)
    return x


def workload(name: str, device='cpu') -> ScanInputs:
    """The named benchmark workload's inputs."""
    w = dict(WORKLOADS[name])
    if name == 'gdn_varlen':
        lens = varlen_lengths(w['n_seqs'], w['len_lo'], w['len_hi'], w['seed'])
        return make_varlen_inputs(lens, w['H'], w['dk'], w['dv'], gate=w['gate'], dtype=w['dtype'],
                                  s0_scale=w['s0_scale'], seed=w['seed'], device=device)
    return make_inputs(w['B'], w['T'], w['H'], w['dk'], w['dv'], gate=w['gate'], dtype=w['dtype'],
                       s0_scale=w['s0_scale'], seed=w['seed'], device=device)


def lm_prompts(n: int, lo: int, hi: int, vocab: int, seed: int) -> list[torch.Tensor]:
    """n prompts with lengths uniform in [lo, hi] and token ids uniform in
    [0, vocab), from `seed` (CPU int64)."""
    gen = torch.Generator('cpu').manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=gen).tolist()
    return [torch.randint(0, vocab, (m,), generator=gen) for m in lens]


def lm_workload(name: str, device='cuda'):
    """(model, prompts, new_tokens) of a generation workload: the GDNLM built
    on `device` from the workload's seed (random init, in its dtype, eval
    mode) and its prompts."""
    from .model import GDNLM
    w = LM_WORKLOADS[name]
    torch.manual_seed(w['seed'])
    with torch.device(device):
        m = GDNLM(**w['model'])
    m = m.to(w['dtype']).eval()
    prompts = lm_prompts(w['n_prompts'], w['len_lo'], w['len_hi'], w['model']['vocab_size'], w['seed'])
    return m, prompts, w['new_tokens']
