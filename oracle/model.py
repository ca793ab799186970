"""CPU composition of the gated delta-rule layer and the GDN language model
from the oracle's pieces: test infrastructure (imported by tests/ only), the
checker for vagus_amd.layer and vagus_amd.model.

Every function here composes functions of oracle/gdr.py, which are pinned
on their own, along the reference's module code:

    layer_forward   GatedDeltaNet.forward (linear_attention.py:829-837) with
                    _heads (:741-753), _gates (:708-739) and _output (:814-825)
    layer_stream    GatedDeltaNet.decode_step (:918-952), token blocks threaded
                    through the state and the conv caches
    rms_norm        RMSNorm (norm_layer.py:15-24)
    swiglu          FFN (ffn.py:46-50)
    lm_forward      GDNLM.forward (gdn_lm.py:188-195) over Block (block.py:54-66)
    lm_greedy       Generator.prefill_ids + gen_ids at temperature 0
                    (generator.py:160-222, sampling.py:30-35), by full recompute

Parameters come as a state_dict of the layer / model (any device and dtype);
everything runs in the dtype of the inputs given (fp64 for the exactness
checks).  Pinned by tests/test_oracle_model.py: the stateless forward equals
the streaming composition (prefill, single tokens, multi-token blocks) and
is causal, as the reference's own module tests require
(tests/test_linear_attention.py:98-132); the LM's greedy tokens by full
recompute equal those of the streaming composition.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import gdr


def _w(sd, name, dtype):
    return sd[name].detach().to('cpu', dtype)


def rms_norm(x, gamma, eps: float = 1e-6):
    """x rsqrt(mean x^2 + eps) in at least fp32, cast back, times gamma."""
    h = gdr._hi(x)
    return (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * gamma.to(x.dtype)


def swiglu(x, l1, l2):
    a, b = torch.chunk(x @ l1.T, 2, dim=-1)
    return (F.silu(a) * b) @ l2.T


def _gates(sd, pre, x, cfg, dtype):
    """(g, beta) as _gates computes them (:708-739), in at least fp32."""
    H, dk = cfg['head_count'], cfg['key_head_dim']
    B, L = x.shape[0], x.shape[1]
    g = beta = None
    if cfg['gate'] == 'scalar':
        A_log, dt = _w(sd, pre + 'A_log', dtype), _w(sd, pre + 'dt_bias', dtype)
        g = -gdr._hi(A_log).exp() * F.softplus(gdr._hi(x @ _w(sd, pre + 'wa.weight', dtype).T) + gdr._hi(dt))
    elif cfg['gate'] == 'vector':
        A_log, dt = _w(sd, pre + 'A_log', dtype), _w(sd, pre + 'dt_bias', dtype)
        f = (x @ _w(sd, pre + 'wa1.weight', dtype).T) @ _w(sd, pre + 'wa2.weight', dtype).T
        g = gdr.gate_activation(f.view(B, L, H, dk), A_log, dt.view(H, dk), cfg.get('gate_lower_bound'))
    if cfg['delta']:
        beta = gdr.beta_sigmoid(x @ _w(sd, pre + 'wb.weight', dtype).T)
    return g, beta


def _output(sd, pre, o, x, cfg, dtype):
    B, L = x.shape[0], x.shape[1]
    H, dv = cfg['head_count'], cfg['value_head_dim']
    gate = (x @ _w(sd, pre + 'wg.weight', dtype).T).view(B, L, H, dv)
    o = gdr.norm_gate(o.to(gate.dtype), gate, _w(sd, pre + 'o_norm.gamma', dtype)).reshape(B, L, H * dv)
    return o @ _w(sd, pre + 'wo.weight', dtype).T


def _proj(sd, pre, x, dtype):
    return tuple(x @ _w(sd, pre + n + '.weight', dtype).T for n in ('wq', 'wk', 'wv'))


def layer_forward(sd, x, cfg, pre: str = ''):
    """GatedDeltaNet.forward on x (B, L, dim) in x's dtype.  cfg: head_count,
    key_head_dim, value_head_dim, short_conv_size, gate, delta (and
    gate_lower_bound); sd: the layer's parameters under prefix `pre`."""
    dtype = x.dtype
    B, L = x.shape[0], x.shape[1]
    H, dk, dv = cfg['head_count'], cfg['key_head_dim'], cfg['value_head_dim']
    qp, kp, vp = _proj(sd, pre, x, dtype)
    if cfg['short_conv_size'] is not None:
        qp = gdr.short_conv(qp, _w(sd, pre + 'conv_q.conv.weight', dtype))[0]
        kp = gdr.short_conv(kp, _w(sd, pre + 'conv_k.conv.weight', dtype))[0]
        vp = gdr.short_conv(vp, _w(sd, pre + 'conv_v.conv.weight', dtype))[0]
    else:
        qp, kp, vp = F.silu(qp), F.silu(kp), F.silu(vp)
    q, k = gdr.l2norm(qp.view(B, L, H, dk)), gdr.l2norm(kp.view(B, L, H, dk))
    v = vp.view(B, L, H, dv)
    g, beta = _gates(sd, pre, x, cfg, dtype)
    o, _ = gdr.recurrent(q, k, v, g, beta, None, scale=dk ** -0.5, delta=cfg['delta'])
    return _output(sd, pre, o, x, cfg, dtype)


def layer_cache(cfg, batch: int, dtype):
    """A fresh streaming cache in the module's format (:888-899)."""
    H, dk, dv, K = cfg['head_count'], cfg['key_head_dim'], cfg['value_head_dim'], cfg['short_conv_size']
    c = {'state': torch.zeros(batch, H, dk, dv, dtype=dtype), 'cache_len': 0}
    if K is not None:
        c.update(qp_cache=torch.zeros(batch, K, H * dk, dtype=dtype), kp_cache=torch.zeros(batch, K, H * dk, dtype=dtype),
                 vp_cache=torch.zeros(batch, K, H * dv, dtype=dtype))
    return c


def layer_stream(sd, x, cfg, cache, pre: str = ''):
    """GatedDeltaNet.decode_step on the block x (B, L, dim): advances `cache`
    (a dict as layer_cache returns) and returns the block's output."""
    dtype = x.dtype
    B, L = x.shape[0], x.shape[1]
    if L == 0:
        return x
    H, dk, dv = cfg['head_count'], cfg['key_head_dim'], cfg['value_head_dim']
    qp, kp, vp = _proj(sd, pre, x, dtype)
    if cfg['short_conv_size'] is not None:
        qp, cache['qp_cache'] = gdr.short_conv(qp, _w(sd, pre + 'conv_q.conv.weight', dtype), cache['qp_cache'])
        kp, cache['kp_cache'] = gdr.short_conv(kp, _w(sd, pre + 'conv_k.conv.weight', dtype), cache['kp_cache'])
        vp, cache['vp_cache'] = gdr.short_conv(vp, _w(sd, pre + 'conv_v.conv.weight', dtype), cache['vp_cache'])
    else:
        qp, kp, vp = F.silu(qp), F.silu(kp), F.silu(vp)
    q, k = gdr.l2norm(qp.view(B, L, H, dk)), gdr.l2norm(kp.view(B, L, H, dk))
    v = vp.view(B, L, H, dv)
    g, beta = _gates(sd, pre, x, cfg, dtype)
    o, S = gdr.recurrent(q, k, v, g, beta, cache['state'], scale=dk ** -0.5, delta=cfg['delta'])
    cache['state'] = S.to(cache['state'].dtype)
    cache['cache_len'] += L
    return _output(sd, pre, o, x, cfg, dtype)


def _block(sd, i, x, cfg, stream_cache=None):
    p = f'blocks.{i}.'
    eps = cfg.get('rmsnorm_eps', 1e-6)
    dtype = x.dtype
    h = rms_norm(x, _w(sd, p + 'rmsnorm1.gamma', dtype), eps)
    if stream_cache is None:
        x = x + layer_forward(sd, h, cfg, p + 'att.')
    else:
        x = x + layer_stream(sd, h, cfg, stream_cache, p + 'att.')
    h = rms_norm(x, _w(sd, p + 'rmsnorm2.gamma', dtype), eps)
    return x + swiglu(h, _w(sd, p + 'ffn.l1.weight', dtype), _w(sd, p + 'ffn.l2.weight', dtype))


def _head(sd, x, cfg):
    dtype = x.dtype
    h = rms_norm(x, _w(sd, 'rms_head.gamma', dtype), cfg.get('rmsnorm_eps', 1e-6))
    head = sd['head.weight'] if 'head.weight' in sd else sd['embedding.weight']
    return h @ head.detach().to('cpu', dtype).T


def lm_forward(sd, tokens, cfg, dtype=torch.float64):
    """GDNLM.forward: tokens (B, L) -> logits (B, L, vocab)."""
    x = _w(sd, 'embedding.weight', dtype)[tokens]
    for i in range(cfg['layer_count']):
        x = _block(sd, i, x, cfg)
    return _head(sd, x, cfg)


def lm_stream(sd, tokens, cfg, caches, dtype=torch.float64):
    """GDNLM.decode_step: consume tokens (B, L) into `caches` (one per layer);
    logits (B, L, vocab)."""
    x = _w(sd, 'embedding.weight', dtype)[tokens]
    for i in range(cfg['layer_count']):
        x = _block(sd, i, x, cfg, caches[i])
    return _head(sd, x, cfg)


def lm_greedy(sd, prompt, steps: int, cfg, dtype=torch.float64):
    """Greedy continuation of one prompt (1-D token tensor) by full recompute:
    each step runs lm_forward over the whole stream and takes the last
    position's argmax.  Returns (tokens (steps,), logits (steps, vocab))."""
    stream = prompt.reshape(1, -1).long()
    toks, logits = [], []
    for _ in range(steps):
        lg = lm_forward(sd, stream, cfg, dtype)[0, -1]
        t = lg.argmax()
        toks.append(t)
        logits.append(lg)
        stream = torch.cat([stream, t.view(1, 1)], dim=1)
    return torch.stack(toks), torch.stack(logits)
