"""Pins of the oracle's layer and LM compositions (oracle/model.py), CPU, fp64.

The reference's module tests (tests/test_linear_attention.py:98-132) define
the layer by relations: the streaming path (decode_step over a prefill
block, single tokens and a multi-token block) reproduces the stateless
forward, and the layer is causal.  The same relations pin the oracle's
composition here; the LM's greedy continuation by full recompute must equal
the streaming one.  The parameters come from vagus_amd's own modules
(constructed on the CPU, no kernel runs), so the state_dict layout the GPU
tests hand the oracle is the one exercised here.
"""
import itertools

import pytest
import torch

from oracle import model as om
from vagus_amd.layer import GatedDeltaNet
from vagus_amd.model import GDNLM

GATES = ('none', 'scalar', 'vector')


def layer_cfg(m: GatedDeltaNet):
    return dict(head_count=m.head_count, key_head_dim=m.key_head_dim, value_head_dim=m.value_head_dim,
                short_conv_size=m.short_conv_size, gate=m.gate, delta=m.delta,
                gate_lower_bound=m.gate_lower_bound)


def make_layer(gate, delta, conv, seed=0, **kw):
    torch.manual_seed(seed)
    m = GatedDeltaNet(dim=32, head_count=2, key_head_dim=8, value_head_dim=16, short_conv_size=conv, gate=gate,
                      delta=delta, gate_rank=4, chunk_size=32, layer_count=4, **kw)
    # nonzero, non-unit norm weights so that they matter
    with torch.no_grad():
        m.o_norm.gamma.uniform_(0.5, 1.5)
        for n in ('conv_q', 'conv_k', 'conv_v'):
            if hasattr(m, n):
                getattr(m, n).conv.weight.normal_(0, 0.5)
    return m.double()


@pytest.mark.parametrize('gate,delta', list(itertools.product(GATES, [True, False])))
@pytest.mark.parametrize('conv', [4, None])
def test_layer_stream_matches_forward(gate, delta, conv):
    m = make_layer(gate, delta, conv)
    sd, cfg = m.state_dict(), layer_cfg(m)
    x = torch.randn(2, 23, 32, dtype=torch.float64)
    ref = om.layer_forward(sd, x, cfg)
    cache = om.layer_cache(cfg, 2, torch.float64)
    parts = [om.layer_stream(sd, x[:, :9], cfg, cache)]
    parts += [om.layer_stream(sd, x[:, t:t + 1], cfg, cache) for t in range(9, 14)]
    parts.append(om.layer_stream(sd, x[:, 14:], cfg, cache))
    out = torch.cat(parts, dim=1)
    assert torch.allclose(out, ref, atol=1e-10, rtol=1e-10)
    assert cache['cache_len'] == 23
    assert torch.equal(om.layer_stream(sd, x[:, :0], cfg, cache), x[:, :0])


def test_layer_bounded_gate_stream_matches_forward():
    m = make_layer('vector', True, 4, gate_lower_bound=-5.0)
    sd, cfg = m.state_dict(), layer_cfg(m)
    x = torch.randn(1, 17, 32, dtype=torch.float64)
    cache = om.layer_cache(cfg, 1, torch.float64)
    out = torch.cat([om.layer_stream(sd, x[:, :5], cfg, cache), om.layer_stream(sd, x[:, 5:], cfg, cache)], 1)
    assert torch.allclose(out, om.layer_forward(sd, x, cfg), atol=1e-10, rtol=1e-10)


def test_layer_causal():
    m = make_layer('vector', True, 4)
    sd, cfg = m.state_dict(), layer_cfg(m)
    x = torch.randn(1, 20, 32, dtype=torch.float64)
    y = om.layer_forward(sd, x, cfg)
    x2 = x.clone()
    x2[:, 12:] += torch.randn(1, 8, 32, dtype=torch.float64)
    y2 = om.layer_forward(sd, x2, cfg)
    assert torch.allclose(y[:, :12], y2[:, :12], atol=1e-13)
    assert not torch.allclose(y[:, 12:], y2[:, 12:])


def tiny_lm(seed=0, gate='scalar'):
    torch.manual_seed(seed)
    m = GDNLM(vocab_size=97, dim=32, layer_count=2, head_count=2, key_head_dim=8, value_head_dim=16,
              gate=gate, gate_rank=4, chunk_size=32)
    with torch.no_grad():
        for blk in m.blocks:
            blk.att.o_norm.gamma.uniform_(0.5, 1.5)
    return m.double()


def lm_cfg(m: GDNLM):
    c = m.config
    return dict(layer_count=c['layer_count'], head_count=c['head_count'], key_head_dim=c['key_head_dim'],
                value_head_dim=c['value_head_dim'], short_conv_size=c['short_conv_size'], gate=c['gate'],
                delta=c['delta'], gate_lower_bound=c['gate_lower_bound'], rmsnorm_eps=c['rmsnorm_eps'])


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_lm_greedy_full_recompute_matches_stream(gate):
    m = tiny_lm(gate=gate)
    sd, cfg = m.state_dict(), lm_cfg(m)
    prompt = torch.randint(0, 97, (11,))
    toks, logits = om.lm_greedy(sd, prompt, 6, cfg)
    # streaming: prompt minus its last token, then one token per step
    caches = [om.layer_cache(cfg, 1, torch.float64) for _ in range(cfg['layer_count'])]
    om.lm_stream(sd, prompt[None, :-1], cfg, caches)
    pending = prompt[-1:]
    for s in range(6):
        lg = om.lm_stream(sd, pending[None], cfg, caches)[0, -1]
        assert torch.allclose(lg, logits[s], atol=1e-10, rtol=1e-10)
        pending = lg.argmax().view(1)
        assert int(pending) == int(toks[s])


def test_lm_tied_head_and_param_layout():
    m = tiny_lm()
    sd = m.state_dict()
    assert m.head.weight is m.embedding.weight
    keys = set(sd)
    for want in ('embedding.weight', 'rms_head.gamma', 'blocks.0.rmsnorm1.gamma', 'blocks.0.rmsnorm2.gamma',
                 'blocks.0.ffn.l1.weight', 'blocks.0.ffn.l2.weight', 'blocks.1.att.wq.weight'):
        assert want in keys, want
    # Llama's SwiGLU sizing: 8/3 dim rounded up to 256 (block.py:43-44)
    assert sd['blocks.0.ffn.l1.weight'].shape == (2 * 256, 32)


# --- closed forms of the oracle's FFN and scalar gates ------------------------

def test_swiglu_closed_form():
    """swiglu(x) = SiLU(first half of l1 x) * (second half) projected by l2
    (ffn.py:46-50).  With l1 = [I; 2I] and l2 = I it is x * 2x / (1 + e^-x)
    elementwise; a swapped pair of halves would give 2x * x / (1 + e^-2x)."""
    import math
    x = torch.tensor([[0.0, 1.0, -1.0, 2.0, -3.0]], dtype=torch.float64)
    n = x.shape[1]
    eye = torch.eye(n, dtype=torch.float64)
    y = om.swiglu(x, torch.cat([eye, 2 * eye]), eye)
    want = torch.tensor([[2 * v * v / (1 + math.exp(-v)) for v in x[0].tolist()]], dtype=torch.float64)
    assert torch.allclose(y, want, rtol=1e-14, atol=1e-14)
    swapped = torch.tensor([[2 * v * v / (1 + math.exp(-2 * v)) for v in x[0].tolist()]], dtype=torch.float64)
    assert not torch.allclose(y, swapped)
    # l2 maps back: a permutation of the hidden units permutes nothing in the result's meaning
    l2 = torch.zeros(2, n, dtype=torch.float64)
    l2[0, 1] = 1.0
    l2[1, 3] = -0.5
    y2 = om.swiglu(x, torch.cat([eye, 2 * eye]), l2)
    assert torch.allclose(y2, torch.tensor([[want[0, 1].item(), -0.5 * want[0, 3].item()]], dtype=torch.float64))


def test_scalar_gates_closed_form():
    """_gates for the scalar gate (linear_attention.py:719-721, :734-735):
    g = -exp(A_log) softplus(W_a x + dt_bias), beta = sigmoid(W_b x), checked
    at points where both have closed values: softplus(0) = ln 2,
    softplus(ln(e - 1)) = 1, sigmoid(0) = 1/2, sigmoid(ln 3) = 3/4."""
    import math
    cfg = dict(head_count=2, key_head_dim=4, value_head_dim=4, gate='scalar', delta=True)
    dim = 3
    x = torch.tensor([[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]]], dtype=torch.float64)     # (B=1, L=2, dim)
    sd = {
        'A_log': torch.tensor([math.log(2.0), 0.0], dtype=torch.float64),
        'dt_bias': torch.tensor([0.0, math.log(math.e - 1.0)], dtype=torch.float64),
        # head 0 reads nothing; head 1 reads -ln(e - 1) of token 1's second feature
        'wa.weight': torch.tensor([[0.0, 0.0, 0.0], [0.0, -math.log(math.e - 1.0), 0.0]], dtype=torch.float64),
        # head 0: 0 everywhere; head 1: ln 3 of the first feature
        'wb.weight': torch.tensor([[0.0, 0.0, 0.0], [math.log(3.0), 0.0, 0.0]], dtype=torch.float64),
    }
    g, beta = om._gates(sd, '', x, cfg, torch.float64)
    ln2 = math.log(2.0)
    want_g = torch.tensor([[[-2.0 * ln2, -1.0],          # token 0: head 0 = -2 ln 2, head 1 = -1 * softplus(ln(e-1)) = -1
                            [-2.0 * ln2, -ln2]]],        # token 1: head 1's pre-activation is 0 -> -ln 2
                          dtype=torch.float64)
    want_b = torch.tensor([[[0.5, 0.75], [0.5, 0.5]]], dtype=torch.float64)
    assert torch.allclose(g, want_g, rtol=1e-14, atol=1e-14), g
    assert torch.allclose(beta, want_b, rtol=1e-14, atol=1e-14), beta
