"""The GDN language model and the ragged greedy generator (vagus_amd.model)
against the oracle's composition (oracle/model.py): a tiny model with the
same weights on both sides.

GPU:
  * fp32 model: each ragged prompt's greedy continuation equals the oracle's
    (full recompute, fp64) token for token, and every step's logits are
    within rel-L2 1e-4;
  * bf16 model: teacher-forced logits (the oracle's tokens fed back) within
    rel-L2 2e-2 at every step;
  * the generator's HIP-graph decode step reproduces the eager step exactly
    (tokens and final states), with eager work between replays;
  * GDNLM.forward's last-position logits equal prefill_packed's.
"""
import pytest
import torch

from oracle import model as om
from vagus_amd.model import GDNLM, RaggedGenerator


def rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def tiny(dtype, gate='scalar', dk=64, seed=0):
    torch.manual_seed(seed)
    m = GDNLM(vocab_size=211, dim=128, layer_count=2, head_count=2, key_head_dim=dk, value_head_dim=64,
              gate=gate, gate_rank=16, chunk_size=64)
    with torch.no_grad():
        for blk in m.blocks:
            blk.att.o_norm.gamma.uniform_(0.5, 1.5)
            for n in ('conv_q', 'conv_k', 'conv_v'):
                getattr(blk.att, n).conv.weight.normal_(0, 0.5)
        m.embedding.weight.normal_(0, 1.0)
    return m.to(device='cuda', dtype=dtype).eval()


def cfg(m):
    c = m.config
    return dict(layer_count=c['layer_count'], head_count=c['head_count'], key_head_dim=c['key_head_dim'],
                value_head_dim=c['value_head_dim'], short_conv_size=c['short_conv_size'], gate=c['gate'],
                delta=c['delta'], gate_lower_bound=c['gate_lower_bound'], rmsnorm_eps=c['rmsnorm_eps'])


def prompts(lens, seed=1, vocab=211):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g) for n in lens]


@pytest.mark.gpu
@pytest.mark.parametrize('gate,dk', [('scalar', 64), ('vector', 64), ('scalar', 32)])
def test_greedy_matches_oracle_fp32(gate, dk):
    m = tiny(torch.float32, gate, dk)
    sd, c = m.state_dict(), cfg(m)
    ps = prompts([5, 70, 19])
    gen = RaggedGenerator(m)
    gen.prefill(ps)
    toks = gen.generate(6).cpu()
    for i, p in enumerate(ps):
        ref_t, ref_l = om.lm_greedy(sd, p, 6, c)
        assert torch.equal(toks[i], ref_t), (i, toks[i].tolist(), ref_t.tolist())
    # the logits along the same streams, teacher-forced through decode_step
    for i, p in enumerate(ps):
        ref_t, ref_l = om.lm_greedy(sd, p, 6, c)
        m.reset_cache(1)
        m.decode_step(p[None, :-1].cuda(), return_logits=False)
        feed = torch.cat([p[-1:], ref_t[:-1]])
        for s in range(6):
            lg = m.decode_step(feed[s].view(1, 1).cuda())[0, -1]
            e = rel(lg, ref_l[s])
            assert e < 1e-4, (gate, i, s, e)
    print(f'[lm fp32] {gate} dk={dk}: greedy tokens equal the oracle\'s', flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_teacher_forced_logits_bf16(gate):
    m = tiny(torch.bfloat16, gate)
    sd, c = m.state_dict(), cfg(m)
    p = prompts([37], seed=2)[0]
    ref_t, ref_l = om.lm_greedy(sd, p, 8, c)
    m.reset_cache(1)
    m.decode_step(p[None, :-1].cuda(), return_logits=False)
    feed = torch.cat([p[-1:], ref_t[:-1]])
    worst = 0.0
    for s in range(8):
        lg = m.decode_step(feed[s].view(1, 1).cuda())[0, -1]
        worst = max(worst, rel(lg, ref_l[s]))
    print(f'[lm bf16] {gate}: worst step logits rel_l2 {worst:.2e}', flush=True)
    assert worst < 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_graph_replay_equals_eager(dtype):
    m = tiny(dtype)
    ps = prompts([9, 64, 130, 1, 33], seed=3)
    gen = RaggedGenerator(m)
    gen.prefill(ps)
    eager = gen.generate(10, graph=False)
    states_e = [blk.att.state.clone() for blk in m.blocks]
    gen.prefill(ps)
    replay = gen.generate(10, graph=True)
    torch.cuda.synchronize()
    assert torch.equal(eager, replay)
    for blk, s in zip(m.blocks, states_e):
        assert torch.equal(blk.att.state, s)
    # a new prefill of the same batch keeps the recorded step: ten replays,
    # one per call, with eager work on the stream between them
    gen.prefill(ps)
    assert gen._graph is not None
    out = []
    for _ in range(10):
        out.append(gen.generate(1, graph=True))
        torch.randn(1000, device='cuda').sum()
    assert torch.equal(torch.cat(out, 1), eager)


@pytest.mark.gpu
def test_forward_and_packed_prefill_agree():
    m = tiny(torch.float32)
    ps = prompts([12, 40], seed=4)
    full = [m(p[None].cuda())[0, -1] for p in ps]
    m.reset_cache(2)
    ids = torch.cat(ps).cuda()
    cu = torch.tensor([0, 12, 52], dtype=torch.int32).cuda()
    last = m.prefill_packed(ids, cu)
    for i in range(2):
        assert rel(last[i], full[i]) < 1e-5


@pytest.mark.gpu
def test_graph_follows_weight_and_cache_changes():
    """A recorded decode step is dropped when what it holds by address
    changes: load_state_dict of other weights (in place, new versions) and a
    cache reset that reallocates (dtype change) both lead to the eager
    tokens, and recording does not advance the layers' cache_len."""
    m, other = tiny(torch.float32, seed=0), tiny(torch.float32, seed=5)
    ps = prompts([9, 40, 3], seed=6)
    gen = RaggedGenerator(m)
    gen.prefill(ps)
    gen.generate(4, graph=True)
    assert gen._graph is not None
    # packed prefill leaves cache_len at 0; the eager first step counts once,
    # the recording and the replays not at all
    assert all(blk.att.cache_len == 1 for blk in m.blocks)
    lens = [blk.att.cache_len for blk in m.blocks]
    gen.generate(1, graph=True)
    assert [blk.att.cache_len for blk in m.blocks] == lens   # replays leave the host counters alone
    m.load_state_dict(other.state_dict())
    gen.prefill(ps)
    replay = gen.generate(6, graph=True)
    ref = RaggedGenerator(other)
    ref.prefill(ps)
    eager = ref.generate(6, graph=False)
    torch.cuda.synchronize()
    assert torch.equal(replay, eager)
    # a different batch size records again; the same size after load_cache keeps the graph valid
    gen.prefill(ps[:2])
    a = gen.generate(3, graph=True)
    ref.prefill(ps[:2])
    b = ref.generate(3, graph=False)
    assert torch.equal(a, b)
