"""Continuous batching of ragged sequences (vagus_amd.serving): ragged
prefill into chosen slots and joint decode of the active slots, against the
oracle run on each sequence alone; and a HIP-graph decode step against the
same step run eagerly.

GPU: each sequence's outputs (through the whole token stream: prefill blocks
and decode tokens) at the 16-bit bar rel_l2 <= 2e-2 against the oracle's
decode_step (fp32 recurrence) on that sequence alone, its final state at the
same bar, its conv caches bit-exact; graph replays bit-identical to eager
calls from the same caches, with host work and input refills between replays.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdr

TOL = 2e-2
H, DK, DV, K = 2, 64, 64, 4


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def _tokens(n, g):
    """Raw projections, gate and beta of n tokens (batch 1)."""
    qp = torch.randn(1, n, H * DK, generator=g).bfloat16()
    kp = torch.randn(1, n, H * DK, generator=g).bfloat16()
    vp = torch.randn(1, n, H * DV, generator=g).bfloat16()
    gl = F.logsigmoid(torch.randn(1, n, H, generator=g) + 4.0)
    beta = torch.sigmoid(torch.randn(1, n, H, generator=g))
    return qp, kp, vp, gl, beta


def _cat(parts):
    return tuple(torch.cat([p[i] for p in parts], 1) for i in range(5))


@pytest.mark.gpu
def test_ragged_prefill_and_joint_decode_match_each_sequence_alone():
    from vagus_amd import serving
    g = torch.Generator().manual_seed(0)
    ws = [(0.5 * torch.randn(d, 1, K, generator=g)) for d in (H * DK, H * DK, H * DV)]
    shape = serving.LayerShape(H=H, dk=DK, dv=DV, conv=K)
    cache = serving.LayerCache(shape, 4, conv_weights=[w.cuda() for w in ws])
    stream = {}                     # sequence -> list of token blocks
    outs = {}                       # sequence -> list of output blocks
    dev = lambda t: t.cuda()

    def run_prefill(seqs, slots, lens):
        blocks = [_tokens(n, g) for n in lens]
        for s, b in zip(seqs, blocks):
            stream.setdefault(s, []).append(b)
        qp, kp, vp, gl, beta = _cat(blocks)
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
        o = serving.prefill(cache, slots, dev(qp), dev(kp), dev(vp), dev(gl), dev(beta), dev(cu))
        for s, a, b in zip(seqs, cu[:-1].tolist(), cu[1:].tolist()):
            outs.setdefault(s, []).append(o[:, a:b].cpu())

    def run_decode(seqs, slots):
        blocks = [_tokens(1, g) for _ in seqs]
        for s, b in zip(seqs, blocks):
            stream[s].append(b)
        qp, kp, vp, gl, beta = (torch.cat([b[i] for b in blocks], 0) for i in range(5))
        o = serving.decode(cache, slots, dev(qp), dev(kp), dev(vp), dev(gl), dev(beta))
        for n, s in enumerate(seqs):
            outs[s].append(o[n:n + 1].cpu())

    print('\n[case] continuous batching: ragged prefill, joint decode, a late joiner', flush=True)
    run_prefill(['A', 'B', 'C'], [2, 0, 3], [5, 37, 70])
    for _ in range(3):
        run_decode(['B', 'A', 'C'], [0, 2, 3])            # a gathered subset of the slots
    run_prefill(['D', 'A'], [1, 2], [11, 6])               # a new sequence joins, A continues with a block
    for _ in range(2):
        run_decode(['B', 'D', 'A', 'C'], [0, 1, 2, 3])     # every slot: updated in place
    slot_of = {'A': 2, 'B': 0, 'C': 3, 'D': 1}
    for s, blocks in stream.items():
        qp, kp, vp, gl, beta = _cat(blocks)
        S0 = torch.zeros(1, H, DK, DV)
        c0 = tuple(torch.zeros(1, K, d).bfloat16() for d in (H * DK, H * DK, H * DV))
        o_ref, S_ref, c_ref = gdr.decode_step(qp, kp, vp, gl, beta, S0, ws, c0, scale=DK ** -0.5)
        o = torch.cat(outs[s], 1)
        eo = _rel(o, o_ref)
        es = _rel(cache.state[slot_of[s]], S_ref[0])
        exact = all(torch.equal(c[slot_of[s]].cpu(), r[0]) for c, r in zip(cache.caches, c_ref))
        print(f'[parity] sequence {s} ({qp.shape[1]} tokens): o={eo:.3e} S={es:.3e} caches exact={exact}',
              flush=True)
        assert eo <= TOL and es <= TOL and exact
        assert cache.length[slot_of[s]] == qp.shape[1]


@pytest.mark.gpu
def test_decode_graph_replays_equal_eager_steps():
    from vagus_amd import serving
    g = torch.Generator().manual_seed(1)
    N, layers = 3, 2
    shape = serving.LayerShape(H=H, dk=DK, dv=DV, conv=K)
    ws = [[(0.5 * torch.randn(d, 1, K, generator=g)).cuda() for d in (H * DK, H * DK, H * DV)]
          for _ in range(layers)]
    caches = [serving.LayerCache(shape, N, conv_weights=ws[i]) for i in range(layers)]
    for c in caches:                                        # start from non-trivial states and caches
        c.state.copy_(0.1 * torch.randn(c.state.shape, generator=g))
        for t in c.caches:
            t.copy_(torch.randn(t.shape, generator=g).bfloat16())
    inputs = [tuple(t.cuda() for t in (torch.randn(N, 1, H * DK, generator=g).bfloat16(),
                                       torch.randn(N, 1, H * DK, generator=g).bfloat16(),
                                       torch.randn(N, 1, H * DV, generator=g).bfloat16(),
                                       F.logsigmoid(torch.randn(N, 1, H, generator=g) + 4.0),
                                       torch.sigmoid(torch.randn(N, 1, H, generator=g))))
              for _ in range(layers)]
    slots = list(range(N))

    def step(cs=caches):
        return [serving.decode(cs[i], slots, *inputs[i]) for i in range(layers)]

    print('\n[case] decode graph: 2 layers x 3 slots, 3 replays', flush=True)
    step()                                                  # the first real step, eager: loads the kernels
    graph = serving.DecodeGraph(step)
    for r in range(3):
        for inp in inputs:                                  # the serving loop refills the static inputs
            for t in inp:
                t.copy_(t.float().mul_(-0.9).add_(0.1).to(t.dtype))
        twins = []                                          # eager twin from the same starting caches
        for i, c in enumerate(caches):
            tw = serving.LayerCache(shape, N, conv_weights=ws[i])
            tw.state.copy_(c.state)
            for a, b in zip(tw.caches, c.caches):
                a.copy_(b)
            twins.append(tw)
        want = step(twins)
        torch.cuda.synchronize()
        got = graph.replay()
        torch.cuda.synchronize()
        same_o = all(torch.equal(a, b) for a, b in zip(got, want))
        same_s = all(torch.equal(c.state, t.state) and all(torch.equal(x, y) for x, y in zip(c.caches, t.caches))
                     for c, t in zip(caches, twins))
        print(f'[parity] replay {r}: outputs equal={same_o} states and caches equal={same_s}', flush=True)
        assert same_o and same_s
