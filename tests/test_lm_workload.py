"""The 1.3B-shape generation workload (vagus_amd.workloads.lm_workload,
gdn_lm_1p3b) at full size on the GPU: the model's parameter count is the
reference layout's (55.7 M per layer plus the 65.5 M tied embedding), ragged
prefill of the 64 prompts and graph-replayed decode run, and the replayed
steps reproduce eager steps exactly from the same prefill.  At full width
(two of its layers: d2048, H16, dk=dv=128, vocab 32000, FFN 5632) the model
is checked against the oracle's forward: greedy tokens in fp32 and the
logits of every step in fp32 and bf16; the fused decode kernel is checked
against the oracle at the layer's exact call (B64 H16, test_decode_conv.py)."""
import pytest
import torch

from vagus_amd import workloads


def test_prompt_draw_is_seeded_and_in_range():
    w = workloads.LM_WORKLOADS['gdn_lm_1p3b']
    a = workloads.lm_prompts(w['n_prompts'], w['len_lo'], w['len_hi'], 32000, w['seed'])
    b = workloads.lm_prompts(w['n_prompts'], w['len_lo'], w['len_hi'], 32000, w['seed'])
    assert len(a) == 64 and all(torch.equal(x, y) for x, y in zip(a, b))
    assert all(64 <= p.numel() <= 2048 for p in a)
    assert all(0 <= int(p.min()) and int(p.max()) < 32000 for p in a)


@pytest.mark.gpu
def test_full_size_generation_graph_equals_eager():
    from vagus_amd.model import RaggedGenerator
    m, prompts, new = workloads.lm_workload('gdn_lm_1p3b')
    n_params = sum(p.numel() for p in m.parameters())
    per_layer = sum(p.numel() for p in m.blocks[0].parameters())
    print(f'[lm 1.3B] params {n_params / 1e9:.3f} B, per layer {per_layer / 1e6:.2f} M', flush=True)
    assert abs(per_layer - 55.7e6) < 0.1e6 and n_params == 24 * per_layer + 32000 * 2048 + 2048   # + rms_head
    gen = RaggedGenerator(m)
    gen.prefill(prompts)
    eager = gen.generate(6, graph=False)
    gen.prefill(prompts)
    replay = gen.generate(6, graph=True)
    torch.cuda.synchronize()
    assert torch.equal(eager, replay)
    assert int(eager.min()) >= 0 and int(eager.max()) < 32000


def _full_width(dtype, layers=2, seed=0):
    """The gdn_lm_1p3b model (d2048, H16, dk=dv=128, vocab 32000, FFN 5632,
    la_fused) cut to `layers` layers, with unit-scale embeddings (so the tied
    head's logits are well separated) and non-trivial norm gains and conv
    taps, on the GPU in `dtype`."""
    from vagus_amd.model import GDNLM
    cfg = dict(workloads.LM_WORKLOADS['gdn_lm_1p3b']['model'], layer_count=layers)
    torch.manual_seed(seed)
    m = GDNLM(**cfg)
    with torch.no_grad():
        m.embedding.weight.normal_(0, 1.0)
        for blk in m.blocks:
            blk.att.o_norm.gamma.uniform_(0.5, 1.5)
            for n in ('conv_q', 'conv_k', 'conv_v'):
                getattr(blk.att, n).conv.weight.normal_(0, 0.5)
    assert m.blocks[0].ffn.hidden_dim == 5632
    return m.to(device='cuda', dtype=dtype).eval()


def _oracle_cfg(m):
    c = m.config
    return dict(layer_count=c['layer_count'], head_count=c['head_count'], key_head_dim=c['key_head_dim'],
                value_head_dim=c['value_head_dim'], short_conv_size=c['short_conv_size'], gate=c['gate'],
                delta=c['delta'], gate_lower_bound=c['gate_lower_bound'], rmsnorm_eps=c['rmsnorm_eps'])


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_full_width_lm_against_oracle(dtype):
    """Two layers of the 1.3B-shape LM at full width against the oracle's
    GDNLM.forward (oracle.model.lm_forward in fp64, gdn_lm.py:188-195) on three
    ragged prompts: the ragged generator's greedy tokens (packed prefill, then
    graph-replayed decode steps) equal the oracle's full-recompute greedy
    tokens in fp32, and the logits along the oracle's tokens, fed back through
    decode_step (the fused one-token kernel), are within rel-L2 1e-4 (fp32) or
    2e-2 (bf16) at every step (the reference's own check,
    tests/test_gdn_lm.py:37-51, pins generation to the full forward)."""
    from oracle import model as om
    from vagus_amd.model import RaggedGenerator
    m = _full_width(dtype)
    sd = {k: v.detach().to('cpu', torch.float64) for k, v in m.state_dict().items()}
    cfg = _oracle_cfg(m)
    g = torch.Generator().manual_seed(7)
    lens, steps = [5, 37, 20], 5
    prompts = [torch.randint(0, 32000, (n,), generator=g) for n in lens]
    print(f'\n[case] full-width 2-layer LM {dtype}: prompts {lens}, {steps} steps', flush=True)
    refs = [om.lm_greedy(sd, p, steps, cfg) for p in prompts]
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    worst = 0.0
    for p, (ref_t, ref_l) in zip(prompts, refs):
        m.reset_cache(1)
        m.decode_step(p[None, :-1].cuda(), return_logits=False)
        feed = torch.cat([p[-1:], ref_t[:-1]])
        for s in range(steps):
            lg = m.decode_step(feed[s].view(1, 1).cuda())[0, -1]
            worst = max(worst, _rel(lg, ref_l[s]))
    print(f'[parity] full-width LM {dtype}: worst step logits rel_l2 {worst:.2e} (tol {tol:g})', flush=True)
    assert worst <= tol
    if dtype == torch.float32:
        gen = RaggedGenerator(m)
        gen.prefill(prompts)
        toks = gen.generate(steps).cpu()
        for i, (ref_t, _) in enumerate(refs):
            assert torch.equal(toks[i], ref_t), (i, toks[i].tolist(), ref_t.tolist())
        print('[parity] full-width LM fp32: generator greedy tokens equal the oracle\'s', flush=True)
