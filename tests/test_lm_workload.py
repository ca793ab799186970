"""The 1.3B-shape generation workload (vagus_amd.workloads.lm_workload,
gdn_lm_1p3b) at full size on the GPU: the model's parameter count is the
reference layout's (55.7 M per layer plus the 65.5 M tied embedding), ragged
prefill of the 64 prompts and graph-replayed decode run, and the replayed
steps reproduce eager steps exactly from the same prefill.  The numerics of
each piece are pinned at smaller shapes against the oracle (test_layer.py,
test_model.py, the kernel tests at the per-layer decode shape B64 H16)."""
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
