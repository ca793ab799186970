"""Write the golden fixtures in this folder (run from the repository root:
``python tests/golden/make_golden.py``).

The reference holds no stored vectors for the scans (its tests are
relational), so the fixtures are produced by the oracle's fp64 token-by-token
recurrence, oracle.gdr.recurrent (linear_attention.py:161-195), from seeded
fp32 inputs.  Each case is one .npz with the fp32 inputs, the expected
outputs (computed in fp64, stored rounded to fp32) and a small JSON header
(shapes, gate form, delta, scale, seed).
The cases cover the three gate forms, both write rules, a partial chunk,
a state carried in and out, a packed batch with empty and sub-chunk segments,
a single-token decode step, and head sizes that need padding.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import gdr  # noqa: E402

# name: (lens or B x T, H, dk, dv, gate, delta, scale, seed)
CASES = {
    'gdn_dense':      dict(B=2, T=70, H=1, dk=64, dv=64, gate='scalar', delta=True, scale=0.125, seed=101),
    'kda_dense':      dict(B=1, T=70, H=1, dk=64, dv=64, gate='vector', delta=True, scale=0.125, seed=102),
    'deltanet':       dict(B=1, T=40, H=1, dk=64, dv=32, gate='none', delta=True, scale=0.125, seed=103),
    'gla_scalar':     dict(B=1, T=45, H=2, dk=32, dv=48, gate='scalar', delta=False, scale=0.2, seed=104),
    'gdn_varlen':     dict(lens=[5, 0, 66, 1, 33], H=1, dk=64, dv=32, gate='scalar', delta=True, scale=0.125,
                           seed=105),
    'kda_varlen':     dict(lens=[17, 64, 0, 9], H=1, dk=64, dv=32, gate='vector', delta=True, scale=0.125,
                           seed=106),
    'decode_step':    dict(B=2, T=1, H=2, dk=64, dv=64, gate='scalar', delta=True, scale=0.125, seed=107),
    'odd_heads':      dict(B=1, T=37, H=3, dk=24, dv=20, gate='vector', delta=True, scale=0.3, seed=108),
}


def inputs(case: dict) -> dict:
    """Seeded fp32 inputs, the distributions of the reference's configs:
    q, k L2-normalised N(0,1), v N(0,1), beta sigmoid(N), g logsigmoid(N + 4),
    entry state 0.1 N(0,1)."""
    gen = torch.Generator().manual_seed(case['seed'])
    if 'lens' in case:
        B, T, N = 1, sum(case['lens']), len(case['lens'])
    else:
        B, T, N = case['B'], case['T'], case['B']
    H, dk, dv = case['H'], case['dk'], case['dv']
    q = torch.nn.functional.normalize(torch.randn(B, T, H, dk, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, dk, generator=gen), dim=-1)
    v = torch.randn(B, T, H, dv, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    gshape = {'none': None, 'scalar': (B, T, H), 'vector': (B, T, H, dk)}[case['gate']]
    g = None if gshape is None else torch.nn.functional.logsigmoid(torch.randn(*gshape, generator=gen) + 4.0)
    S0 = 0.1 * torch.randn(N, H, dk, dv, generator=gen)
    cu = None
    if 'lens' in case:
        cu = torch.tensor(np.cumsum([0] + case['lens']), dtype=torch.int32)
    return dict(q=q, k=k, v=v, g=g, beta=beta, S0=S0, cu=cu)


def expected(case: dict, x: dict):
    """fp64 recurrence per sequence (the packed batch is the concatenation of
    independent segments)."""
    d = lambda t: None if t is None else t.double()
    kw = dict(scale=case['scale'], delta=case['delta'])
    beta = x['beta'] if case['delta'] else None
    if x['cu'] is None:
        return gdr.recurrent(d(x['q']), d(x['k']), d(x['v']), d(x['g']), d(beta), d(x['S0']), **kw)
    return gdr.varlen(gdr.recurrent, d(x['q']), d(x['k']), d(x['v']), d(x['g']), d(beta), d(x['S0']),
                      x['cu'], **kw)


def main():
    for name, case in CASES.items():
        x = inputs(case)
        o, S = expected(case, x)
        arrays = {k: v.numpy() for k, v in x.items() if v is not None}
        arrays['o'] = o.float().numpy()
        arrays['S'] = S.float().numpy()
        arrays['meta'] = np.frombuffer(json.dumps(case).encode(), dtype=np.uint8)
        path = os.path.join(HERE, f'{name}.npz')
        np.savez_compressed(path, **arrays)
        print(f'{name}: {os.path.getsize(path)} bytes', flush=True)


if __name__ == '__main__':
    main()
