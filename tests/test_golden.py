"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle's fp64 recurrence).

CPU: the oracle reproduces every fixture, through the recurrence and through
the chunk forms.  GPU: the HIP chunk and recurrent paths match every fixture,
rel-L2 <= 1e-5 with the fp32 inputs and <= 2e-2 with the inputs rounded to
bf16 (the tolerances of the fp32 reference recurrence).
"""
import glob
import json
import os

import numpy as np
import pytest
import torch

from oracle import gdr

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')
FILES = sorted(glob.glob(os.path.join(GOLDEN, '*.npz')))
NAMES = [os.path.basename(f)[:-4] for f in FILES]


def load(name):
    z = np.load(os.path.join(GOLDEN, f'{name}.npz'))          # allow_pickle defaults to False
    meta = json.loads(bytes(z['meta']).decode())
    t = {k: torch.from_numpy(z[k]) for k in z.files if k != 'meta'}
    return meta, t


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def test_fixture_set_is_complete():
    assert set(NAMES) == {'gdn_dense', 'kda_dense', 'deltanet', 'gla_scalar', 'gdn_varlen', 'kda_varlen',
                          'decode_step', 'odd_heads'}


@pytest.mark.parametrize('name', NAMES)
@pytest.mark.parametrize('form', ['recurrent', 'chunk16', 'chunk64'])
def test_oracle_reproduces_fixture(name, form):
    meta, t = load(name)
    d = lambda k: t[k].double() if k in t else None
    beta = d('beta') if meta['delta'] else None
    if form == 'recurrent':
        fn, kw = gdr.recurrent, {}
    else:
        fn, kw = gdr.chunk, {'chunk_size': int(form[5:])}
    kw.update(scale=meta['scale'], delta=meta['delta'])
    if 'cu' in t:
        o, S = gdr.varlen(fn, d('q'), d('k'), d('v'), d('g'), beta, d('S0'), t['cu'], **kw)
    else:
        o, S = fn(d('q'), d('k'), d('v'), d('g'), beta, d('S0'), **kw)
    # the stored values are the fp64 results rounded to fp32
    assert rel(o, t['o']) < 1e-6 and rel(S, t['S']) < 1e-6


def _gpu_case(name, dtype):
    from vagus_amd import ops
    meta, t = load(name)
    dev = 'cuda'
    q, k, v = (t[n].to(dtype).to(dev) for n in ('q', 'k', 'v'))
    g = t['g'].to(dev) if 'g' in t else None
    beta = t['beta'].to(dev)
    S0 = t['S0'].to(dev)
    cu = t['cu'].to(dev) if 'cu' in t else None
    return ops, meta, t, (q, k, v, g, beta, S0, cu)


@pytest.mark.gpu
@pytest.mark.parametrize('name', NAMES)
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_hip_chunk_matches_fixture(name, dtype):
    ops, meta, t, (q, k, v, g, beta, S0, cu) = _gpu_case(name, dtype)
    print(f'[golden] chunk {name} {dtype}', flush=True)
    o, S = ops.chunk_scan(q, k, v, g, beta if meta['delta'] else None, gate=meta['gate'], delta=meta['delta'],
                          scale=meta['scale'], initial_state=S0, output_final_state=True, cu_seqlens=cu)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert o.dtype == dtype and S.dtype == torch.float32
    assert rel(o, t['o']) <= tol and rel(S, t['S']) <= tol, (rel(o, t['o']), rel(S, t['S']))


@pytest.mark.gpu
@pytest.mark.parametrize('name', NAMES)
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_hip_recurrent_matches_fixture(name, dtype):
    ops, meta, t, (q, k, v, g, beta, S0, cu) = _gpu_case(name, dtype)
    print(f'[golden] recurrent {name} {dtype}', flush=True)
    o, S = ops.hip_recurrent(q, k, v, g, beta if meta['delta'] else None, S0, scale=meta['scale'],
                             delta=meta['delta'], cu_seqlens=cu)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel(o, t['o']) <= tol and rel(S, t['S']) <= tol, (rel(o, t['o']), rel(S, t['S']))
