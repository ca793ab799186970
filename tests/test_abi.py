"""CPU checks of the C ABI and the host-side logic (no GPU needed).

The library must load here (it is built for gfx950 but its host code runs
anywhere), export every symbol include/vagus_gdr.h declares, and reject bad
arguments with the documented status codes before touching a device.
"""
import ctypes
import os
import re

import pytest
import torch

from vagus_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'vagus_gdr.h')


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?(?:int|int64_t|char\s*\*|const char \*)\s*\*?\s*(vgdr_\w+)\s*\(',
                                 text, re.M)))


def test_header_declares_the_bound_symbols():
    syms = header_symbols()
    assert syms == sorted(_lib.SIGNATURES), (syms, sorted(_lib.SIGNATURES))


def test_library_loads_and_exports_every_symbol():
    L = _lib.load()
    for name in header_symbols():
        assert hasattr(L, name), name
    assert L.vgdr_version() >= 100
    assert L.vgdr_varlen_workspace_size(32) == (4 * 32 + 1) * 4
    assert L.vgdr_varlen_workspace_size(-1) == 0


def _chunk_call(fn='vgdr_chunk_fwd', **over):
    a = dict(dtype=1, gate=1, delta=1, q=None, k=None, v=None, g=None, beta=None, o=None, h0=None,
             ht=None, cu=None, ws=None, nbytes=0, B=2, T=0, H=4, dk=128, dv=128, N=2, scale=1.0, chunk=64)
    a.update(over)
    return getattr(_lib.load(), fn)(a['dtype'], a['gate'], a['delta'], a['q'], a['k'], a['v'], a['g'],
                                      a['beta'], a['o'], a['h0'], a['ht'], a['cu'], a['ws'], a['nbytes'],
                                      a['B'], a['T'], a['H'], a['dk'], a['dv'], a['N'], a['scale'],
                                      a['chunk'], None)


def test_argument_checks_return_status_codes():
    L = _lib.load()
    assert _chunk_call(dtype=7) == _lib.VGDR_ERR_INVALID
    assert b'dtype' in L.vgdr_last_error()
    assert _chunk_call(gate=5) == _lib.VGDR_ERR_INVALID
    assert _chunk_call(dk=256) == _lib.VGDR_ERR_UNSUPPORTED
    assert _chunk_call(dv=12) == _lib.VGDR_ERR_UNSUPPORTED
    assert _chunk_call(N=3) == _lib.VGDR_ERR_INVALID            # dense batch: N == B
    assert _chunk_call(cu=8, B=2) == _lib.VGDR_ERR_INVALID      # packed batch needs B == 1
    assert _chunk_call(T=4) == _lib.VGDR_ERR_INVALID            # q/k/v/o missing
    assert _chunk_call(T=4, q=16, k=32, v=48, o=64, g=None) == _lib.VGDR_ERR_INVALID  # gate needs g
    assert _chunk_call(T=4, q=16, k=32, v=48, o=64, g=80, beta=None) == _lib.VGDR_ERR_INVALID
    assert _chunk_call(T=4, q=17, k=32, v=48, o=64, g=80, beta=96) == _lib.VGDR_ERR_INVALID  # alignment
    # the workspace must be present and large enough
    need = L.vgdr_chunk_workspace_size(1, 1, 2, 64, 4, 128, 2, 0, 64)
    # per (chunk, head): TE and A (2 C^2 elements), then the row factors GX, GO,
    # GE (3 C floats), Gc and three floats of padding
    assert need == 2 * 4 * (2 * 64 * 64 * 2 + (3 * 64 + 4) * 4)
    assert _chunk_call(T=64, q=16, k=32, v=48, o=64, g=80, beta=96, ws=None) == _lib.VGDR_ERR_INVALID
    assert _chunk_call(T=64, q=16, k=32, v=48, o=64, g=80, beta=96, ws=4096, nbytes=need - 1) == _lib.VGDR_ERR_INVALID
    assert b'workspace' in L.vgdr_last_error()
    # fp32 with 128-wide keys runs 32-token chunks; packed batches add the segment table
    assert L.vgdr_chunk_workspace_size(0, 1, 1, 64, 1, 128, 1, 0, 64) == 2 * (2 * 32 * 32 * 4 + (3 * 32 + 4) * 4)
    assert L.vgdr_chunk_workspace_size(1, 1, 1, 100, 2, 64, 3, 1, 64) == 256 + (2 + 3) * 2 * (2 * 64 * 64 * 2 + (3 * 64 + 4) * 4)
    # a per-channel gate (16-bit) adds the gated K, Q, K*Gend tiles and Gc per (chunk, head)
    assert L.vgdr_chunk_workspace_size(1, 2, 1, 64, 1, 128, 1, 0, 64) == 2 * 64 * 64 * 2 + 3 * 64 * 128 * 2 + 128 * 4
    assert L.vgdr_chunk_workspace_size(0, 2, 1, 64, 1, 128, 1, 0, 64) == 2 * (2 * 32 * 32 * 4 + (3 * 32 + 4) * 4)
    rc = L.vgdr_recurrent_fwd(1, 1, 1, None, None, None, None, None, None, None, None, None,
                              1, 0, 4, 128, 256, 1, 1.0, None)
    assert rc == _lib.VGDR_ERR_UNSUPPORTED
    assert L.vgdr_varlen_prepare(None, 4, 100, 64, None, None) == _lib.VGDR_ERR_INVALID
    assert L.vgdr_varlen_prepare(None, 0, 0, 64, None, None) == _lib.VGDR_OK


@pytest.mark.parametrize('fn', ['vgdr_chunk_prep', 'vgdr_chunk_state'])
def test_phase_entry_points_check_like_the_fused_one(fn):
    L = _lib.load()
    assert _chunk_call(fn, dtype=7) == _lib.VGDR_ERR_INVALID
    assert fn.encode() in L.vgdr_last_error()
    assert _chunk_call(fn, dk=256) == _lib.VGDR_ERR_UNSUPPORTED
    assert _chunk_call(fn, T=64, q=16, k=32, v=48, o=64, g=80, beta=96, ws=None) == _lib.VGDR_ERR_INVALID
    assert b'workspace' in L.vgdr_last_error()
    assert _chunk_call(fn, B=0, N=0) == _lib.VGDR_OK                  # no sequences: nothing to launch


def test_status_codes_map_to_reference_exceptions():
    _chunk_call(dtype=7)
    with pytest.raises(AssertionError):
        _lib.check(_lib.VGDR_ERR_INVALID)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.VGDR_ERR_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.VGDR_ERR_HIP)


def test_cpu_tensors_fail_loudly():
    q = torch.randn(1, 4, 2, 64)
    with pytest.raises(RuntimeError, match='ROCm GPU'):
        ops.chunk_gated_delta_rule(q, q, q, torch.zeros(1, 4, 2), torch.ones(1, 4, 2))
    with pytest.raises(RuntimeError, match='ROCm GPU'):
        ops.fused_recurrent_kda(q, q, q, torch.zeros(1, 4, 2, 64), torch.ones(1, 4, 2))


def test_missing_library_raises(tmp_path):
    with pytest.raises(RuntimeError, match='not built'):
        _lib.load(str(tmp_path / 'nope.so'))


def test_padding_helpers():
    assert ops._dk_pad(8) == 64 and ops._dk_pad(64) == 64 and ops._dk_pad(100) == 128
    with pytest.raises(NotImplementedError):
        ops._dk_pad(256)
    t = torch.ones(2, 3, 5, 7)
    p = ops._pad_to(t, {1: 16, 2: 8})
    assert p.shape == (2, 3, 8, 16) and p[..., :5, :7].eq(1).all() and p.sum() == t.sum()
    assert ops._pad_to(t, {1: 7}) is t


def test_noalloc_entry_point_rejects_calls_beyond_its_scratch():
    """vgdr_chunk_fwd_noalloc checks the workspace a call needs against the
    library's per-GPU scratch before it touches a device."""
    L = _lib.load()
    limit = 64 << 20
    assert L.vgdr_chunk_workspace_size(_lib.VGDR_BF16, 1, 64, 8192, 16, 128, 64, 0, 64) > limit
    rc = L.vgdr_chunk_fwd_noalloc(_lib.VGDR_BF16, 1, 1, 4096, 8192, 12288, 16384, 20480, 24576, None, None, None,
                                  64, 8192, 16, 128, 128, 64, 0.1, 64, None, None)
    assert rc == _lib.VGDR_ERR_INVALID and b'scratch' in L.vgdr_last_error()
