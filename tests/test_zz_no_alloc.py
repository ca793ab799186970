"""vgdr_chunk_fwd_noalloc: the chunked forward with its workspace in the
library's per-GPU scratch array, through the C ABI, against
vgdr_chunk_fwd_fused with a workspace the caller allocates (same kernels,
so bit-exact), on two calls in a row, the second smaller, plus a packed
batch and a fused-producer call; and the size limit's rejection.
"""
import ctypes

import pytest
import torch

from vagus_amd import _lib, workloads

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def case(msg):
    print(f'\n[case] {msg}', flush=True)


def _p(t):
    return None if t is None else t.data_ptr()


def _run(x, *, gate, noalloc, fusion=None, scale=0.1):
    """One chunk forward through the C ABI; returns (o, final state)."""
    L = _lib.load()
    B, T, H, dk = x.q.shape
    dv = x.v.shape[-1]
    N = B if x.cu_seqlens is None else x.cu_seqlens.numel() - 1
    gk = {'none': _lib.VGDR_GATE_NONE, 'scalar': _lib.VGDR_GATE_SCALAR, 'vector': _lib.VGDR_GATE_VECTOR}[gate]
    o = torch.full((B, T, H, dv), float('nan'), dtype=x.q.dtype, device=DEV)
    S = torch.full((N, H, dk, dv), float('nan'), dtype=torch.float32, device=DEV)
    dt = _lib.VGDR_BF16 if x.q.dtype == torch.bfloat16 else _lib.VGDR_F16
    fz = ctypes.byref(fusion) if fusion is not None else None
    stream = torch.cuda.current_stream().cuda_stream
    head = (dt, gk, 1, _p(x.q), _p(x.k), _p(x.v), _p(x.g if gate != 'none' else None), _p(x.beta), _p(o),
            _p(x.initial_state), _p(S), _p(x.cu_seqlens))
    tail = (B, T, H, dk, dv, N, scale, 64)
    if noalloc:
        rc = L.vgdr_chunk_fwd_noalloc(*head, *tail, fz, stream)
    else:
        nbytes = L.vgdr_chunk_workspace_size(dt, gk, B, T, H, dk, N, int(x.cu_seqlens is not None), 64)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
        rc = L.vgdr_chunk_fwd_fused(*head, _p(ws), nbytes, *tail, fz, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return o, S


def _same(a, b, what):
    assert torch.equal(a[0], b[0]), f'{what}: outputs differ'
    assert torch.equal(a[1], b[1]), f'{what}: final states differ'
    print(f'[no-alloc] {what}: bit-exact', flush=True)


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_noalloc_matches_workspace_entry_point_twice(gate):
    case(f'no-alloc chunk forward, {gate} gate: B4 T700 H8 then B1 T90 H2 (dk=dv=128 bf16)')
    big = workloads.make_inputs(4, 700, 8, 128, 128, gate=gate, dtype=torch.bfloat16, s0_scale=0.2, seed=31).to(DEV)
    small = workloads.make_inputs(1, 90, 2, 128, 128, gate=gate, dtype=torch.bfloat16, s0_scale=0.2,
                                  seed=32).to(DEV)
    ref_big = _run(big, gate=gate, noalloc=False)
    ref_small = _run(small, gate=gate, noalloc=False)
    _same(_run(big, gate=gate, noalloc=True), ref_big, f'{gate} first call (larger)')
    _same(_run(small, gate=gate, noalloc=True), ref_small, f'{gate} second call (smaller)')


def test_noalloc_packed_batch_and_fusion():
    case('no-alloc chunk forward: packed batch with empty and short segments, fused L2 norm and beta sigmoid')
    x = workloads.make_varlen_inputs([300, 0, 5, 64, 129], 4, 128, 64, gate='scalar', dtype=torch.bfloat16,
                                     s0_scale=0.1, seed=33).to(DEV)
    x.q, x.k = 3.0 * x.q, 0.5 * x.k                     # un-normalised rows
    x.beta = torch.logit(x.beta.clamp(1e-4, 1 - 1e-4))  # logits
    fz = _lib.Fusion(1, 1, 0, _lib.VGDR_F32, None, None, 0, 0.0)
    _same(_run(x, gate='scalar', noalloc=True, fusion=fz), _run(x, gate='scalar', noalloc=False, fusion=fz),
          'packed + fused producers')


def test_noalloc_rejects_calls_beyond_the_scratch_size():
    case('no-alloc size limit')
    L = _lib.load()
    # B64 T8192 H16 needs far more than the scratch holds; rejected before any launch
    nbytes = L.vgdr_chunk_workspace_size(_lib.VGDR_BF16, 1, 64, 8192, 16, 128, 64, 0, 64)
    assert nbytes > (64 << 20)
    # null tensor pointers: the size check comes first; were it ever to pass,
    # the null-pointer check refuses the call rather than a kernel launching
    rc = L.vgdr_chunk_fwd_noalloc(_lib.VGDR_BF16, 1, 1, None, None, None, None, None, None, None, None, None,
                                  64, 8192, 16, 128, 128, 64, 0.1, 64, None, None)
    assert rc == _lib.VGDR_ERR_INVALID and b'scratch' in L.vgdr_last_error()
