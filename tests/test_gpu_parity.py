"""GPU parity of the HIP kernels against the CPU oracle (the fp64 token
recurrence and its chunk forms), on identical seeded inputs.

Bars (written into each test): relative L2 error of outputs and final states
<= 1e-5 for fp32 inputs and <= 2e-2 for bf16 / fp16 inputs; integer tables
bit-exact.  rel_l2(x, ref) = ||x - ref||_2 / ||ref||_2, computed in fp64 on
the CPU.  bf16 inputs are rounded first and the oracle consumes the rounded
values, so only the kernels' own arithmetic is measured.
"""
import numpy as np
import pytest
import torch

from oracle import gdr
from vagus_amd import ops, workloads
from vagus_amd import _lib

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
DEV = 'cuda'


def rel_l2(x, ref):
    x, ref = x.detach().double().cpu(), ref.detach().double().cpu()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def case(msg):
    print(f'\n[case] {msg}', flush=True)


def oracle_run(x, *, scale, delta=True, fn=gdr.recurrent):
    """fp64 oracle on the (already rounded) inputs of ScanInputs x (CPU)."""
    d = lambda t: None if t is None else t.double()
    args = (d(x.q), d(x.k), d(x.v), d(x.g), d(x.beta), d(x.initial_state))
    if x.cu_seqlens is not None:
        return gdr.varlen(fn, *args, x.cu_seqlens, scale=scale, delta=delta)
    return fn(*args, scale=scale, delta=delta)


def run_chunk(x, *, scale, delta=True, chunk_size=64):
    y = x.to(DEV)
    if delta:
        gate = 'vector' if (y.g is not None and y.g.dim() == 4) else 'scalar'
        if gate == 'vector':
            return ops.chunk_kda(y.q, y.k, y.v, y.g, y.beta, scale=scale, initial_state=y.initial_state,
                                 output_final_state=True, cu_seqlens=y.cu_seqlens, chunk_size=chunk_size)
        return ops.chunk_gated_delta_rule(y.q, y.k, y.v, y.g, y.beta, scale=scale,
                                          initial_state=y.initial_state, output_final_state=True,
                                          cu_seqlens=y.cu_seqlens, chunk_size=chunk_size)
    return ops.hip_scan(y.q, y.k, y.v, y.g, None, y.initial_state, scale=scale, delta=False,
                        chunk_size=chunk_size, cu_seqlens=y.cu_seqlens)


def check(o, S, ref, dtype, what):
    tol = TOL[dtype]
    eo, es = rel_l2(o, ref[0]), rel_l2(S, ref[1])
    print(f'[parity] {what}: rel_l2 o={eo:.3e} S={es:.3e} (tol {tol:g})', flush=True)
    assert torch.isfinite(o.float()).all() and torch.isfinite(S).all()
    assert eo <= tol, f'{what}: output rel L2 {eo:.3e} > {tol}'
    assert es <= tol, f'{what}: state rel L2 {es:.3e} > {tol}'


# --- recurrent (decode) kernel ---------------------------------------------

@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('gate', ['scalar', 'vector', 'none'])
@pytest.mark.parametrize('delta', [True, False])
def test_recurrent_matches_oracle(dtype, gate, delta):
    case(f'recurrent dtype={dtype} gate={gate} delta={delta} B2 T37 H3 dk64 dv128')
    x = workloads.make_inputs(2, 37, 3, 64, 128, gate=gate, dtype=dtype, s0_scale=0.3, seed=11)
    ref = oracle_run(x, scale=0.125, delta=delta)
    y = x.to(DEV)
    o, S = ops.hip_recurrent(y.q, y.k, y.v, y.g, y.beta, y.initial_state, scale=0.125, delta=delta)
    check(o, S, ref, dtype, f'recurrent {gate} delta={delta}')


def test_decode_step_in_place_and_config4_shape():
    """One decode step at the 1.3B layer shape (B64 H16 dk=dv=128), state updated in place."""
    case('decode in place B64 H16 dk128 dv128 bf16')
    x = workloads.make_inputs(64, 1, 16, 128, 128, gate='scalar', dtype=torch.bfloat16, s0_scale=0.5, seed=5)
    ref = oracle_run(x, scale=128 ** -0.5)
    y = x.to(DEV)
    state = y.initial_state.clone()
    ptr = state.data_ptr()
    o, S = ops.fused_recurrent_gated_delta_rule(y.q, y.k, y.v, y.g, y.beta, initial_state=state,
                                                output_final_state=True, inplace_final_state=True)
    assert S.data_ptr() == ptr
    check(o, state, ref, torch.bfloat16, 'decode step')


# --- chunk kernel ----------------------------------------------------------

def test_chunk_gdn_cpu_workload_fp32():
    """The fp32 CPU workload (B2 T256 H4 dk=dv=64, chunk 64) at 1e-5."""
    case('chunk gdn_cpu fp32')
    x = workloads.workload('gdn_cpu')
    scale = 64 ** -0.5
    ref = oracle_run(x, scale=scale)
    o, S = run_chunk(x, scale=scale)
    check(o, S, ref, torch.float32, 'gdn_cpu fp32 chunk')


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize('gate', ['scalar', 'vector', 'none'])
@pytest.mark.parametrize('delta', [True, False])
@pytest.mark.parametrize('dk', [64, 128])
def test_chunk_matches_oracle(dtype, gate, delta, dk):
    case(f'chunk dtype={dtype} gate={gate} delta={delta} dk={dk} B2 T200 H2 dv128')
    x = workloads.make_inputs(2, 200, 2, dk, 128, gate=gate, dtype=dtype, s0_scale=0.2, seed=7)
    scale = dk ** -0.5
    ref = oracle_run(x, scale=scale, delta=delta)
    o, S = run_chunk(x, scale=scale, delta=delta)
    check(o, S, ref, dtype, f'chunk {gate} delta={delta} dk={dk} {dtype}')


@pytest.mark.parametrize('chunk_size', [32, 64])
def test_chunk_size_option(chunk_size):
    case(f'chunk_size={chunk_size} bf16 gdn')
    x = workloads.make_inputs(1, 150, 2, 128, 64, gate='scalar', dtype=torch.bfloat16, s0_scale=0.1, seed=3)
    ref = oracle_run(x, scale=0.1)
    o, S = run_chunk(x, scale=0.1, chunk_size=chunk_size)
    check(o, S, ref, torch.bfloat16, f'chunk_size {chunk_size}')


def test_chunk_odd_head_dims_are_padded():
    """The reference tests' shapes (dk=8, dv=12) go through zero padding."""
    case('chunk odd dims dk8 dv12 fp32')
    x = workloads.make_inputs(2, 37, 3, 8, 12, gate='scalar', dtype=torch.float32, s0_scale=0.3, seed=0)
    ref = oracle_run(x, scale=0.5)
    o, S = run_chunk(x, scale=0.5)
    assert o.shape == (2, 37, 3, 12) and S.shape == (2, 3, 8, 12)
    check(o, S, ref, torch.float32, 'odd dims')


def test_kda_strong_decay_pairwise_path():
    """Decay ranges beyond the sub-block factorisation limit take the exact path."""
    case('kda strong decay bf16')
    x = workloads.make_inputs(1, 128, 2, 128, 128, gate='vector', dtype=torch.bfloat16, s0_scale=0.1,
                              seed=9, g_shift=-3.0)
    x.g[..., :8] -= 12.0          # channels decaying ~12 nats per token
    ref = oracle_run(x, scale=0.1)
    o, S = run_chunk(x, scale=0.1)
    check(o, S, ref, torch.bfloat16, 'kda strong decay')


# --- packed variable-length batches -----------------------------------------

@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_varlen_matches_oracle(gate):
    lens = [5, 0, 130, 64, 1, 257, 63]
    case(f'varlen {gate} lens={lens} bf16 H2 dk128 dv128')
    x = workloads.make_varlen_inputs(lens, 2, 128, 128, gate=gate, dtype=torch.bfloat16, s0_scale=0.2, seed=4)
    ref = oracle_run(x, scale=0.09)
    o, S = run_chunk(x, scale=0.09)
    check(o, S, ref, torch.bfloat16, f'varlen {gate}')
    # the recurrent kernel on the same packed batch
    y = x.to(DEV)
    o2, S2 = ops.hip_recurrent(y.q, y.k, y.v, y.g, y.beta, y.initial_state, scale=0.09, delta=True,
                               cu_seqlens=y.cu_seqlens)
    check(o2, S2, ref, torch.bfloat16, f'varlen recurrent {gate}')


def test_varlen_segments_isolated_bit_exact():
    lens = [70, 33, 128]
    case(f'varlen isolation lens={lens}')
    x = workloads.make_varlen_inputs(lens, 2, 128, 64, gate='scalar', dtype=torch.bfloat16, s0_scale=0.2, seed=8)
    o, S = run_chunk(x, scale=0.1)
    x2 = workloads.make_varlen_inputs(lens, 2, 128, 64, gate='scalar', dtype=torch.bfloat16, s0_scale=0.2, seed=8)
    x2.v[:, 70:103] += 1.0                          # perturb segment 1 only
    o2, S2 = run_chunk(x2, scale=0.1)
    keep = torch.ones(sum(lens), dtype=torch.bool)
    keep[70:103] = False
    assert torch.equal(o[:, keep.to(DEV)], o2[:, keep.to(DEV)])
    assert torch.equal(S[0], S2[0]) and torch.equal(S[2], S2[2]) and not torch.equal(S[1], S2[1])
    # a segment run alone equals its slot in the packed run, bit for bit
    for n, (s, e) in enumerate([(0, 70), (70, 103), (103, 231)]):
        y = x.to(DEV)
        o1, S1 = ops.chunk_gated_delta_rule(y.q[:, s:e], y.k[:, s:e], y.v[:, s:e], y.g[:, s:e],
                                            y.beta[:, s:e], scale=0.1,
                                            initial_state=y.initial_state[n:n + 1],
                                            output_final_state=True)
        assert torch.equal(o1, o[:, s:e]) and torch.equal(S1, S[n:n + 1])


def test_varlen_schedule_table_bit_exact():
    case('varlen schedule table')
    rng = np.random.default_rng(1)
    L = _lib.load()
    for trial in range(5):
        lens = rng.integers(0, 9000, size=int(rng.integers(1, 200))).tolist()
        cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32, device=DEV)
        N = len(lens)
        ws = torch.empty(L.vgdr_varlen_workspace_size(N), dtype=torch.uint8, device=DEV)
        _lib.check(L.vgdr_varlen_prepare(cu.data_ptr(), N, int(cu[-1]), 64, ws.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream))
        got = ws.view(torch.int32).cpu().numpy()
        want = gdr.chunk_table(cu.cpu(), 64)
        assert np.array_equal(got[:N], want['lens'])
        assert np.array_equal(got[N:2 * N], want['chunks'])
        assert np.array_equal(got[2 * N:3 * N + 1], want['chunk_offsets'])
        assert np.array_equal(got[3 * N + 1:], want['order'])


@pytest.mark.parametrize('gate', ['scalar', 'vector'])
def test_split_phases_equal_fused_call_bit_exact(gate):
    """vgdr_chunk_prep + vgdr_chunk_state (an event between them) == vgdr_chunk_fwd, bit for bit,
    for a dense and a packed batch."""
    case(f'prep + state vs fwd, {gate}')
    dense = workloads.make_inputs(2, 200, 2, 128, 128, gate=gate, dtype=torch.bfloat16, s0_scale=0.1, seed=12)
    packed = workloads.make_varlen_inputs([5, 130, 64, 0, 257], 2, 128, 128, gate=gate, dtype=torch.bfloat16,
                                          s0_scale=0.1, seed=13)
    for x in (dense.to(DEV), packed.to(DEV)):
        kw = dict(gate=gate, delta=True, scale=0.1, initial_state=x.initial_state, output_final_state=True,
                  cu_seqlens=x.cu_seqlens)
        o1, S1 = ops.chunk_scan(x.q, x.k, x.v, x.g, x.beta, **kw)
        o2, S2 = ops.chunk_scan(x.q, x.k, x.v, x.g, x.beta, phase_event=torch.cuda.Event(), **kw)
        assert torch.equal(o1, o2) and torch.equal(S1, S2)


def test_empty_sequence_passes_state_through():
    case('empty input')
    S0 = torch.randn(2, 2, 64, 64, device=DEV)
    q = torch.zeros(2, 0, 2, 64, device=DEV)
    o, S = ops.chunk_gated_delta_rule(q, q, q, torch.zeros(2, 0, 2, device=DEV), torch.zeros(2, 0, 2, device=DEV),
                                      initial_state=S0, output_final_state=True)
    assert o.shape == (2, 0, 2, 64) and torch.equal(S, S0)


def test_module_level_contract_matches_fla_scan():
    """hip_scan returns (o in q.dtype, fp32 S) for every gate form, like fla_scan."""
    case('hip_scan contract')
    for gate in ('scalar', 'vector', 'none'):
        x = workloads.make_inputs(1, 70, 2, 64, 64, gate=gate, dtype=torch.bfloat16, seed=1).to(DEV)
        o, S = ops.hip_scan(x.q, x.k, x.v, x.g, x.beta, None, scale=0.125, delta=True)
        assert o.dtype == torch.bfloat16 and S.dtype == torch.float32 and S.shape == (1, 2, 64, 64)
