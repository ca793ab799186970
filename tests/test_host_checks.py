"""Host-side checks of the packed-batch offsets (ops._check_cu), on the CPU:
the contract is enforced, a tensor that passed is not read back again while
it is unmodified, and an in-place change is checked again."""
import pytest
import torch

from vagus_amd import ops


def test_cu_contract_rejects_bad_tables():
    with pytest.raises(AssertionError, match=r'cu_seqlens\[0\]'):
        ops._check_cu(torch.tensor([1, 4, 9], dtype=torch.int32), 9)
    with pytest.raises(AssertionError, match='packed tokens'):
        ops._check_cu(torch.tensor([0, 4, 8], dtype=torch.int32), 9)
    with pytest.raises(AssertionError, match='non-decreasing'):
        ops._check_cu(torch.tensor([0, 5, 4, 9], dtype=torch.int32), 9)
    with pytest.raises(AssertionError, match='integer'):
        ops._check_cu(torch.tensor([0.0, 9.0]), 9)


def test_cu_checked_once_per_version(monkeypatch):
    cu = torch.tensor([0, 3, 3, 9], dtype=torch.int32)
    ops._check_cu(cu, 9)
    reads = []
    real_to = torch.Tensor.to

    def counting_to(self, *a, **kw):
        reads.append(1)
        return real_to(self, *a, **kw)

    monkeypatch.setattr(torch.Tensor, 'to', counting_to)
    for _ in range(5):
        ops._check_cu(cu, 9)                      # the same unmodified tensor: no read-back
    assert reads == []
    with pytest.raises(AssertionError):
        ops._check_cu(cu, 10)                     # another token count is checked again
    cu[2] = 7                                     # in place: a new version, checked again
    ops._check_cu(cu, 9)
    cu[2] = 1
    with pytest.raises(AssertionError, match='non-decreasing'):
        ops._check_cu(cu, 9)
    # an equal table in a new tensor is checked on its own
    reads.clear()
    ops._check_cu(torch.tensor([0, 3, 3, 9], dtype=torch.int32), 9)
    assert reads
