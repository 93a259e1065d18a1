"""GPU parity: Sinkhorn kernel vs the fp64 oracle (tolerance atol = rtol = 1e-2, the reference's
auto_bench contract; the kernel is expected to be far tighter and that is asserted too)."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _run(x, repeat=10, eps=1e-6):
    print(f"[case] sinkhorn shape={tuple(x.shape)} repeat={repeat}", flush=True)
    y = ops.sinkhorn(x, repeat, eps)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_sinkhorn_config1(device):
    w = workloads.CONFIGS[1](device)
    got = _run(w.tensors["x"], 10)
    want = oracle.sinkhorn(w.tensors["x"].cpu().numpy(), 10, 1e-6)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    assert np.max(np.abs(got - want)) < 1e-5


@pytest.mark.parametrize("shape,repeat", [((1, 1024, 4, 4), 10), ((3, 4, 4), 1), ((1, 4, 4), 20), ((777, 4, 4), 20),
                                          ((2, 65, 4, 4), 3)])
def test_sinkhorn_shapes(device, shape, repeat):
    g = torch.Generator().manual_seed(sum(shape) + repeat)
    x = (torch.randn(shape, generator=g) * 3).to(device)
    got = _run(x, repeat)
    want = oracle.sinkhorn(x.cpu().numpy(), repeat, 1e-6)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    assert np.max(np.abs(got - want)) < 1e-5


def test_sinkhorn_empty_and_errors(device):
    x = torch.empty(0, 4, 4, device=device)
    assert ops.sinkhorn(x).shape == (0, 4, 4)
    with pytest.raises(RuntimeError):
        ops.sinkhorn(torch.zeros(2, 3, 3, device=device))
    with pytest.raises(RuntimeError):
        ops.sinkhorn(torch.zeros(2, 4, 4, device=device, dtype=torch.float64))
    with pytest.raises(RuntimeError):
        ops.sinkhorn(torch.zeros(2, 4, 4, device=device), repeat=0)


def test_sinkhorn_large_doubly_stochastic(device):
    g = torch.Generator(device=device).manual_seed(5)
    x = torch.randn(1 << 20, 4, 4, device=device, generator=g)
    print("[case] sinkhorn 1M matrices", flush=True)
    y = ops.sinkhorn(x, 10, 1e-6)
    torch.cuda.synchronize()
    assert torch.all(y > 0)
    # columns are normalised last: sums are s/(s+eps)
    assert torch.allclose(y.sum(-2), torch.ones(1, device=device), atol=1e-5)
    # rows converge at the algorithm's own rate: compare with the fp64 oracle, not with 1
    want = oracle.sinkhorn(x.cpu().numpy(), 10, 1e-6)
    np.testing.assert_allclose(y.cpu().numpy(), want, atol=1e-2, rtol=1e-2)
    assert np.max(np.abs(y.cpu().numpy() - want)) < 1e-4


@pytest.mark.parametrize("shape,repeat", [((65536, 4, 4), 10), ((65536 + 77, 4, 4), 10), ((3, 25001, 4, 4), 5),
                                          ((786432 + 77, 4, 4), 10), ((2 * 786432 + 5, 4, 4), 2)])
def test_sinkhorn_matrix_per_lane_ragged(device, shape, repeat):
    # batches from 65536 matrices on take the matrix-per-lane kernel; ragged tails leave part of the last
    # wave idle.  Its waves are persistent (12 workgroups of 4 waves per CU: 786432 matrices per stride on 256
    # CUs), so the last two shapes end in a ragged batch reached on a wave's second and third pass.
    g = torch.Generator().manual_seed(sum(shape) + repeat)
    x = (torch.randn(shape, generator=g) * 3).to(device)
    got = _run(x, repeat)
    want = oracle.sinkhorn(x.cpu().numpy(), repeat, 1e-6)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    assert np.max(np.abs(got - want)) < 1e-5
