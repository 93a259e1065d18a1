"""The ops launch on the caller's current stream (the raw handle the wrappers pass to the C-ABI)."""
import pytest
import torch

from kernelswift_amd import ops

pytestmark = pytest.mark.gpu


def test_ops_follow_the_current_stream(device):
    g = torch.Generator(device=device).manual_seed(5)
    x = torch.rand(4096, 4, 4, device=device, generator=g) + 0.1
    want = ops.sinkhorn(x, 10, 1e-6)
    assert ops._stream(x) == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()  # default priority
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert ops._stream(x) == s.cuda_stream
        got = ops.sinkhorn(x, 10, 1e-6)
        done = torch.cuda.Event()
        done.record(s)
    done.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    assert torch.equal(got, want)
