"""ks_sparse_attn_noalloc (the entry point that allocates nothing) against ks_sparse_attn with a caller
workspace, through the C ABI: two calls in a row, the second smaller, bit for bit (the same kernels and
split plan run on the static scratch instead of the workspace), plus the size limit."""
import ctypes

import pytest
import torch

from kernelswift_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(g, B, M, H, Dqk, N, K, device):
    q = torch.randn(B, M, H, Dqk, generator=g).bfloat16().to(device)
    kv = torch.randn(B, N, Dqk, generator=g).bfloat16().to(device)
    sink = torch.randn(H, generator=g).to(device)
    idx = torch.randint(-1, N, (B, M, K), generator=g, dtype=torch.int32).to(device)
    return q, kv, sink, idx


def _with_workspace(lib, q, kv, sink, idx, Dv, stream):
    B, M, H, Dqk = q.shape
    N, K = kv.shape[1], idx.shape[2]
    need = lib.ks_sparse_attn_workspace_size(B, M, H, Dqk, Dv, K)
    # a fresh workspace full of NaN patterns: a partial read before it is written would show in the output
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=q.device)
    out = torch.empty(B, M, H, Dv, dtype=torch.bfloat16, device=q.device)
    _lib.check(lib.ks_sparse_attn(q.data_ptr(), kv.data_ptr(), sink.data_ptr(), idx.data_ptr(), out.data_ptr(),
                                  B, M, H, Dqk, Dv, N, K, Dqk ** -0.5, ws.data_ptr(), need, stream),
               "ks_sparse_attn")
    return out, need


def _no_alloc(lib, q, kv, sink, idx, Dv, stream, out=None):
    B, M, H, Dqk = q.shape
    N, K = kv.shape[1], idx.shape[2]
    if out is None:
        out = torch.empty(B, M, H, Dv, dtype=torch.bfloat16, device=q.device)
    _lib.check(lib.ks_sparse_attn_noalloc(q.data_ptr(), kv.data_ptr(), sink.data_ptr(), idx.data_ptr(),
                                          out.data_ptr(), B, M, H, Dqk, Dv, N, K, Dqk ** -0.5, stream),
               "ks_sparse_attn_noalloc")
    return out


def test_no_alloc_matches_workspace_entry(device):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator().manual_seed(12)
    cases = [(1, 128, 16, 128, 128, 8192, 2048),  # config 3's shape: 8.25 MiB of split partials
             (2, 24, 16, 128, 128, 3000, 1024),   # smaller, after it: the scratch holds the first call's data
             (4, 1, 128, 576, 512, 4096, 2048),   # the MLA decode kernel's split path
             (1, 3, 64, 576, 512, 700, 300)]      # and a smaller one after it
    for B, M, H, Dqk, Dv, N, K in cases:
        print(f"[case] no-alloc sparse attention B={B} M={M} H={H} Dqk={Dqk} K={K}", flush=True)
        q, kv, sink, idx = _inputs(g, B, M, H, Dqk, N, K, device)
        want, need = _with_workspace(lib, q, kv, sink, idx, Dv, stream)
        got = _no_alloc(lib, q, kv, sink, idx, Dv, stream)
        torch.cuda.synchronize()
        assert need > 0, "the case must exercise the split scratch"
        assert torch.equal(got, want)


def test_no_alloc_rejects_shapes_beyond_the_scratch(device):
    lib = _lib.load()
    limit = lib.ks_sparse_attn_noalloc_max_scratch()
    assert limit == 64 << 20
    B, M, H, Dqk, Dv, K = 1, 32, 128, 576, 512, 65536  # 129 MiB of partials: refused before any launch
    assert lib.ks_sparse_attn_workspace_size(B, M, H, Dqk, Dv, K) > limit
    dummy = torch.empty(16, dtype=torch.uint8, device=device)
    p = dummy.data_ptr()
    rc = lib.ks_sparse_attn_noalloc(p, p, p, p, p, B, M, H, Dqk, Dv, 1024, K, 0.1,
                                    torch.cuda.current_stream(device).cuda_stream)
    assert rc == 1 and b"maximum" in lib.ks_last_error()


def test_no_alloc_stale_scratch_invalid_ranges(device):
    # after a call that fills the scratch with valid partials, calls whose split ranges hold only invalid
    # indices (queries whose lists are all -1, or lists shorter than the later ranges): the combine must not
    # read the previous call's partials for them
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator().manual_seed(21)
    big = (1, 128, 16, 128, 128, 8192, 2048)
    for B, M, H, Dqk, Dv, N, K, mode in [(*big, "fill"), (1, 128, 16, 128, 128, 8192, 2048, "half_invalid"),
                                         (*big, "fill"), (2, 40, 16, 128, 128, 8192, 2048, "tail_invalid"),
                                         (4, 1, 128, 576, 512, 4096, 2048, "fill"),
                                         (4, 1, 128, 576, 512, 4096, 2048, "half_invalid")]:
        print(f"[case] no-alloc stale scratch {mode} B={B} M={M} H={H} Dqk={Dqk} K={K}", flush=True)
        q, kv, sink, idx = _inputs(g, B, M, H, Dqk, N, K, device)
        if mode == "half_invalid":
            idx.view(B * M, K)[::2] = -1          # every other query has no valid index at all
        elif mode == "tail_invalid":
            idx[:, :, 40:] = -1                   # only the first range of each list is valid
        want, need = _with_workspace(lib, q, kv, sink, idx, Dv, stream)
        got = _no_alloc(lib, q, kv, sink, idx, Dv, stream)
        torch.cuda.synchronize()
        assert need > 0
        assert torch.equal(got, want)
        if mode == "half_invalid":
            # a query with no valid index: z = sink, the denominator is exp(0) = 1, the output is zero
            assert torch.count_nonzero(got.view(B * M, -1)[::2]) == 0


def test_no_alloc_under_graph_capture(device):
    # one eager call resolves the device's scratch address; a captured call then records kernel launches only
    # (the library issues no memset), and every replay matches the workspace entry's eager result
    lib = _lib.load()
    g = torch.Generator().manual_seed(33)
    B, M, H, Dqk, Dv, N, K = 1, 128, 16, 128, 128, 8192, 2048
    q, kv, sink, idx = _inputs(g, B, M, H, Dqk, N, K, device)
    print("[case] no-alloc sparse attention under graph capture (config 3 shape)", flush=True)
    stream = torch.cuda.current_stream(device).cuda_stream
    want, _ = _with_workspace(lib, q, kv, sink, idx, Dv, stream)
    _no_alloc(lib, q, kv, sink, idx, Dv, stream)  # the warm call
    torch.cuda.synchronize()
    out = torch.zeros(B, M, H, Dv, dtype=torch.bfloat16, device=device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _no_alloc(lib, q, kv, sink, idx, Dv, torch.cuda.current_stream(device).cuda_stream, out=out)
    for r in range(3):
        out.zero_()
        other, _ = _with_workspace(lib, q, kv, sink, idx[:, :, :1024].contiguous(), Dv, stream)  # eager work between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"
        assert other.shape == want.shape
