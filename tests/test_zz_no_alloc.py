"""The allocation-free dispatch entry point (moe_dispatch_noalloc, no reference counterpart)
against moe_dispatch with a caller workspace, through the C ABI.

Two calls in a row share the library's static histogram array; the second has a smaller input, so
a stale histogram from the first call would show. Results must be bit-identical (integer work).
"""
import pytest
import torch

from kernels import _lib
from kernels.workloads import make_workload

pytestmark = pytest.mark.gpu

OUTS = ("counts", "offsets", "tile_offsets", "expert_order", "sorted_token", "sorted_flat",
        "flat_to_sorted", "status")


def _bufs(n, k, e):
    m = max(n * k, 1)
    i32 = dict(device="cuda", dtype=torch.int32)
    return dict(counts=torch.full((e,), -7, **i32), offsets=torch.full((e + 1,), -7, **i32),
                tile_offsets=torch.full((e + 1,), -7, **i32),
                expert_order=torch.full((e,), -7, **i32), sorted_token=torch.full((m,), -7, **i32),
                sorted_flat=torch.full((m,), -7, **i32), flat_to_sorted=torch.full((m,), -7, **i32),
                status=torch.zeros(1, **i32))


def _args(idx, e, b):
    n, k = idx.shape
    return (_lib.ptr(idx), n, k, e, *(_lib.ptr(b[o]) for o in OUTS))


def _with_workspace(idx, e):
    n, k = idx.shape
    b = _bufs(n, k, e)
    ws = torch.empty(max(_lib.lib().moe_get_workspace_size(n, k, e), 256), device="cuda",
                     dtype=torch.uint8)
    _lib.call("moe_dispatch", *_args(idx, e, b), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(idx.device))
    return b


def _noalloc(idx, e):
    n, k = idx.shape
    b = _bufs(n, k, e)
    _lib.call("moe_dispatch_noalloc", *_args(idx, e, b), _lib.stream_of(idx.device))
    return b


def _check(idx, e):
    a = _noalloc(idx, e)
    r = _with_workspace(idx, e)
    torch.cuda.synchronize()
    for o in OUTS:
        assert torch.equal(a[o], r[o]), o


def test_noalloc_dispatch_matches_workspace_dispatch_twice():
    big = make_workload(3, device="cuda", scale=dict(H=8, I=8))["idx"]       # M = 131072, E = 64
    print("[gpu-case] noalloc dispatch: config-3 routing, then a smaller ragged batch", flush=True)
    _check(big, 64)
    g = torch.Generator(device="cuda").manual_seed(1)
    small = torch.randint(0, 200, (3001, 3), generator=g, device="cuda")    # 9 chunks, E = 200
    small[::97, 1] = 200                                                      # out of range
    _check(small, 200)
    _check(small[:100].contiguous(), 200)                                     # one-chunk path


def test_noalloc_dispatch_rejects_beyond_scratch():
    idx = torch.zeros(1, 1, device="cuda", dtype=torch.int64)
    b = _bufs(1, 1, 1024)
    # ceil(2^20 / 1024) * 1024 experts * 4 B = 4 MiB + 4 KiB > 4 MiB: rejected before any launch
    rc = _lib.lib().moe_dispatch_noalloc(_lib.ptr(idx), (1 << 20) + 1024, 1, 1024,
                                         *(_lib.ptr(b[o]) for o in OUTS),
                                         _lib.stream_of(idx.device))
    assert rc == 6
