"""The allocation-free scan (nest_inclusive_scan_u32_noalloc) against the
workspace scan (nest_inclusive_scan_u32) through the C ABI: two calls in a
row on the library's shared scratch, the second smaller, bit-exact, and the
size limit rejected before any launch."""
import ctypes as ct

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _scan_ws(L, x):
    n = x.numel()
    out = torch.empty(n, dtype=torch.int32, device=DEV)
    ws = torch.empty(max(1, L.lib().nest_scan_workspace_size(n)), dtype=torch.uint8, device=DEV)
    L.check(L.lib().nest_inclusive_scan_u32(L.ptr(x), L.ptr(out), n, L.ptr(ws), ws.numel(), L.stream_ptr()),
            "nest_inclusive_scan_u32")
    return out


def _scan_noalloc(L, x, out):
    L.check(L.lib().nest_inclusive_scan_u32_noalloc(L.ptr(x), L.ptr(out), x.numel(), L.stream_ptr()),
            "nest_inclusive_scan_u32_noalloc")
    return out


def test_noalloc_scan_matches_workspace_scan():
    from nest_splat import _lib as L
    rng = np.random.default_rng(7)
    sizes = (3_000_001, 123_457)  # second call smaller: the scratch keeps the first call's partials
    out = torch.full((sizes[0],), -1, dtype=torch.int32, device=DEV)
    for k, n in enumerate(sizes):
        print(f"[noalloc] call {k}: n = {n}", flush=True)
        x_np = rng.integers(0, 64, n, dtype=np.uint32)
        x = torch.from_numpy(x_np.view(np.int32)).to(DEV)
        if k == 1:
            out.fill_(-1)
        _scan_noalloc(L, x, out)
        want = _scan_ws(L, x)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(got[:n], want.cpu().numpy().view(np.uint32))
        np.testing.assert_array_equal(got[:n], np.cumsum(x_np, dtype=np.uint64).astype(np.uint32))
        assert np.all(got[n:] == 0xFFFFFFFF), "wrote past n"
    # a size beyond the scratch is rejected before any launch, outputs untouched
    x = torch.zeros(16, dtype=torch.int32, device=DEV)
    o = torch.full((16,), 5, dtype=torch.int32, device=DEV)
    rc = L.lib().nest_inclusive_scan_u32_noalloc(L.ptr(x), L.ptr(o), L.SCAN_NOALLOC_MAX + 1, L.stream_ptr())
    assert rc == L.NEST_ERR_WORKSPACE
    assert b"exceeds" in L.lib().nest_last_error()
    assert torch.all(o == 5)
    # n on a 4096-item block boundary and n = 1
    for n in (4096 * 37, 1):
        x_np = rng.integers(0, 1000, n, dtype=np.uint32)
        x = torch.from_numpy(x_np.view(np.int32)).to(DEV)
        o = torch.empty(n, dtype=torch.int32, device=DEV)
        _scan_noalloc(L, x, o)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(o.cpu().numpy().view(np.uint32), np.cumsum(x_np, dtype=np.uint64).astype(np.uint32))


def test_noalloc_scan_at_the_scratch_limit():
    """n = NEST_SCAN_NOALLOC_MAX: 65,535 blocks of 4096, so the block partials
    fill the scratch up to its last slot (the grand total); 1 GiB in and out.
    Against the workspace scan, then a smaller call on the same scratch."""
    from nest_splat import _lib as L
    n = L.SCAN_NOALLOC_MAX
    print(f"[noalloc] n = {n} (the limit)", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randint(0, 16, (n,), dtype=torch.int32, device=DEV, generator=g)
    got = torch.empty(n, dtype=torch.int32, device=DEV)
    _scan_noalloc(L, x, got)
    want = _scan_ws(L, x)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    total = int(x.to(torch.int64).sum().item()) & 0xFFFFFFFF
    assert int(got[-1].item()) & 0xFFFFFFFF == total
    del want
    m = 5000
    small = torch.empty(m, dtype=torch.int32, device=DEV)
    _scan_noalloc(L, x[:m].contiguous(), small)
    torch.cuda.synchronize()
    assert torch.equal(small, got[:m])
