"""GPU checks of the binning primitives exported by the C ABI: the stable
pair sort (cub::DeviceRadixSort::SortPairs semantics) and the inclusive scan
(cub::DeviceScan::InclusiveSum), against numpy on the same inputs.  Sizes
cover one partial block, exact block multiples and many blocks; key widths
cover odd and even pass counts; keys are drawn from a small range so that
equal keys (stability) are common."""
import ctypes as ct

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _L():
    from nest_splat import _lib as L
    return L


def _ptr(t):
    return ct.c_void_p(t.data_ptr())


@pytest.mark.parametrize("n,end_bit,key_range", [
    (1, 8, 4), (1000, 8, 16), (4096, 16, 300), (4097, 45, 1 << 40), (50_000, 45, 5000),
    (300_000, 24, 1 << 24), (1_000_003, 64, None),
])
def test_sort_pairs_u64_is_stable_lexsort(n, end_bit, key_range):
    L = _L()
    lib = L.lib()
    rng = np.random.default_rng(n + end_bit)
    if key_range is None:
        keys = rng.integers(0, 1 << 63, n, dtype=np.uint64) | (rng.integers(0, 2, n, dtype=np.uint64) << np.uint64(63))
    else:
        keys = rng.integers(0, key_range, n, dtype=np.uint64)
    keys &= np.uint64((1 << end_bit) - 1) if end_bit < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)
    vals = rng.permutation(n).astype(np.uint32)
    print(f"[case] sort n={n} end_bit={end_bit}", flush=True)
    dev = torch.device("cuda:0")
    k_in = torch.from_numpy(keys.view(np.int64)).to(dev)
    v_in = torch.from_numpy(vals.view(np.int32)).to(dev)
    k_out = torch.empty_like(k_in)
    v_out = torch.empty_like(v_in)
    ws_bytes = lib.nest_sort_workspace_size(n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    L.check(lib.nest_sort_pairs_u64(_ptr(k_in), _ptr(v_in), _ptr(k_out), _ptr(v_out), n, end_bit, _ptr(ws), ws_bytes,
                                    stream), "sort")
    torch.cuda.synchronize()
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(k_out.cpu().numpy().view(np.uint64), keys[order])
    np.testing.assert_array_equal(v_out.cpu().numpy().view(np.uint32), vals[order])
    # inputs are not written
    np.testing.assert_array_equal(k_in.cpu().numpy().view(np.uint64), keys)
    np.testing.assert_array_equal(v_in.cpu().numpy().view(np.uint32), vals)


@pytest.mark.parametrize("n,end_bit", [(5000, 12), (70_000, 21), (5_000_000, 13)])
def test_sort_pairs_u64_ignores_bits_past_end_bit(n, end_bit):
    """cub's SortPairs orders on bits [0, end_bit) only: keys with higher bits
    set keep those bits and their stable order among equal low bits."""
    L = _L()
    lib = L.lib()
    rng = np.random.default_rng(7 * n + end_bit)
    keys = rng.integers(0, 1 << 40, n, dtype=np.uint64)
    vals = rng.permutation(n).astype(np.uint32)
    print(f"[case] sort high bits n={n} end_bit={end_bit}", flush=True)
    dev = torch.device("cuda:0")
    k_in = torch.from_numpy(keys.view(np.int64)).to(dev)
    v_in = torch.from_numpy(vals.view(np.int32)).to(dev)
    k_out = torch.empty_like(k_in)
    v_out = torch.empty_like(v_in)
    ws_bytes = lib.nest_sort_workspace_size(n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    L.check(lib.nest_sort_pairs_u64(_ptr(k_in), _ptr(v_in), _ptr(k_out), _ptr(v_out), n, end_bit, _ptr(ws), ws_bytes,
                                    stream), "sort")
    torch.cuda.synchronize()
    order = np.argsort(keys & np.uint64((1 << end_bit) - 1), kind="stable")
    np.testing.assert_array_equal(k_out.cpu().numpy().view(np.uint64), keys[order])
    np.testing.assert_array_equal(v_out.cpu().numpy().view(np.uint32), vals[order])


@pytest.mark.parametrize("n", [1, 255, 4096, 4097, 1_000_000, 3_000_001])
def test_inclusive_scan_u32(n):
    L = _L()
    lib = L.lib()
    rng = np.random.default_rng(n)
    x = rng.integers(0, 64, n, dtype=np.uint32)
    print(f"[case] scan n={n}", flush=True)
    dev = torch.device("cuda:0")
    a = torch.from_numpy(x.view(np.int32)).to(dev)
    out = torch.empty_like(a)
    ws_bytes = lib.nest_scan_workspace_size(n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    L.check(lib.nest_inclusive_scan_u32(_ptr(a), _ptr(out), n, _ptr(ws), ws_bytes, stream), "scan")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), np.cumsum(x, dtype=np.uint64).astype(np.uint32))
