"""Arrival-counter regions of the in-kernel split merge, at their limits.

A split decode merges its units inside the decode kernel on counters of a
region that no call able to overlap it shares: an eager call uses its
stream's region (64 per device), so streams beyond those take the separate
merge kernel, with the same bits, and the library says so once on stderr;
the per-thread default stream (one handle, many streams) never gets a region.

Named to sort late: it takes every eager region for the rest of the process.
Its checks hold whatever regions earlier tests in the process already took.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem

pytestmark = pytest.mark.gpu

IN_KERNEL, MERGE_KERNEL = 2, 1
STREAM_REGIONS = 64
HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread


def _hip():
    # The HIP runtime this process already loaded (PyTorch's), found by path in
    # the process's mappings rather than by a fixed soname.
    with open("/proc/self/maps") as maps:
        paths = {line.split()[-1] for line in maps if "libamdhip64.so" in line}
    assert paths, "no HIP runtime mapped in this process"
    hip = ctypes.CDLL(sorted(paths)[0])
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return hip


def test_streams_beyond_the_regions_take_the_merge_kernel(gpu_ops, capfd):
    q, kv = device_decode_problem([1800] * 4, 32, 8, 128, 16, dtype=torch.float16, seed=80)
    want = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens).clone()
    hip = _hip()
    handles = []
    for _ in range(STREAM_REGIONS + 8):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        handles.append(h.value)
    modes, outs = [], []
    try:
        for h in handles:
            stream = torch.cuda.ExternalStream(h)
            stream.wait_stream(torch.cuda.current_stream())
            out = torch.full_like(q, float("nan"))
            with torch.cuda.stream(stream):
                gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=out)
            modes.append(_native.core().kl_paged_decode_last_merge())
            outs.append(out)
        torch.cuda.synchronize()
    finally:
        torch.cuda.synchronize()
        for h in handles:
            hip.hipStreamDestroy(h)
    for i, out in enumerate(outs):
        assert torch.equal(out, want), f"stream {i} (merge {modes[i]}) differs"
    # Regions go to streams in call order: in-kernel merges while regions are
    # left (earlier tests in this process may have taken some), then merge
    # kernels; 72 new streams outnumber the 64 regions whatever was taken.
    assert modes[-1] == MERGE_KERNEL, modes
    assert modes == sorted(modes, reverse=True), modes
    assert set(modes) <= {IN_KERNEL, MERGE_KERNEL}, modes
    # Said once per process: now, unless an earlier test used the pool up.
    assert capfd.readouterr().err.count("split-merge counter regions for streams are taken") <= 1


def test_per_thread_default_stream_takes_the_merge_kernel(gpu_ops):
    """Through the C-ABI on hipStreamPerThread, which names a different stream
    on every host thread, so no counter region can belong to it."""
    lib = _native.core()
    q, kv = device_decode_problem([2500] * 6, 32, 8, 128, 16, dtype=torch.float16, seed=81)
    want = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens).clone()
    assert lib.kl_paged_decode_last_merge() == IN_KERNEL
    batch, hq, d = q.shape
    splits, ws = ctypes.c_int(0), ctypes.c_size_t(0)
    assert lib.kl_paged_decode_plan(1, batch, hq, 8, d, 16, kv.block_table.shape[1], 0, 0, ctypes.byref(splits),
                                    ctypes.byref(ws)) == 0
    workspace = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    torch.cuda.synchronize()
    st = lib.kl_paged_decode_attention(1, out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(),
                                       kv.block_table.data_ptr(), kv.seq_lens.data_ptr(), batch, hq, 8, d, 16,
                                       kv.block_table.stride(0), kv.block_table.shape[1], d**-0.5, 0,
                                       workspace.data_ptr(), ws.value, HIP_STREAM_PER_THREAD)
    assert st == 0, _native.last_error()
    assert lib.kl_paged_decode_last_merge() == MERGE_KERNEL
    torch.cuda.synchronize()
    assert torch.equal(out, want)
