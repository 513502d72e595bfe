"""Parity through the C-ABI itself (ctypes, raw device pointers, the current
HIP stream), the way a non-PyTorch caller would bind include/kernel_lab.h, and
operator registration under torch.compile(fullgraph=True)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity, tolerance

pytestmark = pytest.mark.gpu


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rms_norm_through_c_abi(gpu_ops, dtype):
    lib = _native.core()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(16, 4096, generator=g).to("cuda", dtype)
    r = torch.randn(16, 4096, generator=g).to("cuda", dtype)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to("cuda", dtype)
    r0 = r.clone()
    out = torch.empty_like(x)
    st = lib.kl_rms_norm(
        _native.DTYPE_CODES[dtype], out.data_ptr(), x.data_ptr(), r.data_ptr(), w.data_ptr(), 16, 4096, 4096, 1e-6,
        stream_handle(),
    )
    assert st == 0, _native.last_error()
    torch.cuda.synchronize()
    ref_out, ref_res = ref.fused_add_rms_norm(x.cpu(), r0.cpu(), w.cpu())
    assert torch.equal(r.cpu(), ref_res)
    torch.testing.assert_close(out.cpu(), ref_out, **tolerance(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("num_splits", [0, 1, 5, -1])
def test_decode_through_c_abi(gpu_ops, dtype, num_splits):
    lib = _native.core()
    q, kv, _, _ = random_decode_problem([7, 300, 33], 32, 8, 128, 16, dtype=dtype, device="cuda", poison=float("nan"))
    batch, hq, d = q.shape
    hkv, p = kv.k_cache.shape[2], kv.k_cache.shape[1]
    max_pages = kv.block_table.shape[1]
    code = _native.DTYPE_CODES[dtype]
    splits = ctypes.c_int(0)
    ws = ctypes.c_size_t(0)
    st = lib.kl_paged_decode_plan(code, batch, hq, hkv, d, p, max_pages, num_splits, 0, ctypes.byref(splits), ctypes.byref(ws))
    assert st == 0, _native.last_error()
    workspace = torch.empty(max(ws.value, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    args = [code, out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(), kv.block_table.data_ptr(),
            kv.seq_lens.data_ptr(), batch, hq, hkv, d, p, kv.block_table.stride(0), max_pages, d**-0.5, num_splits]
    if ws.value:
        # Too small a workspace is refused before anything launches.
        assert lib.kl_paged_decode_attention(*args, workspace.data_ptr(), ws.value - 1, stream_handle()) == 3
    st = lib.kl_paged_decode_attention(*args, workspace.data_ptr(), ws.value, stream_handle())
    assert st == 0, _native.last_error()
    torch.cuda.synchronize()
    want = ref.paged_decode_attention(q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu())
    decode_parity(out.cpu(), want, dtype)


def test_ops_work_under_torch_compile(gpu_ops):
    """tests/test_cuda_kernels.py:56-66 of the original, plus the decode operator."""
    x = torch.randn(4, 256, device="cuda", dtype=torch.float16)
    w = torch.randn(256, device="cuda", dtype=torch.float16)

    @torch.compile(fullgraph=True)
    def f(x, w):
        out = torch.empty_like(x)
        torch.ops.kernel_lab.rms_norm(out, x, w, 1e-6)
        return out * 2

    torch.testing.assert_close(f(x, w).cpu(), ref.rms_norm(x.cpu(), w.cpu()) * 2, **tolerance(torch.float16))

    q, kv, _, _ = random_decode_problem([7, 40], 8, 2, 64, 16, dtype=torch.float16, device="cuda")

    @torch.compile(fullgraph=True)
    def g(q, k, v, bt, lens, x, r, w):
        out = torch.empty_like(q)
        torch.ops.kernel_lab.paged_decode_attention(out, q, k, v, bt, lens, 0.125)
        y = torch.empty_like(x)
        torch.ops.kernel_lab.fused_add_rmsnorm(y, x, r, w, 1e-6)
        return out * 2, y, r  # doubling is exact, so the check can undo it

    r = torch.randn(4, 256, device="cuda", dtype=torch.float16)
    r0 = r.clone()
    out, y, r_new = g(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, x, r, w)
    want = ref.paged_decode_attention(q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu(), 0.125)
    decode_parity((out / 2).cpu(), want, torch.float16, "under torch.compile")
    ref_y, ref_r = ref.fused_add_rms_norm(x.cpu(), r0.cpu(), w.cpu())
    assert torch.equal(r_new.cpu(), ref_r)
    torch.testing.assert_close(y.cpu(), ref_y, **tolerance(torch.float16))


def test_full_batches_balance_skew_by_default(gpu_ops):
    """64 sequences x 8 KV heads fill the device twice over, and one sequence
    of 4,000 tokens among 63 of 100 (a 250-column table) would leave its
    units to stream alone under one uniform split. The planner's default is
    the balanced schedule (0 splits, a workspace), the same plan as
    KL_SPLITS_BALANCED (-1); KL_DECODE_BALANCE_ALWAYS=0 gives one uniform
    split. The drop-in operator (the reference's schema, no split argument)
    then cuts the long sequence's units over several workgroups and merges
    them in the kernel, matching the oracle; through the C-ABI the balanced
    plan needs its workspace and is refused without one."""
    lib = _native.core()
    lens = [4000] + [100] * 63
    q, kv, _, _ = random_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, device="cuda", poison=float("nan"))
    batch, hq, d = q.shape
    max_pages = kv.block_table.shape[1]
    code = _native.DTYPE_CODES[torch.float16]

    def plan(req):
        splits, ws = ctypes.c_int(0), ctypes.c_size_t(0)
        assert lib.kl_paged_decode_plan(code, batch, hq, 8, d, 16, max_pages, req, 0, ctypes.byref(splits), ctypes.byref(ws)) == 0
        return splits.value, ws.value

    balanced = plan(0)
    assert balanced[0] == 0 and balanced[1] > 0
    assert plan(-1) == balanced
    with _native.decode_switches(balance_always="0"):
        assert plan(0) == (1, 0)
    want = ref.paged_decode_attention(q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu())

    out = torch.full_like(q, float("nan"))
    torch.ops.kernel_lab.paged_decode_attention(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, d**-0.5)
    assert lib.kl_paged_decode_last_merge() == 2, "the long sequence's units should be split and merged in the kernel"
    torch.cuda.synchronize()
    decode_parity(out.cpu(), want, torch.float16, "drop-in operator, 1x4000 + 63x100")

    out = torch.empty_like(q)
    args = [code, out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(), kv.block_table.data_ptr(),
            kv.seq_lens.data_ptr(), batch, hq, 8, d, 16, kv.block_table.stride(0), max_pages, d**-0.5, 0]
    assert lib.kl_paged_decode_attention(*args, None, 0, stream_handle()) == 3
    workspace = torch.empty(balanced[1], dtype=torch.uint8, device="cuda")
    assert lib.kl_paged_decode_attention(*args, workspace.data_ptr(), balanced[1], stream_handle()) == 0
    torch.cuda.synchronize()
    decode_parity(out.cpu(), want, torch.float16, "C-ABI, planner's choice")
