"""gfx950 paged decode over an FP8 (OCP E4M3) KV cache against the CPU oracle.

Caches are quantized per KV head by kernel_lab.kv_cache.quantize_fp8 (spare
pages become NaN codes); the oracle decodes the same codes, so the comparison
isolates the kernel: its arithmetic is the 16-bit path's (exactly decoded
values, fp32 accumulation, P rounded to q's dtype for the MFMA), and the
tolerances are the 16-bit table's.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8, random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity, tolerance

pytestmark = pytest.mark.gpu

QDTYPES = [torch.float16, torch.bfloat16]


def problem(lens, hq, hkv, d, dtype, page=16, seed=0):
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, d, page, dtype=torch.float32, seed=seed, poison=float("nan"))
    kv8, ks, vs = quantize_fp8(kv)
    return q.to(dtype).cuda(), type(kv8)(
        kv8.k_cache.cuda(), kv8.v_cache.cuda(), kv8.block_table.cuda(), kv8.seq_lens.cuda(), page
    ), ks.cuda(), vs.cuda()


def run(ops, q, kv, ks, vs, **kw):
    return ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, k_scale=ks, v_scale=vs, **kw)


def expected(q, kv, ks, vs, scale=None):
    return ref.paged_decode_attention_fp8(
        q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu(), ks.cpu(), vs.cpu(), scale
    )


def check(got, want, dtype):
    got = got.cpu()
    assert torch.isfinite(got).all(), "non-finite output: a NaN spare page or tail leaked in"
    decode_parity(got, want, dtype)


@pytest.mark.parametrize("dtype", QDTYPES)
@pytest.mark.parametrize(("hq", "hkv"), [(8, 8), (16, 4), (8, 1), (32, 8), (32, 1)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_fp8_cache_shapes(gpu_ops, hq, hkv, head_dim, dtype):
    q, kv, ks, vs = problem([1, 15, 16, 17, 300], hq, hkv, head_dim, dtype)
    check(run(gpu_ops, q, kv, ks, vs), expected(q, kv, ks, vs), dtype)


@pytest.mark.parametrize("num_splits", [1, 3, 64, -1])
@pytest.mark.parametrize("dtype", QDTYPES)
def test_fp8_splits_and_balanced_schedule(gpu_ops, num_splits, dtype):
    q, kv, ks, vs = problem([5000, 3, 700, 64], 32, 8, 128, dtype, seed=2)
    check(run(gpu_ops, q, kv, ks, vs, num_splits=num_splits), expected(q, kv, ks, vs), dtype)


@pytest.mark.parametrize("page_size", [16, 32, 64])
def test_fp8_page_sizes(gpu_ops, page_size):
    q, kv, ks, vs = problem([100, 33, 1], 16, 2, 128, torch.float16, page=page_size, seed=4)
    check(run(gpu_ops, q, kv, ks, vs), expected(q, kv, ks, vs), torch.float16)


def test_fp8_scalar_scales_and_custom_scale(gpu_ops):
    """One float for every head (near the quantizer's, so values stay O(1) as
    the tolerance table assumes), and a non-default softmax scale."""
    q, kv, ks, vs = problem([70, 9], 8, 2, 64, torch.bfloat16, seed=8)
    k1, v1 = float(ks.mean()), float(vs.mean())
    got = run(gpu_ops, q, kv, k1, v1, scale=0.05)
    want = expected(q, kv, torch.full((2,), k1), torch.full((2,), v1), scale=0.05)
    check(got, want, torch.bfloat16)


def test_fp8_one_hot_known_answer(gpu_ops):
    """Key 96 at token 13, values = token index, k_scale 0.5, v_scale 2: 26."""
    d = 64
    k = torch.zeros(2, 16, 1, d)
    v = torch.arange(16, dtype=torch.float32)[None, :, None, None].expand(2, 16, 1, d).clone()
    k[1, 13, 0, 0] = 96.0
    k8 = k.to(torch.float8_e4m3fn).cuda()
    v8 = v.to(torch.float8_e4m3fn).cuda()
    bt = torch.tensor([[1]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([16], dtype=torch.int32, device="cuda")
    q = torch.zeros(1, 1, d, dtype=torch.float16, device="cuda")
    q[0, 0, 0] = 1.0
    out = gpu_ops.paged_decode_attention(q, k8, v8, bt, lens, scale=1.0, k_scale=0.5, v_scale=2.0)
    torch.testing.assert_close(out.float().cpu(), torch.full((1, 1, d), 26.0), atol=2e-2, rtol=0)


def test_fp8_llama3_config_b64_ctx4096(gpu_ops):
    """The headline decode shape (32/8/128/16, B=64, 4096 tokens) in FP8."""
    q, kv = device_decode_problem([4096] * 64, 32, 8, 128, 16, dtype=torch.float16)
    kv8, ks, vs = quantize_fp8(kv)
    got = run(gpu_ops, q, kv8, ks, vs)
    rows = [0, 17, 63]
    sub = type(kv8)(kv8.k_cache, kv8.v_cache, kv8.block_table[rows], kv8.seq_lens[rows], 16)
    check(got[rows], expected(q[rows], sub, ks, vs), torch.float16)


def test_fp8_validation(gpu_ops):
    q, kv, ks, vs = problem([20], 8, 2, 64, torch.float16)
    with pytest.raises(ValueError, match="k_scale"):
        gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
    with pytest.raises(ValueError, match="one per KV head"):
        run(gpu_ops, q, kv, torch.ones(3, device="cuda"), vs)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        run(gpu_ops, q.float(), kv, ks, vs)
    q32, kv32, ks32, vs32 = problem([20], 8, 2, 32, torch.float16)
    with pytest.raises(RuntimeError, match="head_dim 64, 128 or 256"):
        run(gpu_ops, q32, kv32, ks32, vs32)
    with pytest.raises(ValueError, match="FP8"):
        gpu_ops.paged_decode_attention(
            q, kv.k_cache.half(), kv.v_cache.half(), kv.block_table, kv.seq_lens, k_scale=ks, v_scale=vs
        )


@pytest.mark.parametrize("num_splits", [0, 4])
def test_fp8_through_c_abi(gpu_ops, num_splits):
    lib = _native.core()
    q, kv, ks, vs = problem([7, 300, 33], 32, 8, 128, torch.bfloat16, seed=9)
    batch, hq, d = q.shape
    code = _native.DTYPE_CODES[torch.bfloat16]
    max_pages = kv.block_table.shape[1]
    splits, ws = ctypes.c_int(0), ctypes.c_size_t(0)
    assert lib.kl_paged_decode_plan(code, batch, hq, 8, d, 16, max_pages, num_splits, 0, ctypes.byref(splits), ctypes.byref(ws)) == 0
    workspace = torch.empty(max(ws.value, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.kl_paged_decode_attention_fp8(
        code, out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(), ks.data_ptr(), vs.data_ptr(),
        kv.block_table.data_ptr(), kv.seq_lens.data_ptr(), batch, hq, 8, d, 16, kv.block_table.stride(0), max_pages,
        d**-0.5, num_splits, workspace.data_ptr(), ws.value, stream,
    )
    assert st == 0, _native.last_error()
    torch.cuda.synchronize()
    check(out, expected(q, kv, ks, vs), torch.bfloat16)
    # Null scales are refused before anything launches.
    assert lib.kl_paged_decode_attention_fp8(
        code, out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(), None, None,
        kv.block_table.data_ptr(), kv.seq_lens.data_ptr(), batch, hq, 8, d, 16, kv.block_table.stride(0), max_pages,
        d**-0.5, num_splits, workspace.data_ptr(), ws.value, stream,
    ) == 1
