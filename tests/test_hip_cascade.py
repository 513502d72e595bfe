"""gfx950 cascade (shared-prefix) decode against the CPU oracle.

Spare pages and the tails of last pages hold NaN, so a read past a prefix or a
suffix, or masking by multiplication, shows up as NaN. Tolerances are the
16-bit table's: the arithmetic is the plain decode's, split in two passes and
merged by the LSE rule.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import random_cascade_problem
from oracle import reference as ref
from tests.conftest import decode_parity, tolerance

pytestmark = pytest.mark.gpu


def run(ops, q, c, **kw):
    return ops.cascade_decode_attention(
        q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, c.prefix_len, c.kv.block_table, c.kv.seq_lens, **kw
    )


def expected(q, c, scale=None):
    return ref.cascade_decode_attention(
        q.cpu().float(), c.kv.k_cache.cpu(), c.kv.v_cache.cpu(), c.prefix_block_table.cpu(), c.prefix_len,
        c.kv.block_table.cpu(), c.kv.seq_lens.cpu(), scale,
    )


def check(got, want, dtype):
    got = got.cpu()
    assert torch.isfinite(got).all(), "non-finite output: a NaN page or tail leaked in"
    decode_parity(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("hq", "hkv"), [(32, 8), (8, 1), (16, 4), (64, 8)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_cascade_shapes(gpu_ops, hq, hkv, head_dim, dtype):
    q, c = random_cascade_problem(300, [1, 17, 0, 64, 250], hq, hkv, head_dim, 16, dtype=dtype, device="cuda")
    check(run(gpu_ops, q, c), expected(q, c), dtype)


@pytest.mark.parametrize("prefix_len", [0, 1, 16, 100, 2500])
def test_cascade_prefix_lengths(gpu_ops, prefix_len):
    q, c = random_cascade_problem(prefix_len, [40, 3, 700], 32, 8, 128, 16, device="cuda", seed=prefix_len)
    check(run(gpu_ops, q, c), expected(q, c), torch.float16)


def test_cascade_without_own_tokens_and_without_any_tokens(gpu_ops):
    q, c = random_cascade_problem(0, [0, 9], 8, 2, 64, 16, device="cuda", seed=5)
    out = run(gpu_ops, q, c)
    assert torch.equal(out[0].cpu(), torch.zeros_like(out[0].cpu()))
    check(out, expected(q, c), torch.float16)
    q, c = random_cascade_problem(77, [0, 0, 5], 8, 2, 64, 16, device="cuda", seed=6)
    check(run(gpu_ops, q, c), expected(q, c), torch.float16)


@pytest.mark.parametrize("page_size", [16, 32, 64])
def test_cascade_page_sizes(gpu_ops, page_size):
    q, c = random_cascade_problem(130, [20, 200], 16, 2, 128, page_size, dtype=torch.bfloat16, device="cuda", seed=7)
    check(run(gpu_ops, q, c, scale=0.07), expected(q, c, 0.07), torch.bfloat16)


def test_cascade_equals_plain_decode_on_concatenated_pages(gpu_ops):
    """A page-aligned prefix followed by the own pages is one block-table row."""
    page = 16
    q, c = random_cascade_problem(512, [100, 1, 1000, 33], 32, 8, 128, page, device="cuda", seed=8)
    npre = c.prefix_block_table.numel()
    rows = []
    for b, n in enumerate(c.kv.seq_lens.tolist()):
        rows.append(torch.cat([c.prefix_block_table, c.kv.block_table[b, : -(-n // page)]]))
    table = torch.zeros(len(rows), max(r.numel() for r in rows), dtype=torch.int32, device="cuda")
    for b, r in enumerate(rows):
        table[b, : r.numel()] = r
    assert npre * page == c.prefix_len
    plain = gpu_ops.paged_decode_attention(q, c.kv.k_cache, c.kv.v_cache, table, c.kv.seq_lens + c.prefix_len)
    torch.testing.assert_close(run(gpu_ops, q, c).cpu(), plain.cpu(), **tolerance(torch.float16))


def test_cascade_llama3_batch64_shared_4096(gpu_ops):
    """64 sequences sharing a 4096-token prefix, 512 own tokens each."""
    q, c = random_cascade_problem(4096, [512] * 64, 32, 8, 128, 16, device="cuda", seed=9)
    got = run(gpu_ops, q, c)
    rows = [0, 31, 63]
    sub = type(c)(type(c.kv)(c.kv.k_cache, c.kv.v_cache, c.kv.block_table[rows], c.kv.seq_lens[rows], 16),
                  c.prefix_block_table, c.prefix_len)
    check(got[rows], expected(q[rows], sub), torch.float16)


def test_cascade_validation(gpu_ops):
    q, c = random_cascade_problem(20, [5], 8, 2, 64, 16, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="fp16 or bf16"):
        run(gpu_ops, q, c)


def test_cascade_through_c_abi(gpu_ops):
    lib = _native.core()
    q, c = random_cascade_problem(200, [30, 0, 90], 32, 8, 128, 16, dtype=torch.bfloat16, device="cuda", seed=10)
    batch, hq, d = q.shape
    code = _native.DTYPE_CODES[torch.bfloat16]
    max_pages = c.kv.block_table.shape[1]
    npre = c.prefix_block_table.numel()
    ws = ctypes.c_size_t(0)
    assert lib.kl_cascade_decode_plan(code, batch, hq, 8, d, 16, npre, max_pages, 0, ctypes.byref(ws)) == 0
    workspace = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
    plen = torch.tensor([c.prefix_len], dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    args = [code, out.data_ptr(), q.data_ptr(), c.kv.k_cache.data_ptr(), c.kv.v_cache.data_ptr(),
            c.prefix_block_table.data_ptr(), plen.data_ptr(), npre, c.kv.block_table.data_ptr(),
            c.kv.seq_lens.data_ptr(), batch, hq, 8, d, 16, c.kv.block_table.stride(0), max_pages, d**-0.5]
    assert lib.kl_cascade_decode_attention(*args, workspace.data_ptr(), ws.value - 256, stream) == 3
    assert lib.kl_cascade_decode_attention(*args, workspace.data_ptr(), ws.value, stream) == 0, _native.last_error()
    torch.cuda.synchronize()
    check(out, expected(q, c), torch.bfloat16)
