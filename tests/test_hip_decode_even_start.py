"""The balanced schedule's even-batch start on full batches.

The planner gives a batch whose units fill the device the balanced schedule
with one workgroup per list unit. When every sequence turns out to have the
same page count, each workgroup's range is one whole unit, which is the cut
of one uniform split. The kernel then starts that unit the way the uniform
kernels do: q and the block-table window are issued before seq_lens arrives,
and there is no scan. Every other batch runs the schedule's scan.

Checks, all through the HIP kernels:
* even batches (including lengths that differ inside the last page) give
  the bits of one uniform split, which runs the same segment code on the
  same cut, and match the unrounded oracle;
* batches that leave the even start (one page more for one sequence, an
  empty sequence, pages below the per-workgroup minimum, more than 256
  sequences) match the oracle;
* the planner reports the balanced schedule (0 splits) for all of them.
"""

from __future__ import annotations

import pytest
import torch

from kernel_lab.kv_cache import device_decode_problem, quantize_fp8
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16

# (label, lens, hq, hkv, head_dim, dtype): every sequence has the same page count.
EVEN = [
    ("paired 32/8 B=64, tails differ", [512 - (i % 16) for i in range(64)], 32, 8, 128, F16),
    ("unpaired 32/8 B=32 bf16", [512] * 32, 32, 8, 128, BF16),
    ("paired 64/8 B=64 bf16", [1024] * 64, 64, 8, 128, BF16),
    ("head_dim 64, 32/8 B=64", [700] * 64, 32, 8, 64, F16),
    ("paired 32/8 B=256", [160] * 256, 32, 8, 128, F16),
]

# Batches that take the schedule's scan.
UNEVEN = [
    ("one sequence one page longer", [512] * 63 + [513], 32, 8, 128, F16),
    ("one empty sequence", [512] * 63 + [-512], 32, 8, 128, F16),  # built with 512 tokens, then emptied
    ("7 pages each (below the workgroup minimum)", [100] * 64, 32, 8, 128, F16),
    ("257 sequences (beyond one scan)", [160] * 257, 32, 8, 128, F16),
    ("1 long among 63 short", [4000] + [100] * 63, 32, 8, 128, BF16),
]


def _oracle(q, kv):
    return ref.paged_decode_attention(q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(),
                                      kv.seq_lens.cpu())


def _planned_balanced(ops, q, kv) -> bool:
    batch, hq, d = q.shape
    splits, _ = ops.plan_decode(q.dtype, batch, hq, kv.k_cache.shape[2], d, kv.k_cache.shape[1],
                                kv.block_table.shape[1])
    return splits == 0


@pytest.mark.parametrize(("label", "lens", "hq", "hkv", "d", "dtype"), EVEN, ids=[c[0] for c in EVEN])
def test_even_batches_equal_one_uniform_split(gpu_ops, label, lens, hq, hkv, d, dtype):
    print(label, flush=True)
    q, kv = device_decode_problem(lens, hq, hkv, d, 16, dtype=dtype, seed=len(lens) + hq, poison=float("nan"))
    assert _planned_balanced(gpu_ops, q, kv), "full batches take the balanced schedule"
    out = torch.full_like(q, float("nan"))
    gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=out)
    uniform = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(out, uniform), f"{label}: differs from one uniform split"
    decode_parity(out, _oracle(q, kv), dtype, label)


@pytest.mark.parametrize(("label", "lens", "hq", "hkv", "d", "dtype"), UNEVEN, ids=[c[0] for c in UNEVEN])
def test_uneven_batches_take_the_scan(gpu_ops, label, lens, hq, hkv, d, dtype):
    print(label, flush=True)
    q, kv = device_decode_problem([abs(n) for n in lens], hq, hkv, d, 16, dtype=dtype, seed=len(lens) + 7,
                                  poison=float("nan"))
    kv.seq_lens.copy_(torch.tensor([max(n, 0) for n in lens], dtype=torch.int32))  # negative: emptied
    assert _planned_balanced(gpu_ops, q, kv)
    out = torch.full_like(q, float("nan"))
    gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=out)
    torch.cuda.synchronize()
    decode_parity(out, _oracle(q, kv), dtype, label)


def test_even_fp8_batch_equals_one_uniform_split(gpu_ops):
    q, kv = device_decode_problem([1024] * 64, 32, 8, 128, 16, dtype=F16, seed=5, poison=float("nan"))
    kv8, ks, vs = quantize_fp8(kv)
    out = torch.full_like(q, float("nan"))
    args = (q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens)
    gpu_ops.paged_decode_attention(*args, k_scale=ks, v_scale=vs, out=out)
    uniform = gpu_ops.paged_decode_attention(*args, k_scale=ks, v_scale=vs, num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(out, uniform)
    want = ref.paged_decode_attention_fp8(q.cpu().float(), kv8.k_cache.cpu(), kv8.v_cache.cpu(), kv8.block_table.cpu(),
                                          kv8.seq_lens.cpu(), ks.cpu(), vs.cpu())
    decode_parity(out, want, F16, "fp8 even batch")
