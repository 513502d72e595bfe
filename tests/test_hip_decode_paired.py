"""Paired decode workgroups (two adjacent KV heads per 8-wave workgroup).

Uniform splits (an explicit split count) pair the units of KV heads 2j and
2j+1 of one sequence, head group and split into one workgroup when the KV
head count is even, head_dim is at most 128 and the pairs alone give each of
MI355X's 256 CUs a workgroup (sequences x KV heads x head groups x splits >=
512). Each half runs the same segment code over the same blocks as the
one-unit workgroup, so the output must be bit-identical with pairing switched
off (``KL_DECODE_PAIRED=0``) and match the oracle. These shapes cover one
split (final outputs written by each half), splits past the end of short
sequences (both halves empty), empty sequences (zeros), two head tiles per
workgroup (GQA group 24), head_dim 32 and 64, and the FP8 cache.

The balanced schedule (the planner's choice below 256 units, and what
``num_splits=BALANCED`` asks for) runs in KV-head pairs on batches with
units >= 512 and one head tile, and on long contexts of small batches (at
least 128 pages per workgroup half, at most 16 segments per pair unit):
checked against the oracle and the unpaired balanced schedule, and, on even
lengths, bit-identical to uniform pairing with the same cut (one pair unit
per workgroup, or uniform splits of the segment length, whose workgroups the
balanced kernel runs in transposed order).
"""

from __future__ import annotations

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8, random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu


def _lens(batch: int, hi: int, seed: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(1, hi + 1, (batch,), generator=g).tolist()


def _empty_rows(batch: int, empty: int) -> list[int]:
    return sorted({(7 * i + 3) % batch for i in range(empty)})


def _both(ops, q, kv, **kw):
    """The decode with pairing as planned and with pairing switched off."""
    paired = ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, **kw)
    with _native.decode_switches(paired="0"):
        single = ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, **kw)
    torch.cuda.synchronize()
    return paired.cpu(), single.cpu()


CASES = [
    # (batch, hq, hkv, head_dim, dtype, max_len, num_splits, empty sequences)
    (64, 32, 8, 128, torch.float16, 700, None, 0),
    (64, 32, 8, 128, torch.bfloat16, 500, None, 5),
    (8, 32, 8, 128, torch.float16, 900, 16, 0),
    (16, 16, 4, 128, torch.bfloat16, 600, 64, 2),
    (64, 192, 8, 128, torch.float16, 200, None, 0),
    (128, 16, 4, 64, torch.float16, 300, None, 3),
    (64, 32, 8, 32, torch.bfloat16, 400, 2, 0),
]


@pytest.mark.parametrize(("batch", "hq", "hkv", "head_dim", "dtype", "max_len", "num_splits", "empty"), CASES)
def test_paired_matches_unpaired_and_oracle(gpu_ops, batch, hq, hkv, head_dim, dtype, max_len, num_splits, empty):
    lens = _lens(batch, max_len, seed=batch + hq + head_dim)
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, head_dim, 16, dtype=dtype, device="cuda", poison=float("nan"))
    empties = _empty_rows(batch, empty)
    kv.seq_lens[empties] = 0  # the fixture needs a token per sequence; these attend over none
    kw = {"num_splits": 1 if num_splits is None else num_splits}  # uniform splits
    paired, single = _both(gpu_ops, q, kv, **kw)
    assert torch.isfinite(paired).all(), "non-finite output: a poisoned page or tail leaked in"
    assert torch.equal(paired, single), "paired workgroups changed the result"
    want = ref.paged_decode_attention(
        q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu()
    )
    decode_parity(paired, want, dtype)
    for b in empties:
        assert not paired[b].any(), "an empty sequence must give zeros"


def test_paired_fp8_cache_matches_unpaired(gpu_ops):
    lens = _lens(64, 600, seed=11)
    q, kv, _, _ = random_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, device="cuda", poison=float("nan"))
    kv8, ks, vs = quantize_fp8(kv)
    k8, v8 = kv8.k_cache, kv8.v_cache
    args = (q, k8, v8, kv.block_table, kv.seq_lens)
    paired = gpu_ops.paged_decode_attention(*args, k_scale=ks, v_scale=vs, num_splits=1)
    with _native.decode_switches(paired="0"):
        single = gpu_ops.paged_decode_attention(*args, k_scale=ks, v_scale=vs, num_splits=1)
    assert torch.equal(paired.cpu(), single.cpu()), "paired workgroups changed the FP8 result"
    want = ref.paged_decode_attention_fp8(
        q.cpu().float(), k8.cpu(), v8.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu(), ks.cpu(), vs.cpu()
    )
    decode_parity(paired.cpu(), want, torch.float16)


# The balanced schedule: the planner's choice below 256 units, or requested
# with num_splits=BALANCED. Batches with units >= 512 or long contexts (an
# even KV head count, one head tile) run it in KV-head pairs; others in single
# heads, which the pairing switch must leave bit-identical.
BALANCED_CASES = [
    # (lens, hq, hkv, head_dim, dtype, num_splits, empty sequences, paired)
    ([700], 32, 8, 128, torch.float16, None, 0, False),
    ([6000, 1, 5, 300, 17, 16, 33, 2048, 15, 1, 4097, 640, 9, 64, 65, 3], 32, 8, 128, torch.float16, None, 2, False),
    ("ragged8", 64, 8, 128, torch.bfloat16, None, 0, False),
    ("ragged64", 32, 8, 128, torch.float16, -1, 4, True),
    ("ragged64", 32, 8, 128, torch.bfloat16, -1, 3, True),
    ("ragged8", 16, 2, 64, torch.bfloat16, None, 1, False),
    ("ragged128", 16, 4, 64, torch.float16, -1, 2, True),
    ([65536] + [2048] * 63, 32, 8, 128, torch.float16, -1, 0, True),
    ([20000] * 8, 32, 8, 128, torch.float16, None, 1, True),  # long contexts of a small batch: paired by default
    ("ragged16long", 32, 8, 128, torch.bfloat16, None, 2, True),
]


def _balanced_lens(spec) -> list[int]:
    if spec == "ragged8":
        return _lens(8, 3000, seed=8)
    if spec == "ragged64":
        return _lens(64, 1500, seed=64)
    if spec == "ragged128":
        return _lens(128, 2500, seed=128)
    if spec == "ragged16long":
        return _lens(16, 30000, seed=16)
    return list(spec)


@pytest.mark.parametrize(("spec", "hq", "hkv", "head_dim", "dtype", "num_splits", "empty", "paired"), BALANCED_CASES)
def test_balanced_schedule_pairing(gpu_ops, spec, hq, hkv, head_dim, dtype, num_splits, empty, paired):
    lens = _balanced_lens(spec)
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, head_dim, 16, dtype=dtype, device="cuda", poison=float("nan"))
    empties = _empty_rows(len(lens), empty)
    kv.seq_lens[empties] = 0
    kw = {} if num_splits is None else {"num_splits": num_splits}
    got, single = _both(gpu_ops, q, kv, **kw)
    if not paired:
        assert torch.equal(got, single), "the pairing switch changed the single-head balanced schedule"
    rows = [b for b in range(len(lens)) if b not in empties][:8]
    want = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu()
    )
    for out in (got, single):
        assert torch.isfinite(out).all(), "non-finite output: a poisoned page or tail leaked in"
        decode_parity(out[rows], want, dtype)
        for b in empties:
            assert not out[b].any(), "an empty sequence must give zeros"


@pytest.mark.parametrize(("batch", "ctx", "dtype"), [(64, 1000, torch.float16), (128, 300, torch.bfloat16)])
def test_paired_balanced_equals_uniform_pairing_on_even_lengths(gpu_ops, batch, ctx, dtype):
    """Even lengths give every workgroup exactly one pair unit, so the balanced
    schedule computes what one uniform split computes, bit for bit."""
    q, kv = device_decode_problem([ctx] * batch, 32, 8, 128, 16, dtype=dtype, seed=batch)
    balanced = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens,
                                              num_splits=gpu_ops.BALANCED)
    uniform = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, num_splits=1)
    assert torch.equal(balanced, uniform)


@pytest.mark.parametrize(
    ("batch", "ctx", "splits", "dtype"),
    [(8, 16384, 8, torch.float16), (8, 40960, 8, torch.bfloat16), (16, 16384, 4, torch.float16)],
)
def test_long_context_pairs_equal_uniform_splits(gpu_ops, batch, ctx, splits, dtype):
    """A small batch of long, even contexts runs the balanced schedule in
    KV-head pairs with its workgroups in transposed order; the cut equals
    uniform splits of the same page count, merged in the same order, so the
    results are bit-identical to the uniform paired kernel's."""
    q, kv = device_decode_problem([ctx] * batch, 32, 8, 128, 16, dtype=dtype, seed=ctx)
    pages = -(-ctx // 16)
    grid = min(256, -(-batch * 4 * pages // 8))
    assert (batch * 4 * pages) % grid == 0 and (batch * 4 * pages // grid) * splits == pages, "not the same cut"
    planned = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
    uniform = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens,
                                             num_splits=splits)
    assert torch.isfinite(planned).all()
    assert torch.equal(planned, uniform)
    rows = [0, batch - 1]
    want = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu()
    )
    decode_parity(planned[rows].cpu(), want, dtype)


@pytest.mark.parametrize(
    ("lens_spec", "head_dim", "page_size", "dtype", "empty"),
    [
        ("even", 64, 64, torch.float16, []),  # 8 x 1875 pages of 64 tokens, head_dim 64
        ("ragged", 128, 32, torch.bfloat16, [2, 5]),  # ragged long contexts, empty sequences
    ],
)
def test_long_context_pairs_other_pages_and_head_dims(gpu_ops, lens_spec, head_dim, page_size, dtype, empty):
    """The long-context pairing rule at other page sizes and head dims: paired
    (planner default), against the unpaired balanced schedule and the oracle,
    with empty sequences zeroed."""
    lens = [120000] * 8 if lens_spec == "even" else _lens(8, 150000, seed=21)
    pages = -(-max(lens) // page_size)
    assert len(lens) * 8 // 2 * pages >= 128 * 256, "not a long-context pairing shape (128 pages per half)"
    q, kv = device_decode_problem(lens, 32, 8, head_dim, page_size, dtype=dtype, seed=page_size)
    if empty:
        kv.seq_lens[empty] = 0
    got, single = _both(gpu_ops, q, kv)
    rows = [b for b in range(len(lens)) if b not in empty][:3]
    want = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu()
    )
    for out in (got, single):
        assert torch.isfinite(out).all()
        decode_parity(out[rows], want, dtype)
        for b in empty:
            assert not out[b].any(), "an empty sequence must give zeros"
