"""The balanced cut's segment charge.

On a batch of at most 256 sequences whose page counts differ, the balanced
schedule's work list gives every unit a few list positions ahead of its
pages (the charge, about what starting a segment costs), so a workgroup
whose range starts a unit takes fewer pages; an even batch (one page count)
and a batch of more than 256 sequences are cut without it. The cases below
reach the cut's edges: ranges that end inside a charge (a batch of one-page
sequences beside a long one, so a workgroup's range is shorter than a
charge), a batch that differs by one page, lengths that differ but not in
pages (no charge), empty sequences, MQA units (merge kernel), paired KV
heads, head_dim 32, 64 and 256, pages of 32, 48, 64 and 256 tokens, the FP8 cache
and a batch past the scan's 256 sequences. A page the cut dropped or took twice changes the output, so
each case checks the oracle on up to 8 sequences (the longest among them),
through the planner and on the balanced schedule, and there the merge kernel
against the in-kernel merge, whose unit ranges are computed by different
code (the merge kernel's list_prefix, the decode kernel's schedule_start),
bit for bit. A seeded sweep of ragged batches of 13-300 sequences (past one
64-lane scan chunk, and past the 256 the charge applies to) checks the same
on the requested balanced schedule.
"""

from __future__ import annotations

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8, random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu


def _lens(spec) -> list[int]:
    if isinstance(spec, str):  # "u<max>x<batch>": uniform in [1, max]
        hi, batch = (int(v) for v in spec[1:].split("x"))
        g = torch.Generator().manual_seed(hi + batch)
        return torch.randint(1, hi + 1, (batch,), generator=g).tolist()
    return list(spec)


CASES = [
    # (lens, hq, hkv, head_dim, dtype, fp8, empty sequences[, page_size])
    ([1] * 63 + [5000], 32, 8, 128, torch.float16, False, []),  # ranges shorter than a charge
    ([2048] * 31 + [2032], 32, 8, 128, torch.float16, False, []),  # one page short: charged
    ([2048] * 31 + [2047], 32, 8, 128, torch.float16, False, []),  # same page counts: even
    ("u2000x32", 32, 8, 128, torch.float16, False, [4, 17]),
    ("u2500x64", 32, 8, 128, torch.bfloat16, False, []),  # paired KV heads
    ("u300x48", 32, 1, 128, torch.bfloat16, False, [0]),  # MQA: merge kernel
    ("u8192x16", 32, 1, 128, torch.bfloat16, False, []),
    ("u3000x64", 16, 2, 64, torch.bfloat16, False, [63]),  # head_dim 64
    ("u1500x40", 32, 8, 128, torch.float16, True, [7]),  # FP8 cache
    ("u600x200", 32, 8, 128, torch.float16, False, []),
    ("u600x300", 32, 8, 128, torch.float16, False, [299]),  # past the scan: no charge
    ("u5000x24", 32, 8, 128, torch.bfloat16, False, [5], 64),  # 64-token pages: 4 blocks per page
    ("u4000x16", 16, 4, 256, torch.float16, False, [], 32),  # head_dim 256, 32-token pages
    ("u3000x40", 8, 2, 32, torch.bfloat16, False, [1]),  # head_dim 32: the charge at its cap
    ("u3000x30", 16, 4, 64, torch.bfloat16, False, [2], 48),  # 48-token pages: block -> page by multiply and shift
    ("u6000x20", 32, 8, 128, torch.float16, False, [], 256),  # 256-token pages: a charge of 2 pages
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("schedule", ["planner", "balanced"])
def test_charged_cut(gpu_ops, case, schedule):
    spec, hq, hkv, head_dim, dtype, fp8, empty = case[:7]
    page_size = case[7] if len(case) > 7 else 16
    lens = _lens(spec)
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, head_dim, page_size, dtype=dtype, device="cuda",
                                        poison=float("nan"))
    kv.seq_lens[empty] = 0
    kw = {} if schedule == "planner" else {"num_splits": gpu_ops.BALANCED}
    if fp8:
        kv8, ks, vs = quantize_fp8(kv)
        run = lambda: gpu_ops.paged_decode_attention(q, kv8.k_cache, kv8.v_cache, kv.block_table, kv.seq_lens,
                                                     k_scale=ks, v_scale=vs, **kw)
    else:
        run = lambda: gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, **kw)
    got = run().cpu()
    assert torch.isfinite(got).all(), "non-finite output: a poisoned page or tail leaked in"
    if schedule == "balanced":
        # (The planner's own choice of schedule depends on whether the
        # in-kernel merge is available, so it is compared on the balanced
        # schedule only.)
        with _native.decode_switches(fused_merge="0"):
            merged = run().cpu()
        assert torch.equal(got, merged), "the in-kernel merge and the merge kernel disagree on the cut"
    for b in empty:
        assert not got[b].any(), "an empty sequence must give zeros"
    live = [b for b in range(len(lens)) if b not in empty]
    longest = max(live, key=lambda b: lens[b])
    rows = sorted({longest, *live[:4], *live[-3:]})
    if fp8:
        want = ref.paged_decode_attention_fp8(
            q[rows].cpu().float(), kv8.k_cache.cpu(), kv8.v_cache.cpu(), kv.block_table[rows].cpu(),
            kv.seq_lens[rows].cpu(), ks.cpu(), vs.cpu()
        )
    else:
        want = ref.paged_decode_attention(
            q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(),
            kv.seq_lens[rows].cpu()
        )
    decode_parity(got[rows], want, dtype)


def _draw_large(seed: int):
    """A seeded ragged batch of 13-300 sequences (past one 64-lane scan chunk,
    some past the 256 the charge applies to), empty sequences included."""
    import random

    rng = random.Random(1000 + seed)
    batch = rng.choice([rng.randint(13, 64), rng.randint(65, 256), rng.randint(257, 300)])
    hq, hkv = rng.choice([(32, 8), (32, 1), (64, 8), (16, 4), (8, 2), (24, 3)])
    head_dim = rng.choice([64, 128])
    page = rng.choice([16, 16, 32])
    dtype = rng.choice([torch.float16, torch.bfloat16])
    hi = rng.choice([300, 2000, 6000])
    lens = [rng.randint(1, hi) for _ in range(batch)]
    if rng.random() < 0.3:  # one long sequence among them
        lens[rng.randrange(batch)] = rng.randint(hi, 4 * hi)
    empty = sorted(rng.sample(range(batch), rng.randint(0, 3)))
    return lens, hq, hkv, head_dim, page, dtype, empty


@pytest.mark.parametrize("seed", range(64))
def test_random_large_batches(gpu_ops, seed):
    lens, hq, hkv, head_dim, page, dtype, empty = _draw_large(seed)
    case = f"seed={seed} B={len(lens)} {hq}/{hkv}/{head_dim} page={page} {dtype} empty={empty}"
    print(case, flush=True)
    q, kv = device_decode_problem(lens, hq, hkv, head_dim, page, dtype=dtype, seed=seed)
    kv.seq_lens[empty] = 0
    run = lambda: gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens,
                                                 num_splits=gpu_ops.BALANCED)
    got = run().cpu()
    with _native.decode_switches(fused_merge="0"):
        merged = run().cpu()
    assert torch.isfinite(got).all(), case
    assert torch.equal(got, merged), case
    for b in empty:
        assert not got[b].any(), case
    live = [b for b in range(len(lens)) if b not in empty]
    longest = max(live, key=lambda b: lens[b])
    rows = sorted({longest, live[0], live[len(live) // 2], live[-1]})
    want = ref.paged_decode_attention(q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(),
                                      kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu())
    decode_parity(got[rows], want, dtype, case)
