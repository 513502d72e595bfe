"""Seeded random sweep of paged decode against the CPU oracle.

Each case draws dtype, head_dim, GQA shape, page size, split request and a
ragged batch (lengths at page boundaries +-1 included, empty sequences
allowed) from a fixed seed, so a failure names a reproducible case. Spare
pages and last-page tails hold NaN."""

from __future__ import annotations

import random

import pytest
import torch

from kernel_lab.kv_cache import random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu

HEAD_DIMS = {torch.float32: [16, 32, 64, 128, 256], torch.float16: [32, 64, 128, 256], torch.bfloat16: [32, 64, 128, 256]}
GQA = [(1, 1), (4, 4), (8, 1), (8, 2), (16, 4), (32, 8), (24, 3), (40, 5), (64, 8), (32, 1), (60, 5), (40, 2), (48, 2)]


def draw_case(seed: int):
    rng = random.Random(seed)
    dtype = rng.choice([torch.float32, torch.float16, torch.bfloat16])
    head_dim = rng.choice(HEAD_DIMS[dtype])
    hq, hkv = rng.choice(GQA)
    page = rng.choice([16, 16, 32, 64, 8, 1] if dtype == torch.float32 else [16, 16, 32, 64, 8])
    batch = rng.randint(1, 12)
    lens = []
    for _ in range(batch):
        kind = rng.random()
        if kind < 0.2:
            lens.append(rng.choice([1, page - 1 if page > 1 else 1, page, page + 1, 2 * page + 1]))
        else:
            lens.append(rng.randint(1, 1200))
    splits = rng.choice([None, None, 1, 2, 3, 7, 64, -1])
    empty = rng.random() < 0.2 and batch > 1
    return dtype, head_dim, hq, hkv, page, lens, splits, empty


@pytest.mark.parametrize("seed", range(160))
def test_random_decode_case(gpu_ops, seed):
    dtype, head_dim, hq, hkv, page, lens, splits, empty = draw_case(seed)
    case = f"seed={seed} dtype={dtype} D={head_dim} hq={hq} hkv={hkv} page={page} lens={lens} splits={splits} empty={empty}"
    print(case, flush=True)
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, head_dim, page, dtype=dtype, device="cuda", seed=seed,
                                        poison=float("nan"), tail=float("nan"))
    if empty:
        kv.seq_lens[0] = 0
    got = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, num_splits=splits)
    want = ref.paged_decode_attention(q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(),
                                      kv.seq_lens.cpu())
    if empty:
        want[0] = 0
    got = got.cpu()
    assert torch.isfinite(got).all(), case
    decode_parity(got, want, dtype, case)
