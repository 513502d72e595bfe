"""The paged-cache builder keeps the original project's paging rules
(kernel_lab/kv_cache.py:33-102 of Markkoby3/Kernel-lab)."""

from __future__ import annotations

import math

import pytest
import torch

from kernel_lab.kv_cache import build_paged_kv, pages_for, random_decode_problem


def test_build_paged_kv_round_trips_and_shuffles_pages():
    keys = [torch.randn(n, 2, 8) for n in (5, 33)]
    values = [torch.randn(n, 2, 8) for n in (5, 33)]
    kv = build_paged_kv(keys, values, page_size=16)
    assert kv.block_table.shape == (2, pages_for(33, 16))
    for b, (k, v) in enumerate(zip(keys, values, strict=True)):
        n = k.shape[0]
        pages = kv.block_table[b, : pages_for(n, 16)].long()
        torch.testing.assert_close(kv.k_cache[pages].reshape(-1, 2, 8)[:n], k)
        torch.testing.assert_close(kv.v_cache[pages].reshape(-1, 2, 8)[:n], v)
    assert kv.block_table[1].tolist() != sorted(kv.block_table[1].tolist())


def test_build_paged_kv_rejects_empty_sequences():
    with pytest.raises(ValueError):
        build_paged_kv([torch.randn(0, 1, 8)], [torch.randn(0, 1, 8)], page_size=16)
    with pytest.raises(ValueError):
        build_paged_kv([], [], page_size=16)


@pytest.mark.parametrize("poison", [1e4, float("nan")])
def test_spare_pages_are_poisoned_and_tails_zero(poison):
    lens = [5, 33, 16]
    keys = [torch.randn(n, 1, 4) for n in lens]
    kv = build_paged_kv(keys, [k.clone() for k in keys], page_size=16, extra_pages=3, poison=poison)
    used = set()
    for b, n in enumerate(lens):
        pages = kv.block_table[b, : pages_for(n, 16)].tolist()
        used.update(pages)
        rem = n - (len(pages) - 1) * 16
        tail = kv.k_cache[pages[-1], rem:]
        assert (tail == 0).all()
    spare = sorted(set(range(kv.k_cache.shape[0])) - used)
    assert len(spare) == 3
    for p in spare:
        block = kv.k_cache[p]
        assert torch.isnan(block).all() if math.isnan(poison) else (block == poison).all()


def test_block_table_padding_is_page_zero():
    kv = build_paged_kv([torch.randn(3, 1, 4), torch.randn(40, 1, 4)], [torch.randn(3, 1, 4), torch.randn(40, 1, 4)], 16)
    assert kv.block_table.dtype == torch.int32
    assert kv.block_table[0, 1:].tolist() == [0, 0]


def test_same_seed_same_problem():
    a = random_decode_problem([7, 20], 4, 2, 16, 16, seed=3)
    b = random_decode_problem([7, 20], 4, 2, 16, 16, seed=3)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1].k_cache, b[1].k_cache)
    assert torch.equal(a[1].block_table, b[1].block_table)


def test_draw_order_is_q_then_keys_then_values():
    """One seeded CPU generator: q first, then every K, then every V (original kv_cache.py:94-101)."""
    lens = [3, 5]
    q, _, keys, values = random_decode_problem(lens, 2, 1, 8, 16, dtype=torch.float32, seed=11)
    g = torch.Generator().manual_seed(11)
    assert torch.equal(q, torch.randn(2, 2, 8, generator=g))
    for k in keys:
        assert torch.equal(k, torch.randn(k.shape[0], 1, 8, generator=g))
    for v in values:
        assert torch.equal(v, torch.randn(v.shape[0], 1, 8, generator=g))
