"""Pins for the cascade (shared-prefix) decode oracle.

The original project ships no cascade implementation (it names the FlashInfer
feature, docs/design.md:96-100), so the definition is attention over the
prefix tokens followed by the sequence's own. Pinned here against the already
pinned paged restatement (page-aligned prefix = one concatenated block table),
against SDPA on contiguous concatenated K/V (an independent library path), and
by its edge cases.
"""

from __future__ import annotations

import pytest
import torch

from kernel_lab.kv_cache import pages_for, random_cascade_problem
from oracle import reference as ref


def _contiguous(kv, table_row, n):
    return ref._gather(kv.k_cache, table_row, n), ref._gather(kv.v_cache, table_row, n)


@pytest.mark.parametrize(("hq", "hkv"), [(8, 2), (8, 8), (32, 1)])
def test_page_aligned_prefix_equals_one_concatenated_table(hq, hkv):
    page = 16
    q, c = random_cascade_problem(64, [5, 40, 17], hq, hkv, 32, page, dtype=torch.float32, seed=1)
    got = ref.cascade_decode_attention(q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, c.prefix_len,
                                       c.kv.block_table, c.kv.seq_lens)
    npre = pages_for(c.prefix_len, page)
    rows = []
    for b, n in enumerate(c.kv.seq_lens.tolist()):
        own = c.kv.block_table[b, : pages_for(n, page)]
        rows.append(torch.cat([c.prefix_block_table[:npre], own]))
    width = max(r.numel() for r in rows)
    table = torch.zeros(len(rows), width, dtype=torch.int32)
    for b, r in enumerate(rows):
        table[b, : r.numel()] = r
    want = ref.paged_decode_attention(q, c.kv.k_cache, c.kv.v_cache, table, c.kv.seq_lens + c.prefix_len)
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("prefix_len", [1, 15, 33, 100])
def test_unaligned_prefix_matches_sdpa_on_concatenated_tokens(prefix_len):
    q, c = random_cascade_problem(prefix_len, [3, 0, 50], 8, 2, 32, 16, dtype=torch.float32, seed=2)
    got = ref.cascade_decode_attention(q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, c.prefix_len,
                                       c.kv.block_table, c.kv.seq_lens)
    pk, pv = _contiguous(c.kv, c.prefix_block_table, prefix_len)
    keys, values = [], []
    for b, n in enumerate(c.kv.seq_lens.tolist()):
        k, v = _contiguous(c.kv, c.kv.block_table[b], n)
        keys.append(torch.cat([pk, k]))
        values.append(torch.cat([pv, v]))
    want = ref.dense_decode_attention(q, keys, values)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)
    assert torch.isfinite(got).all()


def test_empty_prefix_is_plain_decode():
    q, c = random_cascade_problem(0, [7, 30], 8, 2, 32, 16, dtype=torch.float32, seed=3)
    got = ref.cascade_decode_attention(q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, 0,
                                       c.kv.block_table, c.kv.seq_lens)
    want = ref.paged_decode_attention(q, c.kv.k_cache, c.kv.v_cache, c.kv.block_table, c.kv.seq_lens)
    torch.testing.assert_close(got, want, atol=0, rtol=0)


def test_no_tokens_at_all_gives_zeros():
    q, c = random_cascade_problem(0, [0, 5], 4, 2, 32, 16, dtype=torch.float32, seed=4)
    got = ref.cascade_decode_attention(q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, 0,
                                       c.kv.block_table, c.kv.seq_lens)
    assert torch.equal(got[0], torch.zeros_like(got[0])) and torch.isfinite(got[1]).all()
