"""Paged KV caches for tests and benchmarks.

Follows the paging rules of kernel_lab/kv_cache.py:16-102 in the original
project, so the same seed builds the same cache:

* the pool holds sum(cdiv(L_b, page_size)) + ``extra_pages`` pages, all first
  filled with a poison value;
* pages are handed out in the order of ``torch.randperm(total)`` drawn from a
  CPU generator seeded with ``seed``, sequence by sequence;
* the tail of a sequence's last page is ``tail`` (0 in the original: valid
  memory that must never be attended);
* the block table is int32 ``[batch, max_pages]``, padded with page 0 (a real
  page, so kernels must stop at cdiv(L_b, page_size));
* ``random_decode_problem`` draws q, then every K, then every V from one seeded
  CPU generator, as the original does.

Additions for MI355X-scale runs: ``poison`` may be NaN (stricter than 1e4: a
kernel that reads a spare page, or masks by multiplying with 0, turns the
output into NaN), pages are filled with one indexed copy per sequence instead of
a Python loop, and ``device_decode_problem`` builds multi-GB caches directly in
HBM with a device generator.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class PagedKV:
    k_cache: torch.Tensor  # [num_pages, page_size, num_kv_heads, head_dim]
    v_cache: torch.Tensor
    block_table: torch.Tensor  # [batch, max_pages] int32, padded with 0
    seq_lens: torch.Tensor  # [batch] int32
    page_size: int

    @property
    def max_pages(self) -> int:
        return self.block_table.shape[1]


def pages_for(seq_len: int, page_size: int) -> int:
    return (seq_len + page_size - 1) // page_size


def _fill_pages(cache: torch.Tensor, pages: torch.Tensor, src: torch.Tensor, tail: float) -> None:
    """Copy contiguous [L, Hkv, D] tokens into ``pages`` of ``cache`` (in order)."""
    page_size = cache.shape[1]
    n = src.shape[0]
    full = n // page_size
    if full:
        cache.index_copy_(0, pages[:full], src[: full * page_size].reshape(full, page_size, *src.shape[1:]))
    rem = n - full * page_size
    if rem:
        last = int(pages[full])
        cache[last, :rem] = src[full * page_size :]
        cache[last, rem:] = tail


def build_paged_kv(
    keys: list[torch.Tensor],
    values: list[torch.Tensor],
    page_size: int,
    extra_pages: int = 3,
    seed: int = 0,
    poison: float = 1e4,
    tail: float = 0.0,
) -> PagedKV:
    """Page pools built from each sequence's own K and V ([L, Hkv, D] tensors):
    the pages are placed at a seeded random permutation of pool slots.

    ``extra_pages`` unused pages keep the ``poison`` value: reading one makes
    the result visibly wrong.
    """
    if not keys or len(keys) != len(values):
        raise ValueError("need one K and one V tensor per sequence")
    _, num_kv_heads, head_dim = keys[0].shape
    lens = [k.shape[0] for k in keys]
    if min(lens) < 1:
        raise ValueError("every sequence needs at least one cached token")
    needed = [pages_for(n, page_size) for n in lens]
    total = sum(needed) + extra_pages
    device, dtype = keys[0].device, keys[0].dtype

    k_cache = torch.full((total, page_size, num_kv_heads, head_dim), poison, dtype=dtype, device=device)
    v_cache = torch.full_like(k_cache, poison)
    generator = torch.Generator().manual_seed(seed)
    order = torch.randperm(total, generator=generator)

    block_table = torch.zeros((len(keys), max(needed)), dtype=torch.int32)
    cursor = 0
    for b, (k, v) in enumerate(zip(keys, values, strict=True)):
        pages = order[cursor : cursor + needed[b]]
        cursor += needed[b]
        block_table[b, : needed[b]] = pages.to(torch.int32)
        dev_pages = pages.to(device)
        _fill_pages(k_cache, dev_pages, k, tail)
        _fill_pages(v_cache, dev_pages, v, tail)

    return PagedKV(
        k_cache=k_cache,
        v_cache=v_cache,
        block_table=block_table.to(device),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        page_size=page_size,
    )


def random_decode_problem(
    seq_lens: list[int],
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    dtype: torch.dtype = torch.float16,
    device: str | torch.device = "cpu",
    seed: int = 0,
    poison: float = 1e4,
    tail: float = 0.0,
) -> tuple[torch.Tensor, PagedKV, list[torch.Tensor], list[torch.Tensor]]:
    """Seeded N(0, 1) queries, keys and values for sequences of the given
    lengths: returns q, the paged cache, and each sequence's unpaged K and V."""
    generator = torch.Generator().manual_seed(seed)

    def rand(*shape: int) -> torch.Tensor:
        return torch.randn(*shape, generator=generator).to(device=device, dtype=dtype)

    q = rand(len(seq_lens), num_q_heads, head_dim)
    keys = [rand(n, num_kv_heads, head_dim) for n in seq_lens]
    values = [rand(n, num_kv_heads, head_dim) for n in seq_lens]
    kv = build_paged_kv(keys, values, page_size, seed=seed, poison=poison, tail=tail)
    return q, kv, keys, values


def device_decode_problem(
    seq_lens: list[int],
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    dtype: torch.dtype = torch.float16,
    device: str | torch.device = "cuda",
    seed: int = 0,
    extra_pages: int = 3,
    poison: float = float("nan"),
) -> tuple[torch.Tensor, PagedKV]:
    """Same paging rules, generated in device memory (for caches of many GB).

    q, K and V are N(0, 1) from a device generator (a different random stream
    from ``random_decode_problem``); pages are a seeded permutation with
    ``extra_pages`` poisoned spares; tails are zero.
    """
    if min(seq_lens) < 1:
        raise ValueError("every sequence needs at least one cached token")
    gen = torch.Generator(device=device).manual_seed(seed)
    needed = [pages_for(n, page_size) for n in seq_lens]
    total = sum(needed) + extra_pages
    shape = (total, page_size, num_kv_heads, head_dim)
    k_cache = torch.empty(shape, dtype=dtype, device=device)
    v_cache = torch.empty(shape, dtype=dtype, device=device)
    k_cache.normal_(generator=gen)
    v_cache.normal_(generator=gen)
    order = torch.randperm(total, generator=torch.Generator().manual_seed(seed))
    block_table = torch.zeros((len(seq_lens), max(needed)), dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(seq_lens):
        pages = order[cursor : cursor + needed[b]]
        cursor += needed[b]
        block_table[b, : needed[b]] = pages.to(torch.int32)
        rem = n - (needed[b] - 1) * page_size
        if rem < page_size:
            last = int(pages[-1])
            k_cache[last, rem:] = 0
            v_cache[last, rem:] = 0
    spare = order[cursor:].to(device)
    if spare.numel():
        k_cache.index_fill_(0, spare, poison)
        v_cache.index_fill_(0, spare, poison)
    q = torch.randn(len(seq_lens), num_q_heads, head_dim, generator=gen, device=device, dtype=torch.float32).to(dtype)
    kv = PagedKV(
        k_cache=k_cache,
        v_cache=v_cache,
        block_table=block_table.to(device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        page_size=page_size,
    )
    return q, kv


# Largest finite OCP FP8 E4M3 value.
FP8_E4M3_MAX = 448.0


def used_pages(kv: PagedKV) -> torch.Tensor:
    """Distinct pool pages that hold some sequence's tokens (spares excluded)."""
    npages = (kv.seq_lens.to(torch.int64) + kv.page_size - 1) // kv.page_size
    cols = torch.arange(kv.max_pages, device=kv.block_table.device)[None, :] < npages[:, None]
    return torch.unique(kv.block_table[cols].to(torch.int64))


def _head_amax(cache: torch.Tensor, pages: torch.Tensor, chunk: int = 4096) -> torch.Tensor:
    amax = torch.zeros(cache.shape[2], dtype=torch.float32, device=cache.device)
    for i in range(0, pages.numel(), chunk):
        part = cache.index_select(0, pages[i : i + chunk]).float().abs()
        amax = torch.maximum(amax, part.amax(dim=(0, 1, 3)))
    return amax


def quantize_fp8(kv: PagedKV) -> tuple[PagedKV, torch.Tensor, torch.Tensor]:
    """The cache in OCP FP8 E4M3 with one float32 scale per KV head.

    scale_h = max |x| over head h's cached tokens / 448 (spare pages do not
    count), codes = round-to-nearest-even(x / scale_h) as float8_e4m3fn, so
    head h's values are scale_h * code. Values outside E4M3's range (poisoned
    spares) become NaN codes, which a correct kernel never reads.
    """
    pages = used_pages(kv)
    out = []
    scales = []
    for cache in (kv.k_cache, kv.v_cache):
        amax = _head_amax(cache, pages)
        scale = torch.where(amax > 0, amax / FP8_E4M3_MAX, torch.ones_like(amax))
        codes = torch.empty(cache.shape, dtype=torch.float8_e4m3fn, device=cache.device)
        for i in range(0, cache.shape[0], 4096):
            codes[i : i + 4096] = (cache[i : i + 4096].float() / scale[None, None, :, None]).to(torch.float8_e4m3fn)
        out.append(codes)
        scales.append(scale)
    q8 = PagedKV(out[0], out[1], kv.block_table, kv.seq_lens, kv.page_size)
    return q8, scales[0], scales[1]


@dataclass
class CascadeKV:
    """A paged pool holding a shared prefix and each sequence's own tokens."""

    kv: PagedKV  # block_table / seq_lens: each sequence's own tokens (may be 0)
    prefix_block_table: torch.Tensor  # [cdiv(prefix_len, page_size)] int32
    prefix_len: int

    def flattened(self) -> PagedKV:
        """The same attention as plain paged decode: each sequence's table is
        the prefix pages followed by its own (needs a page-aligned prefix)."""
        page = self.kv.page_size
        if self.prefix_len % page:
            raise ValueError("flattening needs prefix_len to be a multiple of page_size")
        own_pages = [pages_for(int(n), page) for n in self.kv.seq_lens.tolist()]
        npre = self.prefix_block_table.numel()
        table = torch.zeros(
            (len(own_pages), npre + max(own_pages + [0])), dtype=torch.int32, device=self.kv.block_table.device
        )
        table[:, :npre] = self.prefix_block_table
        for b, n in enumerate(own_pages):
            table[b, npre : npre + n] = self.kv.block_table[b, :n]
        return PagedKV(self.kv.k_cache, self.kv.v_cache, table, self.kv.seq_lens + self.prefix_len, page)


def random_cascade_problem(
    prefix_len: int,
    seq_lens: list[int],
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    dtype: torch.dtype = torch.float16,
    device: str | torch.device = "cpu",
    seed: int = 0,
    poison: float = float("nan"),
) -> tuple[torch.Tensor, CascadeKV]:
    """Random queries, a shared prefix of ``prefix_len`` tokens and per-sequence
    suffixes of ``seq_lens`` tokens (0 allowed), paged into one pool with the
    rules of build_paged_kv (the prefix is paged first, as one more sequence).
    Spare pages and the tails of last pages hold ``poison``.
    """
    generator = torch.Generator().manual_seed(seed)

    def rand(*shape: int) -> torch.Tensor:
        return torch.randn(*shape, generator=generator).to(dtype=dtype)

    q = rand(len(seq_lens), num_q_heads, head_dim)
    # Every paged "sequence" needs a token; a zero-length prefix or suffix gets
    # one unreferenced token and a length of 0.
    lens = [max(prefix_len, 1)] + [max(n, 1) for n in seq_lens]
    keys = [rand(n, num_kv_heads, head_dim) for n in lens]
    values = [rand(n, num_kv_heads, head_dim) for n in lens]
    # Tails of last pages hold the poison too: only masking keeps them out.
    pool = build_paged_kv(keys, values, page_size, seed=seed, poison=poison, tail=poison)
    npre = pages_for(prefix_len, page_size)
    prefix_table = pool.block_table[0, :npre].clone()
    own = PagedKV(
        k_cache=pool.k_cache.to(device),
        v_cache=pool.v_cache.to(device),
        block_table=pool.block_table[1:].contiguous().to(device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        page_size=page_size,
    )
    return q.to(device), CascadeKV(own, prefix_table.to(device), prefix_len)
