"""Split units merged inside the decode kernel (no merge launch).

On the MFMA path, a unit split over several segments (uniform splits, or a
balanced-schedule workgroup range) with one head tile of at most 8 query
heads is merged by its last segment to finish (MQA and other two-tile units,
and units split so widely that the last segment's merge would be long, keep
the merge kernel, and are checked here too), counted on library-owned arrival counters of a
region that belongs to the call's stream. The merge is the merge kernels' own
routine, so every output must be bit-identical with the fused merge switched
off (``KL_DECODE_FUSED_MERGE=0``), and match the oracle. The counters must be
left at zero by every call (back-to-back calls of different shapes), streams
must not share counters (concurrent streams), and every case checks, through
kl_paged_decode_last_merge, that the merge it expects actually ran. Streams
beyond the library's regions: tests/test_zy_merge_regions.py.
"""

from __future__ import annotations


import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8, random_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu


def _decode(ops, q, kv, out=None, **kw):
    return ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=out, **kw)


def _unfused(fn):
    with _native.decode_switches(fused_merge="0"):
        return fn()


def _lens(batch: int, hi: int, seed: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(1, hi + 1, (batch,), generator=g).tolist()


IN_KERNEL, MERGE_KERNEL = 2, 1  # kl_paged_decode_last_merge: KL_MERGE_IN_KERNEL, KL_MERGE_KERNEL


def _last_merge() -> int:
    return _native.core().kl_paged_decode_last_merge()


CASES = [
    # (lens, hq, hkv, head_dim, dtype, num_splits, empty rows, merge); None = planner
    ([512], 32, 8, 128, torch.float16, None, [], IN_KERNEL),  # B=1: uniform splits
    ([512, 500], 32, 8, 128, torch.float16, None, [], IN_KERNEL),  # balanced, B=2
    ([4096] * 8, 32, 8, 128, torch.float16, None, [], IN_KERNEL),  # balanced, units split 4 ways
    ([65536] + [1024] * 15, 32, 8, 128, torch.float16, None, [], IN_KERNEL),  # skewed, balanced
    ("r24", 64, 8, 128, torch.bfloat16, None, [3, 17], IN_KERNEL),  # G=8, empty sequences
    ("r64", 32, 8, 128, torch.float16, -1, [0, 63], IN_KERNEL),  # balanced on request, full batch
    ([900] * 8, 32, 8, 128, torch.float16, 4, [], IN_KERNEL),  # uniform splits
    ([1, 15, 16, 17, 33, 70, 300, 1025], 16, 4, 64, torch.bfloat16, 16, [2], IN_KERNEL),  # splits past short ones
    ("r16", 8, 8, 32, torch.float16, 5, [], IN_KERNEL),  # G=1, head_dim 32
    ([2000] * 64, 32, 8, 128, torch.float16, 2, [5], IN_KERNEL),  # paired workgroups with splits
    ("m64", 32, 1, 128, torch.bfloat16, None, [9], MERGE_KERNEL),  # MQA: 32-head units, balanced
    ([6000, 30, 2500, 800], 32, 1, 64, torch.float16, 7, [], MERGE_KERNEL),  # MQA, uniform splits, head_dim 64
    ([3000] * 4, 96, 4, 128, torch.float16, None, [], MERGE_KERNEL),  # 24 heads per unit (two head tiles)
    ([32768], 8, 1, 128, torch.float16, None, [], MERGE_KERNEL),  # one unit over 64 splits
    ([2048], 8, 1, 128, torch.float16, None, [], MERGE_KERNEL),  # 16 splits, two heads per wave
    ([1024], 8, 1, 128, torch.float16, None, [], IN_KERNEL),  # 8 splits, two heads per wave
    ([4096, 4000], 32, 8, 128, torch.float16, None, [], IN_KERNEL),  # balanced, 8 short segments per unit
    ([4096, 4000], 64, 8, 128, torch.bfloat16, None, [], IN_KERNEL),  # the same, two heads per wave
    ([8192, 8000], 64, 8, 128, torch.bfloat16, None, [], MERGE_KERNEL),  # 16 segments, two heads per wave
]


def _case_lens(spec):
    if isinstance(spec, str):
        n = int(spec[1:])
        return _lens(n, 8192 if spec[0] == "m" else 3000, seed=n)
    return list(spec)


@pytest.mark.parametrize(("spec", "hq", "hkv", "head_dim", "dtype", "num_splits", "empty", "merge"), CASES)
def test_fused_merge_is_bit_identical(gpu_ops, spec, hq, hkv, head_dim, dtype, num_splits, empty, merge):
    lens = _case_lens(spec)
    q, kv = device_decode_problem(lens, hq, hkv, head_dim, 16, dtype=dtype, seed=len(lens) + hq)
    if empty:
        kv.seq_lens[empty] = 0
    kw = {} if num_splits is None else {"num_splits": num_splits}
    fused = _decode(gpu_ops, q, kv, **kw).cpu()
    assert _last_merge() == merge, "the call did not take the expected merge"
    merged = _unfused(lambda: _decode(gpu_ops, q, kv, **kw)).cpu()
    assert _last_merge() == MERGE_KERNEL
    assert torch.isfinite(fused).all(), "non-finite output: a poisoned page or tail leaked in"
    assert torch.equal(fused, merged), "fused merge differs from the merge kernel"
    for b in empty:
        assert not fused[b].any(), "an empty sequence must give zeros"
    rows = [b for b in range(len(lens)) if b not in empty][:6]
    want = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu()
    )
    decode_parity(fused[rows], want, dtype)


def test_fused_merge_fp8_cache(gpu_ops):
    q, kv, _, _ = random_decode_problem([3000, 20, 700, 1], 32, 8, 128, 16, dtype=torch.bfloat16,
                                        device="cuda", poison=float("nan"))
    kv8, ks, vs = quantize_fp8(kv)
    run = lambda: gpu_ops.paged_decode_attention(q, kv8.k_cache, kv8.v_cache, kv.block_table, kv.seq_lens,
                                                 k_scale=ks, v_scale=vs)
    fused = run().cpu()
    assert torch.equal(fused, _unfused(run).cpu())
    want = ref.paged_decode_attention_fp8(
        q.cpu().float(), kv8.k_cache.cpu(), kv8.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu(), ks.cpu(), vs.cpu()
    )
    decode_parity(fused, want, torch.bfloat16)


def test_counters_are_left_at_zero(gpu_ops):
    """Back-to-back calls whose units overlap in the counter array, with
    different segment counts: a counter left nonzero by one call would make a
    later call merge early or never."""
    problems = []
    for i, (lens, splits) in enumerate([([700] * 8, 3), ([4096] * 2, None), ([300] * 16, 7), ([9000], None)]):
        q, kv = device_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, seed=40 + i)
        kw = {} if splits is None else {"num_splits": splits}
        want = _unfused(lambda q=q, kv=kv, kw=kw: _decode(gpu_ops, q, kv, **kw)).clone()
        problems.append((q, kv, kw, want))
    for _ in range(5):
        for q, kv, kw, want in problems:
            assert torch.equal(_decode(gpu_ops, q, kv, **kw), want)
    torch.cuda.synchronize()


def test_concurrent_streams(gpu_ops):
    """Calls in flight on several streams at once take separate counter
    regions; each stream's results equal the unfused ones."""
    jobs = []
    for i in range(4):
        q, kv = device_decode_problem([2500] * 6, 32, 8, 128, 16, dtype=torch.float16, seed=60 + i)
        want = _unfused(lambda q=q, kv=kv: _decode(gpu_ops, q, kv)).clone()
        jobs.append((torch.cuda.Stream(), q, kv, torch.empty_like(q), want))
    torch.cuda.synchronize()
    for _ in range(3):
        for stream, q, kv, out, _ in jobs:
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(4):
                    _decode(gpu_ops, q, kv, out=out)
        torch.cuda.synchronize()
        for _, _, _, out, want in jobs:
            assert torch.equal(out, want)


@pytest.mark.parametrize(
    ("batch", "hq", "hkv", "max_len", "splits"),
    [
        (64, 8, 2, 32, None),  # 128 units of <= 2 pages: a grid of <= 32 workgroups
        (256, 32, 8, 16, -1),  # paired balanced on request, one page each: 128 workgroups
        (300, 8, 2, 16, -1),   # past the schedule's one-pass scan: 38 workgroups
    ],
)
def test_empty_sequences_beyond_the_grid(gpu_ops, batch, hq, hkv, max_len, splits):
    """Short contexts give a balanced grid smaller than the batch (one
    workgroup per 8 list pages), so workgroup b cannot zero sequence b: every
    empty sequence must still get zeros, with an output buffer that starts as
    NaN, and the rest must equal the merge kernel's result."""
    lens = _lens(batch, max_len, seed=batch)
    q, kv = device_decode_problem(lens, hq, hkv, 128, 16, dtype=torch.float16, seed=batch + 1)
    empty = [1, batch // 2 + 3, batch - 1]
    kv.seq_lens[empty] = 0
    kw = {} if splits is None else {"num_splits": splits}
    fused = _decode(gpu_ops, q, kv, out=torch.full_like(q, float("nan")), **kw).cpu()
    merged = _unfused(lambda: _decode(gpu_ops, q, kv, out=torch.full_like(q, float("nan")), **kw)).cpu()
    for b in empty:
        assert torch.equal(fused[b], torch.zeros_like(fused[b])), f"sequence {b} is empty and must give zeros"
    assert torch.isfinite(fused).all(), "a row was left unwritten"
    assert torch.equal(fused, merged)
    rows = [0, 2, batch // 2, batch - 2]
    want = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table[rows].cpu(), kv.seq_lens[rows].cpu()
    )
    decode_parity(fused[rows], want, torch.float16)


@pytest.mark.parametrize(("lens", "splits"), [([4096] * 8, None), ([900] * 16, 6), ([30000, 40, 500], None)])
def test_fresh_partials_every_call(gpu_ops, lens, splits):
    """New queries on every call, so every call's partials differ from the
    last call's at the same workspace addresses: a merge that read a partial
    before its writer's stores were visible would differ from the merge
    kernel's result."""
    q, kv = device_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, seed=90)
    kw = {} if splits is None else {"num_splits": splits}
    gen = torch.Generator(device="cuda").manual_seed(91)
    for i in range(30):
        q.normal_(generator=gen)
        fused = _decode(gpu_ops, q, kv, **kw)
        merged = _unfused(lambda: _decode(gpu_ops, q, kv, **kw))
        assert torch.equal(fused, merged), f"call {i}: fused merge differs from the merge kernel"
