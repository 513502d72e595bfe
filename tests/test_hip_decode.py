"""gfx950 paged decode attention against the CPU oracle.

Shapes and rules come from the original project's tests
(tests/test_cuda_kernels.py:44-53, tests/test_paged_attention.py:12-106) and the
measured configurations: Llama-3-8B GQA (32/8/128/16, fp16, B 1..64, ctx 512 and
4096, split counts 1/4/16/64 and the planner), ragged-length MQA (32/1/128/16,
bf16, B 64, L ~ U[1, 8192]) and long-context 70B-style GQA (64/8/128/16, bf16,
B 8, ctx 32768). Spare pages hold NaN unless a test says otherwise, so a read of
one, or masking by multiplication, shows up as NaN.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import build_paged_kv, device_decode_problem, random_decode_problem
from kernel_lab.ops import plan_decode
from oracle import reference as ref
from tests.conftest import DTYPES, decode_parity

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_golden.npz"


def run(ops, q, kv, **kw):
    return ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, **kw)


def expected(q, kv, scale=None):
    """The oracle's float32 result before its final rounding to q's dtype
    (q widened exactly; the caches are widened per sequence by the oracle)."""
    return ref.paged_decode_attention(
        q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu(), scale
    )


def check(got, want, dtype, what=""):
    """The reference's tolerance table against the rounded oracle, and at most
    one output ulp (plus 1e-6) from the unrounded one."""
    return decode_parity(got, want, dtype, what)


# ---------------------------------------------------- original test shapes


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hq", "hkv"), [(8, 8), (16, 4), (8, 1), (32, 8)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_native_op_shapes(gpu_ops, hq, hkv, head_dim, dtype):
    """tests/test_cuda_kernels.py:44-53 of the original, with NaN spares."""
    q, kv, _, _ = random_decode_problem(
        [1, 3, 16, 17, 300, 1025], hq, hkv, head_dim, 16, dtype=dtype, device="cuda", poison=float("nan")
    )
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hq", "hkv"), [(4, 4), (8, 2), (8, 1)])
def test_split_kernel_shapes(gpu_ops, hq, hkv, dtype):
    """tests/test_paged_attention.py:25-29: page boundaries 1, 15/16/17, 33, 70; D = 32."""
    q, kv, _, _ = random_decode_problem([1, 15, 16, 17, 33, 70], hq, hkv, 32, 16, dtype=dtype, device="cuda")
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


@pytest.mark.parametrize("num_splits", [1, 2, 3, 5, 64])
@pytest.mark.parametrize("dtype", DTYPES)
def test_split_kv_is_exact_for_any_split_count(gpu_ops, num_splits, dtype):
    """Splits only partition the sum; empty splits get zero weight (tests/test_paged_attention.py:32-37)."""
    q, kv, _, _ = random_decode_problem([1, 15, 16, 17, 33, 70], 4, 2, 32, 16, dtype=dtype, device="cuda")
    check(run(gpu_ops, q, kv, num_splits=num_splits), expected(q, kv), dtype, f"splits={num_splits}")


def test_agrees_with_dense_sdpa(gpu_ops):
    q, kv, keys, values = random_decode_problem([5, 40], 8, 2, 64, 16, dtype=torch.float32, device="cuda")
    want = ref.dense_decode_attention(q.cpu(), [k.cpu() for k in keys], [v.cpu() for v in values])
    check(run(gpu_ops, q, kv), want, torch.float32, "dense SDPA")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("page_size", [16, 32])
@pytest.mark.parametrize("head_dim", [32, 64])
def test_page_and_head_sizes(gpu_ops, page_size, head_dim, dtype):
    q, kv, _, _ = random_decode_problem([3, 50], 4, 2, head_dim, page_size, dtype=dtype, device="cuda")
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


@pytest.mark.parametrize("page_size", [1, 8, 64])
def test_other_page_sizes(gpu_ops, page_size):
    q, kv, _, _ = random_decode_problem([3, 50, 64], 8, 2, 64, page_size, dtype=torch.float16, device="cuda")
    check(run(gpu_ops, q, kv), expected(q, kv), torch.float16)


@pytest.mark.parametrize("page_size", [48, 80, 112])
@pytest.mark.parametrize(("hq", "hkv", "head_dim", "splits"), [(32, 8, 128, 0), (32, 1, 128, 0), (8, 2, 64, 3), (16, 4, 128, -1)])
def test_page_sizes_not_powers_of_two(gpu_ops, page_size, hq, hkv, head_dim, splits):
    """Page sizes that are multiples of 16 but not powers of two: the MFMA
    kernels turn a 16-token block index into its page with a multiply and a
    shift (3, 5 or 7 blocks per page here). Lengths end mid-block, mid-page
    and on page boundaries, and the longest gives every wave blocks across
    many pages."""
    lens = [1, 15, 16, page_size - 1, page_size, page_size + 17, 40 * page_size + 3]
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, head_dim, page_size, dtype=torch.bfloat16, device="cuda",
                                        poison=float("nan"), seed=page_size + hq)
    check(run(gpu_ops, q, kv, num_splits=splits), expected(q, kv), torch.bfloat16, f"page {page_size} splits {splits}")


@pytest.mark.parametrize("poison", [1e4, float("nan")])
@pytest.mark.parametrize("dtype", DTYPES)
def test_reads_only_pages_in_the_block_table(gpu_ops, poison, dtype):
    """Spare pages poisoned (tests/test_paged_attention.py:56-62), and tails too."""
    q, kv, _, _ = random_decode_problem(
        [20, 9, 33], 4, 4, 32, 16, dtype=dtype, device="cuda", poison=poison, tail=poison
    )
    out = run(gpu_ops, q, kv)
    assert torch.isfinite(out).all() and out.abs().max() < 10
    check(out, expected(q, kv), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_nan_tails_under_mfma_tiles(gpu_ops, dtype):
    """Lengths that end mid-block at 128/16 put NaN tokens inside MFMA tiles."""
    q, kv, _, _ = random_decode_problem(
        [1, 5, 17, 31, 47, 100], 32, 8, 128, 16, dtype=dtype, device="cuda", poison=float("nan"), tail=float("nan")
    )
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


def test_max_seq_len_bounds_work_without_changing_results(gpu_ops):
    q, kv, _, _ = random_decode_problem([5, 20], 4, 2, 32, 16, dtype=torch.float32, device="cuda")
    kv.block_table = torch.nn.functional.pad(kv.block_table, (0, 6))  # extra block-table columns
    check(run(gpu_ops, q, kv, max_seq_len=20), expected(q, kv), torch.float32, "max_seq_len=20")
    check(run(gpu_ops, q, kv), expected(q, kv), torch.float32)


def test_strided_block_table(gpu_ops):
    q, kv, _, _ = random_decode_problem([5, 40, 17], 8, 2, 64, 16, dtype=torch.float16, device="cuda")
    wide = torch.zeros(3, kv.block_table.shape[1] + 5, dtype=torch.int32, device="cuda")
    wide[:, : kv.block_table.shape[1]] = kv.block_table
    kv.block_table = wide[:, : kv.block_table.shape[1]]  # row stride > width
    check(run(gpu_ops, q, kv), expected(q, kv), torch.float16)


@pytest.mark.parametrize("dtype", DTYPES)
def test_custom_scale(gpu_ops, dtype):
    q, kv, _, _ = random_decode_problem([12, 40], 2, 2, 32, 16, dtype=dtype, device="cuda")
    check(run(gpu_ops, q, kv, scale=0.05), expected(q, kv, scale=0.05), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_one_hot_attention_returns_that_value(gpu_ops, dtype):
    """tests/test_paged_attention.py:81-91 of the original."""
    head_dim = 32
    keys = [torch.zeros(20, 1, head_dim)]
    values = [torch.arange(20, dtype=torch.float32)[:, None, None].expand(20, 1, head_dim).clone()]
    keys[0][13, 0, 0] = 100.0
    kv = build_paged_kv([k.to("cuda", dtype) for k in keys], [v.to("cuda", dtype) for v in values], page_size=16)
    q = torch.zeros(1, 1, head_dim, device="cuda", dtype=dtype)
    q[0, 0, 0] = 1.0
    out = run(gpu_ops, q, kv, scale=1.0)
    torch.testing.assert_close(out.float(), torch.full_like(out.float(), 13.0), atol=1e-4, rtol=0)


def test_validation(gpu_ops):
    q, kv, _, _ = random_decode_problem([4], 3, 2, 32, 16, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="multiple"):
        run(gpu_ops, q, kv)
    q, kv, _, _ = random_decode_problem([4], 2, 2, 24, 16, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="power of two"):
        run(gpu_ops, q, kv)
    q, kv, _, _ = random_decode_problem([4], 4, 2, 32, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.kernel_lab.paged_decode_attention(
            torch.empty_like(q), q, kv.k_cache, kv.v_cache, kv.block_table.long(), kv.seq_lens, 0.1
        )


def test_empty_sequence_gives_zeros(gpu_ops):
    """seq_len 0 attends over nothing; the original's math (an empty weighted sum) gives 0."""
    q, kv, _, _ = random_decode_problem([4, 9], 4, 2, 64, 16, dtype=torch.float16, device="cuda")
    kv.seq_lens[0] = 0
    for splits in (None, 3):
        out = run(gpu_ops, q, kv, num_splits=splits)
        assert torch.equal(out[0].cpu(), torch.zeros_like(out[0].cpu()))
        want = expected(q[1:], type(kv)(kv.k_cache, kv.v_cache, kv.block_table[1:], kv.seq_lens[1:], 16))
        check(out[1:], want, torch.float16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_golden_vectors(gpu_ops, dtype):
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    for name in names:
        g = {f: data[f"{name}/{f}"] for f in ("q", "k_cache", "v_cache", "block_table", "seq_lens", "scale")}
        q = torch.from_numpy(g["q"]).to("cuda", dtype)
        k = torch.from_numpy(g["k_cache"]).to("cuda", dtype)
        v = torch.from_numpy(g["v_cache"]).to("cuda", dtype)
        bt = torch.from_numpy(g["block_table"]).cuda()
        lens = torch.from_numpy(g["seq_lens"]).cuda()
        out = gpu_ops.paged_decode_attention(q, k, v, bt, lens, float(g["scale"]))
        # Expected values are the float64 brute force, unrounded.
        check(out, torch.from_numpy(data[f"{name}/expected"]), dtype, name)


def test_long_context(gpu_ops):
    """tests/test_paged_attention.py:103-106: [4096, 31, 2000], 32/8/128, fp16."""
    q, kv, _, _ = random_decode_problem([4096, 31, 2000], 32, 8, 128, 16, dtype=torch.float16, device="cuda")
    check(run(gpu_ops, q, kv), expected(q, kv), torch.float16)


# ------------------------------------------------ measured configurations


@pytest.mark.parametrize("batch", [1, 8, 32, 64])
@pytest.mark.parametrize("ctx", [512, 4096])
def test_config2_llama3_gqa(gpu_ops, batch, ctx):
    """32/8/128/16 fp16, NaN spares, splits {1, 4, 16, 64} and the planner."""
    q, kv = device_decode_problem([ctx] * batch, 32, 8, 128, 16, dtype=torch.float16, seed=batch + ctx)
    want = expected(q, kv)
    for splits in (None, 1, 4, 16, 64):
        check(run(gpu_ops, q, kv, num_splits=splits), want, torch.float16, f"B={batch} ctx={ctx} splits={splits}")


def test_config3_ragged_mqa(gpu_ops):
    """32/1/128/16 bf16, B 64, L ~ U[1, 8192] with page-boundary lengths, NaN spares."""
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1, 8193, (64,), generator=g).tolist()
    lens[:9] = [1, 15, 16, 17, 8191, 8192, 4095, 4096, 4097]
    q, kv = device_decode_problem(lens, 32, 1, 128, 16, dtype=torch.bfloat16, seed=3)
    want = expected(q, kv)
    for splits in (None, 1, 7, 64):
        check(run(gpu_ops, q, kv, num_splits=splits), want, torch.bfloat16, f"ragged MQA splits={splits}")


@pytest.mark.parametrize("page", [16, 32, 64])
@pytest.mark.parametrize(("dtype", "hq", "splits"), [(torch.float16, 32, 1), (torch.bfloat16, 64, 1), (torch.float16, 32, 2)])
def test_long_segments_refill_the_block_table_window(gpu_ops, page, dtype, hq, splits):
    """Head_dim 128 with one head tile loads K and V straight into LDS and
    reads each wave's block-table entries from a 64-block window in LDS that
    is refilled ahead of use. Segments of 8,000+ tokens give every wave well
    over 128 blocks (several refills), the lengths end mid-block and mid-page,
    and the pages are scattered over the cache."""
    lens = [8 * 1024 + 5, 6 * 1024 - 1, 9 * 1024 + page + 3]
    q, kv, _, _ = random_decode_problem(lens, hq, 8, 128, page, dtype=dtype, device="cuda", poison=float("nan"),
                                        seed=page + hq)
    check(run(gpu_ops, q, kv, num_splits=splits), expected(q, kv), dtype, f"page {page} splits {splits}")


@pytest.mark.parametrize(
    ("hq", "hkv", "ctx", "dtype"),
    [
        (32, 8, 4096, torch.float16),  # 32 uniform splits, merge kernel
        (32, 8, 1024, torch.float16),  # 8 splits, merged in the kernel
        (64, 8, 32768, torch.bfloat16),
        (8, 1, 32768, torch.float16),  # 64 splits of one KV head
        (32, 1, 20000, torch.bfloat16),  # two head tiles; the length ends mid-page
        (32, 4, 8190, torch.float16),
    ],
)
def test_single_sequence_uniform_splits(gpu_ops, hq, hkv, ctx, dtype):
    """A batch of one sequence takes uniform splits of >= 8 pages (it cannot be
    skewed); many-way splits at long contexts, checked against the unrounded
    oracle, with NaN in every unused page."""
    q, kv, _, _ = random_decode_problem([ctx], hq, hkv, 128, 16, dtype=dtype, device="cuda", poison=float("nan"),
                                        seed=ctx + hq)
    pages = kv.block_table.shape[1]
    splits, _ = plan_decode(dtype, 1, hq, hkv, 128, 16, pages, 0)
    assert splits > 1 and -(-pages // splits) >= 8, (splits, pages)  # uniform (0 would be the balanced schedule)
    check(run(gpu_ops, q, kv), expected(q, kv), dtype, f"{hq}/{hkv} ctx {ctx} splits {splits}")


def test_config4_long_context_gqa(gpu_ops):
    """64/8/128/16 bf16, B 8, ctx 32768; the planner picks the splits."""
    q, kv = device_decode_problem([32768] * 8, 64, 8, 128, 16, dtype=torch.bfloat16, seed=4)
    check(run(gpu_ops, q, kv), expected(q, kv), torch.bfloat16, "ctx 32768")


def test_config4_131072_context(gpu_ops):
    """64/8/128/16 bf16, B 8, ctx 131072 (4.3 GB of cache), planner splits.

    Every sequence is checked against the oracle (each is served by its own
    workgroups and merges, so a fault anywhere in the grid shows; about 3 s
    of CPU), and pinned once more by linearity in V: doubling V doubles the
    output bit for bit (products and fp32 sums scale exactly by 2, the
    log-sum-exp merge weights do not change, and rounding commutes with a
    power of two).
    """
    q, kv = device_decode_problem([131072] * 8, 64, 8, 128, 16, dtype=torch.bfloat16, seed=5)
    got = run(gpu_ops, q, kv)
    assert torch.isfinite(got).all()
    want = ref.paged_decode_attention(
        q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu()
    )
    check(got, want, torch.bfloat16, "ctx 131072, all 8 sequences")
    kv.v_cache.mul_(2)  # NaN spares stay NaN; N(0,1) values stay far from overflow
    doubled = run(gpu_ops, q, kv)
    assert torch.equal(doubled, got * 2), "output is not exactly linear in V"


# ------------------------------------------- balanced schedule (planner path)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_balanced_schedule_many_short_sequences(gpu_ops, dtype):
    """240 one-page units: each workgroup's range spans many whole units."""
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(1, 17, (30,), generator=g).tolist()
    q, kv, _, _ = random_decode_problem(lens, 32, 8, 128, 16, dtype=dtype, device="cuda", poison=float("nan"))
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("hq", "hkv"), [(32, 1), (8, 2), (64, 8)])
def test_balanced_schedule_ragged_lengths(gpu_ops, dtype, hq, hkv):
    """One long sequence among short and empty-page-boundary ones: units split
    across workgroups, ranges spanning unit and sequence boundaries."""
    lens = [6000, 1, 5, 300, 17, 16, 33, 2048, 15, 1]
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype, device="cuda", poison=float("nan"))
    check(run(gpu_ops, q, kv), expected(q, kv), dtype)


def test_balanced_schedule_with_empty_sequences(gpu_ops):
    q, kv, _, _ = random_decode_problem([300, 7, 1000, 9], 16, 4, 64, 16, dtype=torch.float16, device="cuda")
    kv.seq_lens[1] = 0
    kv.seq_lens[3] = 0
    out = run(gpu_ops, q, kv)
    assert torch.equal(out[1].cpu(), torch.zeros_like(out[1].cpu()))
    assert torch.equal(out[3].cpu(), torch.zeros_like(out[3].cpu()))
    keep = [0, 2]
    sub = type(kv)(kv.k_cache, kv.v_cache, kv.block_table[keep], kv.seq_lens[keep], 16)
    check(out[keep], expected(q[keep], sub), torch.float16)


def test_planner_and_uniform_splits_agree(gpu_ops):
    """The balanced schedule and uniform splits partition the same sum."""
    q, kv, _, _ = random_decode_problem([5000, 3, 700], 32, 8, 128, 16, dtype=torch.float32, device="cuda")
    kv16 = type(kv)(kv.k_cache.half(), kv.v_cache.half(), kv.block_table, kv.seq_lens, 16)
    want = expected(q.half(), kv16)
    check(run(gpu_ops, q.half(), kv16), want, torch.float16, "planner")
    check(run(gpu_ops, q.half(), kv16, num_splits=7), want, torch.float16, "7 splits")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_balanced_schedule_over_64_sequences(gpu_ops, dtype):
    """More sequences than lanes in a wave: the schedule scans seq_lens in
    64-sequence chunks (planner path, MQA so units stay under the CU count)."""
    g = torch.Generator().manual_seed(12)
    lens = torch.randint(1, 1500, (150,), generator=g).tolist()
    lens[3] = 4000
    q, kv, _, _ = random_decode_problem(lens, 8, 1, 128, 16, dtype=dtype, device="cuda", poison=float("nan"))
    kv.seq_lens[70] = 0
    kv.seq_lens[149] = 0
    out = run(gpu_ops, q, kv)
    assert torch.equal(out[70].cpu(), torch.zeros_like(out[70].cpu()))
    keep = [i for i in range(150) if i not in (70, 149)]
    sub = type(kv)(kv.k_cache, kv.v_cache, kv.block_table[keep], kv.seq_lens[keep], 16)
    check(out[keep], expected(q[keep], sub), dtype)


@pytest.mark.parametrize(("lens", "hq", "hkv"), [([9000] + [700] * 69, 32, 8), ([1] * 40 + [3000] * 3, 64, 8)])
def test_requested_balanced_schedule_on_full_batches(gpu_ops, lens, hq, hkv):
    """num_splits=BALANCED with more (sequence, KV head) units than CUs."""
    from kernel_lab import ops

    q, kv, _, _ = random_decode_problem(lens, hq, hkv, 128, 16, dtype=torch.float16, device="cuda", poison=float("nan"))
    check(run(gpu_ops, q, kv, num_splits=ops.BALANCED), expected(q, kv), torch.float16)


def test_requested_balanced_schedule_falls_back_for_fp32(gpu_ops):
    from kernel_lab import ops

    q, kv, _, _ = random_decode_problem([300, 20], 8, 2, 64, 16, dtype=torch.float32, device="cuda")
    check(run(gpu_ops, q, kv, num_splits=ops.BALANCED), expected(q, kv), torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(32, 8, 128), (8, 1, 64), (16, 16, 256)])
def test_forced_valu_kernel_on_mfma_shapes(gpu_ops, hq, hkv, head_dim, dtype):
    """KL_DECODE_FORCE_VALU=1 runs the VALU kernel (the benchmarks' comparison
    path) on shapes the MFMA kernel normally takes; both must match the oracle."""
    q, kv, _, _ = random_decode_problem([1, 40, 300, 17], hq, hkv, head_dim, 16, dtype=dtype, device="cuda",
                                        poison=float("nan"))
    with _native.decode_switches(force_valu="1"):
        check(run(gpu_ops, q, kv), expected(q, kv), dtype)
        check(run(gpu_ops, q, kv, num_splits=3), expected(q, kv), dtype)
