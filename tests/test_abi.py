"""The C-ABI library: it loads, exports every symbol include/kernel_lab.h
declares, and its host-only paths (status codes, argument checks, the split
planner) behave as documented. Nothing here launches a kernel."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from kernel_lab import _native, ops

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kernel_lab.h"

pytestmark = pytest.mark.skipif(not _native.loaded(), reason=_native.why_unavailable())


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    assert "kl_rms_norm" in names and "kl_paged_decode_attention" in names and "kl_paged_decode_plan" in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.CORE_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in kernel_lab.h but not exported"


def test_python_signatures_cover_the_header():
    assert set(declared_functions()) == set(_native.SIGNATURES)


def test_status_strings():
    lib = _native.core()
    assert lib.kl_status_string(0) == b"success"
    assert b"argument" in lib.kl_status_string(1)
    assert b"unknown" in lib.kl_status_string(99)
    assert lib.kl_version() >= 100


def test_rms_norm_argument_errors_need_no_gpu():
    lib = _native.core()
    # rows == 0 is a successful no-op, even with null pointers.
    assert lib.kl_rms_norm(1, None, None, None, None, 0, 4096, 4096, 1e-6, None) == 0
    assert lib.kl_rms_norm(1, None, None, None, None, 4, 4096, 4096, 1e-6, None) == 1
    assert b"non-null" in lib.kl_last_error()
    assert lib.kl_rms_norm(1, 16, 16, None, 16, 4, 4096, 100, 1e-6, None) == 1
    assert b"stride" in lib.kl_last_error()
    assert lib.kl_rms_norm(1, 16, 16, None, 16, -1, 4096, 4096, 1e-6, None) == 1


def test_decode_argument_errors_need_no_gpu():
    lib = _native.core()
    # batch == 0: no-op.
    assert lib.kl_paged_decode_attention(1, *([None] * 6), 0, 32, 8, 128, 16, 256, 256, 0.1, 0, None, 0, None) == 0
    # Group not a divisor.
    assert lib.kl_paged_decode_attention(1, *([None] * 6), 2, 3, 2, 32, 16, 4, 4, 0.1, 0, None, 0, None) == 1
    assert b"multiple" in lib.kl_last_error()
    # Unsupported head_dim.
    assert lib.kl_paged_decode_attention(1, *([None] * 6), 2, 4, 2, 24, 16, 4, 4, 0.1, 0, None, 0, None) == 2


@pytest.mark.parametrize(
    ("batch", "hkv", "max_pages", "cus", "want"),
    [
        (64, 8, 256, 256, 1),  # 512 units already fill 256 CUs
        (32, 8, 256, 256, 1),  # 256 units: one per CU
        (1, 8, 256, 256, 32),  # one sequence: splits keep >= 8 pages
        (1, 8, 64, 256, 8),
        (2, 8, 256, 256, 16),  # several sequences: splits keep >= 16 pages
        (8, 8, 256, 256, 4),
        (8, 8, 2048, 256, 4),
        (1, 1, 3, 256, 1),  # a 3-page table is one split
        (1, 1, 8192, 256, 64),  # capped at 64 splits
        (64, 1, 512, 256, 4),
    ],
)
def test_planner_fills_the_device(batch, hkv, max_pages, cus, want):
    """Uniform-split rule (fp32 takes it at every size)."""
    splits, ws = ops.plan_decode(torch.float32, batch, hkv * 4, hkv, 128, 16, max_pages, 0, cus)
    assert splits == want
    if splits > 1:
        assert ws >= batch * hkv * 4 * splits * (128 + 1) * 4
    else:
        assert ws == 0


@pytest.mark.parametrize(
    ("batch", "hkv", "hq", "max_pages", "balanced"),
    [
        (64, 8, 32, 255, True),  # full batch, short table: balanced (the even cut is decided on the device)
        (32, 8, 32, 128, True),
        (64, 8, 32, 256, True),
        (256, 8, 32, 64, True),
        (32, 8, 32, 4096, True),  # 128 pair units: one 8-wave workgroup per CU, two segments each
        (64, 8, 128, 255, False),  # 16 heads per workgroup: split units need the merge launch; short table: uniform
        (64, 8, 128, 256, True),  # ... long table: balanced
        (1024, 16, 64, 8192, False),  # balanced workspace would exceed 16 MiB: uniform
        (8, 8, 32, 256, True),  # fewer units than CUs: balanced at any table length
        (2, 8, 32, 32, True),
        (64, 1, 4, 512, True),
        (1, 8, 32, 32, False),  # one sequence cannot be skewed: uniform splits
        (1, 1, 4, 2048, False),
    ],
)
def test_planner_balances_uneven_batches_by_default(batch, hkv, hq, max_pages, balanced):
    """fp16/bf16: pages are balanced across sequences on the device (reported
    as 0 splits, with a workspace of partial slots) when the units do not
    fill the device, and on full batches, where one long sequence among short
    ones would otherwise set the time. A full batch gets one workgroup per
    list unit: on an even batch that is one uniform split's cut, which the
    kernel detects from seq_lens. Full batches whose split units could not be
    merged in the kernel (more than 8 query heads per workgroup) keep one
    uniform split on short tables."""
    splits, ws = ops.plan_decode(torch.float16, batch, hq, hkv, 128, 16, max_pages, 0, 256)
    if balanced:
        assert splits == 0 and 0 < ws <= 16 << 20
        units = batch * hkv  # one head group: at most 16 query heads per KV head here
        paired = hkv % 2 == 0 and (units >= 512 or units // 2 * max_pages >= 256 * 128 and units // 2 * 16 >= 256)
        lunits = units // 2 if paired else units
        if units >= 256 and lunits >= 256:  # one workgroup per list unit, a slot per workgroup and unit
            grid = min(lunits, -(-lunits * max_pages // 8))
            slots = (grid + lunits) * (2 if paired else 1)
            heads = min(hq // hkv, 16)
            assert ws == _align(slots * heads * 128 * 4) + _align(slots * heads * 4)
    elif batch == 1:
        # The uniform rule with >= 8 pages per split, at most 64 splits.
        assert splits == min(-(-256 // hkv), -(-max_pages // 8), 64) and ws > 0
    else:
        assert splits == 1 and ws == 0


@pytest.mark.parametrize(("batch", "hkv", "max_pages"), [(64, 8, 256), (32, 8, 256), (128, 8, 64), (64, 1, 512)])
def test_balanced_planner_on_request(batch, hkv, max_pages):
    """KL_DECODE_BALANCE_ALWAYS=1 gives every fp16/bf16 batch the balanced
    schedule. With an even KV head count and units >= 2 x CUs the list runs in
    KV-head pairs, with a partial slot per half; a full batch gets one
    workgroup per list unit."""
    with _native.decode_switches(balance_always="1"):
        splits, ws = ops.plan_decode(torch.float16, batch, hkv * 4, hkv, 128, 16, max_pages, 0, 256)
    units = batch * hkv
    long_pairs = units // 2 * max_pages >= 256 * 128 and units // 2 * 16 >= 256
    paired = hkv % 2 == 0 and (units >= 512 or long_pairs)
    lunits = units // 2 if paired else units
    floor = lunits if units >= 256 and lunits >= 256 else 256 if paired else max(256, units)
    grid = min(floor, -(-lunits * max_pages // 8))
    slots = (grid + lunits) * (2 if paired else 1)
    assert splits == 0 and ws == _align(slots * 4 * 128 * 4) + _align(slots * 4 * 4)
    with _native.decode_switches(balance_always="0"):
        uniform = ops.plan_decode(torch.float16, batch, hkv * 4, hkv, 128, 16, max_pages, 0, 256)[0]
    assert uniform >= 1 if units >= 256 else uniform == 0  # fewer units than CUs: balanced regardless


def _align(n: int) -> int:
    return -(-n // 256) * 256


@pytest.mark.parametrize(
    ("batch", "hkv", "max_pages", "paired"),
    [
        (8, 8, 2048, True),  # 32 pair units x 2048 pages: 256 pages per workgroup half, 8 segments each
        (8, 8, 8192, True),
        (16, 8, 1024, True),
        (8, 8, 1024, True),  # exactly 128 pages per half
        (8, 8, 1023, False),
        (8, 8, 256, False),  # 32 pages per half: the 8-wave start costs more than pairing gains
        (2, 8, 8192, False),  # 8 pair units: 32 segments each
        (12, 2, 8192, False),  # 12 pair units: more than 16 segments each
        (8, 1, 32768, False),  # one KV head: nothing to pair
        (2, 1, 2048, False),  # at most 64 workgroups per list unit
        (2, 8, 256, False),  # 16 short segments per unit: cut 8 ways instead
        (3, 8, 128, False),
        (2, 8, 512, False),  # 32-page segments: 16 of them
        (3, 8, 336, False),  # 24 units, 11 segments of 31 pages: never more workgroups than before the cut
    ],
)
def test_planner_pairs_long_contexts_of_small_batches(batch, hkv, max_pages, paired):
    """Fewer units than CUs (balanced by default): the list runs in KV-head
    pairs when every workgroup half gets >= 128 pages and a pair unit at most
    16 segments. The workspace is exact: a partial slot per list workgroup and
    list unit, two per slot when paired; a list unit takes at most 64
    workgroups."""
    splits, ws = ops.plan_decode(torch.float16, batch, hkv * 4, hkv, 128, 16, max_pages, 0, 256)
    units = batch * hkv
    lunits = units // 2 if paired else units
    grid = min(256, -(-lunits * max_pages // 8), lunits * 64)
    segments = -(-grid // lunits)
    if not paired and segments > 8 and lunits * 8 >= 128 and max_pages < 32 * segments:
        grid = min(grid, lunits * max(8, -(-max_pages // 32)))  # units merged in the kernel: at most 8 short segments
    slots = (grid + lunits) * (2 if paired else 1)
    assert splits == 0
    assert ws == _align(slots * 4 * 128 * 4) + _align(slots * 4 * 4)


def test_requested_balanced_schedule_at_any_batch():
    """KL_SPLITS_BALANCED (-1) picks the balanced schedule whatever the planner
    default; the VALU path (fp32) takes the planner's uniform splits."""
    with _native.decode_switches(balance_always="0"):
        assert ops.plan_decode(torch.float16, 64, 32, 8, 128, 16, 256, 0, 256)[0] == 1
        splits, ws = ops.plan_decode(torch.float16, 64, 32, 8, 128, 16, 256, ops.BALANCED, 256)
    units = 64 * 8  # paired: 256 workgroups and 256 pair units, two slots each
    assert splits == 0 and ws >= (256 + units // 2) * 2 * 4 * (128 + 1) * 4
    assert ops.plan_decode(torch.float32, 64, 32, 8, 128, 16, 256, ops.BALANCED, 256) == ops.plan_decode(
        torch.float32, 64, 32, 8, 128, 16, 256, 0, 256
    )
    with pytest.raises(ValueError):
        ops.plan_decode(torch.float16, 2, 4, 2, 32, 16, 4, -2)


@pytest.mark.parametrize(("max_pages", "balanced"), [(4194239, True), (4194240, False)])
def test_balanced_schedule_needs_list_lengths_in_32_bits(max_pages, balanced):
    """The balanced kernel sums 64 sequences' list lengths (each unit's pages
    plus a charge of at most 64 positions) in 32-bit lanes: 64 x 8 units x
    (max_pages + 64) must stay below 2^31, or the planner keeps uniform
    splits, also when the balanced schedule is requested."""
    for requested in (0, ops.BALANCED):
        splits, ws = ops.plan_decode(torch.float16, 64, 32, 8, 128, 16, max_pages, requested, 256)
        if balanced:
            assert splits == 0 and ws > 0
        else:
            assert splits >= 1


@pytest.mark.parametrize(("requested", "max_pages", "want"), [(1, 5, 1), (2, 5, 2), (3, 5, 3), (5, 5, 5), (64, 5, 5), (4, 7, 4), (5, 7, 4)])
def test_requested_splits_normalise_like_the_original(requested, max_pages, want):
    """pages_per_split = cdiv(max_pages, S); S = cdiv(max_pages, pages_per_split)
    (kernel_lab/triton_kernels/paged_attention.py:210-211)."""
    splits, _ = ops.plan_decode(torch.float32, 2, 4, 2, 32, 16, max_pages, requested, 256)
    assert splits == want


@pytest.mark.parametrize("dtype", [-1, 3, 7, 1 << 30])
def test_out_of_range_dtypes_are_rejected(dtype):
    """A C caller may pass any int as kl_dtype; the library checks it (the
    enum is int-based in C++, so such a value is well-defined there too)."""
    lib = _native.core()
    splits, ws = ctypes.c_int(-5), ctypes.c_size_t(7)
    assert lib.kl_paged_decode_plan(dtype, 2, 8, 2, 128, 16, 4, 0, 256, ctypes.byref(splits), ctypes.byref(ws)) == 2
    assert b"dtype" in lib.kl_last_error()
    assert lib.kl_rms_norm(dtype, 16, 16, None, 16, 4, 4096, 4096, 1e-6, None) == 2
    assert lib.kl_paged_decode_attention(dtype, 16, 16, 16, 16, 16, 16, 2, 8, 2, 128, 16, 4, 4, 0.1, 0, None, 0,
                                         None) == 2


def test_planner_rejects_bad_shapes():
    with pytest.raises(ValueError, match="multiple"):
        ops.plan_decode(torch.float16, 2, 3, 2, 128, 16, 4)
    with pytest.raises(ValueError):
        ops.plan_decode(torch.float16, 2, 4, 2, 24, 16, 4)


def test_one_hip_runtime_in_process():
    """The libraries bind to the HIP runtime PyTorch already loaded."""
    maps = Path("/proc/self/maps").read_text()
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(paths) <= 1, paths


def test_planner_choices_fit_the_no_allocation_array():
    """kl_paged_decode_attention_noalloc holds 16 MiB of split workspace per
    device; every plan the planner makes by itself (num_splits 0) on MI355X's
    256 CUs must fit it, across batch sizes, GQA layouts, head dims, context
    widths and dtypes."""
    lib = _native.core()
    splits, ws = ctypes.c_int(0), ctypes.c_size_t(0)
    worst = (0, None)
    for code in (0, 1, 2):
        for batch in (1, 2, 3, 7, 8, 16, 31, 32, 33, 63, 64, 100, 127, 128, 255, 256, 257, 511, 512, 1024):
            for hq, hkv in ((32, 8), (32, 1), (64, 8), (8, 1), (16, 16), (40, 5), (64, 2), (128, 8), (64, 1), (96, 4)):
                for d in (32, 64, 128, 256):
                    for max_pages in (1, 32, 256, 2048, 8192):
                        st = lib.kl_paged_decode_plan(code, batch, hq, hkv, d, 16, max_pages, 0, 256,
                                                      ctypes.byref(splits), ctypes.byref(ws))
                        if st != 0:
                            continue  # shapes the dtype has no kernel for (fp32 head_dim 256 x 64 lanes ...)
                        if ws.value > worst[0]:
                            worst = (ws.value, (code, batch, hq, hkv, d, max_pages))
    assert 0 < worst[0] <= 16 << 20, worst


def test_switches_are_read_once_and_on_reload(monkeypatch):
    """The library reads its KL_DECODE_* switches once per process: a change to
    the environment alone leaves the plan as it was (the last plan is also
    remembered per thread, and must not outlive the switches), and
    kl_paged_decode_reload_options() applies it."""
    args = (torch.float16, 64, 32, 8, 128, 16, 256, 0, 256)  # full batch, 256 pages: balanced
    assert ops.plan_decode(*args)[0] == 0
    monkeypatch.setenv("KL_DECODE_BALANCE_ALWAYS", "0")
    assert ops.plan_decode(*args)[0] == 0, "the environment was re-read without a reload"
    lib = _native.core()
    try:
        assert lib.kl_paged_decode_reload_options() == 0
        assert ops.plan_decode(*args)[0] == 1
    finally:
        monkeypatch.delenv("KL_DECODE_BALANCE_ALWAYS")
        lib.kl_paged_decode_reload_options()
    assert ops.plan_decode(*args)[0] == 0


def test_remembered_plan_follows_its_arguments():
    """Alternating two shapes returns each one's own plan every time."""
    a = (torch.float16, 64, 32, 8, 128, 16, 256, 0, 256)
    b = (torch.float16, 8, 32, 8, 128, 16, 32, 0, 256)
    first = ops.plan_decode(*a), ops.plan_decode(*b)
    for _ in range(3):
        assert (ops.plan_decode(*a), ops.plan_decode(*b)) == first
    assert first[0] != first[1]
