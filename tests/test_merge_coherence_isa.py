"""The in-kernel split merge's memory ordering, pinned at the instruction level.

A unit split over several workgroups is merged by the last of them to
arrive, inside the decode kernel. The protocol does not use agent-scope
release/acquire fences (on gfx950 they are a write-back and an invalidate of
the whole L2, measured at up to 66 % of a call's time). It relies instead on
the coherence policy of the accesses themselves: every partial is stored with
the `sc1` bit (device-coherent: written through the XCD's non-coherent L2),
each wave waits for its stores to complete before the workgroup barrier, one
lane then adds to the unit's arrival counter with a returning atomic, and the
last arriver reads the partials with `sc1` loads (which do not hit stale L2
lines) issued only after the atomic returned.

This test compiles the decode source for gfx950 (device code only, no GPU)
and checks, in the uniform split kernel that merges in-kernel, that the
encoding the argument depends on is what the compiler emitted: all partial
stores (`buffer_store`) and all merge loads (`buffer_load` not into LDS) carry
`sc1`, the arrival counter is a returning global atomic add, its reset is an
`sc1` store, and no whole-cache fence was added. A compiler change in these
encodings fails here instead of silently weakening the merge.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "kernel-lab_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else shutil.which("hipcc")
KERNEL = "_ZN2kl12_GLOBAL__N_118decode_mfma_kernelINS_3F16ES2_Li128ELi1EEEvNS0_10DecodeArgsE"


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory) -> list[str]:
    if HIPCC is None:
        pytest.skip("hipcc not found")
    out = tmp_path_factory.mktemp("isa") / "paged_decode.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", f"-I{ROOT / 'include'}", f"-I{CSRC}",
           str(CSRC / "paged_decode.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    lines = out.read_text().splitlines()
    start = next(i for i, line in enumerate(lines) if line.startswith(KERNEL + ":"))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    return [line.strip() for line in lines[start:end] if line.startswith("\t") and not line.strip().startswith(";")]


def _ops(asm: list[str], pattern: str) -> list[str]:
    return [line for line in asm if re.match(pattern, line)]


def test_partials_are_stored_device_coherent(kernel_asm):
    stores = _ops(kernel_asm, r"buffer_store_")
    assert stores, "no partial stores found"
    assert all(" sc1" in s for s in stores), [s for s in stores if " sc1" not in s]


def test_merge_loads_are_device_coherent(kernel_asm):
    loads = [ld for ld in _ops(kernel_asm, r"buffer_load_dwordx4") if not ld.endswith(" lds")]
    assert loads, "no merge loads found"
    assert all(" sc1" in ld for ld in loads), [ld for ld in loads if " sc1" not in ld]


def test_arrival_counter_is_a_returning_atomic_add_reset_coherently(kernel_asm):
    adds = _ops(kernel_asm, r"global_atomic_add ")
    assert len(adds) == 1 and " sc0" in adds[0], adds  # sc0 on an atomic: returns the old value
    resets = [s for s in _ops(kernel_asm, r"global_store_dword ") if " sc1" in s]
    assert resets, "the counter reset is not a device-coherent store"


def test_no_whole_cache_fences(kernel_asm):
    assert not _ops(kernel_asm, r"buffer_(wbl2|inv)"), "an L2 write-back or invalidate appeared in the decode kernel"
