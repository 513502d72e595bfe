"""The committed per-kernel register/spill report is current, and no kernel
spills to scratch.

The report (profiles/kernel_resources_gfx950.md) is the compiler's
kernel-resource-usage remarks for every kernel instance the library builds.
This test compiles the device code again (about a minute, no GPU), compares
the result with the committed file, and checks every row: a kernel that
needs scratch memory has spilled registers to HBM, which costs the decode
and RMSNorm kernels their bandwidth. SGPR spills are allowed: the compiler
keeps them in VGPR lanes, not in memory.
"""

from __future__ import annotations

import importlib.util
import shutil
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REPORT = ROOT / "profiles" / "kernel_resources_gfx950.md"
BUILD = ROOT / "kernel-lab_amd" / "build.py"

pytestmark = pytest.mark.skipif(
    shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc not installed"
)


def _build_module():
    spec = importlib.util.spec_from_file_location("kernel_lab_build", BUILD)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def _rows(text: str) -> list[dict[str, str]]:
    rows, header = [], None
    for line in text.splitlines():
        if line.startswith("| kernel |"):
            header = [c.strip() for c in line.strip("|").split("|")]
        elif line.startswith("| `") and header:
            rows.append(dict(zip(header, (c.strip().strip("`") for c in line.strip("|").split("|")))))
    return rows


@pytest.fixture(scope="module")
def regenerated() -> str:
    return _build_module().resource_report()


def test_report_matches_the_sources(regenerated):
    committed = REPORT.read_text()
    assert regenerated == committed, (
        "profiles/kernel_resources_gfx950.md is stale; regenerate it with "
        "`python kernel-lab_amd/build.py --resource-report profiles/kernel_resources_gfx950.md`"
    )


def test_no_kernel_spills_to_scratch(regenerated):
    rows = _rows(regenerated)
    assert len(rows) > 100, "expected every decode and RMSNorm instance in the report"
    for r in rows:
        assert r["scratch B/lane"] == "0" and r["VGPR spill"] == "0", f"{r['kernel']} spills: {r}"
        assert int(r["VGPRs"]) + int(r["AGPRs"]) <= 512, r


def test_headline_kernels_are_listed(regenerated):
    names = {r["kernel"] for r in _rows(regenerated)}
    for kernel in ("decode_mfma_balanced_kernel<F16, F16, 128, 1, 2>", "rms_norm_reg_kernel<BF16, 8, 2, true>",
                   "decode_mfma_paired_kernel<F16, F16, 128, 1>", "rms_norm_staged_kernel<BF16, 8, true>"):
        assert kernel in names, kernel
