"""The C-ABI header is plain C: a C99 program includes it, links the built
library and runs every host-only path (status codes, planners, argument
checks). Nothing here touches a GPU."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from kernel_lab import _native

ROOT = Path(__file__).resolve().parents[1]

PROGRAM = r"""
#include <stdio.h>
#include "kernel_lab.h"

int main(void) {
  int splits = -7;
  size_t ws = 1;
  printf("version %d\n", kl_version());
  printf("ok %s\n", kl_status_string(KL_OK));
  /* Planner: pure host arithmetic with an explicit CU count. */
  int st = kl_paged_decode_plan(KL_DTYPE_F16, 64, 32, 8, 128, 16, 128, 0, 256, &splits, &ws);
  printf("plan64 %d %d %d\n", st, splits, ws > 0);
  st = kl_paged_decode_plan(KL_DTYPE_F16, 64, 128, 8, 128, 16, 128, 0, 256, &splits, &ws);
  printf("plan64g16 %d %d %zu\n", st, splits, ws);
  st = kl_paged_decode_plan(KL_DTYPE_F16, 64, 32, 8, 128, 16, 256, 0, 256, &splits, &ws);
  printf("plan64long %d %d %d\n", st, splits, ws > 0);
  st = kl_paged_decode_plan(KL_DTYPE_F16, 1, 32, 8, 128, 16, 256, 0, 256, &splits, &ws);
  printf("plan1 %d %d %d\n", st, splits, ws > 0);
  st = kl_paged_decode_plan(KL_DTYPE_F16, 4, 32, 8, 128, 16, 256, 0, 256, &splits, &ws);
  printf("plan4 %d %d %d\n", st, splits, ws > 0);
  st = kl_paged_decode_plan(KL_DTYPE_F16, 64, 32, 8, 128, 16, 256, KL_SPLITS_BALANCED, 256, &splits, &ws);
  printf("planbal %d %d %d\n", st, splits, ws > 0);
  size_t cws = 0;
  st = kl_cascade_decode_plan(KL_DTYPE_BF16, 64, 32, 8, 128, 16, 256, 32, 256, &cws);
  printf("cascade %d %d\n", st, cws > 0);
  /* Argument errors are reported before any launch. */
  st = kl_paged_decode_plan(KL_DTYPE_F16, 2, 3, 2, 128, 16, 4, 0, 256, &splits, &ws);
  printf("badgroup %d %s\n", st, kl_last_error());
  st = kl_rms_norm(KL_DTYPE_BF16, 0, 0, 0, 0, 0, 4096, 4096, 1e-6f, 0);
  printf("norows %d\n", st);
  st = kl_rms_norm(KL_DTYPE_BF16, 0, 0, 0, 0, 4, 4096, 4096, 1e-6f, 0);
  printf("nullptr %d\n", st);
  st = kl_paged_decode_attention_fp8(KL_DTYPE_F32, 0, 0, 0, 0, 0, 0, 0, 0, 1, 8, 2, 128, 16, 4, 4, 0.1f, 0, 0, 0, 0);
  printf("fp8f32 %d\n", st);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None or not _native.loaded(), reason="needs gcc and the built library")
def test_header_compiles_as_c99_and_links(tmp_path):
    src = tmp_path / "abi.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "abi"
    lib_dir = _native.CORE_PATH.parent
    subprocess.run(
        ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{ROOT / 'include'}", str(src),
         f"-L{lib_dir}", "-lkernel_lab", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)],
        check=True,
    )
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()
    got = dict(line.split(" ", 1) for line in out)
    assert int(got["version"]) >= 100
    assert got["ok"] == "success"
    assert got["plan64"] == "0 0 1"  # a full batch: balanced, the even cut decided on the device
    st, splits, ws = got["plan64g16"].split()
    assert st == "0" and splits == "1" and int(ws) == 0  # 16 heads per workgroup, short table: one uniform split
    assert got["plan64long"] == "0 0 1"  # a long table on a full batch: balanced
    assert got["plan1"] == "0 32 1"  # one sequence: 32 uniform splits of 8 pages
    assert got["plan4"] == "0 0 1"  # a few sequences: balanced schedule
    assert got["planbal"] == "0 0 1"
    assert got["cascade"] == "0 1"
    assert got["badgroup"].startswith("1 ") and "multiple" in got["badgroup"]
    assert got["norows"] == "0"
    assert got["nullptr"] == "1"
    assert got["fp8f32"] == "2"
