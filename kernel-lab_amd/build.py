"""Build the kernel_lab native libraries in-tree for MI355X (gfx950).

    python kernel-lab_amd/build.py            # build both libraries
    python kernel-lab_amd/build.py --check    # also compile every HIP source with -Werror
    python kernel-lab_amd/build.py --resource-report profiles/kernel_resources_gfx950.md
                                              # per-kernel registers, spills, occupancy, LDS

Outputs (next to the Python package, so they travel with the source tree):

* ``kernel_lab/libkernel_lab.so`` -- the HIP kernels behind the C-ABI declared in
  ``include/kernel_lab.h``. No PyTorch inside; any FFI can load it.
* ``kernel_lab/_C.so`` -- the PyTorch-ROCm operator registrations
  (``torch.ops.kernel_lab.*``), linked against ``libkernel_lab.so``.

Both link the HIP runtime by its soname (``libamdhip64.so.7``). PyTorch-ROCm
ships its own copy with the same soname and loads it on ``import torch``; the
dynamic loader then binds these libraries to that copy, so one process never
carries two HIP runtimes.

Environment:
  KERNEL_LAB_ARCH   offload target (default gfx950)
  HIPCC             compiler driver (default /opt/rocm/bin/hipcc, else hipcc on PATH)
"""

from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
PKG = HERE / "kernel_lab"
INCLUDE = HERE.parent / "include"

HIP_SOURCES = ["rmsnorm.hip", "paged_decode.hip"]
HOST_SOURCES = ["status.cpp"]

# Packed-FP32 VALU forms are disabled on purpose: scalar and float2 code must
# not be turned into v_pk_*_f32 by the compiler.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    if Path("/opt/rocm/bin/hipcc").exists():
        return "/opt/rocm/bin/hipcc"
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; set HIPCC")
    return found


def _arch() -> str:
    return os.environ.get("KERNEL_LAB_ARCH", "gfx950")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_core(out_dir: Path = PKG, werror: bool = False) -> Path:
    """Compile the HIP kernels and the C-ABI into libkernel_lab.so."""
    out = out_dir / "libkernel_lab.so"
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={_arch()}", *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}"]
    if werror:
        cmd += ["-Wall", "-Werror"]
    cmd += [str(CSRC / s) for s in HIP_SOURCES + HOST_SOURCES]
    cmd += ["-Wl,-soname,libkernel_lab.so", "-o", str(tmp)]
    _run(cmd)
    tmp.replace(out)
    return out


def build_torch(out_dir: Path = PKG) -> Path:
    """Compile torch_bindings.cpp into _C.so (host C++, linked to libkernel_lab.so)."""
    import torch
    from torch.utils import cpp_extension

    out = out_dir / "_C.so"
    tmp = out.with_suffix(".so.tmp")
    includes = cpp_extension.include_paths(device_type="cuda")
    libdirs = [str(Path(torch.__file__).parent / "lib")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C",
        *[f"-I{p}" for p in includes],
        f"-I{INCLUDE}",
        str(CSRC / "torch_bindings.cpp"),
        *[f"-L{p}" for p in libdirs],
        f"-L{out_dir}",
        "-lkernel_lab",
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN",
        "-o",
        str(tmp),
    ]
    _run(cmd)
    tmp.replace(out)
    return out


def check_sources() -> None:
    """Compile-only check of every HIP source with -Wall -Werror (no link)."""
    for src in HIP_SOURCES:
        _run(
            [_hipcc(), f"--offload-arch={_arch()}", *HIP_FLAGS, "-Wall", "-Werror", f"-I{INCLUDE}",
             f"-I{CSRC}", "-c", str(CSRC / src), "-o", os.devnull]
        )


# Fields of the compiler's kernel-resource-usage remarks, in report order.
RESOURCE_FIELDS = [
    ("VGPRs", "VGPRs"),
    ("AGPRs", "AGPRs"),
    ("TotalSGPRs", "SGPRs"),
    ("ScratchSize [bytes/lane]", "scratch B/lane"),
    ("VGPRs Spill", "VGPR spill"),
    ("SGPRs Spill", "SGPR spill"),
    ("Occupancy [waves/SIMD]", "waves/SIMD"),
    ("LDS Size [bytes/block]", "LDS B/block"),
]
_REMARK = re.compile(r"remark:\s+(.*?)\s+\[-Rpass-analysis=kernel-resource-usage\]")


def _short_name(demangled: str) -> str:
    """'void kl::(anonymous namespace)::k<kl::F16, 128>(kl::(anonymous namespace)::A)' -> 'k<F16, 128>'."""
    name = demangled.replace("kl::(anonymous namespace)::", "").replace("kl::", "")
    name = name[5:] if name.startswith("void ") else name
    depth = 0
    for i, ch in enumerate(name):  # cut the parameter list: the first '(' outside template brackets
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            return name[:i]
    return name


def resource_usage(src: str) -> list[dict[str, str]]:
    """Per-kernel register, scratch, occupancy and LDS figures of one HIP source
    as the compiler reports them for the offload target (device code only)."""
    cmd = [_hipcc(), f"--offload-arch={_arch()}", *HIP_FLAGS, "--cuda-device-only", "-c",
           "-Rpass-analysis=kernel-resource-usage", f"-I{INCLUDE}", f"-I{CSRC}", str(CSRC / src), "-o", os.devnull]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stderr[-4000:]}")
    rows: list[dict[str, str]] = []
    for line in proc.stderr.splitlines():
        m = _REMARK.search(line)
        if m is None:
            continue
        key, _, value = m.group(1).partition(":")
        if key == "Function Name":
            rows.append({"mangled": value.strip()})
        elif rows:
            rows[-1][key.strip()] = value.strip()
    filt = shutil.which("c++filt")
    mangled = [r["mangled"] for r in rows]
    names = mangled
    if filt and mangled:
        names = subprocess.run([filt], input="\n".join(mangled), capture_output=True, text=True).stdout.splitlines()
    for row, name in zip(rows, names):
        row["kernel"] = _short_name(name)
    return sorted(rows, key=lambda r: r["kernel"])


def resource_report() -> str:
    """Markdown table of resource_usage over every HIP source."""
    version = subprocess.run([_hipcc(), "--version"], capture_output=True, text=True).stdout.splitlines()
    compiler = next((v.strip() for v in version if v.startswith("HIP version")), "unknown")
    lines = [
        f"# Kernel resources on {_arch()} (compiler report)",
        "",
        "Registers, scratch (spills), occupancy and LDS of every kernel instance the",
        "library builds, from the compiler's kernel-resource-usage remarks. Generated",
        "from the repository root by",
        "",
        f"    python kernel-lab_amd/build.py --resource-report profiles/kernel_resources_{_arch()}.md",
        "",
        "which compiles each source for the device alone with the library's flags and",
        "`-Rpass-analysis=kernel-resource-usage`. `tests/test_resource_report.py`",
        "regenerates it, fails if it differs from this file, and fails if any kernel",
        "uses scratch. gfx950 gives a lane 512 registers (VGPRs + AGPRs, allocated in",
        "blocks of 8) shared by the waves on its SIMD; waves/SIMD is the occupancy",
        "those registers and the LDS leave. SGPR spills live in VGPR lanes, not in",
        "memory.",
        "",
        f"{compiler}",
    ]
    for src in HIP_SOURCES:
        rows = resource_usage(src)
        lines += ["", f"## {src} ({len(rows)} kernels)", "",
                  "| kernel | " + " | ".join(label for _, label in RESOURCE_FIELDS) + " |",
                  "|---|" + "---:|" * len(RESOURCE_FIELDS)]
        for r in rows:
            lines.append(f"| `{r['kernel']}` | " + " | ".join(r.get(key, "?") for key, _ in RESOURCE_FIELDS) + " |")
    return "\n".join(lines) + "\n"


def build(check: bool = False) -> list[Path]:
    if check:
        check_sources()
    return [build_core(), build_torch()]


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--check", action="store_true", help="also compile every HIP source with -Werror")
    parser.add_argument("--resource-report", metavar="PATH", type=Path,
                        help="write the per-kernel register/spill report to PATH and exit (no build)")
    args = parser.parse_args(argv)
    if args.resource_report is not None:
        args.resource_report.write_text(resource_report())
        print(args.resource_report)
        return 0
    for path in build(check=args.check):
        print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
