"""Headline benchmark: achieved HBM GB/s of one decode-layer step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is the hot path once over synthetic data already resident in HBM:

1. paged decode attention, Llama-3-8B GQA (32 query heads, 8 KV heads,
   head_dim 128, 16-token pages), fp16, batch 64, context 4096, NaN-poisoned
   spare pages, split count from the planner;
2. fused residual-add + RMSNorm, 4096 x 8192, bf16, residual updated in place.

The decode streams 1.07 GB of KV cache per step, which evicts the 256 MB
Infinity Cache, so the RMSNorm's 128 MB of inputs come from HBM every step
too. Outputs are checked against the CPU oracle before anything is timed.

Four live passes, after W warm-up steps:
* throughput pass: the K steps back to back with nothing between the kernels,
  timed between two device synchronisations;
* kernel pass: the same K steps with a HIP event pair on the launch stream
  around each operator. Measured on MI355X, an event's timestamp packet
  between two kernels leaves the GPU idle ~5 us (16 us per step, 7 %), so
  events stay out of the throughput pass; the pair around one launch also
  spans its dispatch, 2-4 % above the kernel's traced duration;
* dominant-kernel pass: K launches of the dominant kernel (decode) back to
  back inside one event pair on the launch stream; per launch this is the
  kernel's duration plus the gap between two launches, and it gives the
  roofline figure;
* flushed dominant-kernel pass: K launches of the dominant kernel, each after
  a read of a 1 GiB buffer (so no input is left in the 256 MB Infinity Cache,
  and the first K/V loads miss the translation caches as a cold call's do),
  each inside its own event pair; the median is reported beside the
  back-to-back figure (`us_per_launch_flushed`).

One JSON line goes to stdout:
* value: algorithmic bytes of the K steps / wall time of the throughput pass
  (GB/s);
* kernels: per-operator HIP-event time (kernel pass), GB/s and fraction of the
  8 TB/s peak;
* roofline: the dominant kernel (decode) against HBM peak, with its HBM
  traffic per launch measured in this run: two child passes of this script
  under `rocprofv3 --pmc` (FETCH_SIZE, then WRITE_SIZE, one counter per pass,
  each under its own kill timer) run two decode steps and a 1 GiB elementwise
  copy, and each counter is scaled by what it reads for the copy, whose bytes
  are known (on gfx950 FETCH_SIZE reads half of them); null, with the reason,
  when a pass fails or --no-counters is given;
* cpu_baseline: the CPU oracle (float32 PyTorch restatement of the original's
  reference.py) on a bounded sample of the same workload, on this host's
  cores (threads = the process's CPU affinity), with the CPU model and the
  torch version.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import platform
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "kernel-lab_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

from kernel_lab import _native  # noqa: E402
from kernel_lab.bench.roofline import MI355X, decode_attention_work, lookup, rms_norm_work  # noqa: E402
from kernel_lab.kv_cache import device_decode_problem  # noqa: E402

METRIC = "achieved HBM GB/s + % of peak: paged decode (B=64, ctx 4k) and add-RMSNorm"
DECODE = {"batch": 64, "ctx": 4096, "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128, "page_size": 16}
RMS = {"tokens": 4096, "hidden": 8192}
COPY_BYTES = 1 << 30  # calibration copy: reads and writes this many bytes per dispatch
FLUSH_BYTES = 1 << 30  # read before each launch of the flushed pass (> the 256 MB Infinity Cache)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def counter_probe(device: torch.device) -> None:
    """Child mode (under rocprofv3 --pmc): two decode steps of the workload and
    two 1 GiB elementwise copies, the counters' calibration kernel."""
    lens, q, kv, _, _, _ = build_inputs(device)
    out = torch.empty_like(q)
    for _ in range(2):
        torch.ops.kernel_lab.paged_decode_attention(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens,
                                                    DECODE["head_dim"] ** -0.5)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.add(src, 0.0, out=dst)  # one read and one write of every byte
    torch.cuda.synchronize()


def _counter_means(csv_path: Path, counter: str) -> dict[str, float]:
    """Mean value per dispatch of `counter` for the decode kernel and for the
    calibration copy (the two largest elementwise dispatches: the input
    set-up runs smaller elementwise kernels too)."""
    decode: list[float] = []
    elementwise: list[float] = []
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name = row.get("Kernel_Name", "")
            if "decode_mfma" in name:
                decode.append(float(row["Counter_Value"]))
            elif "elementwise" in name:
                elementwise.append(float(row["Counter_Value"]))
    out = {}
    if decode:
        out["decode"] = sum(decode) / len(decode)
    if len(elementwise) >= 2:
        out["copy"] = sum(sorted(elementwise)[-2:]) / 2
    return out


def measure_traffic(timeout_s: int = 150) -> tuple[float | None, str]:
    """HBM bytes per decode launch from this run's counters: one rocprofv3 --pmc
    pass per counter over a child run of this script, each counter scaled by
    its reading for the 1 GiB copy. Returns (bytes, how it was obtained)."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    per_launch = 0.0
    notes = []
    with tempfile.TemporaryDirectory(prefix="kl_pmc_") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", counter, "--kernel-trace", "-f", "csv",
                   "-d", tmp, "-o", counter, "--", sys.executable, str(Path(__file__).resolve()), "--counter-probe"]
            log(f"counter pass: {counter}")
            proc = subprocess.run(cmd, capture_output=True, text=True, cwd=tmp)
            files = list(Path(tmp).rglob(f"{counter}_counter_collection.csv"))
            if not files:
                return None, f"{counter} pass produced no counters (exit {proc.returncode}): {proc.stderr[-200:]}"
            means = _counter_means(files[0], counter)
            if "decode" not in means or "copy" not in means:
                return None, f"{counter} pass: kernels missing from the counter file"
            scale = COPY_BYTES / (means["copy"] * 1024)  # counters count KiB
            per_launch += means["decode"] * 1024 * scale
            notes.append(f"{counter} {means['decode']:.1f} KiB/launch x {scale:.3f} (copy-calibrated)")
    return per_launch, "; ".join(notes)


def build_inputs(device: torch.device):
    lens = [DECODE["ctx"]] * DECODE["batch"]
    q, kv = device_decode_problem(
        lens, DECODE["num_q_heads"], DECODE["num_kv_heads"], DECODE["head_dim"], DECODE["page_size"],
        dtype=torch.float16, device=device, seed=0,
    )
    gen = torch.Generator(device=device).manual_seed(1)
    shape = (RMS["tokens"], RMS["hidden"])
    x = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
    res = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(RMS["hidden"], generator=gen, device=device)).to(torch.bfloat16)
    return lens, q, kv, x, res, w


def check_outputs(q, kv, out, x, res_before, res_after, w, y) -> dict:
    """Compare a sample of every output with the CPU oracle before timing."""
    from oracle import reference as ref

    rows = [0, 17, 63]
    sub_bt = kv.block_table[rows].cpu()
    want32 = ref.paged_decode_attention(
        q[rows].cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), sub_bt, kv.seq_lens[rows].cpu(),
        DECODE["head_dim"] ** -0.5,
    )
    want = want32.to(q.dtype)
    got = out[rows].cpu()
    dec_err = (got.float() - want.float()).abs().max().item()
    torch.testing.assert_close(got, want, atol=2e-3, rtol=2e-3)
    # Distance to the unrounded float32 result in fp16 ulps of that result
    # (0.5 is a correctly rounded output of the same float32 value).
    _, e = torch.frexp(want32.double().abs())
    ulp = torch.pow(2.0, torch.clamp(e.double() - 11, min=-24))
    dec_ulps = ((got.double() - want32.double()).abs() / ulp).max().item()
    sel = torch.tensor([0, 1, 2047, 4095])
    ref_y, ref_res = ref.fused_add_rms_norm(x[sel].cpu(), res_before[sel].cpu(), w.cpu())
    assert torch.equal(res_after[sel].cpu(), ref_res), "residual not bit-exact"
    rms_err = (y[sel].cpu().float() - ref_y.float()).abs().max().item()
    torch.testing.assert_close(y[sel].cpu(), ref_y, atol=1.6e-2, rtol=1.6e-2)
    return {"decode_max_abs_err": dec_err, "decode_max_err_ulps_vs_fp32": round(dec_ulps, 3),
            "rmsnorm_max_abs_err": rms_err}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(q, kv, x, res, w, dec_bytes: float, rms_bytes: float, budget_s: float) -> dict:
    """The CPU oracle on a bounded sample of the step, on this host's cores:
    threads = the CPUs this process may run on."""
    from oracle import reference as ref

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    qc = q[:4].cpu()
    kc, vc = kv.k_cache.cpu(), kv.v_cache.cpu()
    btc, lc = kv.block_table[:4].cpu(), kv.seq_lens[:4].cpu()
    xc, rc, wc = x[:256].cpu(), res[:256].cpu(), w.cpu()

    def timed(fn, budget):
        fn()  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return el / n, n

    t_dec, n_dec = timed(lambda: ref.paged_decode_attention(qc, kc, vc, btc, lc, DECODE["head_dim"] ** -0.5), budget_s / 2)
    t_rms, n_rms = timed(lambda: ref.fused_add_rms_norm(xc, rc, wc, 1e-6), budget_s / 2)
    # Extrapolate the sample to one whole step: 4 of 64 sequences, 256 of 4096 rows.
    step_s = t_dec * (DECODE["batch"] / 4) + t_rms * (RMS["tokens"] / 256)
    return {
        "value": round((dec_bytes + rms_bytes) / step_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"oracle/reference.py (float32 PyTorch CPU) on 4 of 64 decode sequences ({n_dec} runs, "
            f"{t_dec * 1e3:.1f} ms each) and 256 of 4096 RMSNorm rows ({n_rms} runs, {t_rms * 1e3:.2f} ms each), "
            f"extrapolated to one step of the same workload ({step_s * 1e3:.1f} ms)"
        ),
        "decode_gbps": round(dec_bytes / (t_dec * DECODE["batch"] / 4) / 1e9, 3),
        "rmsnorm_gbps": round(rms_bytes / (t_rms * RMS["tokens"] / 256) / 1e9, 3),
        "cpu_model": _cpu_model(),
        "torch": torch.__version__,
    }


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--only", choices=["decode", "rmsnorm"], help="time one operator (for profiling runs)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-oracle timing")
    parser.add_argument("--no-counters", action="store_true", help="skip the rocprofv3 traffic passes")
    parser.add_argument("--counter-probe", action="store_true", help=argparse.SUPPRESS)
    args = parser.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): the decode and "
            "RMSNorm kernels need no collectives (decode shards by batch, KV head or page range; RMSNorm by "
            "rows), and this build measures one GPU's share of the workload.",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("No GPU device: bench.py needs an MI355X.", file=sys.stderr)
        return 2
    if not _native.loaded():
        print(f"kernel_lab native libraries missing: {_native.why_unavailable()}", file=sys.stderr)
        return 2

    device = torch.device("cuda:0")
    if args.counter_probe:
        counter_probe(device)
        return 0
    name = torch.cuda.get_device_name(device)
    peak = lookup(name) or lookup(torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]) or MI355X
    log(f"device: {name}; peak {peak.dram_gbps} GB/s ({peak.name})")

    lens, q, kv, x, res, w = build_inputs(device)
    out = torch.empty_like(q)
    y = torch.empty_like(x)
    scale = DECODE["head_dim"] ** -0.5
    op_dec = torch.ops.kernel_lab.paged_decode_attention
    op_rms = torch.ops.kernel_lab.fused_add_rms_norm

    dec_work = decode_attention_work(lens, DECODE["num_q_heads"], DECODE["num_kv_heads"], DECODE["head_dim"], 2)
    rms_work = rms_norm_work(RMS["tokens"], RMS["hidden"], 2, fused_residual=True)
    do_dec = args.only in (None, "decode")
    do_rms = args.only in (None, "rmsnorm")

    # Correctness first (as the original harness does: a wrong result is never timed).
    res_before = res.clone()
    op_dec(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, scale)
    op_rms(y, x, res, w, 1e-6)
    torch.cuda.synchronize()
    errors = check_outputs(q, kv, out, x, res_before, res, w, y)
    del res_before
    log(f"outputs match the oracle: {errors}")

    def step():
        if do_dec:
            op_dec(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, scale)
        if do_rms:
            op_rms(y, x, res, w, 1e-6)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Throughput pass: nothing between the kernels.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    log(f"throughput pass: {args.steps} steps in {wall * 1e3:.2f} ms")

    # Kernel pass: HIP events on the launch stream around each operator.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    stream = torch.cuda.current_stream()
    for i in range(args.steps):
        ev[i][0].record(stream)
        if do_dec:
            op_dec(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, scale)
        ev[i][1].record(stream)
        if do_rms:
            op_rms(y, x, res, w, 1e-6)
        ev[i][2].record(stream)
    torch.cuda.synchronize()
    log(f"kernel pass: {args.steps} steps")

    dec_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    rms_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / args.steps
    step_bytes = (dec_work.bytes if do_dec else 0) + (rms_work.bytes if do_rms else 0)
    value = step_bytes * args.steps / wall / 1e9

    def kernel_entry(work, ms):
        gbps = work.bytes / (ms * 1e-3) / 1e9
        return {"us": round(ms * 1e3, 2), "gbps": round(gbps, 1), "frac_of_peak": round(gbps / peak.dram_gbps, 4)}

    kernels = {}
    if do_dec:
        kernels["paged_decode_attention"] = kernel_entry(dec_work, dec_ms) | {"bytes": dec_work.bytes}
    if do_rms:
        kernels["fused_add_rms_norm"] = kernel_entry(rms_work, rms_ms) | {"bytes": rms_work.bytes}
    for op, entry in kernels.items():
        if entry["frac_of_peak"] > 0.92:
            # The reference runbook's sanity check (docs/gpu-runbook.md:75-76).
            log(f"warning: {op} above 92 % of peak: check the byte count and cache residency")

    dom_work = dec_work if do_dec else rms_work
    dom_op = (lambda: op_dec(out, q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, scale)) if do_dec else (
        lambda: op_rms(y, x, res, w, 1e-6))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        dom_op()
    e1.record(stream)
    torch.cuda.synchronize()
    dom_ms = e0.elapsed_time(e1) / args.steps
    log(f"dominant-kernel pass: {args.steps} launches, {dom_ms * 1e3:.2f} us each")
    achieved = dom_work.bytes / (dom_ms * 1e-3) / 1e9

    # Flushed pass: a 1 GiB read before every launch, an event pair around each.
    flush = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=device)
    flushed = []
    for _ in range(args.steps):
        flush.sum()
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record(stream)
        dom_op()
        f1.record(stream)
        f1.synchronize()
        flushed.append(f0.elapsed_time(f1))
    del flush
    flushed.sort()
    flushed_ms = flushed[len(flushed) // 2]
    log(f"flushed dominant-kernel pass: {args.steps} launches, median {flushed_ms * 1e3:.2f} us")
    traffic, traffic_note = None, "not measured (--no-counters or a single-operator run)"
    if do_dec and not args.no_counters:
        traffic, traffic_note = measure_traffic()
    roofline = {
        "kernel": "paged_decode_attention" if do_dec else "fused_add_rms_norm",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": peak.dram_gbps,
        "unit": "GB/s",
        "frac": round(achieved / peak.dram_gbps, 4),
        "us_per_launch": round(dom_ms * 1e3, 2),
        # A 1 GiB read before each launch, an event pair around it, median.
        "us_per_launch_flushed": round(flushed_ms * 1e3, 2),
        "frac_flushed": round(dom_work.bytes / (flushed_ms * 1e-3) / 1e9 / peak.dram_gbps, 4),
        "traffic": None if traffic is None else round(traffic),
        "traffic_over_algorithmic": None if traffic is None else round(traffic / dom_work.bytes, 4),
        "traffic_source": traffic_note,
    }

    baseline = None
    if not args.no_cpu_baseline and args.only is None:
        log("timing the CPU oracle on a bounded sample ...")
        baseline = cpu_baseline(q, kv, x, res, w, dec_work.bytes, rms_work.bytes, args.cpu_budget)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16/bf16",
        "data": "synthetic (device N(0,1) q/K/V, NaN-poisoned spare pages; x, residual N(0,1), w = 1 + N(0,0.1))",
        "config": {
            "workload": (
                "decode step: paged decode 32/8/128/16 fp16 B=64 ctx=4096 + fused add+RMSNorm 4096x8192 bf16"
                if args.only is None
                else f"{args.only} only"
            ),
            "decode": DECODE | {"dtype": "float16"},
            "rmsnorm": RMS | {"dtype": "bfloat16"},
            "device": name,
        },
        "frac_of_peak": round(value / peak.dram_gbps, 4),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": baseline,
        "check": errors,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
