"""Benchmark the gfx950 kernels against PyTorch GPU baselines and report roofline efficiency.

    python -m kernel_lab.bench all --dtype float16 --out results/

Suites (the original harness, kernel_lab/bench/__main__.py:95-216, widened to
the measured configurations):

* rmsnorm: fused add+RMSNorm at tokens {1, 16, 128, 1024, 4096} x hidden
  {4096, 8192};
* decode: Llama-3-8B GQA (32/8/128/16) at batch {1, 8, 32, 64} x context
  {512, 4096} with the planner and with fixed splits; ragged-length MQA and
  GQA (32/1/128 and 32/8/128, batch 64, L ~ U[1, 8192]); long-context 70B-style GQA
  (64/8/128, batch 8, contexts 32768 and 131072);
* decode-fp8: the FP8 (E4M3) cache against a 16-bit cache holding the same
  values, at the headline, ragged and long-context shapes;
* cascade: shared-prefix decode against plain paged decode over the same
  pages (prefixes of 4096-32768 tokens shared by 16-64 sequences);
* copy: a 1 GiB device copy (the streaming ceiling, and the counter
  calibration kernel for the profiles);
* configs: each measured configuration's planner call (fused add+RMSNorm at
  every token count and hidden size in bf16 and fp16, Llama-3-8B decode at
  batch {1, 8, 32, 64} x context {512, 4096}, ragged MQA, long-context
  64/8/128), writing ``order.json`` with ``--out``; ``attribute --trace
  run_kernel_trace.csv --order order.json`` then gives each configuration's
  median kernel time from a rocprofv3 kernel trace of that run (no GPU
  needed).

Every implementation is checked against the PyTorch baseline before it is
timed; a wrong result is reported as such, never as a speed. Timing: HIP
events on the launch stream around each call, median of --reps calls, with a
read of a >= 512 MiB buffer before every call so inputs are not served from the
256 MiB Infinity Cache (a read leaves clean lines, so no write-back lands in
the timed call). GB/s uses the algorithmic byte model in roofline.py.

A case's tensors go back to PyTorch's caching allocator, never to the driver
(no empty_cache between cases): on MI355X, handing a 2 GiB block back to the
driver slowed the next calls of an HBM-bound kernel by ~5 % (32/8/128 fp16
B=64 ctx 4096 decode 158.8 -> 166.5 us) until about 2 s had passed, and made
every case after the first look 5 % slower.
"""

from __future__ import annotations

import argparse
import json
import sys
from collections.abc import Callable
from dataclasses import asdict, dataclass
from pathlib import Path

import torch

from kernel_lab import _native, ops
from kernel_lab.bench.roofline import GPUPeak, Work, decode_attention_work, lookup, rms_norm_work
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8, random_cascade_problem

DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


@dataclass
class Row:
    kernel: str
    shape: str
    impl: str
    us: float | None
    gbps: float | None
    pct_peak_bw: float | None
    speedup: float | None
    max_abs_err: float | None
    note: str = ""


class Timer:
    """HIP-event timing with an Infinity Cache flush (a large read) before each call."""

    def __init__(self, reps: int, flush_mb: int) -> None:
        self.reps = reps
        n = max(flush_mb, 0) * (1 << 20) // 4
        self.flush_buf = torch.ones(n, dtype=torch.float32, device="cuda") if n else None

    def flush(self) -> None:
        if self.flush_buf is not None:
            self.flush_buf.sum()

    def __call__(self, fn: Callable[[], object]) -> float:
        """Median time of one call in microseconds."""
        for _ in range(3):
            fn()
        times = []
        for _ in range(self.reps):
            self.flush()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            fn()
            end.record()
            end.synchronize()
            times.append(start.elapsed_time(end) * 1e3)
        times.sort()
        return times[len(times) // 2]


# Achieved bandwidth above this fraction of the spec-sheet peak is flagged.
SUSPECT_FRACTION = 0.92


def _checked(fn: Callable[[], torch.Tensor], expected: torch.Tensor, atol: float) -> tuple[float | None, str]:
    """Runs fn once and compares it with the baseline's output: (max |error|,
    "" when within atol, else why it will not be timed)."""
    try:
        got = fn()
    except Exception as exc:  # unsupported shape, out of memory, no such backend
        return None, f"skipped: {exc}"[:120]
    err = float((got.float() - expected.float()).abs().max())
    return err, "" if err <= atol else "WRONG RESULT, not timed"  # NaN is never <= atol


def measure(
    kernel: str,
    shape: str,
    impls: dict[str, Callable[[], torch.Tensor]],
    work: Work | dict[str, Work],
    peak: GPUPeak | None,
    baseline: str,
    atol: float,
    timer: Callable[[Callable[[], object]], float],
) -> list[Row]:
    """Check every implementation against the baseline's output first, then
    time only those that agree (a wrong result is never reported as a speed),
    and report each with bandwidth from the byte model and speedup over the
    baseline. Implementations may write into one shared output tensor, so
    the baseline's result is copied before the others run."""
    expected = impls[baseline]().clone()
    verdict = {name: _checked(fn, expected, atol) for name, fn in impls.items()}
    elapsed: dict[str, float] = {}
    for name, (err, why) in verdict.items():
        if not why:
            elapsed[name] = timer(impls[name])
    base_us = elapsed.get(baseline)
    rows = []
    for name, (err, why) in verdict.items():
        us = elapsed.get(name)
        if us is None:
            rows.append(Row(kernel, shape, name, None, None, None, None, err, why))
            continue
        nbytes = (work[name] if isinstance(work, dict) else work).bytes
        gbps = nbytes / us / 1e3  # bytes per microsecond -> GB/s
        share = gbps / peak.dram_gbps if peak else None
        # Above ~92 % of the spec sheet the byte count is wrong or the data came
        # from cache, not HBM (the original runbook's check, docs/gpu-runbook.md:75-76).
        flag = "above 92 % of peak: check the byte count and cache residency" if share and share > SUSPECT_FRACTION else ""
        rows.append(Row(kernel, shape, name, round(us, 2), round(gbps, 1),
                        None if share is None else round(100 * share, 1),
                        round(base_us / us, 2) if base_us else None, err, flag))
    print(f"measured {kernel} {shape}: {len(elapsed)} of {len(impls)} timed", file=sys.stderr, flush=True)
    return rows


# ------------------------------------------------------------------ RMSNorm


def rmsnorm_suite(dtype: torch.dtype, peak: GPUPeak | None, timer, compile_baseline: bool) -> list[Row]:
    """Fused add+RMSNorm against PyTorch (the original harness's suite,
    kernel_lab/bench/__main__.py:95-118 there, at the measured token counts).

    Baselines: torch eager (an add kernel writes the sum, the norm reads it
    back) and torch.compile of the same function. The compiled graph returns
    the normed output and the new residual, so it moves the bytes the fused
    operator moves; a second compiled row returns the normed output alone, as
    the original harness's does, and is credited with only the bytes it
    moves (x and the residual read, the output written). Inductor rounds the
    sum to the storage type before normalising (emulate_precision_casts), as
    eager and the operator do; without it the compiled outputs differ from
    eager's by up to two bf16 ulps and fail the check."""
    import torch._inductor.config as inductor_config

    inductor_config.emulate_precision_casts = True
    elem = torch.tensor([], dtype=dtype).element_size()
    rows: list[Row] = []
    for hidden in (4096, 8192):
        for tokens in (1, 16, 128, 1024, 4096):
            g = torch.Generator(device="cuda").manual_seed(tokens + hidden)
            x = torch.randn(tokens, hidden, generator=g, device="cuda").to(dtype)
            r = torch.randn(tokens, hidden, generator=g, device="cuda").to(dtype)
            w = (1 + 0.1 * torch.randn(hidden, generator=g, device="cuda")).to(dtype)
            out = torch.empty_like(x)
            res = r.clone()

            def add_norm(x, r, w):
                s = x + r  # eager: the add writes the sum, the norm reads it back
                return torch.nn.functional.rms_norm(s, (s.shape[-1],), w, eps=1e-6), s

            def norm_only(x, r, w):
                s = x + r
                return torch.nn.functional.rms_norm(s, (s.shape[-1],), w, eps=1e-6)

            def hip(x=x, r=r, w=w, out=out, res=res):
                # Functional form for the check: refresh the residual from r first.
                res.copy_(r)
                torch.ops.kernel_lab.fused_add_rms_norm(out, x, res, w, 1e-6)
                return out

            def hip_inplace(x=x, w=w, out=out, res=res):
                torch.ops.kernel_lab.fused_add_rms_norm(out, x, res, w, 1e-6)
                return out

            work = rms_norm_work(tokens, hidden, elem, fused_residual=True)
            impls: dict[str, Callable[[], torch.Tensor]] = {
                "torch eager": lambda x=x, r=r, w=w: add_norm(x, r, w)[0]
            }
            works: dict[str, Work] = {"torch eager": work}
            if compile_baseline:
                # A fresh compile per shape: every shape gets its own static-shape
                # graph, and no shape falls back to eager at dynamo's recompile limit.
                torch._dynamo.reset()
                both = torch.compile(add_norm)
                only = torch.compile(norm_only)
                impls["torch.compile"] = lambda x=x, r=r, w=w, f=both: f(x, r, w)[0]
                works["torch.compile"] = work
                name = "torch.compile, normed output only (the original harness's)"
                impls[name] = lambda x=x, r=r, w=w, f=only: f(x, r, w)
                works[name] = Work(bytes=3 * tokens * hidden * elem + hidden * elem, flops=work.flops)
            impls["hip"] = hip
            works["hip"] = work
            atol = 2e-2 if dtype != torch.float32 else 1e-4
            got = measure("fused_add_rms_norm", f"{tokens}x{hidden}", impls, works, peak, "torch eager", atol, timer)
            # The check above ran the functional form (residual refreshed from r);
            # time the operator itself, updating the residual in place as a model does.
            for row in got:
                if row.impl == "hip" and row.us is not None:
                    us = timer(hip_inplace)
                    row.us = round(us, 2)
                    row.gbps = round(work.bytes / (us * 1e-6) / 1e9, 1)
                    row.pct_peak_bw = round(100 * row.gbps / peak.dram_gbps, 1) if peak else None
                    base = next((r.us for r in got if r.impl == "torch eager" and r.us), None)
                    row.speedup = round(base / us, 2) if base else None
                    row.note = "in-place operator"
                    if peak and row.gbps > SUSPECT_FRACTION * peak.dram_gbps:
                        row.note += "; above 92 % of peak: check the byte count and cache residency"
            rows += got
    return rows


# ------------------------------------------------------- decode attention


def _padded_kv(cache: torch.Tensor, block_table: torch.Tensor) -> torch.Tensor:
    """Every sequence's pages gathered into one padded [B, L, Hkv, D] tensor
    (L = block-table width x page size); tokens past a sequence's length are
    whatever its last and padding pages hold."""
    batch, width = block_table.shape
    return cache[block_table.long()].reshape(batch, width * cache.shape[1], cache.shape[2], cache.shape[3])


def _valid_tokens(block_table: torch.Tensor, seq_lens: torch.Tensor, page: int) -> torch.Tensor:
    positions = torch.arange(block_table.shape[1] * page, device=seq_lens.device)
    return positions[None, :] < seq_lens[:, None].long()  # [B, L]


def torch_sdpa_decode(q, k_cache, v_cache, block_table, seq_lens, scale, padded: bool = True):
    """The original harness's PyTorch baseline (kernel_lab/bench/__main__.py:128-139
    there): pages gathered into padded K/V, then scaled_dot_product_attention.

    Only SDPA's fused kernels may serve the call: its math fallback runs
    batched 16-bit products (torch.bmm) whose right operand is a transposed
    view of K, a form reported to fault GPUs on the MI355X pool this was built
    on, so it is never run. On this build's SDPA (probed on MI355X, fp16 and
    bf16), the flash kernel takes grouped-query heads only without a mask,
    and the memory-efficient kernel takes a mask only with K/V expanded to
    every query head. So a batch whose sequences all fill the block table
    (`padded` False) runs flash with grouped heads; otherwise K/V are expanded
    and the padding masked.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    batch, hq, _ = q.shape
    page, hkv = k_cache.shape[1], k_cache.shape[2]
    keys = _padded_kv(k_cache, block_table).transpose(1, 2)  # [B, Hkv, L, D]
    values = _padded_kv(v_cache, block_table).transpose(1, 2)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        if not padded:
            out = torch.nn.functional.scaled_dot_product_attention(
                q.unsqueeze(2), keys, values, scale=scale, enable_gqa=True
            )
        else:
            keep = _valid_tokens(block_table, seq_lens, page)[:, None, None, :]
            out = torch.nn.functional.scaled_dot_product_attention(
                q.unsqueeze(2), keys.repeat_interleave(hq // hkv, dim=1), values.repeat_interleave(hq // hkv, dim=1),
                attn_mask=keep, scale=scale,
            )
    return out.squeeze(2)


def torch_paged_decode(q, k_cache, v_cache, block_table, seq_lens, scale):
    """Plain PyTorch without SDPA: the same gather, then softmax(q K^T) V as two
    batched products on contiguous operands (K^T materialised), the products
    that are safe for 16-bit data on this platform."""
    batch, hq, d = q.shape
    hkv = k_cache.shape[2]
    keys_t = _padded_kv(k_cache, block_table).permute(0, 2, 3, 1).contiguous()  # [B, Hkv, D, L]
    values = _padded_kv(v_cache, block_table).permute(0, 2, 1, 3).contiguous()  # [B, Hkv, L, D]
    scores = torch.matmul(q.reshape(batch, hkv, hq // hkv, d), keys_t).float() * scale  # [B, Hkv, G, L]
    keep = _valid_tokens(block_table, seq_lens, k_cache.shape[1])[:, None, None, :]
    probs = torch.softmax(scores.masked_fill(~keep, float("-inf")), dim=-1).to(q.dtype)
    return torch.matmul(probs, values).reshape(batch, hq, d)


def decode_cases(dtype: torch.dtype) -> list[tuple[str, list[int], int, int, torch.dtype]]:
    cases = []
    for batch in (1, 8, 32, 64):
        for ctx in (512, 4096):
            cases.append((f"32/8/128 b{batch} ctx{ctx}", [ctx] * batch, 32, 8, dtype))
    g = torch.Generator().manual_seed(3)
    ragged = torch.randint(1, 8193, (64,), generator=g).tolist()
    cases.append(("32/1/128 b64 ragged U[1,8192]", ragged, 32, 1, torch.bfloat16 if dtype != torch.float32 else dtype))
    cases.append(("32/8/128 b64 ragged U[1,8192]", ragged, 32, 8, dtype))
    # One long sequence among short ones: splits sized from the block table's
    # width leave most of the work to the long sequence's few workgroups.
    cases.append(("32/8/128 b16 skewed 1x65536+15x1024", [65536] + [1024] * 15, 32, 8, dtype))
    cases.append(("32/8/128 b64 skewed 1x65536+63x2048", [65536] + [2048] * 63, 32, 8, dtype))
    for ctx in (32768, 131072):
        cases.append((f"64/8/128 b8 ctx{ctx}", [ctx] * 8, 64, 8, torch.bfloat16 if dtype != torch.float32 else dtype))
    return cases


def _forced_valu(fn: Callable[[], torch.Tensor]) -> torch.Tensor:
    """Runs fn with the library's 16-bit decode sent to its VALU kernel."""
    with _native.decode_switches(force_valu="1"):
        return fn()


def _unpaired(fn: Callable[[], torch.Tensor]) -> torch.Tensor:
    """Runs fn with paired workgroups (two adjacent KV heads per 8-wave
    workgroup) switched off."""
    with _native.decode_switches(paired="0"):
        return fn()


def decode_suite(
    dtype: torch.dtype,
    peak: GPUPeak | None,
    timer,
    splits: list[int],
    baseline_max_bytes: float,
    shape: str | None = None,
) -> list[Row]:
    rows: list[Row] = []
    d, page = 128, 16
    for label, lens, hq, hkv, dt in decode_cases(dtype):
        if shape and shape not in label:
            continue
        q, kv = device_decode_problem(lens, hq, hkv, d, page, dtype=dt, device="cuda")
        args = (q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
        scale = d**-0.5
        elem = torch.tensor([], dtype=dt).element_size()
        work = decode_attention_work(lens, hq, hkv, d, elem)
        out = torch.empty_like(q)
        out2 = torch.empty_like(q)
        impls: dict[str, Callable[[], torch.Tensor]] = {}
        # The gather baseline materialises padded K/V; skip it where that would be huge.
        gather_bytes = 2 * kv.block_table.numel() * page * hkv * d * elem
        if gather_bytes <= baseline_max_bytes:
            padded = any(n != kv.block_table.shape[1] * page for n in lens)
            sdpa = lambda a=args, s=scale, p=padded: torch_sdpa_decode(*a, s, p)  # noqa: E731
            try:
                sdpa()
                impls["torch (gather + SDPA)"] = sdpa  # the original harness's baseline
            except RuntimeError as exc:  # no fused SDPA kernel for this case
                rows.append(Row("paged_decode", label, "torch (gather + SDPA)", None, None, None, None, None,
                                f"skipped: {exc}"[:120]))
            impls["torch (gather + matmul)"] = lambda a=args, s=scale: torch_paged_decode(*a, s)
        impls["hip split-KV (planner)"] = lambda a=args, s=scale, o=out: ops.paged_decode_attention(*a, s, out=o)
        if dt != torch.float32:
            if hkv % 2 == 0:
                impls["hip unpaired (planner)"] = lambda a=args, s=scale, o=out2: _unpaired(
                    lambda: ops.paged_decode_attention(*a, s, out=o)
                )
            impls["hip VALU kernel (planner)"] = lambda a=args, s=scale, o=out2: _forced_valu(
                lambda: ops.paged_decode_attention(*a, s, out=o)
            )
        for n in splits:
            impls[f"hip splits={n}"] = lambda a=args, s=scale, o=out, n=n: ops.paged_decode_attention(
                *a, s, num_splits=n, out=o
            )
        baseline = next(iter(impls))
        atol = 2e-2 if dt != torch.float32 else 1e-3
        rows += measure("paged_decode", label, impls, work, peak, baseline, atol, timer)
        del q, kv, args, out, out2, impls
    return rows


def decode_fp8_cases() -> list[tuple[str, list[int], int, int, torch.dtype]]:
    g = torch.Generator().manual_seed(3)
    ragged = torch.randint(1, 8193, (64,), generator=g).tolist()
    return [
        ("32/8/128 b1 ctx4096", [4096], 32, 8, torch.float16),
        ("32/8/128 b8 ctx4096", [4096] * 8, 32, 8, torch.float16),
        ("32/8/128 b64 ctx4096", [4096] * 64, 32, 8, torch.float16),
        ("32/1/128 b64 ragged U[1,8192]", ragged, 32, 1, torch.bfloat16),
        ("64/8/128 b8 ctx32768", [32768] * 8, 64, 8, torch.bfloat16),
        ("64/8/128 b8 ctx131072", [131072] * 8, 64, 8, torch.bfloat16),
    ]


def decode_fp8_suite(peak: GPUPeak | None, timer, shape: str | None = None) -> list[Row]:
    """FP8 (E4M3, per-KV-head scales) cache against the 16-bit cache holding the
    same values: E4M3 values are exact in fp16/bf16, so both compute the same
    attention and the rows show what halving the KV bytes buys."""
    rows: list[Row] = []
    d, page = 128, 16
    for label, lens, hq, hkv, dt in decode_fp8_cases():
        if shape and shape not in label:
            continue
        q, kv = device_decode_problem(lens, hq, hkv, d, page, dtype=dt, device="cuda")
        kv8, ks, vs = quantize_fp8(kv)
        # The same values in the 16-bit format (exact), scales applied.
        kv.k_cache.copy_(kv8.k_cache.to(dt) * ks.to(dt)[None, None, :, None])
        kv.v_cache.copy_(kv8.v_cache.to(dt) * vs.to(dt)[None, None, :, None])
        scale = d**-0.5
        out16, out8 = torch.empty_like(q), torch.empty_like(q)
        a16 = (q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
        a8 = (q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens)
        impls: dict[str, Callable[[], torch.Tensor]] = {
            f"hip {str(dt).split('.')[-1]} cache (same values)": lambda: ops.paged_decode_attention(
                *a16, scale, out=out16
            ),
            "hip fp8 cache (planner)": lambda: ops.paged_decode_attention(*a8, scale, out=out8, k_scale=ks, v_scale=vs),
        }
        if hkv % 2 == 0:
            impls["hip fp8 cache unpaired (planner)"] = lambda: _unpaired(
                lambda: ops.paged_decode_attention(*a8, scale, out=out8, k_scale=ks, v_scale=vs)
            )
        w16 = decode_attention_work(lens, hq, hkv, d, 2)
        w8 = decode_attention_work(lens, hq, hkv, d, 2, kv_elem_bytes=1)
        work = {name: (w8 if "fp8" in name else w16) for name in impls}
        baseline = next(iter(impls))
        # Scales rounded to the 16-bit type make the two caches differ by a rounding.
        rows += measure("paged_decode_fp8", label, impls, work, peak, baseline, 3e-2, timer)
        del q, kv, kv8, a16, a8, out16, out8, impls
    return rows


# ------------------------------------------------------------------ cascade


def cascade_cases() -> list[tuple[str, int, list[int], int, int, torch.dtype]]:
    return [
        ("32/8/128 b64 prefix 4096 + 512 own", 4096, [512] * 64, 32, 8, torch.float16),
        ("32/8/128 b32 prefix 16384 + 256 own", 16384, [256] * 32, 32, 8, torch.float16),
        ("64/8/128 b16 prefix 32768 + 1024 own", 32768, [1024] * 16, 64, 8, torch.bfloat16),
    ]


def cascade_suite(peak: GPUPeak | None, timer, shape: str | None = None) -> list[Row]:
    """Shared-prefix decode against plain paged decode over the same pages
    (each sequence's table = prefix pages + own pages). GB/s counts the bytes
    each must read: the prefix once for cascade, once per sequence for plain."""
    rows: list[Row] = []
    d, page = 128, 16
    for label, plen, lens, hq, hkv, dt in cascade_cases():
        if shape and shape not in label:
            continue
        q, c = random_cascade_problem(plen, lens, hq, hkv, d, page, dtype=dt, device="cuda")
        flat = c.flattened()
        scale = d**-0.5
        o_plain, o_casc = torch.empty_like(q), torch.empty_like(q)
        impls: dict[str, Callable[[], torch.Tensor]] = {
            "hip paged decode (planner)": lambda: ops.paged_decode_attention(
                q, flat.k_cache, flat.v_cache, flat.block_table, flat.seq_lens, scale, out=o_plain
            ),
            "hip cascade": lambda: ops.cascade_decode_attention(
                q, c.kv.k_cache, c.kv.v_cache, c.prefix_block_table, c.prefix_len, c.kv.block_table,
                c.kv.seq_lens, scale, out=o_casc
            ),
        }
        elem = 2
        plain = decode_attention_work([plen + n for n in lens], hq, hkv, d, elem)
        prefix_once = decode_attention_work([plen + sum(lens)], hq, hkv, d, elem)
        # q and out are counted for every sequence, the prefix's K/V once.
        q_out = 2 * len(lens) * hq * d * elem
        casc = Work(bytes=prefix_once.bytes - 2 * hq * d * elem + q_out, flops=plain.flops)
        work = {"hip paged decode (planner)": plain, "hip cascade": casc}
        rows += measure("cascade_decode", label, impls, work, peak, "hip paged decode (planner)", 3e-2, timer)
        del q, c, flat, o_plain, o_casc, impls
    return rows


# ------------------------------------------------------------------- copy


def copy_suite(peak: GPUPeak | None, timer, mib: int = 1024) -> list[Row]:
    """A plain device-to-device copy of ``mib`` MiB (torch ``copy_``): the
    practical streaming ceiling, and the known-size kernel that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (it reads and writes exactly mib MiB)."""
    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    work = Work(bytes=2 * n * 4, flops=0)
    rows = measure("copy", f"{mib} MiB", {"torch copy_": lambda: y.copy_(x)}, work, peak, "torch copy_", 0.0, timer)
    del x, y
    return rows


# ------------------------------------------------------- BASELINE configs

WARMUP_CALLS = 3  # Timer's untimed calls before the timed ones


def baseline_config_cases() -> list[tuple[str, str, dict]]:
    """The measured configurations, in a fixed order: (config, label, spec)."""
    cases = []
    for dt in (torch.bfloat16, torch.float16):
        for hidden in (4096, 8192):
            for tokens in (1, 16, 128, 1024, 4096):
                cases.append(("cfg1", f"{str(dt)[6:]} {tokens}x{hidden}",
                              {"kind": "rms", "tokens": tokens, "hidden": hidden, "dtype": dt}))
    for batch in (1, 8, 32, 64):
        for ctx in (512, 4096):
            cases.append(("cfg2", f"32/8/128 fp16 B={batch} ctx {ctx}",
                          {"kind": "decode", "lens": [ctx] * batch, "hq": 32, "hkv": 8, "dtype": torch.float16}))
    g = torch.Generator().manual_seed(3)
    ragged = torch.randint(1, 8193, (64,), generator=g).tolist()
    cases.append(("cfg3", "32/1/128 bf16 B=64 L~U[1,8192]",
                  {"kind": "decode", "lens": ragged, "hq": 32, "hkv": 1, "dtype": torch.bfloat16}))
    for ctx in (32768, 131072):
        cases.append(("cfg4", f"64/8/128 bf16 B=8 ctx {ctx}",
                      {"kind": "decode", "lens": [ctx] * 8, "hq": 64, "hkv": 8, "dtype": torch.bfloat16}))
    return cases


def configs_suite(peak: GPUPeak | None, timer, shape: str | None = None) -> tuple[list[Row], list[dict]]:
    """Each measured configuration's planner call: checked once against the
    PyTorch computation, then timed (WARMUP_CALLS + reps calls). The second
    result lists the cases in launch order with their call counts, so a
    rocprofv3 kernel trace of this run can be attributed (``attribute``)."""
    rows: list[Row] = []
    order: list[dict] = []
    for cfg, label, spec in baseline_config_cases():
        if shape and shape not in label:
            continue
        dt = spec["dtype"]
        elem = torch.tensor([], dtype=dt).element_size()
        if spec["kind"] == "rms":
            gen = torch.Generator(device="cuda").manual_seed(spec["tokens"] + spec["hidden"])
            x = torch.randn(spec["tokens"], spec["hidden"], generator=gen, device="cuda").to(dt)
            r = torch.randn(spec["tokens"], spec["hidden"], generator=gen, device="cuda").to(dt)
            w = (1 + 0.1 * torch.randn(spec["hidden"], generator=gen, device="cuda")).to(dt)
            out = torch.empty_like(x)
            res = r.clone()
            s = x + r
            expected = torch.nn.functional.rms_norm(s, (s.shape[-1],), w, eps=1e-6)
            fn = lambda x=x, w=w, out=out, res=res: torch.ops.kernel_lab.fused_add_rms_norm(out, x, res, w, 1e-6)
            work = rms_norm_work(spec["tokens"], spec["hidden"], elem, fused_residual=True)
            kernel = "fused_add_rms_norm"
        else:
            q, kv = device_decode_problem(spec["lens"], spec["hq"], spec["hkv"], 128, 16, dtype=dt, device="cuda")
            out = torch.empty_like(q)
            args = (q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
            scale = 128 ** -0.5
            expected = torch_paged_decode(*args, scale)
            fn = lambda a=args, o=out: ops.paged_decode_attention(*a, scale, out=o)
            work = decode_attention_work(spec["lens"], spec["hq"], spec["hkv"], 128, elem)
            kernel = "paged_decode"
        fn()
        err = (out.float() - expected.float()).abs().max().item()
        atol = 2e-2
        if not err <= atol:
            rows.append(Row(kernel, f"{cfg} {label}", "hip (planner)", None, None, None, None, err,
                            "WRONG RESULT, not timed"))
            order.append({"cfg": cfg, "case": label, "calls": 1, "bytes": work.bytes})
            continue
        us = timer(fn)
        gbps = work.bytes / (us * 1e-6) / 1e9
        pct = round(100 * gbps / peak.dram_gbps, 1) if peak else None
        rows.append(Row(kernel, f"{cfg} {label}", "hip (planner)", round(us, 2), round(gbps, 1), pct, None, err))
        order.append({"cfg": cfg, "case": label, "calls": 1 + WARMUP_CALLS + timer.reps, "timed": timer.reps,
                      "bytes": work.bytes})
        del expected, out
    return rows, order


# Kernels of this library in a kernel trace: the main launch of a call, and the
# merge launches that follow it in the same call.
_MAIN_KERNELS = ("decode_mfma", "decode_valu", "rms_norm")
_MERGE_KERNELS = ("decode_merge", "cascade_merge")


def attribute_trace(trace_csv: Path, order: list[dict]) -> str:
    """Median kernel time per case from a rocprofv3 ``--kernel-trace`` CSV of
    a ``configs`` run: the library's dispatches in start order are its calls
    (a main kernel plus any merge kernel), the cases' call counts cut them
    into cases, and each case's last ``timed`` calls give the medians."""
    import csv
    import statistics

    with open(trace_csv) as f:
        recs = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    calls: list[list] = []  # [kernel, main ns, merge ns]
    for r in recs:
        name = r["Kernel_Name"].replace("void kl::(anonymous namespace)::", "").split("(kl::")[0].replace("kl::", "")
        dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        if any(k in name for k in _MAIN_KERNELS):
            calls.append([name, dur, 0])
        elif any(k in name for k in _MERGE_KERNELS) and calls:
            calls[-1][2] += dur
    need = sum(c["calls"] for c in order)
    if len(calls) != need:
        raise ValueError(f"trace holds {len(calls)} calls of this library, the run made {need}")
    lines = [
        "| config | case | kernel | kernel µs | merge µs | algorithmic bytes | GB/s | % of peak |",
        "|---|---|---|---:|---:|---:|---:|---:|",
    ]
    i = 0
    for c in order:
        grp = calls[i : i + c["calls"]][-c.get("timed", 1):]
        i += c["calls"]
        main_ns = statistics.median(g[1] for g in grp)
        merge_ns = statistics.median(g[2] for g in grp)
        kernels = ", ".join(sorted({g[0] for g in grp}))
        gbps = c["bytes"] / (main_ns + merge_ns)
        lines.append(f"| {c['cfg']} | {c['case']} | {kernels} | {main_ns / 1e3:,.1f} | {merge_ns / 1e3:,.1f} | "
                     f"{c['bytes']:,} | {gbps:,.0f} | {100 * gbps / 8000:.1f} |")
    return "\n".join(lines) + "\n"


# --------------------------------------------------------------------- report


def _cell(value: float | None, unit: str = "") -> str:
    return "-" if value is None else f"{value}{unit}"


# (heading, alignment, cell) for each column of the results table.
_COLUMNS: tuple[tuple[str, str, Callable[[Row], str]], ...] = (
    ("Kernel", "---", lambda r: r.kernel),
    ("Shape", "---", lambda r: r.shape),
    ("Implementation", "---", lambda r: f"{r.impl} ({r.note})" if r.note else r.impl),
    ("Time (µs)", "---:", lambda r: _cell(r.us)),
    ("GB/s", "---:", lambda r: _cell(r.gbps)),
    ("% peak BW", "---:", lambda r: _cell(r.pct_peak_bw, "%")),
    ("Speedup", "---:", lambda r: _cell(r.speedup, "x")),
    ("Max err", "---:", lambda r: "-" if r.max_abs_err is None else f"{r.max_abs_err:.1e}"),
)


def to_markdown(rows: list[Row], header: str) -> str:
    """A markdown table of the rows under `header`; untimed rows show why."""
    table = ["| " + " | ".join(c[0] for c in _COLUMNS) + " |", "|" + "|".join(c[1] for c in _COLUMNS) + "|"]
    table += ["| " + " | ".join(c[2](r) for c in _COLUMNS) + " |" for r in rows]
    return "\n".join([header, "", *table]) + "\n"


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(
        prog="python -m kernel_lab.bench", description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter
    )
    parser.add_argument("suite", choices=["rmsnorm", "decode", "decode-fp8", "cascade", "copy", "configs",
                                          "attribute", "all"])
    parser.add_argument("--dtype", choices=list(DTYPES), default="float16")
    parser.add_argument("--peak-gbps", type=float, help="override the spec-sheet DRAM bandwidth")
    parser.add_argument("--no-compile", action="store_true", help="skip the torch.compile RMSNorm baseline")
    parser.add_argument("--splits", type=int, nargs="*", default=[1, 4, 16, 64], help="fixed split counts to time")
    parser.add_argument("--reps", type=int, default=50)
    parser.add_argument("--flush-mb", type=int, default=1024, help="read this much between timed calls (0: none)")
    parser.add_argument("--baseline-max-gb", type=float, default=8.0, help="skip the gather baseline above this")
    parser.add_argument("--out", type=Path, help="directory for results.json and results.md")
    parser.add_argument("--shape", help="run only the cases whose shape label contains this text")
    parser.add_argument("--trace", type=Path, help="attribute: a rocprofv3 kernel_trace.csv of a configs run")
    parser.add_argument("--order", type=Path, help="attribute: the configs run's order.json")
    args = parser.parse_args(argv)

    if args.suite == "attribute":  # no GPU needed
        if not args.trace or not args.order:
            print("attribute needs --trace and --order", file=sys.stderr)
            return 2
        print(attribute_trace(args.trace, json.loads(args.order.read_text())), end="")
        return 0

    if not torch.cuda.is_available():
        print("No GPU device: the benchmarks need an AMD Instinct GPU (MI355X).", file=sys.stderr)
        return 2
    if not ops.available():
        print(f"kernel_lab kernels unavailable: {ops.why_unavailable()}", file=sys.stderr)
        return 2

    name = torch.cuda.get_device_name()
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    peak = lookup(name) or lookup(arch)
    if args.peak_gbps:
        peak = GPUPeak(name, args.peak_gbps, peak.fp16_tflops if peak else 0.0)
    dtype = DTYPES[args.dtype]
    print(f"GPU: {name} ({arch}); peak DRAM: {peak.dram_gbps if peak else 'unknown'} GB/s; dtype: {args.dtype}",
          file=sys.stderr)
    timer = Timer(args.reps, args.flush_mb)

    rows: list[Row] = []
    if args.suite in ("rmsnorm", "all"):
        rows += rmsnorm_suite(dtype, peak, timer, compile_baseline=not args.no_compile)
    if args.suite in ("decode", "all"):
        rows += decode_suite(dtype, peak, timer, args.splits, args.baseline_max_gb * 1e9, args.shape)
    if args.suite in ("decode-fp8", "all"):
        rows += decode_fp8_suite(peak, timer, args.shape)
    if args.suite in ("cascade", "all"):
        rows += cascade_suite(peak, timer, args.shape)
    if args.suite == "copy":
        rows += copy_suite(peak, timer)
    order = None
    if args.suite == "configs":
        got, order = configs_suite(peak, timer, args.shape)
        rows += got

    header = (
        f"### {name} ({arch}), {args.dtype}\n\nPeak DRAM bandwidth used for %: "
        f"{peak.dram_gbps if peak else 'unknown'} GB/s. Speedup is vs the first PyTorch baseline per shape; "
        f"{args.flush_mb} MiB read before every timed call."
    )
    table = to_markdown(rows, header)
    print(table)
    if args.out:
        args.out.mkdir(parents=True, exist_ok=True)
        meta = {"gpu": name, "arch": arch, "dtype": args.dtype, "torch": torch.__version__,
                "peak_dram_gbps": peak.dram_gbps if peak else None, "flush_mb": args.flush_mb, "reps": args.reps}
        (args.out / "results.json").write_text(json.dumps({"meta": meta, "rows": [asdict(r) for r in rows]}, indent=2))
        (args.out / "results.md").write_text(table)
        if order is not None:
            (args.out / "order.json").write_text(json.dumps(order, indent=2))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
