"""Roofline byte/FLOP model: the original project's known answers
(tests/test_roofline.py:9-47 of Markkoby3/Kernel-lab) plus the MI355X entry."""

from __future__ import annotations

import pytest

from kernel_lab.bench import roofline


def test_rms_norm_bytes_count_each_tensor_once():
    w = roofline.rms_norm_work(rows=2, hidden=8, elem_bytes=2, fused_residual=True)
    assert w.bytes == 2 * 8 * 2 * 4 + 8 * 2  # x, residual in; out, residual out; + weight
    assert roofline.rms_norm_work(2, 8, 2, False).bytes == 2 * 8 * 2 * 2 + 8 * 2


def test_decode_attention_is_memory_bound_on_every_listed_gpu():
    work = roofline.decode_attention_work([4096] * 8, 32, 8, 128, elem_bytes=2)
    assert 3.5 < work.intensity < 4.5  # GQA group 4: about 4 FLOPs per byte of KV
    for gpu in roofline.GPU_PEAKS:
        assert work.intensity < gpu.ridge_flops_per_byte


def test_decode_kv_bytes():
    work = roofline.decode_attention_work([10, 20], num_q_heads=4, num_kv_heads=2, head_dim=8, elem_bytes=2)
    assert work.bytes == 2 * 30 * 2 * 8 * 2 + 2 * 2 * 4 * 8 * 2
    assert work.flops == 4 * 30 * 4 * 8


def test_fp8_cache_halves_the_kv_bytes():
    w16 = roofline.decode_attention_work([4096] * 64, 32, 8, 128, 2)
    w8 = roofline.decode_attention_work([4096] * 64, 32, 8, 128, 2, kv_elem_bytes=1)
    q_out = 2 * 64 * 32 * 128 * 2
    assert w8.bytes - q_out == (w16.bytes - q_out) // 2 and w8.flops == w16.flops


def test_baseline_floors():
    """Algorithmic bytes at the headline shapes (8.0 TB/s floors in the build's targets)."""
    rms = roofline.rms_norm_work(4096, 8192, 2, True)
    assert rms.bytes == 268_451_840
    dec = roofline.decode_attention_work([4096] * 64, 32, 8, 128, 2)
    assert dec.bytes == 1_074_790_400
    assert dec.flops == 4_294_967_296
    assert abs(dec.bytes / (roofline.MI355X.dram_gbps * 1e9) * 1e6 - 134.35) < 0.01


@pytest.mark.parametrize(
    ("device", "expected"),
    [
        ("AMD Instinct MI355X", "MI355X"),
        ("AMD Instinct MI300X", "MI300X"),
        ("AMD Instinct MI300X VF", "MI300X"),
        ("gfx950", "MI355X"),
        ("NVIDIA H100 80GB HBM3", "H100 80GB HBM3"),
        ("NVIDIA A100 80GB PCIe", "A100 80GB PCIe"),
        ("NVIDIA L40", "L40"),
        ("NVIDIA L40S", "L40S"),
        ("Tesla T4", None),
        ("NVIDIA H100 PCIe", "H100 PCIe"),
        ("NVIDIA A100-SXM4-80GB", "A100-SXM4-80GB"),
        ("NVIDIA A100-PCIE-40GB", "A100"),
        ("NVIDIA L4", "L4"),
        ("NVIDIA A10G", "A10G"),
        ("NVIDIA GeForce RTX 4090", "RTX 4090"),
    ],
)
def test_gpu_lookup(device, expected):
    peak = roofline.lookup(device)
    assert (peak.name if peak else None) == expected


def test_mi355x_ridge():
    assert 300 < roofline.MI355X.ridge_flops_per_byte < 330


def test_markdown_marks_skips_and_wrong_results():
    from kernel_lab.bench.__main__ import Row, to_markdown

    rows = [
        Row("k", "s", "torch", 10.0, 100.0, 50.0, 1.0, 0.0),
        Row("k", "s", "bad", None, None, None, None, 0.5, "WRONG RESULT, not timed"),
    ]
    text = to_markdown(rows, "### test")
    assert "| k | s | torch | 10.0 | 100.0 | 50.0% | 1.0x | 0.0e+00 |" in text
    assert "bad (WRONG RESULT, not timed)" in text


def test_measure_flags_bandwidth_above_92_percent_of_peak():
    """The reference runbook's sanity check (docs/gpu-runbook.md:75-76): above
    ~92 % of peak the byte count is wrong or the data came from cache."""
    import torch

    from kernel_lab.bench.__main__ import measure

    work = roofline.Work(bytes=8e9, flops=0.0)  # 8 GB: 1000 us is 8 TB/s
    impls = {"base": lambda: torch.zeros(4), "ok": lambda: torch.zeros(4), "suspect": lambda: torch.zeros(4)}
    times = iter([2000.0, 1100.0, 1050.0])  # 50 %, 90.9 %, 95.2 % of 8 TB/s
    rows = measure("k", "s", impls, work, roofline.MI355X, "base", 0.0, lambda fn: next(times))
    notes = {r.impl: r.note for r in rows}
    assert notes["base"] == "" and notes["ok"] == ""
    assert "above 92 %" in notes["suspect"]


def test_cli_without_gpu_exits_cleanly(capsys):
    import torch

    from kernel_lab.bench.__main__ import main

    if torch.cuda.is_available():
        pytest.skip("GPU present")
    assert main(["rmsnorm"]) == 2
    assert "No GPU device" in capsys.readouterr().err


def test_decode_cases_cover_the_measured_configs():
    import torch

    from kernel_lab.bench.__main__ import decode_cases

    labels = [c[0] for c in decode_cases(torch.float16)]
    assert "32/8/128 b64 ctx4096" in labels and "32/8/128 b1 ctx512" in labels
    assert any("ragged" in s for s in labels) and "64/8/128 b8 ctx131072" in labels
    ragged = next(c for c in decode_cases(torch.float16) if "ragged" in c[0])
    assert ragged[2:] == (32, 1, torch.bfloat16) and len(ragged[1]) == 64
    assert 1 <= min(ragged[1]) and max(ragged[1]) <= 8192


def test_config_cases_cover_every_measured_config():
    """The configs suite runs every measured configuration: cfg1 (fused
    add+RMSNorm, bf16 and fp16, tokens {1, 16, 128, 1024, 4096} x hidden
    {4096, 8192}), cfg2 (32/8/128 fp16, B {1, 8, 32, 64} x ctx {512, 4096}),
    cfg3 (ragged MQA) and cfg4 (64/8/128 bf16 B=8, ctx 32768 and 131072)."""
    import torch

    from kernel_lab.bench.__main__ import baseline_config_cases

    cases = baseline_config_cases()
    by_cfg = {}
    for cfg, _, spec in cases:
        by_cfg.setdefault(cfg, []).append(spec)
    assert len(by_cfg["cfg1"]) == 20
    assert {(s["tokens"], s["hidden"]) for s in by_cfg["cfg1"]} == {
        (t, h) for t in (1, 16, 128, 1024, 4096) for h in (4096, 8192)
    }
    assert {(len(s["lens"]), s["lens"][0]) for s in by_cfg["cfg2"]} == {
        (b, c) for b in (1, 8, 32, 64) for c in (512, 4096)
    }
    (mqa,) = by_cfg["cfg3"]
    assert (mqa["hq"], mqa["hkv"], mqa["dtype"], len(mqa["lens"])) == (32, 1, torch.bfloat16, 64)
    assert {s["lens"][0] for s in by_cfg["cfg4"]} == {32768, 131072}
    assert all(s["hq"] == 64 and s["hkv"] == 8 and len(s["lens"]) == 8 for s in by_cfg["cfg4"])


def test_attribute_trace_assigns_calls_in_order(tmp_path):
    """Dispatches of other kernels are skipped, a merge kernel is added to the
    call before it, and each case's medians come from its last timed calls."""
    from kernel_lab.bench.__main__ import attribute_trace

    rows = []
    t = 0

    def dispatch(name, dur):
        nonlocal t
        rows.append((name, t, t + dur))
        t += dur + 100

    flush = "void at::native::reduce_kernel<512, 1>(float)"
    # Case A: 4 calls (1 check + 1 warm-up + 2 timed), one kernel each.
    for dur in (9_000, 8_000, 5_000, 7_000):
        dispatch(flush, 50_000)
        dispatch("void kl::(anonymous namespace)::decode_mfma_kernel<kl::F16, kl::F16, 128, 1>"
                 "(kl::(anonymous namespace)::DecodeArgs)", dur)
    # Case B: 3 calls (check + 2 timed), each a decode kernel then a merge kernel.
    for dur, merge in ((20_000, 9_000), (10_000, 2_000), (12_000, 4_000)):
        dispatch("void kl::(anonymous namespace)::decode_mfma_balanced_kernel<kl::BF16, kl::BF16, 128, 2, 1>"
                 "(kl::(anonymous namespace)::DecodeArgs)", dur)
        dispatch("void kl::(anonymous namespace)::decode_merge_balanced_kernel<kl::BF16>"
                 "(kl::(anonymous namespace)::DecodeArgs, int)", merge)
    path = tmp_path / "run_kernel_trace.csv"
    path.write_text("Kernel_Name,Start_Timestamp,End_Timestamp\n" +
                    "".join(f'"{n}",{s},{e}\n' for n, s, e in reversed(rows)))
    order = [
        {"cfg": "cfgA", "case": "a", "calls": 4, "timed": 2, "bytes": 48_000},
        {"cfg": "cfgB", "case": "b", "calls": 3, "timed": 2, "bytes": 28_000},
    ]
    table = attribute_trace(path, order).splitlines()
    assert table[2] == "| cfgA | a | decode_mfma_kernel<F16, F16, 128, 1> | 6.0 | 0.0 | 48,000 | 8 | 0.1 |"
    assert table[3] == ("| cfgB | b | decode_mfma_balanced_kernel<BF16, BF16, 128, 2, 1> | 11.0 | 3.0 | "
                        "28,000 | 2 | 0.0 |")
    with pytest.raises(ValueError, match="trace holds"):
        attribute_trace(path, order[:1])
