"""Pins the CPU oracle before anything is checked against it.

Each check uses something the oracle's code does not share: PyTorch library
routines (F.rms_norm, SDPA), closed forms, invariants, the original project's
known answers, a float64 brute force, and committed golden vectors. The
planted-mistake tests show the golden vectors reject plausible bugs (GQA
mapping, scale, length, page order, rounding point).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kernel_lab.kv_cache import build_paged_kv, random_decode_problem
from oracle import brute
from oracle import reference as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_decode_golden() -> dict[str, dict[str, np.ndarray]]:
    data = np.load(GOLDEN / "decode_golden.npz")
    cases: dict[str, dict[str, np.ndarray]] = {}
    for key in data.files:
        name, field = key.split("/")
        cases.setdefault(name, {})[field] = data[key]
    return cases


def load_rms_golden() -> dict[str, dict[str, np.ndarray]]:
    data = np.load(GOLDEN / "rmsnorm_golden.npz")
    cases: dict[str, dict[str, np.ndarray]] = {}
    for key in data.files:
        name, field = key.split("/")
        cases.setdefault(name, {})[field] = data[key]
    return cases


DECODE_GOLDEN = load_decode_golden()
RMS_GOLDEN = load_rms_golden()


def golden_tensors(case: dict[str, np.ndarray], dtype: torch.dtype = torch.float32):
    return (
        torch.from_numpy(case["q"].astype(np.float32)).to(dtype),
        torch.from_numpy(case["k_cache"].astype(np.float32)).to(dtype),
        torch.from_numpy(case["v_cache"].astype(np.float32)).to(dtype),
        torch.from_numpy(case["block_table"]),
        torch.from_numpy(case["seq_lens"]),
        float(case["scale"]),
    )


# ------------------------------------------------------------------ RMSNorm


def test_rms_norm_unit_rms_output():
    """With weight 1 and eps 0 the output has mean square 1 (original tests/test_reference.py:12-15).
    The oracle computes in float32, so float32 tolerance."""
    x = torch.randn(8, 512, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    y = ref.rms_norm(x, torch.ones(512, dtype=torch.float64), eps=0.0)
    torch.testing.assert_close(y.pow(2).mean(-1), torch.ones(8, dtype=torch.float64), atol=1e-6, rtol=1e-6)


def test_rms_norm_matches_torch_builtin():
    x = torch.randn(4, 64)
    w = torch.randn(64)
    torch.testing.assert_close(ref.rms_norm(x, w, eps=1e-5), torch.nn.functional.rms_norm(x, (64,), w, eps=1e-5))


def test_rms_norm_closed_form():
    """x = [3, 4]: mean square 12.5, so y = x / sqrt(12.5) * w exactly (to fp32)."""
    x = torch.tensor([[3.0, 4.0]])
    w = torch.tensor([2.0, -1.0])
    want = torch.tensor([[3.0 / math.sqrt(12.5) * 2.0, -4.0 / math.sqrt(12.5)]])
    torch.testing.assert_close(ref.rms_norm(x, w, eps=0.0), want, atol=1e-7, rtol=1e-7)


@pytest.mark.parametrize("name", sorted(RMS_GOLDEN))
def test_rms_norm_golden(name):
    case = RMS_GOLDEN[name]
    x = torch.from_numpy(case["x"].astype(np.float32))
    w = torch.from_numpy(case["weight"].astype(np.float32))
    eps = float(case["eps"])
    got = ref.rms_norm(x, w, eps)
    torch.testing.assert_close(got, torch.from_numpy(case["expected_rms_x"]), atol=2e-6, rtol=2e-6)


@pytest.mark.parametrize("name", sorted(RMS_GOLDEN))
def test_fused_residual_is_the_correctly_rounded_sum(name):
    """fp16: dtype(f32(x) + f32(r)) equals the float64 sum rounded once (24 >= 2*11 + 2)."""
    case = RMS_GOLDEN[name]
    x = torch.from_numpy(case["x"])
    r = torch.from_numpy(case["residual"])
    w = torch.from_numpy(case["weight"])
    out, res = ref.fused_add_rms_norm(x, r, w, float(case["eps"]))
    assert torch.equal(res, torch.from_numpy(case["expected_residual_f16"]))
    torch.testing.assert_close(out.float(), torch.from_numpy(case["expected_out_f16_res"]), atol=2e-3, rtol=2e-3)


def test_fused_residual_bf16_correctly_rounded():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    r = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    _, res = ref.fused_add_rms_norm(x, r, torch.ones(256, dtype=torch.bfloat16))
    exact = (x.double() + r.double()).to(torch.bfloat16)
    assert torch.equal(res, exact)


def test_rms_norm_brute_force_agrees():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 5, 48, generator=g)
    w = torch.randn(48, generator=g)
    want = brute.rms_norm_f64(x.numpy(), w.numpy(), 1e-6)
    torch.testing.assert_close(ref.rms_norm(x, w, 1e-6).double(), torch.from_numpy(want), atol=1e-5, rtol=1e-5)


def test_zero_rows_stay_finite():
    assert torch.isfinite(ref.rms_norm(torch.zeros(2, 32), torch.ones(32), eps=1e-6)).all()


# --------------------------------------------------------- decode attention


@pytest.mark.parametrize("name", sorted(DECODE_GOLDEN))
def test_decode_golden(name):
    q, k, v, bt, lens, scale = golden_tensors(DECODE_GOLDEN[name])
    got = ref.paged_decode_attention(q, k, v, bt, lens, scale)
    assert torch.isfinite(got).all(), "a NaN-poisoned spare page leaked into the result"
    torch.testing.assert_close(
        got.double(), torch.from_numpy(DECODE_GOLDEN[name]["expected"]), atol=1e-5, rtol=1e-5
    )


@pytest.mark.parametrize(("hq", "hkv"), [(4, 4), (8, 2), (8, 1), (32, 8), (32, 1)])
def test_paged_reference_matches_dense_sdpa(hq, hkv):
    """Original tests/test_reference.py:27-35: paged restatement vs SDPA on contiguous K/V."""
    q, kv, keys, values = random_decode_problem([1, 16, 17, 50], hq, hkv, 32, 16, dtype=torch.float32)
    torch.testing.assert_close(
        ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens),
        ref.dense_decode_attention(q, keys, values),
        atol=1e-5,
        rtol=1e-5,
    )


def test_one_hot_attention_returns_that_value():
    """Original tests/test_paged_attention.py:81-91: one key far more aligned than the rest."""
    head_dim = 32
    keys = [torch.zeros(20, 1, head_dim)]
    values = [torch.arange(20, dtype=torch.float32)[:, None, None].expand(20, 1, head_dim).clone()]
    keys[0][13, 0, 0] = 100.0
    kv = build_paged_kv(keys, values, page_size=16)
    q = torch.zeros(1, 1, head_dim)
    q[0, 0, 0] = 1.0
    out = ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, scale=1.0)
    torch.testing.assert_close(out, torch.full_like(out, 13.0), atol=1e-4, rtol=0)


def test_single_token_returns_its_value():
    q, kv, _, values = random_decode_problem([1], 4, 2, 32, 16, dtype=torch.float32)
    out = ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
    want = values[0][0].repeat_interleave(2, dim=0)  # query head h reads kv head h // 2
    torch.testing.assert_close(out[0], want, atol=0, rtol=0)


def test_equal_scores_average_the_values():
    """Identical keys give a uniform softmax: the output is the mean of V."""
    n = 37
    keys = [torch.ones(n, 1, 16)]
    values = [torch.randn(n, 1, 16)]
    kv = build_paged_kv(keys, values, page_size=16)
    q = torch.randn(1, 3, 16)
    out = ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
    torch.testing.assert_close(out[0], values[0][:, 0].mean(0).expand(3, 16), atol=1e-6, rtol=1e-6)


def test_poisoned_spare_pages_are_never_read():
    """Original tests/test_paged_attention.py:56-62 with 1e4, and NaN (stricter)."""
    for poison in (1e4, float("nan")):
        q, kv, _, _ = random_decode_problem([20, 9], 4, 4, 32, 16, dtype=torch.float32, poison=poison)
        out = ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
        assert torch.isfinite(out).all() and out.abs().max() < 10


def test_decode_brute_force_agrees_on_random_problem():
    q, kv, _, _ = random_decode_problem([3, 16, 17, 40], 6, 3, 32, 16, dtype=torch.float32, seed=7)
    want = brute.decode_f64(
        q.numpy(), kv.k_cache.numpy(), kv.v_cache.numpy(), kv.block_table.numpy(), kv.seq_lens.numpy(), 32**-0.5
    )
    got = ref.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens)
    torch.testing.assert_close(got.double(), torch.from_numpy(want), atol=1e-5, rtol=1e-5)


# ------------------------------------------------- planted mistakes are caught


def _planted(variant: str):
    """A copy of the oracle's decode with one plausible mistake planted in it."""

    def run(q, k_cache, v_cache, block_table, seq_lens, scale):
        batch, hq, d = q.shape
        p, hkv = k_cache.shape[1], k_cache.shape[2]
        group = hq // hkv
        out = torch.empty_like(q)
        for b in range(batch):
            length = int(seq_lens[b]) + (1 if variant == "length+1" else 0)
            pages = block_table[b, : (length + p - 1) // p].long()
            if variant == "page_order" and pages.numel() > 1:
                pages = pages.flip(0)
            k = k_cache[pages].reshape(-1, hkv, d)[:length].float()
            v = v_cache[pages].reshape(-1, hkv, d)[:length].float()
            if variant == "gqa_tiled":
                kk = k.permute(1, 0, 2).repeat(group, 1, 1)
                vv = v.permute(1, 0, 2).repeat(group, 1, 1)
            else:
                kk = k.permute(1, 0, 2).repeat_interleave(group, dim=0)
                vv = v.permute(1, 0, 2).repeat_interleave(group, dim=0)
            s = torch.einsum("hd,hld->hl", q[b].float(), kk)
            s = s if variant == "no_scale" else s * scale
            pr = torch.softmax(s, dim=-1)
            out[b] = torch.einsum("hl,hld->hd", pr, vv)
        return out

    return run


@pytest.mark.parametrize("variant", ["gqa_tiled", "no_scale", "length+1", "page_order"])
def test_golden_vectors_reject_planted_mistakes(variant):
    rejected = 0
    for case in DECODE_GOLDEN.values():
        q, k, v, bt, lens, scale = golden_tensors(case)
        got = _planted(variant)(q, k, v, bt, lens, scale).double()
        want = torch.from_numpy(case["expected"])
        if not torch.allclose(got, want, atol=1e-5, rtol=1e-5, equal_nan=False):
            rejected += 1
    assert rejected > 0, f"golden vectors did not catch the planted mistake {variant!r}"
    # And the unmutated copy passes, so the rejection is the mistake's doing.
    for case in DECODE_GOLDEN.values():
        q, k, v, bt, lens, scale = golden_tensors(case)
        got = _planted("none")(q, k, v, bt, lens, scale).double()
        torch.testing.assert_close(got, torch.from_numpy(case["expected"]), atol=1e-5, rtol=1e-5)


def test_rms_golden_rejects_rounding_after_normalising():
    """Normalising the unrounded fp32 sum (the wrong rounding point) changes the result."""
    mismatched = 0
    for case in RMS_GOLDEN.values():
        x = torch.from_numpy(case["x"])
        r = torch.from_numpy(case["residual"])
        w = torch.from_numpy(case["weight"])
        wrong = ref.rms_norm(x.float() + r.float(), w.float(), float(case["eps"])).to(torch.float16)
        right = torch.from_numpy(case["expected_out_f16_res"]).to(torch.float16)
        mismatched += int(not torch.equal(wrong, right))
    assert mismatched > 0
