"""Pins for the FP8 (OCP E4M3) KV-cache oracle and the quantizing fixture.

The original project has no FP8 implementation to compare against (it lists
the format as planned work, README.md:98), so the oracle's definition is the
16-bit path's math on dequantised values. What pins it: the E4M3 decoding
checked code by code against the OCP bit layout, scale identities that hold
bit for bit with power-of-two scales, a float64 brute force, and a one-hot
known answer that a swapped or misplaced scale gets wrong.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from kernel_lab.kv_cache import FP8_E4M3_MAX, build_paged_kv, quantize_fp8, random_decode_problem, used_pages
from oracle import brute
from oracle import reference as ref


def test_torch_e4m3_widening_matches_the_ocp_bit_layout():
    table = brute.e4m3_table()
    got = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    nan = np.isnan(table)
    assert list(np.flatnonzero(nan)) == [0x7F, 0xFF]
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], table[~nan])
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(table[~nan]))
    assert table[0x7E] == FP8_E4M3_MAX and table[0x01] == 2.0**-9


def test_e4m3_layout_spot_values():
    """Hand-decoded codes: 0x38 = 1.0, 0x3C = 1.5, 0xC0 = -2.0, 0x08 = 2^-6 (smallest normal)."""
    assert brute.e4m3_decode(0x38) == 1.0
    assert brute.e4m3_decode(0x3C) == 1.5
    assert brute.e4m3_decode(0xC0) == -2.0
    assert brute.e4m3_decode(0x08) == 2.0**-6
    assert brute.e4m3_decode(0x80) == 0.0 and math.copysign(1.0, brute.e4m3_decode(0x80)) == -1.0


def _fp8_problem(lens, hq, hkv, d, page=16, seed=0, poison=float("nan")):
    q, kv, _, _ = random_decode_problem(lens, hq, hkv, d, page, dtype=torch.float32, seed=seed, poison=poison)
    kv8, ks, vs = quantize_fp8(kv)
    return q, kv, kv8, ks, vs


def test_quantizer_scales_and_round_trip():
    q, kv, kv8, ks, vs = _fp8_problem([40, 17, 5], 8, 2, 64)
    pages = used_pages(kv)
    for cache, codes, s in ((kv.k_cache, kv8.k_cache, ks), (kv.v_cache, kv8.v_cache, vs)):
        x = cache[pages]
        back = codes[pages].float() * s[None, None, :, None]
        amax = x.abs().amax(dim=(0, 1, 3))
        torch.testing.assert_close(s, amax / FP8_E4M3_MAX)
        # Largest code of each head is +-448 exactly; errors within half an E4M3 ulp.
        assert torch.equal(codes[pages].float().abs().amax(dim=(0, 1, 3)), torch.full_like(s, FP8_E4M3_MAX))
        bound = torch.maximum(x.abs() * 2.0**-4, (2.0**-10) * s[None, None, :, None].expand_as(x))
        assert ((back - x).abs() <= bound * (1 + 1e-6)).all()


def test_quantized_spares_stay_nan():
    _, kv, kv8, _, _ = _fp8_problem([20, 9], 4, 4, 64)
    spare = torch.ones(kv.k_cache.shape[0], dtype=torch.bool)
    spare[used_pages(kv)] = False
    assert spare.any() and torch.isnan(kv8.k_cache[spare].float()).all()


def test_fp8_oracle_equals_the_16bit_math_on_dequantised_values():
    q, kv, kv8, ks, vs = _fp8_problem([33, 7, 64], 8, 4, 64, seed=3)
    got = ref.paged_decode_attention_fp8(q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens, ks, vs)
    table = torch.from_numpy(brute.e4m3_table())
    k = table[kv8.k_cache.view(torch.uint8).long()] * ks.double()[None, None, :, None]
    v = table[kv8.v_cache.view(torch.uint8).long()] * vs.double()[None, None, :, None]
    want = brute.decode_f64(q.numpy(), k.numpy(), v.numpy(), kv.block_table.numpy(), kv.seq_lens.numpy(), 64**-0.5)
    torch.testing.assert_close(got.double(), torch.from_numpy(want), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("c", [0.5, 4.0])
def test_k_scale_folds_into_the_score_scale(c):
    """q.(c k) * s == q.k * (c s) bit for bit when c is a power of two."""
    q, _, kv8, ks, vs = _fp8_problem([25, 50], 8, 2, 64, seed=5)
    args = (q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens)
    a = ref.paged_decode_attention_fp8(*args, ks * c, vs, scale=0.1)
    b = ref.paged_decode_attention_fp8(*args, ks, vs, scale=0.1 * c)
    assert torch.equal(a, b)
    assert not torch.allclose(a, ref.paged_decode_attention_fp8(*args, ks, vs, scale=0.1))


def test_v_scale_multiplies_the_output():
    q, _, kv8, ks, vs = _fp8_problem([25, 50], 8, 2, 64, seed=6)
    args = (q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens, ks)
    assert torch.equal(ref.paged_decode_attention_fp8(*args, vs * 2), 2 * ref.paged_decode_attention_fp8(*args, vs))


def test_fp8_one_hot_known_answer_with_scales():
    """One-hot of the original tests (13.0) with E4M3-exact values: key 96 at
    token 13, values = token index; k_scale 0.5 keeps token 13 dominant
    (score 48), v_scale 2 doubles it: 26. Swapping the scales gives 13."""
    d = 64
    keys = [torch.zeros(16, 1, d)]
    keys[0][13, 0, 0] = 96.0
    values = [torch.arange(16, dtype=torch.float32)[:, None, None].expand(16, 1, d).clone()]
    kv = build_paged_kv(keys, values, page_size=16)
    k8 = kv.k_cache.to(torch.float8_e4m3fn)
    v8 = kv.v_cache.to(torch.float8_e4m3fn)
    assert torch.equal(k8.float()[kv.block_table[0, 0]], kv.k_cache[kv.block_table[0, 0]])  # exact codes
    q = torch.zeros(1, 1, d, dtype=torch.float16)
    q[0, 0, 0] = 1.0
    out = ref.paged_decode_attention_fp8(
        q, k8, v8, kv.block_table, kv.seq_lens, torch.tensor([0.5]), torch.tensor([2.0]), scale=1.0
    )
    torch.testing.assert_close(out.float(), torch.full((1, 1, d), 26.0), atol=1e-3, rtol=0)
