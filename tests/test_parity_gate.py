"""The decode parity gate itself (tests/conftest.py: decode_parity, ulp_of), on the CPU.

The gate bounds every output element by one output ulp of the unrounded
float32 oracle plus 1e-6. These tests pin what it accepts and rejects:

* ulp spacings at known points of each format (normal, subnormal, zero);
* a correctly rounded result passes, one off by two ulps fails;
* at the magnitude of a 131,072-token context (rms about 0.005), an error
  the original project's 1.6e-2 bf16 tolerance cannot see (a dropped
  segment's worth) fails;
* an emulation of the decode's PV step: softmax weights rounded once to bf16
  (what the kernel did before it split them) fail the gate at a 4,096-token
  context, and the high/low split the kernel uses now passes it.
"""

from __future__ import annotations

import pytest
import torch

from tests.conftest import decode_parity, tolerance, ulp_of


@pytest.mark.parametrize(
    ("x", "dtype", "spacing"),
    [
        (1.0, torch.float16, 2.0**-10),
        (1.5, torch.float16, 2.0**-10),
        (0.026, torch.float16, 2.0**-16),
        (2.0**-20, torch.float16, 2.0**-24),  # subnormal
        (0.0, torch.float16, 2.0**-24),
        (1.0, torch.bfloat16, 2.0**-7),
        (-3.0, torch.bfloat16, 2.0**-6),
        (0.0046, torch.bfloat16, 2.0**-15),
        (0.0, torch.bfloat16, 2.0**-133),
        (1.0, torch.float32, 2.0**-23),
    ],
)
def test_ulp_spacing(x, dtype, spacing):
    assert float(ulp_of(torch.tensor([x]), dtype)[0]) == spacing


def test_ulp_matches_nextafter_for_representable_values():
    g = torch.Generator().manual_seed(0)
    for dtype in (torch.float16, torch.bfloat16):
        v = (torch.randn(4000, generator=g) * 10.0 ** torch.randint(-6, 3, (4000,), generator=g)).to(dtype)
        v = v[v != 0].float()
        up = torch.nextafter(v.to(dtype).float().double(), torch.tensor(float("inf"), dtype=torch.float64))
        # next representable value of `dtype` above |v|: add one to the bit pattern of |v|
        bits = v.abs().to(dtype).view(torch.int16) + 1
        nxt = bits.view(dtype).double()
        assert torch.equal(nxt - v.abs().double(), ulp_of(v, dtype)), dtype
        assert (up > v.double()).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rounded_result_passes_and_two_ulps_fail(dtype):
    g = torch.Generator().manual_seed(1)
    want = torch.randn(4, 8, 128, generator=g) * 0.03
    decode_parity(want.to(dtype), want, dtype, "rounded")
    bad = want.to(dtype).clone()
    flat = bad.view(-1)
    i = int(want.abs().view(-1).argmax())
    flat[i] = (want.view(-1)[i] + 2 * ulp_of(want.view(-1)[i : i + 1], dtype)[0]).to(dtype)
    with pytest.raises(AssertionError, match="unrounded oracle"):
        decode_parity(bad, want, dtype, "two ulps")


def test_dropped_segment_at_long_context_fails_but_passes_the_table():
    """At ctx 131,072 with N(0,1) data the output rms is about 0.0046; losing
    one of 16 segments moves outputs by about a quarter of that, well inside
    the original 1.6e-2 bf16 tolerance."""
    g = torch.Generator().manual_seed(2)
    want = torch.randn(2, 64, 128, generator=g) * 0.0046
    got = (want + torch.randn(want.shape, generator=g) * 0.0046 / 4).to(torch.bfloat16)
    torch.testing.assert_close(got, want.to(torch.bfloat16), **tolerance(torch.bfloat16))  # the table is blind
    with pytest.raises(AssertionError, match="unrounded oracle"):
        decode_parity(got, want, torch.bfloat16, "dropped segment")


def _pv(p: torch.Tensor, v: torch.Tensor, l: torch.Tensor, mode: str, dtype: torch.dtype) -> torch.Tensor:
    """sum_t p[h, t] v[t, d] / l[h] with p carried as the kernel carries it."""
    if mode == "rounded":
        w = p.to(dtype).double()
    else:  # split: E(p) + E(p - E(p)), each product exact, summed in float64
        hi = p.to(dtype)
        lo = (p - hi.float()).to(dtype)
        w = hi.double() + lo.double()
    return (w @ v.double()) / l.double()[:, None]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_softmax_weight_format(dtype):
    """Emulates one KV head of the decode (8 query heads, 4,096 tokens, N(0,1)
    q, K, V in `dtype`): scores and weights in float32 as the kernel makes
    them, the PV sum exact. Weights rounded once to bf16 leave outputs near
    zero several ulps off the float32 oracle; the split passes."""
    g = torch.Generator().manual_seed(3)
    heads, length, d = 8, 4096, 128
    q = torch.randn(heads, d, generator=g).to(dtype).float()
    k = torch.randn(length, d, generator=g).to(dtype).float()
    v = torch.randn(length, d, generator=g).to(dtype).float()
    s = (q @ k.T) * (d**-0.5) * 1.4426950408889634  # log2 domain
    p = torch.exp2(s - s.max(dim=1, keepdim=True).values)
    l = p.sum(dim=1)
    want = torch.softmax((q @ k.T) * d**-0.5, dim=1) @ v  # the oracle's float32 math
    split = _pv(p, v, l, "split", dtype).float().to(dtype)
    decode_parity(split, want, dtype, "split weights")
    if dtype == torch.bfloat16:
        rounded = _pv(p, v, l, "rounded", dtype).float().to(dtype)
        with pytest.raises(AssertionError, match="unrounded oracle"):
            decode_parity(rounded, want, dtype, "bf16 weights")
