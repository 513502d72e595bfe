"""Seeded random sweep of RMSNorm / fused add+RMSNorm against the CPU oracle.

Each case draws dtype, row count, hidden size (odd, prime, vector-aligned and
past the register-resident limit), row stride and start alignment of x, eps,
and whether a residual is fused, from a fixed seed. The residual must match
bit for bit; the output within the tolerance table (and 1 ulp for 16-bit)."""

from __future__ import annotations

import random

import pytest
import torch

from oracle import reference as ref
from tests.conftest import tolerance, ulp_distance

pytestmark = pytest.mark.gpu


def draw_case(seed: int):
    rng = random.Random(seed)
    dtype = rng.choice([torch.float32, torch.float16, torch.bfloat16])
    hidden = rng.choice([1, 7, 8, 63, 100, 127, 1000, 4096, 4097, 5120, 8191, 8192, 13824, 16384, 70001])
    rows = rng.choice([1, 2, 3, 17, 64, 300])
    pad = rng.choice([0, 0, 1, 8, 33])  # extra row elements: stride = hidden + pad
    offset = rng.choice([0, 0, 1, 8])  # x starts this many elements into its buffer
    eps = rng.choice([1e-6, 1e-5, 1e-3])
    fused = rng.random() < 0.6
    return dtype, rows, hidden, pad, offset, eps, fused


@pytest.mark.parametrize("seed", range(96))
def test_random_rmsnorm_case(gpu_ops, seed):
    dtype, rows, hidden, pad, offset, eps, fused = draw_case(seed)
    case = f"seed={seed} dtype={dtype} rows={rows} hidden={hidden} pad={pad} offset={offset} eps={eps} fused={fused}"
    print(case, flush=True)
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(rows * (hidden + pad) + offset, generator=g).to(dtype).cuda()
    x = base[offset:].as_strided((rows, hidden), (hidden + pad, 1))
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype).cuda()
    out = torch.empty(rows, hidden, dtype=dtype, device="cuda")
    if fused:
        r = torch.randn(rows, hidden, generator=g).to(dtype).cuda()
        r_in = r.clone()
        torch.ops.kernel_lab.fused_add_rms_norm(out, x, r, w, eps)
        want_out, want_res = ref.fused_add_rms_norm(x.cpu(), r_in.cpu(), w.cpu(), eps)
        assert torch.equal(r.cpu(), want_res), case
    else:
        torch.ops.kernel_lab.rms_norm(out, x, w, eps)
        want_out = ref.rms_norm(x.cpu(), w.cpu(), eps)
    torch.testing.assert_close(out.cpu(), want_out, **tolerance(dtype), msg=lambda m: f"{case}: {m}")
    if dtype != torch.float32:
        assert ulp_distance(out.cpu(), want_out) <= 1, case
