"""gfx950 RMSNorm / fused add+RMSNorm against the CPU oracle.

Shapes: the original project's native-op tests (tests/test_cuda_kernels.py:17-41),
its Triton tests (tests/test_rmsnorm.py:12-65), and the measured configs
(16x4096 fp32; {1,16,128,1024,4096} x {4096,8192} fp16/bf16). The updated
residual must match bit for bit; the normed output within the original
tolerance table, with the ulp distance to the oracle reported as at most 1.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as ref
from tests.conftest import DTYPES, tolerance, ulp_distance

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "rmsnorm_golden.npz"


def make(shape, dtype, seed=0, device="cuda"):
    """x, r ~ N(0,1), w = 1 + N(0, 0.1), drawn in that order (original tests/test_rmsnorm.py:14-19)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g).to(dtype)
    r = torch.randn(*shape, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(dtype)
    return x.to(device), r.to(device), w.to(device)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 64), (3, 100), (8, 4096), (2, 5, 8192), (1, 16), (4, 256), (2, 3, 128), (7, 1000)])
def test_rms_norm(gpu_ops, shape, dtype):
    x, _, w = make(shape, dtype)
    got = gpu_ops.rms_norm(x, w)
    want = ref.rms_norm(x.cpu(), w.cpu())
    torch.testing.assert_close(got.cpu(), want, **tolerance(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(3, 100), (16, 4096), (1, 16), (4, 256), (2, 3, 128), (7, 1000)])
def test_fused_add_rms_norm(gpu_ops, shape, dtype):
    x, r, w = make(shape, dtype)
    out, res = gpu_ops.fused_add_rms_norm(x, r, w)
    ref_out, ref_res = ref.fused_add_rms_norm(x.cpu(), r.cpu(), w.cpu())
    assert torch.equal(res.cpu(), ref_res), "residual must match bit for bit"
    torch.testing.assert_close(out.cpu(), ref_out, **tolerance(dtype))
    if dtype != torch.float32:
        assert ulp_distance(out.cpu(), ref_out) <= 1


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tokens", [1, 16, 128, 1024, 4096])
@pytest.mark.parametrize("hidden", [4096, 8192])
def test_fused_add_rms_norm_benchmark_shapes(gpu_ops, tokens, hidden, dtype):
    x, r, w = make((tokens, hidden), dtype, seed=tokens + hidden)
    r_in = r.clone()
    out = torch.empty_like(x)
    torch.ops.kernel_lab.fused_add_rms_norm(out, x, r, w, 1e-6)  # in place, as a model calls it
    ref_out, ref_res = ref.fused_add_rms_norm(x.cpu(), r_in.cpu(), w.cpu())
    assert torch.equal(r.cpu(), ref_res)
    torch.testing.assert_close(out.cpu(), ref_out, **tolerance(dtype))
    assert ulp_distance(out.cpu(), ref_out) <= 1


def test_config0_fp32_16x4096(gpu_ops):
    """16 x 4096 fp32, eps 1e-6; residual bit-exact."""
    x, r, w = make((16, 4096), torch.float32)
    out, res = gpu_ops.fused_add_rms_norm(x, r, w, 1e-6)
    ref_out, ref_res = ref.fused_add_rms_norm(x.cpu(), r.cpu(), w.cpu(), 1e-6)
    assert torch.equal(res.cpu(), ref_res)
    torch.testing.assert_close(out.cpu(), ref_out, atol=1e-5, rtol=1e-5)


def test_golden_vectors(gpu_ops):
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    for name in names:
        x = torch.from_numpy(data[f"{name}/x"]).cuda()
        r = torch.from_numpy(data[f"{name}/residual"]).cuda()
        w = torch.from_numpy(data[f"{name}/weight"]).cuda()
        eps = float(data[f"{name}/eps"])
        out, res = gpu_ops.fused_add_rms_norm(x, r, w, eps)
        assert torch.equal(res.cpu(), torch.from_numpy(data[f"{name}/expected_residual_f16"]))
        want = torch.from_numpy(data[f"{name}/expected_out_f16_res"])
        torch.testing.assert_close(out.cpu().float(), want, atol=2e-3, rtol=2e-3)
        y = gpu_ops.rms_norm(x.float(), w.float(), eps)
        torch.testing.assert_close(y.cpu(), torch.from_numpy(data[f"{name}/expected_rms_x"]), atol=1e-5, rtol=1e-5)


def test_unaligned_rows_take_scalar_path(gpu_ops):
    base = torch.randn(4, 130, device="cuda", dtype=torch.float16)
    x = base[:, 1:101]  # misaligned start and odd width: no 16-byte vector loads
    w = torch.randn(100, device="cuda", dtype=torch.float16)
    torch.testing.assert_close(gpu_ops.rms_norm(x, w).cpu(), ref.rms_norm(x.cpu(), w.cpu()), **tolerance(torch.float16))
    out = torch.empty(4, 100, device="cuda", dtype=torch.float16)
    torch.ops.kernel_lab.rms_norm(out, x, w, 1e-6)  # strided rows straight into the operator
    torch.testing.assert_close(out.cpu(), ref.rms_norm(x.cpu(), w.cpu()), **tolerance(torch.float16))


def test_strided_rows_are_supported(gpu_ops):
    base = torch.randn(4, 192, device="cuda")
    x = base[:, :128]  # row stride 192, not 128
    w = torch.ones(128, device="cuda")
    torch.testing.assert_close(gpu_ops.rms_norm(x, w).cpu(), ref.rms_norm(x.cpu(), w.cpu()), atol=1e-5, rtol=1e-5)


def test_inputs_are_not_modified(gpu_ops):
    x, r, w = make((3, 64), torch.float32)
    x0, r0 = x.clone(), r.clone()
    gpu_ops.fused_add_rms_norm(x, r, w)
    assert torch.equal(x, x0) and torch.equal(r, r0)


def test_zero_rows_stay_finite(gpu_ops):
    x = torch.zeros(2, 32, device="cuda")
    assert torch.isfinite(gpu_ops.rms_norm(x, torch.ones(32, device="cuda"), eps=1e-6)).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(
    ("hidden", "fused"),
    [(16384, True), (65536, True), (100000, True), (300000, True), (300000, False), (40001, True), (12289, False)],
)
def test_wide_rows(gpu_ops, hidden, fused, dtype):
    """Rows past the register-resident limit (16-bit > 65,536, fp32 > 32,768
    aligned; > 8,192 unaligned) take the LDS-staged kernel: the row's first
    48 KiB come back from LDS and the rest is formed again from x and the
    residual, whose new value must still be written exactly once."""
    x, r, w = make((3, hidden), dtype, seed=hidden)
    if fused:
        out, res = gpu_ops.fused_add_rms_norm(x, r, w)
        ref_out, ref_res = ref.fused_add_rms_norm(x.cpu(), r.cpu(), w.cpu())
        assert torch.equal(res.cpu(), ref_res)
    else:
        out = gpu_ops.rms_norm(x, w)
        ref_out = ref.rms_norm(x.cpu(), w.cpu())
    torch.testing.assert_close(out.cpu(), ref_out, **tolerance(dtype))
    if dtype != torch.float32:
        assert ulp_distance(out.cpu(), ref_out) <= 1


@pytest.mark.parametrize(
    "layout",
    ["sliced rows", "every other middle row", "transposed leading dims", "size-one middle", "expanded rows"],
)
def test_rows_of_any_leading_layout(gpu_ops, layout):
    """The operator addresses x's rows with one stride when its leading
    dimensions nest (each spans the next), and reads a contiguous copy when
    they do not (or rows would overlap); either way the result is the oracle's."""
    base = torch.randn(4, 6, 288, device="cuda", dtype=torch.float16)
    w = (1 + 0.1 * torch.randn(256, device="cuda")).half()
    x = {
        "sliced rows": base[:, :, :256],  # row stride 288
        "every other middle row": base[:, ::2, :256],  # nested: 1728 = 576 x 3
        "transposed leading dims": base.transpose(0, 1)[:, :, :256],  # 288 != 1728 x 4: copied
        "size-one middle": base[:, 2:3, :256],  # a size-1 dimension has any stride
        "expanded rows": base[0, 0, :256].expand(5, 256),  # row stride 0: copied
    }[layout]
    out = torch.empty(x.shape, device="cuda", dtype=torch.float16)
    torch.ops.kernel_lab.rms_norm(out, x, w, 1e-6)
    want = ref.rms_norm(x.cpu(), w.cpu())
    torch.testing.assert_close(out.cpu(), want, **tolerance(torch.float16))
    assert ulp_distance(out.cpu(), want) <= 1


def test_validation_errors(gpu_ops):
    x = torch.randn(2, 32, device="cuda")
    with pytest.raises(ValueError, match="does not match"):
        gpu_ops.rms_norm(x, torch.ones(16, device="cuda"))
    with pytest.raises(ValueError, match="same shape"):
        gpu_ops.fused_add_rms_norm(x, torch.randn(2, 16, device="cuda"), torch.ones(32, device="cuda"))
    with pytest.raises(RuntimeError, match="share a dtype"):
        torch.ops.kernel_lab.rms_norm(torch.empty_like(x), x, torch.ones(32, device="cuda", dtype=torch.float16), 1e-6)


def test_empty_rows_are_a_no_op(gpu_ops):
    x = torch.empty(0, 64, device="cuda", dtype=torch.float16)
    assert gpu_ops.rms_norm(x, torch.ones(64, device="cuda", dtype=torch.float16)).shape == (0, 64)


def test_alias_schema(gpu_ops):
    """torch.ops.kernel_lab.fused_add_rmsnorm is the same operator under the north-star spelling."""
    x, r, w = make((5, 4096), torch.bfloat16)
    r1, r2 = r.clone(), r.clone()
    o1, o2 = torch.empty_like(x), torch.empty_like(x)
    torch.ops.kernel_lab.fused_add_rms_norm(o1, x, r1, w, 1e-6)
    torch.ops.kernel_lab.fused_add_rmsnorm(o2, x, r2, w, 1e-6)
    assert torch.equal(o1, o2) and torch.equal(r1, r2)
