"""Python entry points for the gfx950 kernels (``torch.ops.kernel_lab.*``).

Functions and arguments follow the original project's wrappers:

* ``rms_norm`` / ``fused_add_rms_norm`` / ``paged_decode_attention`` as in
  kernel_lab/cuda_ops.py:31-61 (caller-facing functional forms; the operators
  themselves mutate caller-allocated outputs);
* ``paged_decode_attention(..., num_splits=, max_seq_len=)`` and the
  ``ValueError`` validation of kernel_lab/triton_kernels/paged_attention.py:176-211
  and kernel_lab/triton_kernels/rmsnorm.py:59-115.

Every call runs the HIP kernels. There is no CPU or PyTorch fallback: without
the native libraries or a GPU the calls raise.
"""

from __future__ import annotations

import ctypes

import torch

from kernel_lab import _native

# num_splits value asking for the device-balanced schedule (KL_SPLITS_BALANCED).
BALANCED = -1

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)


def available() -> bool:
    return _native.available()


def why_unavailable() -> str:
    return _native.why_unavailable()


# ------------------------------------------------------------------ RMSNorm


def _check_rms(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None) -> None:
    if x.dim() < 1 or weight.dim() != 1 or x.shape[-1] != weight.shape[0]:
        raise ValueError(f"hidden size {x.shape[-1] if x.dim() else None} does not match weight {tuple(weight.shape)}")
    if residual is not None and residual.shape != x.shape:
        raise ValueError("residual must have the same shape as x")


def _rows_view(x: torch.Tensor) -> torch.Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """y = x / sqrt(mean(x^2) + eps) * weight over the last dimension."""
    _check_rms(x, weight, None)
    _native.require_ops()
    x = _rows_view(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    torch.ops.kernel_lab.rms_norm(out, x, weight.contiguous(), eps)
    return out


def fused_add_rms_norm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """Functional form: returns (out, new_residual) and leaves ``residual`` untouched.

    Use ``fused_add_rms_norm_`` (or the operator directly) to update the
    residual in place without the copy.
    """
    _check_rms(x, weight, residual)
    _native.require_ops()
    x = _rows_view(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    new_residual = residual.contiguous().clone()
    torch.ops.kernel_lab.fused_add_rms_norm(out, x, new_residual, weight.contiguous(), eps)
    return out, new_residual


def fused_add_rms_norm_(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """In-place pre-norm step: residual += x (rounded to its dtype), returns rmsnorm(residual)."""
    _check_rms(x, weight, residual)
    _native.require_ops()
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    torch.ops.kernel_lab.fused_add_rms_norm(out, _rows_view(x), residual, weight, eps)
    return out


# ---------------------------------------------------------- decode attention


def _check_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if q.dim() != 3 or k_cache.dim() != 4:
        raise ValueError("q is [batch, heads, head_dim] and the caches are [pages, page_size, kv_heads, head_dim]")
    _, num_q_heads, head_dim = q.shape
    _, page_size, num_kv_heads, head_dim_kv = k_cache.shape
    if head_dim_kv != head_dim or v_cache.shape != k_cache.shape:
        raise ValueError("q, k_cache and v_cache disagree on shape")
    if num_kv_heads < 1 or num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim must be a power of two in [16, 256], got {head_dim}")
    if page_size < 1:
        raise ValueError(f"page_size must be >= 1, got {page_size}")
    if q.stride(-1) != 1 or k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise ValueError("the head dimension must be contiguous")


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
    num_splits: int | None = None,
    max_seq_len: int | None = None,
    out: torch.Tensor | None = None,
    k_scale: torch.Tensor | float | None = None,
    v_scale: torch.Tensor | float | None = None,
) -> torch.Tensor:
    """Single-token decode attention over a paged KV cache (NHD layout).

    ``num_splits`` overrides the split planner (``None`` or 0: planner;
    ``BALANCED`` (-1): pages of all sequences cut into equal per-workgroup
    ranges on the device, for batches of very uneven lengths).
    ``max_seq_len`` bounds the work per sequence; without it the block table's
    width is used, so ``seq_lens`` is never read back to the host.

    A ``torch.float8_e4m3fn`` cache holds FP8 codes; ``k_scale`` and
    ``v_scale`` (one float32 per KV head, or one float for all) give head h's
    values as ``k_scale[h] * k`` and ``v_scale[h] * v``. q is then float16 or
    bfloat16 and the output has q's dtype.
    """
    _check_decode(q, k_cache, v_cache)
    _native.require_ops()
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if k_cache.dtype == torch.float8_e4m3fn or v_cache.dtype == torch.float8_e4m3fn:
        if k_scale is None or v_scale is None:
            raise ValueError("an FP8 cache needs k_scale and v_scale")
        hkv = k_cache.shape[2]
        ks = _head_scales(k_scale, hkv, q.device)
        vs = _head_scales(v_scale, hkv, q.device)
        torch.ops.kernel_lab.paged_decode_attention_fp8(
            out, q, k_cache, v_cache, block_table, seq_lens, scale, ks, vs, int(num_splits or 0), int(max_seq_len or 0)
        )
        return out
    if k_scale is not None or v_scale is not None:
        raise ValueError("k_scale and v_scale apply to an FP8 (float8_e4m3fn) cache only")
    if num_splits is None and max_seq_len is None:
        torch.ops.kernel_lab.paged_decode_attention(out, q, k_cache, v_cache, block_table, seq_lens, scale)
    else:
        torch.ops.kernel_lab.paged_decode_attention.splits(
            out, q, k_cache, v_cache, block_table, seq_lens, scale, int(num_splits or 0), int(max_seq_len or 0)
        )
    return out


def cascade_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    prefix_block_table: torch.Tensor,
    prefix_len: int | torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode with a prefix shared by every sequence (cascade attention).

    Sequence b attends over the ``prefix_len`` tokens on pages
    ``prefix_block_table`` (1-D int32, shared) followed by its own
    ``seq_lens[b]`` tokens on ``block_table[b]``; both sets of pages live in
    ``k_cache`` / ``v_cache``. ``prefix_len`` may be a one-element int32 device
    tensor (no host sync) or an int. The prefix's K/V is streamed once per 32
    query heads of the whole batch instead of once per sequence.
    """
    _check_decode(q, k_cache, v_cache)
    _native.require_ops()
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if not isinstance(prefix_len, torch.Tensor):
        prefix_len = torch.tensor([int(prefix_len)], dtype=torch.int32, device=q.device)
    prefix_block_table = prefix_block_table.reshape(-1).to(torch.int32).contiguous()
    torch.ops.kernel_lab.cascade_decode_attention(
        out, q, k_cache, v_cache, prefix_block_table, prefix_len.reshape(1), block_table, seq_lens, scale
    )
    return out


def _head_scales(s: torch.Tensor | float, num_kv_heads: int, device: torch.device) -> torch.Tensor:
    """Per-KV-head float32 scales on the device: a tensor of num_kv_heads
    values, or one number (or one-element tensor) for every head."""
    t = torch.as_tensor(s, dtype=torch.float32, device=device).reshape(-1)
    if t.numel() == 1:
        t = t.expand(num_kv_heads)
    if t.numel() != num_kv_heads:
        raise ValueError(f"expected {num_kv_heads} scales (one per KV head), got {t.numel()}")
    return t.contiguous()


def plan_decode(
    dtype: torch.dtype,
    batch: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    max_pages: int,
    num_splits: int = 0,
    cu_count: int = 0,
) -> tuple[int, int]:
    """(num_splits, workspace_bytes) the launch will use; host arithmetic only."""
    splits = ctypes.c_int(0)
    ws = ctypes.c_size_t(0)
    status = _native.core().kl_paged_decode_plan(
        _native.DTYPE_CODES[dtype],
        batch,
        num_q_heads,
        num_kv_heads,
        head_dim,
        page_size,
        max_pages,
        num_splits,
        cu_count,
        ctypes.byref(splits),
        ctypes.byref(ws),
    )
    if status != _native.KL_OK:
        raise ValueError(f"{_native.status_string(status)}: {_native.last_error()}")
    return splits.value, ws.value
