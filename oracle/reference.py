"""Float32 PyTorch CPU restatement of kernel_lab/reference.py (Markkoby3/Kernel-lab).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Math is float32; values are
rounded to the input dtype exactly where the original rounds them: the updated
residual (before it is normalised) and each output.
"""

from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dim (reference.py:13-17)."""
    xf = x.float()
    rstd = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * rstd * weight.float()).to(x.dtype)


def fused_add_rms_norm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """(rms_norm(new_residual), new_residual) with new_residual = dtype(f32(x) + f32(residual))
    (reference.py:20-30): the sum is rounded before it is normalised."""
    new_residual = (x.float() + residual.float()).to(x.dtype)
    return rms_norm(new_residual, weight, eps), new_residual


def _gather(cache: torch.Tensor, block_table_row: torch.Tensor, length: int) -> torch.Tensor:
    """The first `length` tokens of one sequence as [L, Hkv, D] float32 (reference.py:58-61)."""
    page_size = cache.shape[1]
    pages = block_table_row[: (length + page_size - 1) // page_size].long()
    return cache[pages].reshape(-1, cache.shape[2], cache.shape[3])[:length].float()


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
) -> torch.Tensor:
    """Single-token decode attention over a paged KV cache (reference.py:33-68).

    Query head h uses KV head h // (Hq / Hkv), as repeat_interleave does in the
    original; here the group is a view ([Hkv, G, D]) instead of a copy, so a
    131072-token sequence does not materialise G copies of its K and V.
    """
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    scale = head_dim**-0.5 if scale is None else scale
    lens = [int(n) for n in seq_lens.tolist()]
    table = block_table.cpu()
    out = torch.empty_like(q)
    for b in range(batch):
        k = _gather(k_cache, table[b], lens[b])  # [L, Hkv, D]
        v = _gather(v_cache, table[b], lens[b])
        qb = q[b].float().reshape(num_kv_heads, group, head_dim)
        scores = torch.einsum("hgd,lhd->hgl", qb, k) * scale
        probs = torch.softmax(scores, dim=-1)
        out[b] = torch.einsum("hgl,lhd->hgd", probs, v).reshape(num_q_heads, head_dim).to(q.dtype)
    return out


def paged_decode_attention_fp8(
    q: torch.Tensor,
    k_codes: torch.Tensor,
    v_codes: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    scale: float | None = None,
) -> torch.Tensor:
    """Decode over an OCP FP8 E4M3 cache (float8_e4m3fn codes, same layout):
    KV head h's values are k_scale[h] * e4m3(code) and v_scale[h] * e4m3(code),
    then exactly the float32 math of paged_decode_attention, output in q's dtype.

    The original project lists this cache format as planned work
    (README.md:98) and ships no implementation, so its definition is the
    16-bit path's math on the dequantised values.
    """
    ks = k_scale.float().cpu().reshape(1, 1, -1, 1)
    vs = v_scale.float().cpu().reshape(1, 1, -1, 1)
    k = k_codes.cpu().float() * ks
    v = v_codes.cpu().float() * vs
    return paged_decode_attention(q.cpu(), k, v, block_table, seq_lens, scale)


def cascade_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    prefix_block_table: torch.Tensor,
    prefix_len: int,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
) -> torch.Tensor:
    """Shared-prefix decode: sequence b attends over the prefix's first
    prefix_len tokens (pages prefix_block_table) followed by its own seq_lens[b]
    tokens, with paged_decode_attention's float32 math over the concatenation.

    The original project names this FlashInfer feature (docs/design.md:96-100)
    without implementing it; its definition is attention over the concatenated
    token sequence.
    """
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    scale = head_dim**-0.5 if scale is None else scale
    ptable = prefix_block_table.cpu().reshape(-1)
    pk = _gather(k_cache, ptable, prefix_len)
    pv = _gather(v_cache, ptable, prefix_len)
    lens = [int(n) for n in seq_lens.tolist()]
    table = block_table.cpu()
    out = torch.empty_like(q)
    for b in range(batch):
        k = torch.cat([pk, _gather(k_cache, table[b], lens[b])])
        v = torch.cat([pv, _gather(v_cache, table[b], lens[b])])
        if k.shape[0] == 0:
            out[b] = 0
            continue
        qb = q[b].float().reshape(num_kv_heads, group, head_dim)
        probs = torch.softmax(torch.einsum("hgd,lhd->hgl", qb, k) * scale, dim=-1)
        out[b] = torch.einsum("hgl,lhd->hgd", probs, v).reshape(num_q_heads, head_dim).to(q.dtype)
    return out


def dense_decode_attention(
    q: torch.Tensor, keys: list[torch.Tensor], values: list[torch.Tensor], scale: float | None = None
) -> torch.Tensor:
    """Same computation on contiguous per-sequence K/V ([L, Hkv, D]) through SDPA
    (reference.py:71-87): an independent path (explicit repeat_interleave, library
    attention) used to cross-check the paged restatement."""
    num_q_heads = q.shape[1]
    rows = []
    for b, (k, v) in enumerate(zip(keys, values, strict=True)):
        group = num_q_heads // k.shape[1]
        kk = k.permute(1, 0, 2).repeat_interleave(group, dim=0).float()
        vv = v.permute(1, 0, 2).repeat_interleave(group, dim=0).float()
        o = torch.nn.functional.scaled_dot_product_attention(q[b].float().unsqueeze(1), kk, vv, scale=scale)
        rows.append(o.squeeze(1).to(q.dtype))
    return torch.stack(rows)
