"""Float64 NumPy brute force, written independently of oracle/reference.py.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Small inputs only: the
decode loops run over every (sequence, query head, token) in Python.

It follows the definitions, not the restatement: explicit per-token page
lookup through the block table, the GQA rule "query head h reads KV head
h // group", a max-subtracted softmax, and float64 throughout.
"""

from __future__ import annotations

import numpy as np


def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * weight over the last axis, in float64."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    out = np.empty_like(x)
    flat_in = x.reshape(-1, x.shape[-1])
    flat_out = out.reshape(-1, x.shape[-1])
    for i, row in enumerate(flat_in):
        ms = float(np.dot(row, row)) / row.size
        flat_out[i] = row / np.sqrt(ms + eps) * w
    return out


def decode_f64(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    block_table: np.ndarray,
    seq_lens: np.ndarray,
    scale: float,
) -> np.ndarray:
    """softmax(scale * q.K^T) V per (sequence, query head), token by token, float64."""
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache, dtype=np.float64)
    v_cache = np.asarray(v_cache, dtype=np.float64)
    batch, num_q_heads, head_dim = q.shape
    page_size, num_kv_heads = k_cache.shape[1], k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    out = np.zeros((batch, num_q_heads, head_dim), dtype=np.float64)
    for b in range(batch):
        length = int(seq_lens[b])
        for h in range(num_q_heads):
            kvh = h // group
            scores = np.empty(length, dtype=np.float64)
            vals = np.empty((length, head_dim), dtype=np.float64)
            for t in range(length):
                page = int(block_table[b, t // page_size])
                scores[t] = scale * float(np.dot(q[b, h], k_cache[page, t % page_size, kvh]))
                vals[t] = v_cache[page, t % page_size, kvh]
            if length == 0:
                continue
            w = np.exp(scores - scores.max())
            out[b, h] = (w[:, None] * vals).sum(axis=0) / w.sum()
    return out


def e4m3_decode(code: int) -> float:
    """Value of an OCP FP8 E4M3 ("e4m3fn") code, from the bit layout alone:
    sign bit 7, exponent bits 6-3 (bias 7), mantissa bits 2-0; exponent 0 is
    subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinities."""
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return float("nan")
    if exp == 0:
        return sign * (man / 8.0) * 2.0**-6
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def e4m3_table() -> np.ndarray:
    """Float64 values of all 256 E4M3 codes, indexed by code."""
    return np.array([e4m3_decode(c) for c in range(256)], dtype=np.float64)
