"""Write the golden vectors in tests/golden/ (run from the repository root):

    python tests/golden/make_golden.py

Inputs come from a seeded NumPy PCG64 stream and are rounded to fp16, so the
same values are exact in fp16 and fp32. Expected outputs come from the float64
brute force in oracle/brute.py, which is independent of the float32
restatement the tests check. The original project ships no golden files, so
these vectors are this build's own; the original tests' known answers (one-hot
attention, byte counts) are asserted directly in the tests.

Decode cases cover page boundaries (L = 1, 15/16/17, 31/33), GQA, MQA (group
32), MHA, page sizes 16 and 32, head dims 32..256, and NaN-poisoned spare
pages (never read by a correct implementation).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.brute import decode_f64, rms_norm_f64  # noqa: E402

OUT = Path(__file__).resolve().parent

DECODE_CASES = {
    # name: (seq_lens, num_q_heads, num_kv_heads, head_dim, page_size)
    "gqa_d32_p16": ([1, 15, 16, 17, 33, 70], 8, 2, 32, 16),
    "mqa_d64_p16": ([33, 5], 8, 1, 64, 16),
    "mha_d64_p32": ([31, 70], 4, 4, 64, 32),
    "llama_d128_p16": ([16, 40], 32, 8, 128, 16),
    "mqa_g32_d128_p16": ([47, 200], 32, 1, 128, 16),
    "gqa_d256_p16": ([50], 4, 2, 256, 16),
}

RMS_CASES = {
    # name: (rows, hidden, eps)
    "odd_3x100": (3, 100, 1e-6),
    "llama_2x4096": (2, 4096, 1e-6),
    "tiny_1x64": (1, 64, 1e-5),
}


def f16(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16)


def decode_case(rng: np.random.Generator, lens, hq, hkv, d, p) -> dict[str, np.ndarray]:
    needed = [(n + p - 1) // p for n in lens]
    extra = 3
    total = sum(needed) + extra
    k_cache = np.full((total, p, hkv, d), np.nan, dtype=np.float16)
    v_cache = np.full_like(k_cache, np.nan)
    order = rng.permutation(total)
    table = np.zeros((len(lens), max(needed)), dtype=np.int32)
    q = f16(rng.standard_normal((len(lens), hq, d)))
    cursor = 0
    for b, n in enumerate(lens):
        k = f16(rng.standard_normal((n, hkv, d)))
        v = f16(rng.standard_normal((n, hkv, d)))
        for j in range(needed[b]):
            page = int(order[cursor])
            cursor += 1
            table[b, j] = page
            lo, hi = j * p, min((j + 1) * p, n)
            k_cache[page, : hi - lo] = k[lo:hi]
            v_cache[page, : hi - lo] = v[lo:hi]
            k_cache[page, hi - lo :] = 0
            v_cache[page, hi - lo :] = 0
    seq_lens = np.asarray(lens, dtype=np.int32)
    scale = d**-0.5
    expected = decode_f64(q, k_cache, v_cache, table, seq_lens, scale)
    return {
        "q": q,
        "k_cache": k_cache,
        "v_cache": v_cache,
        "block_table": table,
        "seq_lens": seq_lens,
        "scale": np.float64(scale),
        "expected": expected,
    }


def rms_case(rng: np.random.Generator, rows, hidden, eps) -> dict[str, np.ndarray]:
    x = f16(rng.standard_normal((rows, hidden)))
    r = f16(rng.standard_normal((rows, hidden)))
    w = f16(1.0 + 0.1 * rng.standard_normal(hidden))
    # Correctly rounded fp16 sum: float64 add (exact here) then one rounding.
    res16 = (x.astype(np.float64) + r.astype(np.float64)).astype(np.float16)
    return {
        "x": x,
        "residual": r,
        "weight": w,
        "eps": np.float64(eps),
        "expected_residual_f16": res16,
        "expected_out_f16_res": rms_norm_f64(res16.astype(np.float64), w, eps).astype(np.float32),
        "expected_rms_x": rms_norm_f64(x.astype(np.float64), w, eps).astype(np.float32),
    }


def main() -> int:
    rng = np.random.Generator(np.random.PCG64(20261201))
    decode = {}
    for name, (lens, hq, hkv, d, p) in DECODE_CASES.items():
        for key, val in decode_case(rng, lens, hq, hkv, d, p).items():
            decode[f"{name}/{key}"] = val
    np.savez_compressed(OUT / "decode_golden.npz", **decode)
    rms = {}
    for name, (rows, hidden, eps) in RMS_CASES.items():
        for key, val in rms_case(rng, rows, hidden, eps).items():
            rms[f"{name}/{key}"] = val
    np.savez_compressed(OUT / "rmsnorm_golden.npz", **rms)
    for f in ("decode_golden.npz", "rmsnorm_golden.npz"):
        print(OUT / f, (OUT / f).stat().st_size, "bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
