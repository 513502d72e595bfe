"""kl_paged_decode_attention_noalloc: the decode with its split workspace in a
library-owned device array instead of a caller workspace, for callers that
cannot allocate (graph capture, allocation-free serving loops).

Called through the C-ABI (ctypes, raw pointers, the current stream), it must
give exactly the bits of kl_paged_decode_attention with a caller workspace
(same planner, same kernels), on consecutive calls whose second input is
smaller than the first (the array keeps the last call's contents), with the
in-kernel merge, the merge kernel and one split; and it must refuse a plan
that needs more than the array holds, before launching anything.

Under HIP graph capture (its main use) two captured calls replay with the
bits of the same calls made eagerly, and a process whose first call is made
during a capture (so the device's array is looked up there) works too.

Named to sort last: the round's end runs ``pytest -x``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem
from oracle import reference as ref
from tests.conftest import decode_parity

pytestmark = pytest.mark.gpu

KL_ERR_WORKSPACE = 3
KL_MERGE_NONE = 0


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _args(q, kv, out, num_splits):
    batch, hq, d = q.shape
    p, hkv = kv.k_cache.shape[1], kv.k_cache.shape[2]
    return [_native.DTYPE_CODES[q.dtype], out.data_ptr(), q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(),
            kv.block_table.data_ptr(), kv.seq_lens.data_ptr(), batch, hq, hkv, d, p, kv.block_table.stride(0),
            kv.block_table.shape[1], d**-0.5, num_splits]


def _with_workspace(q, kv, num_splits):
    """The existing entry point, with a caller workspace sized by the planner."""
    lib = _native.core()
    batch, hq, d = q.shape
    p, hkv = kv.k_cache.shape[1], kv.k_cache.shape[2]
    splits, ws = ctypes.c_int(0), ctypes.c_size_t(0)
    st = lib.kl_paged_decode_plan(_native.DTYPE_CODES[q.dtype], batch, hq, hkv, d, p, kv.block_table.shape[1],
                                  num_splits, 0, ctypes.byref(splits), ctypes.byref(ws))
    assert st == 0, _native.last_error()
    workspace = torch.empty(max(ws.value, 1), dtype=torch.uint8, device="cuda")
    out = torch.full_like(q, float("nan"))
    st = lib.kl_paged_decode_attention(*_args(q, kv, out, num_splits), workspace.data_ptr(), ws.value, _stream())
    assert st == 0, _native.last_error()
    torch.cuda.synchronize()
    return out, ws.value


def _no_alloc(q, kv, num_splits):
    out = torch.full_like(q, float("nan"))
    st = _native.core().kl_paged_decode_attention_noalloc(*_args(q, kv, out, num_splits), _stream())
    assert st == 0, _native.last_error()
    torch.cuda.synchronize()
    return out


# (lens, hq, hkv, dtype, num_splits): each pair of consecutive cases runs the
# larger input first, then a smaller one.
CALLS = [
    ([3000, 17, 2500, 900, 4096, 1, 2048, 300], 32, 8, torch.float16, 0),  # balanced, in-kernel merge
    ([700, 40], 32, 8, torch.float16, 0),  # smaller: fewer slots of the same array
    ([6000, 1, 5, 300, 17, 16, 33, 2048], 32, 1, torch.bfloat16, 0),  # MQA units: the merge kernel
    ([900, 31], 32, 1, torch.bfloat16, 0),
    ([1500] * 6, 32, 8, torch.float16, 5),  # uniform splits
    ([200] * 3, 32, 8, torch.float16, 2),
]


@pytest.mark.parametrize("first", [0, 2, 4])
def test_no_alloc_matches_workspace_entry_point(gpu_ops, first):
    """Two calls in a row, the second with a smaller input: every output equals
    the caller-workspace entry point's, bit for bit, and the oracle."""
    for i, (lens, hq, hkv, dtype, splits) in enumerate(CALLS[first : first + 2]):
        what = f"call {i}: B={len(lens)} {hq}/{hkv} {dtype} splits={splits}"
        print(what, flush=True)
        q, kv = device_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype, seed=first + i)
        want_bits, ws_bytes = _with_workspace(q, kv, splits)
        assert i > 0 or ws_bytes > 0, "the first call of each pair must use the workspace"
        got = _no_alloc(q, kv, splits)
        assert torch.equal(got, want_bits), f"{what}: differs from kl_paged_decode_attention"
        want = ref.paged_decode_attention(
            q.cpu().float(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_table.cpu(), kv.seq_lens.cpu()
        )
        decode_parity(got, want, dtype, what)


def test_no_alloc_single_split_needs_no_workspace(gpu_ops):
    """One requested split needs no workspace either way."""
    q, kv = device_decode_problem([512] * 64, 32, 8, 128, 16, dtype=torch.float16, seed=9)
    want_bits, ws_bytes = _with_workspace(q, kv, 1)
    assert ws_bytes == 0
    assert torch.equal(_no_alloc(q, kv, 1), want_bits)


def test_no_alloc_full_batch_default(gpu_ops):
    """A batch that fills the device takes the balanced schedule by default
    (one workgroup per unit, a workspace of partial slots): the even batch
    and then a smaller skewed one, both bit-identical to the workspace entry
    point."""
    for i, lens in enumerate(([512] * 64, [2000] + [100] * 39)):
        q, kv = device_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, seed=40 + i)
        want_bits, ws_bytes = _with_workspace(q, kv, 0)
        assert ws_bytes > 0
        assert torch.equal(_no_alloc(q, kv, 0), want_bits), f"call {i}"


def test_no_alloc_refuses_plans_beyond_its_array(gpu_ops):
    """64 explicit splits over a 64-sequence batch need 67 MB of partials: the
    call is refused before any launch, with the sizes in the message, and
    reports no merge even right after a call that merged in the kernel."""
    lens, hq, hkv, dtype, splits = CALLS[0]
    q0, kv0 = device_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype, seed=12)
    _no_alloc(q0, kv0, splits)
    # In the kernel when this stream holds a counter region, else the merge kernel.
    assert _native.core().kl_paged_decode_last_merge() != KL_MERGE_NONE
    q, kv = device_decode_problem([4096] * 64, 32, 8, 128, 16, dtype=torch.float16, seed=10)
    out = torch.full_like(q, float("nan"))
    st = _native.core().kl_paged_decode_attention_noalloc(*_args(q, kv, out, 64), _stream())
    assert st == KL_ERR_WORKSPACE
    msg = _native.last_error()
    assert "no-allocation" in msg and str(16 << 20) in msg, msg
    assert _native.core().kl_paged_decode_last_merge() == KL_MERGE_NONE, "a refused call merged nothing"
    torch.cuda.synchronize()
    assert torch.isnan(out).all(), "a refused call must not write"


def test_no_alloc_batch_zero_is_a_no_op(gpu_ops):
    q, kv = device_decode_problem([16], 8, 2, 128, 16, dtype=torch.float16, seed=11)
    args = _args(q, kv, q, 0)
    args[7] = 0  # batch
    assert _native.core().kl_paged_decode_attention_noalloc(*args, _stream()) == 0


def _capture(fn):
    """fn recorded into a graph on torch's capture stream (no warm-up call)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_no_alloc_graph_replays_match_eager(gpu_ops):
    """Two calls captured into one graph share the library's array one after
    the other on the capture stream; four replays, with eager work and
    synchronisations between them, each give the bits of the same two calls
    made eagerly."""
    probs = [device_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype, seed=20 + i)
             for i, (lens, hq, hkv, dtype, _) in enumerate(CALLS[:2])]
    want = [_no_alloc(q, kv, 0) for q, kv in probs]
    outs = [torch.full_like(q, float("nan")) for q, _ in probs]

    def run():
        for (q, kv), out in zip(probs, outs):
            st = _native.core().kl_paged_decode_attention_noalloc(*_args(q, kv, out, 0), _stream())
            assert st == 0, _native.last_error()

    g = _capture(run)
    for rep in range(4):
        for out in outs:
            out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for j, (out, w) in enumerate(zip(outs, want)):
            assert torch.equal(out, w), f"replay {rep}, call {j}: differs from the eager call"
        probs[0][0].mul_(1.0)  # eager work between replays
        torch.cuda.synchronize()


def _first_call_captured() -> None:
    """Body of the child process below: the process's first no-allocation
    call is recorded into a graph, then replayed three times."""
    lens, hq, hkv, dtype, splits = CALLS[0]
    q, kv = device_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype, seed=30)
    want, _ = _with_workspace(q, kv, splits)
    out = torch.full_like(q, float("nan"))
    status = []
    g = _capture(lambda: status.append(
        _native.core().kl_paged_decode_attention_noalloc(*_args(q, kv, out, splits), _stream())))
    assert status == [0], _native.last_error()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from the workspace entry point"
    print("first call captured: ok", flush=True)


def test_no_alloc_first_call_under_capture(gpu_ops):
    """In a fresh process, the first call (which looks up the device's array)
    is made while a graph is being captured."""
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(root), str(root / "kernel-lab_amd"), env.get("PYTHONPATH", "")])
    code = "from tests.test_zz_no_alloc import _first_call_captured; _first_call_captured()"
    print("child process: first no-allocation call under graph capture", flush=True)
    proc = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True, text=True,
                          timeout=100)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-3000:]
    assert "first call captured: ok" in proc.stdout
