"""The operators under HIP graph capture, as a serving loop runs them.

Each graph is replayed several times with eager work and synchronisations
between replays, and every replay is checked against the eager result (a
graph node that only works on its first replay must fail here)."""

from __future__ import annotations

import pytest
import torch

from kernel_lab import _native
from kernel_lab.kv_cache import device_decode_problem, quantize_fp8

pytestmark = pytest.mark.gpu


def capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up outside the graph (allocations, library state)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize(
    ("lens", "hq", "hkv", "dtype", "splits"),
    [
        ([4096] * 16, 32, 8, torch.float16, None),  # one split
        ([5000, 3, 700, 64], 32, 8, torch.bfloat16, None),  # balanced schedule + merge
        ([900] * 8, 32, 8, torch.float16, 4),  # uniform splits + merge
        ([300, 40], 8, 2, torch.float32, None),  # VALU kernel
        ([(37 * i) % 6000 + 1 for i in range(64)], 32, 1, torch.bfloat16, None),  # ragged MQA: charged cut, merge kernel
        ([(53 * i) % 3000 + 1 for i in range(64)], 32, 8, torch.float16, None),  # ragged full batch: pairs, in-kernel merge
    ],
)
def test_decode_graph_replays_match_eager(gpu_ops, lens, hq, hkv, dtype, splits):
    q, kv = device_decode_problem(lens, hq, hkv, 128, 16, dtype=dtype)
    out = torch.empty_like(q)
    run = lambda: gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens,
                                                 num_splits=splits, out=out)
    want = run().clone()
    g = capture(run)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"
        q.mul_(1.0)  # eager work between replays
        torch.cuda.synchronize()


def test_decode_graph_sees_new_inputs(gpu_ops):
    """A captured graph reads the buffers' current contents on every replay."""
    q, kv = device_decode_problem([700, 30], 16, 4, 64, 16, dtype=torch.float16)
    out = torch.empty_like(q)
    run = lambda: gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=out)
    g = capture(run)
    q.copy_(torch.randn_like(q))
    want = gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens).clone()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_fp8_and_rmsnorm_graph_replays(gpu_ops):
    q, kv = device_decode_problem([2048] * 8, 32, 8, 128, 16, dtype=torch.float16)
    kv8, ks, vs = quantize_fp8(kv)
    x = torch.randn(64, 4096, device="cuda", dtype=torch.bfloat16)
    res0 = torch.randn_like(x)
    w = torch.ones(4096, device="cuda", dtype=torch.bfloat16)
    out, y, res = torch.empty_like(q), torch.empty_like(x), res0.clone()

    def step():
        gpu_ops.paged_decode_attention(q, kv8.k_cache, kv8.v_cache, kv8.block_table, kv8.seq_lens,
                                       k_scale=ks, v_scale=vs, out=out)
        torch.ops.kernel_lab.fused_add_rms_norm(y, x, res, w, 1e-6)

    step()
    want_out, want_y, want_res = out.clone(), y.clone(), res.clone()
    # The residual is reset by an elementwise kernel (a copy could record a
    # memcpy node); then the step.
    g = capture(lambda: (torch.add(res0, 0, out=res), step()))
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out) and torch.equal(y, want_y) and torch.equal(res, want_res), i


def test_concurrent_replays_of_two_graphs(gpu_ops):
    """Two decode graphs captured on torch's shared capture stream, replayed
    at the same time on two streams, twenty times. Each captured call merges
    its split units inside the decode kernel, on arrival counters of its own
    capture: graphs that shared counters would count each other's arrivals and
    merge early (stale partials) or never (the output left as NaN)."""
    jobs = []
    for i, lens in enumerate(([4096] * 8, [3000, 17, 2500, 900, 4096, 1, 2048, 300])):
        q, kv = device_decode_problem(lens, 32, 8, 128, 16, dtype=torch.float16, seed=70 + i)
        outs = [torch.empty_like(q) for _ in range(4)]

        def run(q=q, kv=kv, outs=outs):
            for o in outs:
                gpu_ops.paged_decode_attention(q, kv.k_cache, kv.v_cache, kv.block_table, kv.seq_lens, out=o)

        run()
        want = [o.clone() for o in outs]
        g = capture(run)
        assert _native.core().kl_paged_decode_last_merge() == 2, "captured calls should merge in-kernel"
        # A graph reads its inputs where they were at capture: they must stay
        # allocated while it replays (the closure alone does not hold them
        # once the next iteration rebinds it).
        jobs.append((g, outs, want, torch.cuda.Stream(), (q, kv)))
    torch.cuda.synchronize()
    for rep in range(20):
        for _, outs, _, _, _ in jobs:
            for o in outs:
                o.fill_(float("nan"))
        for g, _, _, stream, _ in jobs:
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                g.replay()
        torch.cuda.synchronize()
        for i, (_, outs, want, _, _) in enumerate(jobs):
            for o, w in zip(outs, want):
                assert torch.equal(o, w), f"replay {rep} of graph {i} differs from eager"
