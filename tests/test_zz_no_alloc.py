"""The allocation-free decode entry point (lkv_decode_attn_noalloc) against lkv_decode_attn.

Both entry points run the same kernels with the same split count; the allocation-free one keeps
the split states in the library's static per-GPU scratch instead of a caller workspace, so its
outputs and LSEs must equal lkv_decode_attn's bit for bit.  Two calls in a row, the second with a
smaller input (the scratch still holds the first call's states), a one-split call (one split keeps
no split state: lkv_decode_workspace_bytes is 0, so the call neither looks up nor touches the
scratch), then a call whose split states exceed the scratch, which is rejected before any launch.
A fresh process whose first allocation-free call is made under HIP graph capture (the scratch's
address is looked up by that call) replays the graph with eager work between the replays, each
replay equal to lkv_decode_attn bit for bit.  The calls go through the C ABI (lastkv_amd.ops fills
the argument struct and calls the library with ctypes).
"""

from __future__ import annotations

import os
import subprocess
import sys
import textwrap

import pytest
import torch

from lastkv_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _segments(seed, B, Hkv, T0, n1):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda *shape: torch.randn(shape, generator=g, device=DEV).bfloat16()
    older = ops.TiledKV(rnd(B, Hkv, -(-T0 // 32), 4096), rnd(B, Hkv, -(-T0 // 32), 4096))
    ring = ops.TiledKV(rnd(B, Hkv, -(-(n1 + 40) // 32), 4096), rnd(B, Hkv, -(-(n1 + 40) // 32), 4096))
    vscale = torch.rand(Hkv, generator=g, device=DEV) + 0.5
    return dict(older=older, older_len=T0, vscale=vscale, local=ring, local_len=n1, local_start=37), g


@pytest.mark.parametrize("B,Hq,Hkv,T0,n1,splits", [(16, 32, 8, 4000, 300, 8), (3, 8, 2, 700, 41, 5), (2, 12, 4, 90, 7, 1)])
def test_noalloc_decode_equals_workspace_decode(B, Hq, Hkv, T0, n1, splits):
    seg, g = _segments(B * 131 + splits, B, Hkv, T0, n1)
    q = torch.randn((B, Hq, 128), generator=g, device=DEV).bfloat16()
    print(f"B={B} Hq={Hq} Hkv={Hkv} older={T0} local={n1} splits={splits}: "
          f"{ops.decode_workspace_bytes(B, Hq, splits)} bytes of split state", flush=True)
    lse_w = torch.empty((B, Hq), dtype=torch.float32, device=DEV)
    lse_n = torch.full((B, Hq), 7.0, dtype=torch.float32, device=DEV)
    out_w = ops.decode_attention(q, lse=lse_w, num_splits=splits, **seg)
    out_n = torch.full_like(out_w, 3.0)
    ops.decode_attention(q, lse=lse_n, num_splits=splits, out=out_n, no_alloc=True, **seg)
    torch.cuda.synchronize()
    assert torch.equal(out_w, out_n)
    assert torch.equal(lse_w, lse_n)


def test_noalloc_decode_rejects_split_state_beyond_the_scratch():
    B, Hq, Hkv, splits = 64, 64, 8, 16  # 64 * 64 * 16 * 520 bytes > 16 MiB
    seg, g = _segments(5, B, Hkv, 64, 8)
    q = torch.randn((B, Hq, 128), generator=g, device=DEV).bfloat16()
    assert ops.decode_workspace_bytes(B, Hq, splits) > 16 << 20
    with pytest.raises(RuntimeError, match="static scratch"):
        ops.decode_attention(q, num_splits=splits, no_alloc=True, **seg)
    out = ops.decode_attention(q, num_splits=2, no_alloc=True, **seg)  # 8.5 MB: fits
    torch.cuda.synchronize()
    assert torch.equal(out, ops.decode_attention(q, num_splits=2, **seg))


_CAPTURE_SCRIPT = textwrap.dedent("""
    import sys
    import torch
    from lastkv_amd import ops

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(3)
    B, Hq, Hkv, T0, splits = 8, 32, 8, 3000, 6
    rnd = lambda *shape: torch.randn(shape, generator=g, device=dev).bfloat16()
    older = ops.TiledKV(rnd(B, Hkv, -(-T0 // 32), 4096), rnd(B, Hkv, -(-T0 // 32), 4096))
    vscale = torch.rand(Hkv, generator=g, device=dev) + 0.5
    q = rnd(B, Hq, 128)
    want = ops.decode_attention(q, older=older, older_len=T0, vscale=vscale, num_splits=splits)
    out = torch.zeros_like(want)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):  # the first allocation-free call of this process
        ops.decode_attention(q, older=older, older_len=T0, vscale=vscale, num_splits=splits, out=out, no_alloc=True)
    scratch = torch.randn(512, 512, device=dev)
    for i in range(4):
        out.zero_()
        scratch = scratch @ scratch.T * 1e-3  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(out, want):
            print(f"replay {i} differs", flush=True)
            sys.exit(1)
    print("captured allocation-free decode: 4 replays equal lkv_decode_attn", flush=True)
""")


def test_noalloc_decode_first_call_under_graph_capture():
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=repo + os.pathsep + os.environ.get("PYTHONPATH", ""))
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT], cwd=repo, env=env, capture_output=True, text=True,
                          timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "4 replays equal" in proc.stdout
