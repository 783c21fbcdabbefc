"""Host logic of the serving path on the CPU: the per-row segment plan against the oracle's
region plan (itself pinned by enumeration against the reference test's cache invariants), and the
page allocator's bookkeeping under a random open / grow / close workload, and the serving model's
fused projection weights."""

from __future__ import annotations

import numpy as np
import pytest

from lastkv_amd import ops
from lastkv_amd.serving import PageAllocator, plan_row
from oracle import attention as A


@pytest.mark.parametrize("chunk", [1, 4, 12, 32, 48, 64])
def test_plan_row_matches_oracle_regions(chunk):
    R = ops.ring_tokens_for_chunk(chunk)
    for p in range(5 * chunk):
        for n in range(1, chunk - p % chunk + 1):
            older, local, start = plan_row(p, n, chunk, R)
            reg = A.plan_regions(p + n - 1, chunk)  # the row's last query decides the segments
            assert older == reg.older[1]
            assert local == reg.current[1] - reg.recent[0]
            assert start == reg.recent[0] % R
            assert local <= 2 * chunk <= R
            # every query of the row sees the same segments
            for t in range(p, p + n):
                r = A.plan_regions(t, chunk)
                assert r.older == reg.older and r.recent == reg.recent


def test_plan_row_rejects_rows_across_a_boundary():
    with pytest.raises(ValueError, match="cross"):
        plan_row(40, 10, 48, 128)
    with pytest.raises(ValueError):
        plan_row(0, 0, 48, 128)


def test_page_allocator_random_workload():
    rng = np.random.default_rng(3)
    pages, width, scratch = 40, 12, 999
    al = PageAllocator(max_slots=5, pages=pages, width=width, scratch=scratch)
    length = {}
    for _ in range(2000):
        op = rng.integers(3)
        if op == 0 and len(length) < 5:
            s = al.open_slot()
            assert s not in length and (al.table[s] == scratch).all()
            length[s] = 0
        elif op == 1 and length:
            s = int(rng.choice(list(length)))
            grow = length[s] + int(rng.integers(1, 70))
            need = -(-grow // 32) - int(al.used[s])
            if grow > width * 32:
                with pytest.raises(ValueError):
                    al.reserve(s, grow)
            elif need > al.free_pages:
                with pytest.raises(RuntimeError):
                    al.reserve(s, grow)
            else:
                lo, hi = al.reserve(s, grow)
                assert hi - lo == max(0, need)
                length[s] = grow
        elif op == 2 and length:
            s = int(rng.choice(list(length)))
            al.close_slot(s)
            del length[s]
            assert (al.table[s] == scratch).all()
        owned = np.concatenate([al.table[s, : al.used[s]] for s in length]) if length else np.zeros(0)
        assert len(set(owned.tolist())) == owned.size  # no page in two places
        assert owned.size + al.free_pages == pages
        for s, n in length.items():
            assert al.used[s] == -(-n // 32)
            assert (al.table[s, al.used[s]:] == scratch).all()


def test_fuse_linears_aliases_weights_in_place():
    """One fused [sum(out), in] weight / bias whose row ranges are the modules' own parameters:
    same values, no copy, reused by a second call, written through by load_state_dict."""

    import torch

    from lastkv_amd.serving import fuse_linears

    torch.manual_seed(3)
    mods = [torch.nn.Linear(16, n, bias=True) for n in (8, 4, 4)]
    before = [(m.weight.detach().clone(), m.bias.detach().clone()) for m in mods]
    x = torch.randn(5, 16)
    want = torch.cat([m(x) for m in mods], dim=-1).detach()
    w, b = fuse_linears(mods)
    assert w.shape == (16, 16) and b.shape == (16,)
    for m, (w0, b0), r0 in zip(mods, before, (0, 8, 12)):
        assert torch.equal(m.weight, w0) and torch.equal(m.bias, b0)
        assert m.weight.data_ptr() == w[r0:].data_ptr() and m.bias.data_ptr() == b[r0:].data_ptr()
    torch.testing.assert_close(torch.nn.functional.linear(x, w, b), want, rtol=0, atol=1e-6)
    w2, b2 = fuse_linears(mods)
    assert w2 is w and b2 is b
    mods[1].load_state_dict({"weight": before[1][0] * 2, "bias": before[1][1] * 2})
    assert torch.equal(w[8:12], before[1][0] * 2) and torch.equal(b[8:12], before[1][1] * 2)
    mixed = [torch.nn.Linear(16, 4, bias=True), torch.nn.Linear(16, 4, bias=False)]
    with pytest.raises(ValueError, match="bias"):
        fuse_linears(mixed)
