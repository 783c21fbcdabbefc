"""GPU parity of the serving fast path (lastkv_amd.serving) over one paged pool.

1. ``run_layer`` against a contiguous twin: per sequence a LastKVCache driven by the same C-ABI
   calls the drop-in attention makes (contiguous ring + shared store, boundary blend right at the
   boundary).  The same arithmetic runs in the same order on both sides, so with one decode split
   the outputs of every layer at every step are bit-identical, over ragged steps (prompt pieces of
   different lengths in one step, uniform prefill steps, padded decode steps) that cross several
   chunk boundaries with a chunk size that straddles page boundaries.
2. ``LastKVServingModel`` (ragged continuous batching through the tiny model) against the oracle
   model run per sequence, with the noise-floor criterion of the drop-in model's tests: no further
   from the fp32-attention oracle than the reference's own bf16 path is.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from lastkv_amd.llm import LastKVCache
from lastkv_amd.serving import LastKVFastPath, LastKVPagePool, LastKVServingModel

from test_gpu_llm import _no_worse_than_reference_bf16, _o16, _o32, _tiny

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rotary(positions: torch.Tensor):
    inv = 1.0 / (10000.0 ** (torch.arange(0, 128, 2, device=positions.device).float() / 128))
    f = positions[..., None].float() * inv
    emb = torch.cat((f, f), -1)
    return emb.cos().bfloat16(), emb.sin().bfloat16()


class _Twin:
    """One sequence on contiguous buffers, called exactly as LastKVAttention.forward calls the kernels."""

    def __init__(self, layers, Hkv, C, cap, params, blend):
        self.cache = LastKVCache(layers, C, capacity_tokens=cap)
        self.cache.reserve(1, Hkv, torch.device(DEV), cap)
        self.params, self.blend, self.C, self.layers = params, blend, C, layers

    def layer(self, l, q, k, v, Hq, Hkv):
        c, C = self.cache, self.C
        n = q.shape[0]
        p0 = c.seen_tokens
        qn_w, kn_w, eps, vs = self.params[l]
        cos, sin = _rotary(torch.arange(p0, p0 + n, device=DEV)[None, :])
        ring = c.ring(l)
        qn = ops.qkv_epilogue(q.reshape(1, n, -1), k.reshape(1, n, -1), v.reshape(1, n, -1), cos, sin, num_q_heads=Hq,
                              num_kv_heads=Hkv, q_norm_weight=qn_w, k_norm_weight=kn_w, eps=eps, positions=p0,
                              ring=ring, deep=c.store if l == self.layers - 1 else None)
        rec = max(0, (p0 + n - 1) // C * C - C)
        seg = dict(older=c.store, older_len=rec, vscale=vs, local=ring, local_len=p0 + n - rec,
                   local_start=rec % c.ring_tokens)
        if n == 1:
            return ops.decode_attention(qn.view(1, Hq, 128), num_splits=1, **seg).view(1, Hq, 128)
        return ops.prefill_attention(qn, causal=True, num_splits=1, **seg).view(n, Hq, 128)

    def advance(self, n):
        c = self.cache
        c.seen_tokens += n
        if c.seen_tokens % self.C == 0:
            alpha, om, s = self.blend
            ops.blend_chunk(c.ring_k, c.ring_v, c.store, batch=1, chunk_start=c.seen_tokens - self.C, chunk_len=self.C,
                            alpha=alpha, one_minus_alpha=om, vscale=s)


def test_run_layer_bit_exact_vs_contiguous_twin():
    g = torch.Generator(device=DEV).manual_seed(5)
    layers, Hq, Hkv, C, cap = 3, 8, 2, 48, 640
    params = []
    for l in range(layers):
        w = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
        vs = (torch.rand(Hkv, generator=g, device=DEV) + 0.4).bfloat16().float()
        params.append((w, w.flip(0).contiguous(), 1e-5, vs))
    alpha = torch.rand(layers * Hkv, generator=g, device=DEV).bfloat16().float()
    blend = (alpha, (1 - alpha).bfloat16().float(), torch.cat([p[3] for p in params]))
    pool = LastKVPagePool(num_layers=layers, kv_heads=Hkv, chunk_size=C, max_slots=4, source_pages=64,
                          max_tokens_per_slot=cap, device=DEV)
    fast = LastKVFastPath(pool, num_q_heads=Hq, layer_params=params, blend=blend, rotary=_rotary, max_batch=6,
                          num_splits=1)
    slots = [fast.add_sequence() for _ in range(3)]
    twins = [_Twin(layers, Hkv, C, cap, params, blend) for _ in slots]
    # (rows of (sequence, tokens), pad_to)
    schedule = [([(0, 48), (1, 20), (2, 5)], None), ([(1, 28), (0, 48), (2, 43)], None),
                ([(0, 48), (1, 48), (2, 48)], None), ([(2, 30), (0, 1)], None)]
    schedule += [([(0, 1), (1, 1)], 4)] * 3 + [([(0, 1), (1, 1), (2, 1)], None)] * 2
    schedule += [([(2, 16)], None), ([(0, 2), (1, 1), (2, 3)], None)] + [([(1, 1), (2, 1), (0, 1)], 5 if i % 2 else None) for i in range(60)]
    for step, (rows, pad) in enumerate(schedule):
        fast.prepare([(slots[i], n) for i, n in rows], pad_to=pad)
        T = fast.tokens
        q = torch.randn((T, Hq * 128), generator=g, device=DEV).bfloat16()
        k = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        v = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        for l in range(layers):
            out = torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV)
            fast.run_layer(l, q, k, v, out)
            start = 0
            for i, n in rows:
                sl = slice(start, start + n)
                want = twins[i].layer(l, q[sl], k[sl], v[sl], Hq, Hkv)
                assert torch.equal(out[sl], want), f"step {step} layer {l} sequence {i}"
                start += n
        for i, n in rows:
            twins[i].advance(n)
            assert fast.seen(slots[i]) == twins[i].cache.seen_tokens
    print(f"{len(schedule)} steps, final lengths {[fast.seen(s) for s in slots]}", flush=True)
    for s in slots:
        fast.free_sequence(s)
    assert pool.free_pages == 64


@pytest.mark.parametrize("seed", range(8))
def test_run_layer_random_schedules_bit_exact_vs_twins(seed):
    """Seeded random serving schedules against contiguous twins, bit for bit at every layer of every
    step (one decode split on both sides): GQA 1-8 over 1-4 kv heads, a chunk size of 8-100 tokens,
    up to 4 live sequences with random targets, arriving at random steps and freed when done (so
    slots and pages are reused), each step scheduling a random subset of them with prompt pieces up
    to the next chunk boundary or single tokens, and padded decode steps; at the end every page is
    back in the pool."""

    rng = np.random.default_rng(300 + seed)
    g = torch.Generator(device=DEV).manual_seed(300 + seed)
    layers, cap, live_max = 2, 480, 4
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    C = int(rng.choice([8, 24, 32, 40, 64, 100]))
    params = []
    for _ in range(layers):
        w = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
        vs = (torch.rand(Hkv, generator=g, device=DEV) + 0.4).bfloat16().float()
        params.append((w, w.flip(0).contiguous(), 1e-5, vs))
    alpha = torch.rand(layers * Hkv, generator=g, device=DEV).bfloat16().float()
    blend = (alpha, (1 - alpha).bfloat16().float(), torch.cat([p[3] for p in params]))
    pool = LastKVPagePool(num_layers=layers, kv_heads=Hkv, chunk_size=C, max_slots=live_max,
                          source_pages=live_max * cap // 32 + 4, max_tokens_per_slot=cap, device=DEV)
    free0 = pool.free_pages
    fast = LastKVFastPath(pool, num_q_heads=Hq, layer_params=params, blend=blend, rotary=_rotary,
                          max_batch=live_max + 2, num_splits=1)
    live = {}  # slot -> (twin, target length, prompt length)
    started = steps = 0
    while steps < 200 and (live or started < 16):
        while len(live) < live_max and started < 16 and (not live or rng.random() < 0.4):
            target = int(rng.integers(2, 240 if rng.random() < 0.7 else cap))
            live[fast.add_sequence()] = (_Twin(layers, Hkv, C, cap, params, blend), target,
                                         int(rng.integers(1, target)))
            started += 1
        rows = []
        for slot, (_, target, prompt) in live.items():
            if len(live) > 1 and rng.random() < 0.2:
                continue  # not in this step
            p = fast.seen(slot)
            room = min(target - p, C - p % C)
            rows.append((slot, int(rng.integers(1, room + 1)) if p < prompt else 1))
        if not rows:
            continue
        decode = all(n == 1 for _, n in rows)
        pad = len(rows) + int(rng.integers(1, 3)) if decode and rng.random() < 0.3 else None
        fast.prepare(rows, pad_to=pad)
        T = fast.tokens
        q = torch.randn((T, Hq * 128), generator=g, device=DEV).bfloat16()
        k = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        v = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        label = f"seed {seed} (Hq {Hq}, Hkv {Hkv}, C {C}) step {steps} rows {[(n, fast.seen(sl) - n) for sl, n in rows]}"
        for l in range(layers):
            out = torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV)
            fast.run_layer(l, q, k, v, out)
            start = 0
            for slot, n in rows:
                sl = slice(start, start + n)
                want = live[slot][0].layer(l, q[sl], k[sl], v[sl], Hq, Hkv)
                assert torch.equal(out[sl], want), f"{label}: layer {l} slot {slot}"
                start += n
        for slot, n in rows:
            live[slot][0].advance(n)
            assert fast.seen(slot) == live[slot][0].cache.seen_tokens
        for slot in [sl for sl, (_, target, _) in live.items() if fast.seen(sl) >= target]:
            fast.free_sequence(slot)
            del live[slot]
        steps += 1
    for slot in list(live):
        fast.free_sequence(slot)
    assert pool.free_pages == free0
    print(f"seed {seed}: Hq {Hq} Hkv {Hkv} C {C}, {steps} steps, {started} sequences", flush=True)


def test_serving_model_ragged_batches_match_oracle():
    oracle, ours = _tiny(chunk=8)
    lengths = [37, 22, 50]
    gen = torch.Generator().manual_seed(8)
    seqs = [torch.randint(3, 97, (n,), generator=gen).to(DEV) for n in lengths]
    runner = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=64)
    slots = [runner.add_sequence() for _ in seqs]
    fed = [0] * len(seqs)
    got = [[] for _ in seqs]  # (position of the row's last token, logits)
    pieces = [5, 3, 8, 1, 8, 2, 7]
    step = 0
    with torch.inference_mode():
        while any(f < len(s) for f, s in zip(fed, seqs)):
            rows, owners = [], []
            for i, s in enumerate(seqs):
                if fed[i] >= len(s):
                    continue
                p = runner.fast.seen(slots[i])
                take = min(len(s) - fed[i], 8 - p % 8, pieces[(step + i) % len(pieces)] if fed[i] < 24 else 1)
                rows.append((slots[i], s[fed[i]:fed[i] + take]))
                owners.append((i, fed[i] + take - 1))
                fed[i] += take
            logits = runner.step(rows)
            for (i, pos), row in zip(owners, logits):
                got[i].append((pos, row.float()))
            step += 1
        for i, s in enumerate(seqs):
            want, _ = _o32(oracle)(s[None])
            ref16, _ = _o16(oracle)(s[None])
            pos = [p for p, _ in got[i]]
            mine = torch.stack([r for _, r in got[i]])[None]
            _no_worse_than_reference_bf16(mine, want[:, pos].float(), ref16[:, pos].float(),
                                          f"serving sequence {i} ({len(pos)} steps)")
    print(f"{step} ragged steps", flush=True)


def test_serving_generate_runs_and_frees_pages():
    _, ours = _tiny(chunk=8)
    runner = LastKVServingModel(ours, max_batch=3, max_tokens_per_slot=96)
    total = runner.pool.free_pages
    prompts = [torch.tensor([1, 5, 17, 33, 2, 9], device=DEV), torch.arange(3, 30, device=DEV)]
    with torch.inference_mode():
        out = runner.generate(prompts, 12, prefill_chunk=5)
        again = runner.generate(prompts, 12, prefill_chunk=5)  # reused slots and pages, same ids
    for a, b, p in zip(out, again, prompts):
        assert a.shape[0] == p.numel() + 12
        assert torch.equal(a[: p.numel()], p.cpu())
        assert torch.equal(a, b)
    assert runner.pool.free_pages == total



def _prefill(runner, slots, prompts, chunk):
    """Feed each prompt in pieces cut at chunk boundaries; returns each row's next greedy id."""

    nxt = []
    for slot, p in zip(slots, prompts):
        fed = 0
        while fed < p.numel():
            take = min(p.numel() - fed, chunk - runner.fast.seen(slot) % chunk)
            logits = runner.step([(slot, p[fed:fed + take])])
            fed += take
        nxt.append(logits[0].argmax())
    return torch.stack(nxt)


def test_decode_graph_replays_match_eager_steps():
    """DecodeGraph against eager LastKVServingModel.step on a second runner over the same model:
    3 sequences prefilled eagerly, then 40 decode steps at C = 8 (boundary commits and ring wraps
    run in the host prologue between replays), with unrelated eager work and synchronisations
    between the replays; every replay's logits and greedy ids equal the eager step's."""

    _, ours = _tiny(chunk=8)
    eager = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=96, num_splits=2)
    graphed = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=96, num_splits=2)
    prompts = [torch.arange(3, 14, device=DEV), torch.tensor([1, 5, 17, 33, 2], device=DEV),
               torch.arange(40, 61, device=DEV)]
    se = [eager.add_sequence() for _ in prompts]
    sg = [graphed.add_sequence() for _ in prompts]
    with torch.inference_mode():
        t_eager = _prefill(eager, se, prompts, 8)
        t_graph = _prefill(graphed, sg, prompts, 8)
        assert torch.equal(t_eager, t_graph)
        graph = graphed.decode_graph(sg)
        scratch = torch.randn(256, 256, device=DEV)
        for i in range(40):
            le = eager.step([(s, t_eager[j:j + 1]) for j, s in enumerate(se)])
            lg, ng = graph.step(t_graph)
            assert torch.equal(le, lg), f"step {i}: replay logits differ from the eager step"
            t_eager = le.argmax(-1)
            assert torch.equal(t_eager, ng), f"step {i}: greedy ids differ"
            t_graph = ng.clone()
            scratch = scratch @ scratch.T * 1e-3  # the program's own eager work between replays
            if i % 3 == 0:
                torch.cuda.synchronize()
    assert graphed.fast.seen(sg[0]) == eager.fast.seen(se[0]) == prompts[0].numel() + 40


@pytest.mark.parametrize("contract", ["hf", "vllm"])
def test_vllm_impl_adapter_runs_the_fast_path(contract):
    """lastkv_amd.vllm_backend.LastKVAttentionImpl.forward (the reference's Impl contract,
    vllm_backend.py:637-717) over steps prepared on the current fast path: a ragged prefill step,
    a uniform prefill step and padded decode steps crossing a chunk boundary.  vLLM hands it padded
    buffers (more rows than num_actual_tokens); rows past the real tokens must come back zero and
    the real rows must equal LastKVFastPath.run_layer's output bit for bit."""

    from types import SimpleNamespace

    from lastkv_amd import vllm_backend as VB

    _, ours = _tiny(chunk=8)
    cfg = ours.config
    Hq, Hkv, L = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
    runner = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=64, contract=contract)
    fast = runner.fast
    slots = [runner.add_sequence() for _ in range(3)]
    impl = VB.LastKVAttentionImpl(Hq, 128, 128 ** -0.5, Hkv, None, None, "auto")
    g = torch.Generator(device=DEV).manual_seed(9)
    steps = [([(slots[0], 5), (slots[1], 3), (slots[2], 8)], None), ([(s, 2) for s in slots], None)]
    steps += [([(s, 1) for s in slots], 4)] * 6
    VB.set_current(fast)
    try:
        for i, (rows, pad) in enumerate(steps):
            fast.prepare(rows, pad_to=pad)
            T = fast.tokens
            actual = sum(n for _, n in rows)
            for l in range(L):
                q = torch.randn((T + 3, Hq * 128), generator=g, device=DEV).bfloat16()
                k = torch.randn((T + 3, Hkv * 128), generator=g, device=DEV).bfloat16()
                v = torch.randn((T + 3, Hkv * 128), generator=g, device=DEV).bfloat16()
                out = torch.full((T + 3, Hq, 128), 7.0, dtype=torch.bfloat16, device=DEV)
                got = impl.forward(SimpleNamespace(rmarin_layer_index=l), q, k, v, None,
                                   SimpleNamespace(num_actual_tokens=actual), out)
                ref = torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV)
                fast.run_layer(l, q[:T], k[:T], v[:T], ref)
                assert got is out
                assert torch.equal(out[:actual], ref[:actual]), f"step {i} layer {l}"
                assert not out[actual:].any(), f"step {i} layer {l}: padded rows not zero"
        assert impl.forward(SimpleNamespace(rmarin_layer_index=0), q, k, v, None, None, out) is out and not out.any()
    finally:
        VB.set_current(None)


@pytest.mark.parametrize("contract", ["hf", "vllm"])
def test_merged_check_reports_two_pass_agreement(contract, monkeypatch, capsys):
    """LASTKV_MERGED_CHECK=1 (the reference's RMARIN_MERGED_CHECK, fastpath.py:198-202, 737-773):
    every eager layer call is recomputed in two passes from the same pool (older segment, ring
    segment, exact LSE merge) and reported; over uniform prefill, ragged and padded decode steps
    that cross chunk boundaries the one-pass output stays within 1e-2 (rel-L2) of it, half the
    reference's reporting threshold (the two-pass result rounds each pass to bf16 before the merge:
    measured worst 2.9e-3 with the HF contract, 3.9e-3 with the vLLM one).  Mode 2 hands
    the two-pass result to the model; under graph capture nothing is checked and replays still
    equal eager steps."""

    import ast

    monkeypatch.setenv("LASTKV_MERGED_CHECK", "1")
    g = torch.Generator(device=DEV).manual_seed(11)
    layers, Hq, Hkv, C, cap = 2, 8, 2, 48, 640
    params = []
    for l in range(layers):
        w = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
        vs = (torch.rand(Hkv, generator=g, device=DEV) + 0.4).bfloat16().float()
        params.append((w, w.flip(0).contiguous(), 1e-5, vs))
    alpha = torch.rand(layers * Hkv, generator=g, device=DEV).bfloat16().float()
    blend = (alpha, (1 - alpha).bfloat16().float(), torch.cat([p[3] for p in params]))
    pool = LastKVPagePool(num_layers=layers, kv_heads=Hkv, chunk_size=C, max_slots=4, source_pages=64,
                          max_tokens_per_slot=cap, device=DEV)
    fast = LastKVFastPath(pool, num_q_heads=Hq, layer_params=params, blend=blend, rotary=_rotary, max_batch=6,
                          contract=contract)
    assert fast.check and not fast.check_replace
    slots = [fast.add_sequence() for _ in range(3)]
    schedule = [([(0, 48), (1, 48), (2, 48)], None), ([(0, 48), (1, 20), (2, 5)], None),
                ([(1, 28), (0, 48), (2, 43)], None), ([(0, 1), (1, 1)], 4), ([(2, 30), (0, 2), (1, 1)], None)]
    schedule += [([(0, 1), (1, 1), (2, 1)], 5 if i % 2 else None) for i in range(20)]
    calls = 0
    for rows, pad in schedule:
        fast.prepare([(slots[i], n) for i, n in rows], pad_to=pad)
        T = fast.tokens
        q = torch.randn((T, Hq * 128), generator=g, device=DEV).bfloat16()
        k = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        v = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
        for l in range(layers):
            fast.run_layer(l, q, k, v, torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV))
            calls += 1
    reports = [ast.literal_eval(line)["lastkv_merged_check"] for line in capsys.readouterr().out.splitlines()
               if line.startswith("{'lastkv_merged_check'")]
    assert len(reports) == calls, (len(reports), calls)
    worst = max(r["rel"] for r in reports)
    with capsys.disabled():
        print(f"{contract}: {calls} layer calls checked, worst rel-L2 {worst:.2e}", flush=True)
    assert worst < 1e-2
    assert any(r["older"][0] > 0 for r in reports), "no call had an older segment"

    # mode 2: the output is the two-pass result
    fast.check_replace = True
    fast.prepare([(slots[i], 1) for i in range(3)])
    T = fast.tokens
    q = torch.randn((T, Hq * 128), generator=g, device=DEV).bfloat16()
    k = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
    v = torch.randn((T, Hkv * 128), generator=g, device=DEV).bfloat16()
    out = torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV)
    fast.run_layer(0, q, k, v, out)
    rep = [ast.literal_eval(line)["lastkv_merged_check"] for line in capsys.readouterr().out.splitlines()
           if line.startswith("{'lastkv_merged_check'")]
    assert len(rep) == 1 and torch.isfinite(out.float()).all()


def test_merged_check_skips_graph_capture(monkeypatch, capsys):
    """With the check on, a captured decode step checks nothing and its replays equal eager steps
    (the eager runner's calls, and the graph's one eager warm-up step, are checked and left
    unchanged)."""

    monkeypatch.setenv("LASTKV_MERGED_CHECK", "1")
    _, ours = _tiny(chunk=8)
    eager = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=96, num_splits=2)
    graphed = LastKVServingModel(ours, max_batch=4, max_tokens_per_slot=96, num_splits=2)
    assert eager.fast.check and graphed.fast.check
    prompts = [torch.arange(3, 14, device=DEV), torch.tensor([1, 5, 17, 33, 2], device=DEV)]
    se = [eager.add_sequence() for _ in prompts]
    sg = [graphed.add_sequence() for _ in prompts]
    with torch.inference_mode():
        t_eager = _prefill(eager, se, prompts, 8)
        t_graph = _prefill(graphed, sg, prompts, 8)
        graph = graphed.decode_graph(sg)
        capsys.readouterr()
        for i in range(12):
            le = eager.step([(s, t_eager[j:j + 1]) for j, s in enumerate(se)])
            lg, ng = graph.step(t_graph)
            assert torch.equal(le, lg), f"step {i}"
            t_eager, t_graph = le.argmax(-1), ng.clone()
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("{'lastkv_merged_check'")]
    # the eager runner's 12 steps and the graph's eager warm-up step before its capture
    assert len(lines) == 13 * len(ours.model.layers), len(lines)
