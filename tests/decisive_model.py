"""A LastKV model whose greedy decisions are decisive by construction (test helper, GPU tests).

Random-init weights make argmax a near-tie at a sizeable fraction of steps, so two correct bf16
implementations diverge within 64 greedy steps.  This builder writes weights whose attention is
one-hot with score gaps of hundreds, whose hidden states carry exact copies of cached values,
and whose lm_head separates the winner from every other token by a wide margin, while the
generated ids still depend on which cache region (older shared segment or local ring) holds the
key that each query finds.

Construction, for every kv head g (all q heads of its group identical):
  - token u's embedding holds unit codes kappa[g, u] (48-d key code), kappa[g, sigma[u]] (the
    key code of the token u looks up), nu[g, u] and nu2[g, u] (32-d value codes);
  - every layer's k_proj / q_proj copy the key / query code into the 48 head dims of the 24
    slowest rotary pairs (which turn by < 0.1 rad over the test's positions), q/k RMSNorm gains
    are 8, so a query scores ~720 on the key of its target token and ~360 or less elsewhere;
  - v_proj copies nu (layers 0 .. L-2) or nu2 (the final layer, whose K/V form the shared
    cache), so layer 0's output at a decode step is nu[x] (x found in the local ring: the recent
    chunk, blended with small alpha, or the current chunk) or s * nu2[x] (x found in the older
    segment, read through the final layer's K/V);
  - o_proj writes layer l's head outputs into a home of the residual stream of its own; the MLP
    writes only into dims no projection reads; lm_head reads layer 0's home: next_local[x] has
    row nu[., x], next_older[x] has row nu2[., x].
Prompts are distinct tokens of the lower half of the vocabulary; sigma maps every token to a
prompt token; next_local / next_older are disjoint injections of the prompt tokens into the
upper half.  The greedy continuation is then, in closed form,
  t_{n+1} = next_older[x] if x sits before rec else next_local[x],   x = sigma[t_n],
with rec = max(0, floor(p / C) * C - C) for the query position p.
"""

from __future__ import annotations

import torch

from oracle import model as M

KEY_CODE = 48  # head dims of the 24 slowest rotary pairs
VALUE_CODE = 32
NORM_GAIN = 8.0
ALPHA_LOGIT = -2.5  # alpha = 0.076: the recent chunk is mostly the layer's own K/V


def slow_rotary_dims(head_dim: int = 128) -> torch.Tensor:
    half = head_dim // 2
    pairs = torch.arange(half - KEY_CODE // 2, half)
    return torch.cat([pairs, pairs + half])


def _unit(shape, gen):
    x = torch.randn(shape, generator=gen)
    return x / x.norm(dim=-1, keepdim=True)


def build(cfg: M.Config, prompt_len: int, seed: int = 0, device="cpu"):
    """Returns (oracle model in fp32 on ``device``, tables) for ``cfg``; tables (on the CPU) hold
    sigma, next_local, next_older and the prompt token pool.  The codes and tables are drawn on
    the CPU; the MLP's N(0, 0.02) weights with a generator on ``device``."""

    H, Hkv, D, d, L, V = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size,
                          cfg.num_hidden_layers, cfg.vocab_size)
    G = H // Hkv
    kc, vc = KEY_CODE, VALUE_CODE
    key0, qry0 = 0, Hkv * kc
    nu0, nu20 = 2 * Hkv * kc, 2 * Hkv * kc + Hkv * vc
    home0 = 2 * Hkv * (kc + vc)
    free0 = home0 + L * Hkv * vc
    assert D == 128 and free0 + 64 <= d and 4 * prompt_len <= V
    gen = torch.Generator().manual_seed(seed)
    pool = torch.randperm(V // 2, generator=gen)[:prompt_len]
    upper = V // 2 + torch.randperm(V - V // 2, generator=gen)[:2 * prompt_len]
    next_local = torch.full((V,), -1, dtype=torch.long)
    next_older = torch.full((V,), -1, dtype=torch.long)
    next_local[pool] = upper[:prompt_len]
    next_older[pool] = upper[prompt_len:]
    sigma = pool[torch.randint(0, prompt_len, (V,), generator=gen)]
    kappa = _unit((Hkv, V, kc), gen)
    nu = _unit((Hkv, V, vc), gen)
    nu2 = _unit((Hkv, V, vc), gen)

    with torch.device(device):
        model = M.ForCausalLM(cfg)
    wgen = torch.Generator(device=device).manual_seed(seed)
    slow = slow_rotary_dims(D)
    kappa, nu, nu2, sigma = (t.to(device) for t in (kappa, nu, nu2, sigma))
    pool_d, nl_d, no_d = pool.to(device), next_local.to(device), next_older.to(device)
    with torch.no_grad():
        for w in (mlp_w for layer in model.model.layers
                  for mlp_w in (layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight, layer.mlp.down_proj.weight)):
            w.normal_(0.0, 0.02, generator=wgen)
        for norm in [model.model.norm] + [n for layer in model.model.layers
                                          for n in (layer.input_layernorm, layer.post_attention_layernorm)]:
            norm.weight.fill_(1.0)
        E = model.model.embed_tokens.weight
        E.zero_()
        for g in range(Hkv):
            E[:, key0 + g * kc:key0 + (g + 1) * kc] = kappa[g]
            E[:, qry0 + g * kc:qry0 + (g + 1) * kc] = kappa[g, sigma]
            E[:, nu0 + g * vc:nu0 + (g + 1) * vc] = nu[g]
            E[:, nu20 + g * vc:nu20 + (g + 1) * vc] = nu2[g]
        E[:, free0:].normal_(0.0, 0.02, generator=wgen)
        for l, layer in enumerate(model.model.layers):
            att, mlp = layer.self_attn, layer.mlp
            for w in (att.q_proj.weight, att.k_proj.weight, att.v_proj.weight, att.o_proj.weight):
                w.zero_()
            vsrc = nu20 if l == L - 1 else nu0
            home = home0 + l * Hkv * vc
            ak, av = torch.arange(kc, device=device), torch.arange(vc, device=device)
            sl = slow.to(device)
            for g in range(Hkv):
                att.k_proj.weight[g * D + sl, key0 + g * kc + ak] = 1.0
                att.v_proj.weight[g * D + av, vsrc + g * vc + av] = 1.0
                for h in range(g * G, (g + 1) * G):
                    att.q_proj.weight[h * D + sl, qry0 + g * kc + ak] = 1.0
                    att.o_proj.weight[home + g * vc + av, h * D + av] = 1.0 / G
            att.q_norm.weight.fill_(NORM_GAIN)
            att.k_norm.weight.fill_(NORM_GAIN)
            att.prev_chunk_alphas.fill_(ALPHA_LOGIT)
            att.deep_v_scale.copy_(torch.empty(Hkv).uniform_(0.8, 1.2, generator=gen))
            mlp.down_proj.weight[:free0].zero_()
        lm = model.lm_head.weight
        lm.zero_()
        for g in range(Hkv):
            cols = home0 + g * vc + torch.arange(vc, device=device)
            lm[nl_d[pool_d][:, None], cols[None, :]] = nu[g, pool_d]
            lm[no_d[pool_d][:, None], cols[None, :]] = nu2[g, pool_d]
    return model.eval(), dict(sigma=sigma.cpu(), next_local=next_local, next_older=next_older, pool=pool)


def prompts(tables, batch: int, seed: int = 1) -> torch.Tensor:
    """``batch`` prompts, each the whole prompt pool in its own order (distinct tokens)."""

    gen = torch.Generator().manual_seed(seed)
    pool = tables["pool"]
    return torch.stack([pool[torch.randperm(pool.numel(), generator=gen)] for _ in range(batch)])


def expected_ids(tables, prompt: torch.Tensor, steps: int, chunk: int) -> torch.Tensor:
    """The closed-form greedy continuation of ``prompt`` [B, P] (module docstring)."""

    sigma, nl, no = tables["sigma"], tables["next_local"], tables["next_older"]
    out = []
    for row in prompt.tolist():
        where = {tok: i for i, tok in enumerate(row)}
        t, ids = row[-1], []
        for n in range(steps):
            p = len(row) - 1 + n
            rec = max(0, p // chunk * chunk - chunk)
            x = int(sigma[t])
            t = int(no[x] if where[x] < rec else nl[x])
            ids.append(t)
        out.append(ids)
    return torch.tensor(out, dtype=torch.long)
