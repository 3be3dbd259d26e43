"""The DRAM-tier variants through the engine-neutral driver: a decode loop on
``LocksConfig(variant="mem-v" | "mem-kv")`` equals the resident ``fast``
variant bit for bit (the reference's tier invariant, tier/__init__.py:8-16),
with the whole control plane running: per-step staging lifecycle in the
prologue, per-layer write_kv, residency plan + fetch between selection and
the decode (tier/tier.py:239-301, :386-466, :704-784).

The mem-v engine's cache holds K only in earnest: its V half is NaN from the
start, so every V byte the decode reads comes from the tier's hot slots,
staging pool or pinned pool.  Small hot buffers force LRU evictions and
installs that run out of slots; prefill chunks, an arrival and a stalled
step run through the lifecycle.  After every step the tier's invariants hold
(maps mutual inverses, staging blocks partitioned, no overflow of staging).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PAGE, D = 16, 128


@pytest.mark.parametrize("variant,hot_slots", [("mem-v", 6), ("mem-kv", 6), ("mem-v", 0)])
def test_tier_engine_equals_resident(variant, hot_slots):
    import torch
    from locks.backend.engine import LocksEngine
    from locks.config import LocksConfig

    L, n_kv, G, R, MAXLEN = 3, 2, 4, 2, 16 * 40
    MP = MAXLEN // PAGE
    NB = R * MP + 4
    g = torch.Generator().manual_seed(7)
    res = [torch.zeros(NB, 2, PAGE, n_kv, D, dtype=torch.bfloat16, device="cuda") for _ in range(L)]
    tie = [torch.zeros_like(c) for c in res]
    for c in tie:
        c[:, 1] = float("nan")                       # V lives only in the tier
    perm = torch.randperm(NB, generator=g)[: R * MP].view(R, MP).to(torch.int32)
    bt = perm.cuda()
    kw = dict(num_heads_q=n_kv * G, num_heads_kv=n_kv, head_dim=D, block_size=PAGE,
              max_num_seqs=R, max_model_len=MAXLEN, max_num_batched_tokens=256)
    e_res = LocksEngine(LocksConfig(budget_pages=4), res, **kw)
    e_tie = LocksEngine(LocksConfig(variant=variant, budget_pages=4, hot_slots=hot_slots), tie, **kw)
    tier = e_tie.tier
    print(f"[tier-eng] {variant} hot_slots={tier.S} staging blocks={tier.NV}", flush=True)
    scale = 1.0 / math.sqrt(D)

    lens, qlen = [150], [150]
    for step in range(30):
        if step == 6:
            lens, qlen = lens + [90], [1, 90]
        n = len(lens)
        qs = np.concatenate([[0], np.cumsum(qlen)])
        sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
        qsd = torch.tensor(qs, dtype=torch.int32, device="cuda")
        e_res.prologue(bt, sl, qsd, n, np.array(lens), qs)
        e_tie.prologue(bt, sl, qsd, n, np.array(lens), qs)
        toks = [(r, p) for r in range(n) for p in range(lens[r] - qlen[r], lens[r])]
        for layer in range(L):
            kv = torch.randn(len(toks), 2, n_kv, D, generator=g).to(torch.bfloat16).cuda()
            for i, (r, p) in enumerate(toks):
                b = int(perm[r, p // PAGE])
                res[layer][b, :, p % PAGE] = kv[i]
                tie[layer][b, 0, p % PAGE] = kv[i, 0]
                if variant == "mem-kv":
                    pass                             # K stays resident too: summaries read it
            e_res.write_kv(layer, kv[:, 0], kv[:, 1])
            e_tie.write_kv(layer, kv[:, 0].contiguous(), kv[:, 1].contiguous())
        if all(x == 1 for x in qlen):
            q = [torch.randn(n, n_kv * G, D, generator=g).to(torch.bfloat16).cuda() for _ in range(L)]
            for layer in range(L):
                o_res = torch.empty(n, n_kv * G, D, dtype=torch.bfloat16, device="cuda")
                o_tie = torch.full_like(o_res, float("nan"))
                e_res.forward(q[layer], res[layer], bt, sl, n, scale, o_res)
                e_tie.forward(q[layer], tie[layer], bt, sl, n, scale, o_tie)
                torch.cuda.synchronize()
                assert torch.equal(e_res.st.page_table, e_tie.st.page_table), (step, layer)
                assert torch.equal(o_res.view(torch.int16), o_tie.view(torch.int16)), (step, layer)
            hits = int((tier.lru > 0).sum())
            print(f"[tier-eng] step {step} lens {lens} ok; touched slots {hits}", flush=True)
        tier.check_invariants()
        assert int(tier.stg_overflow.item()) == 0
        if step != 14:
            lens = [x + 1 for x in lens]
        qlen = [1] * len(lens)
