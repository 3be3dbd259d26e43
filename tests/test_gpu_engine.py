"""End-to-end decode loop through the engine-neutral driver (LocksEngine).

Steps mimic a serving engine: a prefill step (dense attention, keys written
after the prologue), then single-token decode steps whose new key and value
are written before attention, an arrival and a frozen drain replay.  After
every decode step:

* the page tables equal those of a fresh state whose summaries are built
  from scratch out of the current cache (so the refresh gate kept every
  scored summary current, with no stale or missing page);
* the output equals fp32 softmax attention over exactly the selected pages
  (max abs 2e-2, mean rel 1e-3);
* with a budget that covers every page, the output equals dense attention.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PAGE, D = 16, 128


def _attend(q, K, V, bt, sl, tab, cnt, r, kh, G, scale):
    """fp32 attention of request r, kv head kh's query heads over the listed
    logical pages (tokens past seq_len masked)."""
    import torch
    pages = tab[r, kh, : cnt[r, kh]].tolist()
    toks = [p * PAGE + t for p in pages for t in range(PAGE) if p * PAGE + t < sl[r]]
    blk = [int(bt[r, t // PAGE]) for t in toks]
    k = torch.stack([K[b, t % PAGE, kh] for b, t in zip(blk, toks)]).float()
    v = torch.stack([V[b, t % PAGE, kh] for b, t in zip(blk, toks)]).float()
    qq = q[r, kh * G:(kh + 1) * G].float()
    p = torch.softmax((qq @ k.T) * scale, dim=-1)
    return p @ v


def _run(budget_pages, steps, check_fresh, full_budget=False, kv_first=False):
    import torch
    from locks.backend.engine import LocksEngine
    from locks.config import LocksConfig
    from locks.selection import Rki4State, derive_page_params, rki4_build_bulk
    from locks.backend import _runtime

    L, n_kv, G, R, MAXLEN = 3, 2, 4, 2, 16 * 40
    MP = MAXLEN // PAGE
    NB = R * MP + 4
    g = torch.Generator().manual_seed(5)
    if kv_first:                                 # vLLM 0.11 layout (2, NB, page, n_kv, d)
        caches = [torch.zeros(2, NB, PAGE, n_kv, D, dtype=torch.bfloat16, device="cuda")
                  for _ in range(L)]
    else:
        caches = [torch.zeros(NB, 2, PAGE, n_kv, D, dtype=torch.bfloat16, device="cuda")
                  for _ in range(L)]

    def halves(c):
        return (c[0], c[1]) if kv_first else (c[:, 0], c[:, 1])
    perm = torch.randperm(NB, generator=g)[: R * MP].view(R, MP).to(torch.int32)
    bt = perm.cuda()
    cfg = LocksConfig(budget_pages=budget_pages, sink_pages=1, window_pages=1)
    eng = LocksEngine(cfg, caches, num_heads_q=n_kv * G, num_heads_kv=n_kv, head_dim=D,
                      block_size=PAGE, max_num_seqs=R, max_model_len=MAXLEN)
    scale = 1.0 / math.sqrt(D)

    def write(r, pos):
        b = int(perm[r, pos // PAGE])
        for c in caches:
            kv = torch.randn(2, n_kv, D, generator=g).to(torch.bfloat16).cuda()
            Kc, Vc = halves(c)
            Kc[b, pos % PAGE] = kv[0]
            Vc[b, pos % PAGE] = kv[1]

    lens, qlen = [150], [150]                    # prefill of request 0
    worst = 0.0
    for step in range(steps):
        if step == 6:                            # request 1 arrives (prefill 90)
            lens, qlen = lens + [90], [1, 90]
        n = len(lens)
        qs = np.concatenate([[0], np.cumsum(qlen)])
        sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
        qsd = torch.tensor(qs, dtype=torch.int32, device="cuda")
        eng.prologue(bt, sl, qsd, n, np.array(lens), qs)
        decode = all(x == 1 for x in qlen)
        if not decode:                           # dense attention step: keys land after
            for r in range(n):
                for pos in range(lens[r] - qlen[r], lens[r]):
                    write(r, pos)
        else:
            for r in range(n):
                write(r, lens[r] - 1)            # the new token, before attention
            q = [torch.randn(n, n_kv * G, D, generator=g).to(torch.bfloat16).cuda() for _ in range(L)]
            outs = []
            for layer in range(L):
                out = torch.empty(n, n_kv * G, D, dtype=torch.bfloat16, device="cuda")
                eng.forward(q[layer], caches[layer], bt, sl, n, scale, out)
                tab = eng.st.page_table.clone()
                cnt = eng.st.page_cnt.clone()
                outs.append((out, tab, cnt))
            torch.cuda.synchronize()
            print(f"[case] engine budget={budget_pages} step={step} lens={lens}", flush=True)
            if check_fresh:
                fresh = Rki4State("cuda", num_layers=L, num_blocks=NB, n_kv=n_kv, G=G,
                                  head_dim=D, page=PAGE, max_reqs=R, max_pages=MP,
                                  budget=0.1, budget_pages=budget_pages)
                fresh._layer_of = {c.data_ptr(): i for i, c in enumerate(caches)}
                ks = [halves(c)[0] for c in caches]
                settled = sl[:n] - 1
                rki4_build_bulk(fresh, ks, bt, settled, n, int(settled.max()) // PAGE)
                derive_page_params(fresh, sl, n)
            for layer in range(L):
                out, tab, cnt = outs[layer]
                K, V = halves(caches[layer])
                if check_fresh:
                    _runtime._rki4_select_adapter(q[layer], caches[layer], bt, sl, fresh, n,
                                                  scale, cfg)
                    for r in range(n):
                        for kh in range(n_kv):
                            c = int(cnt[r, kh])
                            assert c == int(fresh.page_cnt[r, kh])
                            assert torch.equal(tab[r, kh, :c], fresh.page_table[r, kh, :c]), \
                                (step, layer, r, kh)
                esum = rsum = 0.0
                for r in range(n):
                    for kh in range(n_kv):
                        if full_budget:              # every page selected: dense attention
                            assert int(cnt[r, kh]) == -(-lens[r] // PAGE)
                        # bf16 output vs the bf16-rounded fp32 reference
                        ref = _attend(q[layer], K, V, bt, lens, tab, cnt, r, kh, G, scale)
                        ref = ref.to(torch.bfloat16).float()
                        err = (out[r, kh * G:(kh + 1) * G].float() - ref).abs()
                        worst = max(worst, float(err.max()))
                        assert float(err.max()) <= 2e-2, (step, layer, r, kh)
                        esum += float(err.sum())
                        rsum += float(ref.abs().sum())
                assert esum / rsum <= 1e-3, (step, layer, esum / rsum)
        if step != 14:                           # step 15 replays step 14's lengths
            lens = [x + 1 for x in lens]
        qlen = [1] * len(lens)
    return worst


def test_engine_decode_loop_selection_and_output():
    _run(budget_pages=4, steps=26, check_fresh=True)


def test_engine_full_budget_equals_dense():
    """Every page selected: the sparse output is dense attention."""
    _run(budget_pages=64, steps=10, check_fresh=False, full_budget=True)


def test_engine_kv_first_cache_layout():
    """The (2, num_blocks, page, n_kv, d) cache layout of vLLM 0.11."""
    _run(budget_pages=4, steps=12, check_fresh=True, kv_first=True)
