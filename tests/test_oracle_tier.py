"""Pins of the DRAM tier oracle (oracle/tier_oracle.py) by properties its
sequential loops do not restate (CPU only).

A seeded serving scenario (prefills, a shared prefix block, decodes with
fresh page selections, an arrival) drives the oracle step by step with small
hot buffers so pages are evicted; after every step:

* source rule (the reason the tier exists): for every selected page of every
  (request, kv head), the bytes the decode's select rule reads -- hot slot if
  the page is complete and mapped, else the staging block, else the pinned
  pool -- are exactly the V (and K) written for that page;
* I1 no lost V (staging.py:590-604): every complete page is staged or flushed
  in every layer; I3 staging blocks: assigned + free partition [0, NV);
* I2/I3 residency (residency.py:602-765 R1-R3): page2slot and slot2page are
  mutual inverses and hot[slot] holds slot2page[slot]'s bytes;
* exact LRU, checked against each call's before/after maps without the
  oracle's argmin: every evicted page's slot was last used no later than
  every slot that kept a page it was not asked for (ties: lower slot first),
  installs = distinct missing complete pages (min with the free slots), and
  no page that was selected this call is evicted;
* a brute-force check of the victim order on tiny pools (every LRU order of
  3-4 slots against a direct "oldest first" simulation).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import tier_oracle as T

PAGE, D = 16, 8


def _bf(rng, *shape):
    return rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)


class Scenario:
    """Block tables, token writes and page selections of a few requests."""

    def __init__(self, seed, L=2, n_kv=2, NB=48, S=4, NV=40, R=3, MP=12, max_tokens=96,
                 offload_k=False):
        self.rng = np.random.default_rng(seed)
        self.L, self.n_kv, self.NB, self.R, self.MP = L, n_kv, NB, R, MP
        self.st = T.new_state(L=L, NB=NB, n_kv=n_kv, S=S, NV=NV, page=PAGE, d=D,
                              max_tokens=max_tokens, offload_k=offload_k)
        perm = self.rng.permutation(NB)
        self.bt = np.full((R, MP), -1, np.int32)
        for r in range(R):
            self.bt[r] = perm[r * MP:(r + 1) * MP]
        self.bt[2, 0] = self.bt[0, 0]              # request 2 shares request 0's first block
        # true bytes per (layer, block, token, kv): V and K
        self.V = np.zeros((L, NB, PAGE, n_kv, D), np.uint16)
        self.K = np.zeros_like(self.V)
        self.lens = []

    def step(self, new, grow):
        """new: {r: (ctx_cached, qlen)} arrivals; grow: decode the others."""
        st, rng = self.st, self.rng
        sl, ql = [], []
        for r in range(len(self.lens) + len(new)):
            if r < len(self.lens):
                self.lens[r] += 1 if grow else 0
                sl.append(self.lens[r])
                ql.append(1 if grow else 0)
            else:
                ctx, q = new[r]
                self.lens.append(ctx + q)
                sl.append(ctx + q)
                ql.append(q)
        n = len(sl)
        qsl = np.concatenate([[0], np.cumsum(ql)]).astype(np.int64)
        T.invalidate_written(st, self.bt, sl, qsl)
        T.staging_begin_step(st, self.bt, sl, qsl, int(qsl[-1]), max_flush=64)
        toks = [(r, pos) for r in range(n) for pos in range(sl[r] - ql[r], sl[r])]
        for layer in range(self.L):
            val = _bf(rng, len(toks), self.n_kv, D)
            key = _bf(rng, len(toks), self.n_kv, D)
            for i, (r, pos) in enumerate(toks):
                b = self.bt[r, pos // PAGE]
                self.V[layer, b, pos % PAGE] = val[i]
                self.K[layer, b, pos % PAGE] = key[i]
            T.scatter_kv(st, layer, val, key if st["offload_k"] else None)
        self.check_staging(sl)
        if not grow and new:                       # prefill step: no selection
            return sl, None
        plans = []
        for layer in range(self.L):
            tab, cnt = self.select(sl)
            before = (st["page2slot"][layer].copy(), st["slot2page"][layer].copy(),
                      st["lru"][layer].copy())
            miss, vict, fetch = T.gather_plan(st, layer, tab, cnt, self.bt, sl, n)
            T.gather_fetch(st, layer, fetch)
            plans.append((layer, tab, cnt, before, miss, vict, fetch))
            self.check_lru(layer, tab, cnt, sl, before, fetch)
            self.check_sources(layer, tab, cnt, sl)
        self.check_residency()
        return sl, plans

    def select(self, sl):
        """Random kept pages per (request, kv head): sink, window, and a few
        middle pages (what the decode reads; selection itself is not under test)."""
        n = len(sl)
        tab = np.full((n, self.n_kv, self.MP), -1, np.int32)
        cnt = np.zeros((n, self.n_kv), np.int32)
        for r in range(n):
            npg = -(-sl[r] // PAGE)
            for kv in range(self.n_kv):
                mid = list(range(1, max(npg - 1, 1)))
                pick = sorted(set([0, npg - 1] + list(self.rng.choice(mid, min(3, len(mid)),
                                                                       replace=False))))
                tab[r, kv, :len(pick)] = pick
                cnt[r, kv] = len(pick)
        return tab, cnt

    def check_staging(self, sl):
        st = self.st
        vbo = st["vbo"]
        assigned = vbo[vbo >= 0]
        free = st["free_stack"][: st["free_top"]]
        assert sorted(assigned.tolist() + free.tolist()) == list(range(st["NV"]))
        for r, s in enumerate(sl):
            for p in range(s // PAGE):              # complete pages: staged or flushed
                b = self.bt[r, p]
                assert vbo[b] >= 0 or st["pool_valid"][:, :, b].all(), (r, p)

    def check_residency(self):
        st = self.st
        for l in range(self.L):
            for kv in range(self.n_kv):
                for slot, b in enumerate(st["slot2page"][l, kv]):
                    if b >= 0:
                        assert st["page2slot"][l, kv, b] == slot
                        assert np.array_equal(st["hot"][l, kv, slot], self.V[l, b, :, kv])
                for b, slot in enumerate(st["page2slot"][l, kv]):
                    if slot >= 0:
                        assert st["slot2page"][l, kv, slot] == b

    def check_sources(self, layer, tab, cnt, sl):
        st = self.st
        for r in range(len(sl)):
            for kv in range(self.n_kv):
                for pt in tab[r, kv, :cnt[r, kv]]:
                    b = self.bt[r, pt]
                    complete = (pt + 1) * PAGE <= sl[r]
                    slot, vb = st["page2slot"][layer, kv, b], st["vbo"][b]
                    if complete and slot >= 0:
                        got = st["hot"][layer, kv, slot]
                        gk = st["hot_k"][layer, kv, slot] if st["offload_k"] else None
                    elif vb >= 0:
                        got = st["v_pool"][layer, vb, :, kv]
                        gk = st["k_pool"][layer, vb, :, kv] if st["offload_k"] else None
                    else:
                        got = st["pool"][layer, b, kv]
                        gk = st["pool_k"][layer, b, kv] if st["offload_k"] else None
                    valid = min(PAGE, sl[r] - pt * PAGE)
                    assert np.array_equal(got[:valid], self.V[layer, b, :valid, kv]), (r, kv, pt)
                    if gk is not None:
                        assert np.array_equal(gk[:valid], self.K[layer, b, :valid, kv])

    def check_lru(self, layer, tab, cnt, sl, before, fetch):
        st = self.st
        p2s0, s2p0, lru0 = before
        s2p1 = st["slot2page"][layer]
        for kv in range(self.n_kv):
            asked = {int(self.bt[r, pt]) for r in range(len(sl)) for pt in tab[r, kv, :cnt[r, kv]]
                     if (pt + 1) * PAGE <= sl[r]}
            hits = {b for b in asked if p2s0[kv, b] >= 0}
            missing = asked - hits
            touched = {int(p2s0[kv, b]) for b in hits}
            installs = [(b, s) for (k, b, s) in fetch if k == kv]
            free_slots = [s for s in range(st["S"]) if s not in touched]
            assert len(installs) == min(len(missing), len(free_slots))
            assert {b for b, _ in installs} <= missing
            replaced = {s for _, s in installs}
            assert not (replaced & touched)
            # every replaced slot is no younger than every kept, untouched slot
            kept = [s for s in free_slots if s not in replaced]
            for s in replaced:
                for t in kept:
                    assert (lru0[kv, s], s) < (lru0[kv, t], t), (kv, s, t)
            # install order = oldest slot first for the earliest miss
            order = sorted(replaced, key=lambda s: (lru0[kv, s], s))
            assert [s for _, s in installs] == order
            for b in asked:                        # every asked page resident unless slots ran out
                if len(missing) <= len(free_slots):
                    assert st["page2slot"][layer, kv, b] >= 0
            for s in range(st["S"]):
                if s not in replaced:
                    assert s2p1[kv, s] == s2p0[kv, s]


@pytest.mark.parametrize("offload_k", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tier_oracle_serving_scenario(seed, offload_k):
    sc = Scenario(seed, offload_k=offload_k)
    sc.step({0: (0, 40)}, grow=False)                     # prefill request 0 (2.5 pages)
    for _ in range(20):
        sc.step({}, grow=True)
    sc.step({1: (0, 33), 2: (16, 20)}, grow=False)        # arrivals; request 2 shares a block
    for _ in range(40):
        sc.step({}, grow=True)
    st = sc.st
    # 4 hot slots against up to 3 requests x 5 pages: installs run out of
    # slots (the overflow latch), staging never does
    assert st["res_overflow"] == 1 and st["stg_overflow"] == 0
    assert (st["pool_valid"] == 1).sum() > 0 and (st["slot2page"] >= 0).all()


def test_lru_order_brute_force():
    """Tiny pools: for every LRU clock assignment of 4 slots and 1-4 missing
    pages, gather_plan's victims are the slots a direct simulation picks
    (repeatedly the untouched slot with the oldest clock, lowest slot on a
    tie), in that order."""
    import itertools
    for clocks in itertools.product(range(3), repeat=4):
        for n_miss in range(1, 5):
            st = T.new_state(L=1, NB=16, n_kv=1, S=4, NV=4, page=PAGE, d=D, max_tokens=4)
            st["lru"][0, 0] = clocks
            st["clock"] = 5
            for s in range(4):                              # slots hold blocks 8..11
                st["page2slot"][0, 0, 8 + s] = s
                st["slot2page"][0, 0, s] = 8 + s
            bt = np.arange(16, dtype=np.int32)[None]
            tab = np.full((1, 1, 16), -1, np.int32)
            tab[0, 0, :n_miss] = np.arange(n_miss)               # blocks 0.. missing
            tab[0, 0, n_miss] = 8                                # one hit: slot 0 touched
            cnt = np.array([[n_miss + 1]], np.int32)
            _, vict, fetch = T.gather_plan(st, 0, tab, cnt, bt, [16 * 16], 1)
            avail = [(c, s) for s, c in enumerate(clocks) if s != 0]
            expect = [s for _, s in sorted(avail)][:n_miss]
            assert [s for (_, _, s) in fetch] == expect, (clocks, n_miss)
            assert vict[(0, 0)] == expect + [-1] * (n_miss - len(expect))
            assert st["res_overflow"] == (1 if n_miss > 3 else 0)
