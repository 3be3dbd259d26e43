"""GPU parity of the DRAM tier's control plane (csrc/locks_tier.hip through the
C ABI, via locks.tier.Tier) against the CPU oracle (oracle/tier_oracle.py).

A seeded serving scenario (prefills, a block shared by two requests, decode
steps with fresh page selections per layer, arrivals, small hot buffers so
pages are evicted and installs run out of slots) is applied to both.  After
every step every piece of state must be identical:

* residency: page2slot, slot2page, pool_valid, the slots' LRU order (the GPU
  keeps one clock per (layer, kv head), the reference one global clock; the
  order of the clocks inside each (layer, kv head) is what eviction reads),
  per-(request, kv head) miss lists and victims, the fetch list, overflow;
* staging: vbo, v_flushed, the free stack, the flush list, the token slot
  mapping, overflow;
* bytes: every occupied hot slot, every pool-valid pinned page, every
  assigned staging block, of every layer (V, and K for mem-kv).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import tier_oracle as T

pytestmark = pytest.mark.gpu


def say(*a):
    print("[tier-ctl]", *a, flush=True)


def _lru_order(lru):
    """Slots of each (kv head) sorted by (clock, slot)."""
    return np.stack([np.lexsort((np.arange(row.size), row)) for row in lru])


class Both:
    def __init__(self, seed, *, L, n_kv, NB, S, R, MP, page, d, max_tokens, offload_k):
        import torch
        from locks.tier import Tier
        self.rng = np.random.default_rng(seed)
        self.L, self.n_kv, self.NB, self.R, self.MP, self.page, self.d = L, n_kv, NB, R, MP, page, d
        self.g = Tier("cuda", num_layers=L, num_blocks=NB, n_kv=n_kv, head_dim=d, page=page,
                      hot_slots=S, max_reqs=R, max_pages=MP, max_tokens=max_tokens,
                      offload_k=offload_k)
        self.o = T.new_state(L=L, NB=NB, n_kv=n_kv, S=S, NV=self.g.NV, page=page, d=d,
                             max_tokens=max_tokens, offload_k=offload_k)
        perm = self.rng.permutation(NB)
        self.bt = perm[: R * MP].reshape(R, MP).astype(np.int32)
        self.bt[R - 1, 0] = self.bt[0, 0]               # a shared prefix block
        self.bt_d = torch.from_numpy(self.bt).cuda()
        self.lens = []

    def step(self, new, grow):
        import torch
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
        qsl = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
        sl_d = torch.tensor(sl, dtype=torch.int32, device="cuda")
        qsl_d = torch.from_numpy(qsl).cuda()
        ntok = int(qsl[-1])
        self.g.begin_step(self.bt_d, sl_d, qsl_d, n, ntok)
        T.invalidate_written(self.o, self.bt, sl, qsl)
        T.staging_begin_step(self.o, self.bt, sl, qsl, ntok, max_flush=self.g.MAXF)
        for layer in range(self.L):
            val = self.rng.integers(0, 1 << 16, (ntok, self.n_kv, self.d), dtype=np.uint16)
            key = self.rng.integers(0, 1 << 16, (ntok, self.n_kv, self.d), dtype=np.uint16)
            # NaN bit patterns would survive the copies, but keep them finite anyway
            val &= 0xBFFF
            key &= 0xBFFF
            dv = torch.from_numpy(val.view(np.int16)).view(torch.bfloat16).cuda()
            dk = torch.from_numpy(key.view(np.int16)).view(torch.bfloat16).cuda()
            self.g.write_kv(layer, dv, dk if self.g.offload_k else None, ntok)
            T.scatter_kv(self.o, layer, val, key if self.o["offload_k"] else None)
        torch.cuda.synchronize()
        self.compare_staging()
        if not grow and new:
            return
        for layer in range(self.L):
            tab, cnt = self.select(sl)
            pt = torch.full((self.R, self.n_kv, self.MP), -1, dtype=torch.int32)
            pt[:n] = torch.from_numpy(tab)
            pc = torch.zeros((self.R, self.n_kv), dtype=torch.int32)
            pc[:n] = torch.from_numpy(cnt)
            self.g.step(layer, pt.cuda(), pc.cuda(), self.bt_d, sl_d, n)
            miss, vict, fetch = T.gather_plan(self.o, layer, tab, cnt, self.bt, sl, n)
            T.gather_fetch(self.o, layer, fetch)
            torch.cuda.synchronize()
            self.compare_plan(layer, n, miss, vict, fetch)
        self.compare_residency()

    def select(self, sl):
        n = len(sl)
        tab = np.full((n, self.n_kv, self.MP), -1, np.int32)
        cnt = np.zeros((n, self.n_kv), np.int32)
        for r in range(n):
            npg = -(-sl[r] // self.page)
            for kv in range(self.n_kv):
                mid = list(range(1, max(npg - 1, 1)))
                k = min(int(self.rng.integers(1, 6)), len(mid))
                pick = sorted(set([0, npg - 1] + list(self.rng.choice(mid, k, replace=False))))
                tab[r, kv, :len(pick)] = pick
                cnt[r, kv] = len(pick)
        return tab, cnt

    def _np(self, t):
        import torch
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    def compare_staging(self):
        g, o = self.g, self.o
        assert np.array_equal(self._np(g.vbo), o["vbo"])
        assert np.array_equal(self._np(g.v_flushed), o["v_flushed"])
        top = int(g.free_top.item())
        assert top == o["free_top"]
        assert np.array_equal(self._np(g.free_stack)[:top], o["free_stack"][:top])
        assert np.array_equal(self._np(g.v_slot_mapping), o["v_slot_mapping"])
        assert int(g.stg_overflow.item()) == o["stg_overflow"]
        assert np.array_equal(self._np(g.pool_valid), o["pool_valid"])
        vbo = o["vbo"]
        vp = self._np(g.v_pool)
        for b in np.nonzero(vbo >= 0)[0]:
            assert np.array_equal(vp[:, vbo[b]], o["v_pool"][:, vbo[b]]), f"staging block of {b}"
            if o["offload_k"]:
                assert np.array_equal(self._np(g.k_pool)[:, vbo[b]], o["k_pool"][:, vbo[b]])
        pool = self._np(g.pool)
        for l, kv, b in zip(*np.nonzero(o["pool_valid"] == 1)):
            assert np.array_equal(pool[l, b, kv], o["pool"][l, b, kv]), ("pool", l, b, kv)
            if o["offload_k"]:
                assert np.array_equal(self._np(g.pool_k)[l, b, kv], o["pool_k"][l, b, kv])

    def compare_plan(self, layer, n, miss, vict, fetch):
        g = self.g
        mc, mp, vi = self._np(g.miss_cnt), self._np(g.miss_pages), self._np(g.victims)
        for r in range(n):
            for kv in range(self.n_kv):
                m = miss[(r, kv)]
                assert mc[r, kv] == len(m), (layer, r, kv)
                assert mp[r, kv, :len(m)].tolist() == m, (layer, r, kv)
                assert vi[r, kv, :len(m)].tolist() == vict[(r, kv)], (layer, r, kv)
        fc, fl = self._np(g.fetch_cnt), self._np(g.fetch_list)
        got = [(kv, int(fl[kv, u, 0]), int(fl[kv, u, 1])) for kv in range(self.n_kv)
               for u in range(fc[kv])]
        assert got == fetch, (layer, got, fetch)
        assert int(g.res_overflow.item()) == self.o["res_overflow"]

    def compare_residency(self):
        g, o = self.g, self.o
        assert np.array_equal(self._np(g.page2slot), o["page2slot"])
        assert np.array_equal(self._np(g.slot2page), o["slot2page"])
        assert np.array_equal(self._np(g.pool_valid), o["pool_valid"])
        gl = self._np(g.lru)
        for l in range(self.L):
            assert np.array_equal(_lru_order(gl[l]), _lru_order(o["lru"][l])), ("lru order", l)
        hot = self._np(g.hot)
        for l, kv, s in zip(*np.nonzero(o["slot2page"] >= 0)):
            assert np.array_equal(hot[l, kv, s], o["hot"][l, kv, s]), ("hot", l, kv, s)
            if o["offload_k"]:
                assert np.array_equal(self._np(g.hot_k)[l, kv, s], o["hot_k"][l, kv, s])
        g.check_invariants()


CASES = [  # (seed, L, n_kv, NB, S, R, MP, page, d, max_tokens, offload_k)
    (0, 2, 2, 96, 4, 3, 24, 16, 64, 96, False),
    (1, 2, 2, 96, 6, 3, 24, 16, 128, 96, True),
    (2, 3, 4, 160, 9, 3, 40, 32, 64, 256, False),
    (3, 1, 8, 64, 5, 2, 20, 64, 128, 128, True),
]


@pytest.mark.parametrize("seed,L,n_kv,NB,S,R,MP,page,d,max_tokens,offload_k", CASES)
def test_tier_control_plane_matches_oracle(seed, L, n_kv, NB, S, R, MP, page, d, max_tokens,
                                           offload_k):
    say("case", seed, L, n_kv, NB, S, R, MP, page, d, max_tokens, "mem-kv" if offload_k else "mem-v")
    b = Both(seed, L=L, n_kv=n_kv, NB=NB, S=S, R=R, MP=MP, page=page, d=d,
             max_tokens=max_tokens, offload_k=offload_k)
    b.step({0: (0, min(max_tokens, 3 * page - 5))}, grow=False)
    for _ in range(page + 3):
        b.step({}, grow=True)
    arrivals = {r: ((page if r == R - 1 else 0), min(max_tokens // 2, 2 * page + 3)) for r in range(1, R)}
    b.step(arrivals, grow=False)
    for _ in range(2 * page + 5):
        b.step({}, grow=True)
    say("steps done; evictions seen:", int((b.o["lru"] > 0).sum()), "overflow", b.o["res_overflow"])
