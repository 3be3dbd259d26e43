"""CPU restatement of the DRAM tier's control plane (TEST INFRASTRUCTURE ONLY:
imported by tests/ alone; the product path never calls it).

Follows the reference's per-step tier lifecycle (src/locks/tier/), as
sequential numpy / Python loops over one state dict:

* residency (tier/residency.py): invalidate_written (:271-307, :389-419),
  gather_plan = miss_diff (:51-88) + select_victims (:91-145) with the
  clock advance (:437-459), gather_fetch (:216-268, :461-488);
* staging (tier/staging.py): begin_step (:373-442) = vflush_clear
  (:125-138), flush_collect (:141-191), flush_copy (:247-277), valloc
  (:194-221), vslot (:224-244); scatter_kv (:57-82, :444-460).

Where the reference leaves an order to GPU atomics (the flush list and the
free-stack pushes of one flush_collect block, the flat fetch list), this
restatement fixes it to ascending page order (flush list, free stack) and to
(kv head, install order) for the fetch list, the orders the HIP kernels use;
the fetch list is a set for every reader (each entry copies one page to its
own slot).  The copy-engine transport (build/issue_dma_plan), the K5 claim
machinery (owner, gen, pending -2 slots) and prefill leases are not restated:
this build does not implement them.

Buffers (numpy, bf16 as uint16 bits):
  hot (L, n_kv, S, page, d), page2slot (L, n_kv, NB), slot2page (L, n_kv, S),
  lru (L, n_kv, S), pool_valid (L, n_kv, NB), clock (scalar; the reference's
  one global clock), v_pool (L, NV, page, n_kv, d), vbo (NB,), v_flushed
  (NB,), free_stack (NV,), free_top, v_slot_mapping (max_tokens,), pool (L,
  NB, n_kv, page, d), overflow flags; *_k twins when offload_k.
"""
from __future__ import annotations

import numpy as np


def new_state(*, L, NB, n_kv, S, NV, page, d, max_tokens, offload_k=False):
    """Fresh tier state (residency.py:313-387, staging.py:291-371)."""
    u16, i32 = np.uint16, np.int32
    st = dict(
        L=L, NB=NB, n_kv=n_kv, S=S, NV=NV, page=page, d=d, offload_k=offload_k,
        hot=np.zeros((L, n_kv, S, page, d), u16),
        page2slot=np.full((L, n_kv, NB), -1, i32),
        slot2page=np.full((L, n_kv, S), -1, i32),
        lru=np.zeros((L, n_kv, S), i32),
        pool_valid=np.zeros((L, n_kv, NB), np.int8),
        clock=1, res_overflow=0,
        v_pool=np.zeros((L, NV, page, n_kv, d), u16),
        vbo=np.full((NB,), -1, i32),
        v_flushed=np.zeros((NB,), i32),
        free_stack=np.arange(NV, dtype=i32),
        free_top=NV, stg_overflow=0,
        v_slot_mapping=np.full((max_tokens,), -1, np.int64),
        pool=np.zeros((L, NB, n_kv, page, d), u16),
    )
    if offload_k:
        st["hot_k"] = np.zeros_like(st["hot"])
        st["k_pool"] = np.zeros_like(st["v_pool"])
        st["pool_k"] = np.zeros_like(st["pool"])
    return st


def _written(bt, sl, qsl, page):
    """(r, ctx, first written page, last written page) of every request with
    tokens this step (staging.py:487-506)."""
    for r in range(len(sl)):
        s, ql = int(sl[r]), int(qsl[r + 1] - qsl[r])
        if s <= 0:
            continue
        yield r, s, ql


def invalidate_written(st, bt, sl, qsl):
    """residency.py:271-307: drop pool validity and hot residency of every page
    (re)written this step, all layers.  Guard is sl > 0 only (a request with
    ql = 0 re-invalidates its partial tail page, as the reference does)."""
    page, n_kv = st["page"], st["n_kv"]
    for r, s, ql in _written(bt, sl, qsl, page):
        p0, p1 = (s - ql) // page, (s - 1) // page
        for p in range(p0, p1 + 1):
            blk = int(bt[r, p])
            for l in range(st["L"]):
                for kv in range(n_kv):
                    st["pool_valid"][l, kv, blk] = 0
                    slot = int(st["page2slot"][l, kv, blk])
                    if slot >= 0:
                        st["slot2page"][l, kv, slot] = -1
                    if slot != -1:
                        st["page2slot"][l, kv, blk] = -1


def gather_plan(st, layer, tab, cnt, bt, sl, n_req):
    """residency.py:437-459 (clock += 1), miss_diff :51-88, select_victims
    :91-145.  Returns (miss_pages {(r, kv): [blk...]}, victims {(r, kv):
    [slot or -1 ...]}, fetch list [(kv, blk, slot)] in (kv, install) order)."""
    page, S, n_kv = st["page"], st["S"], st["n_kv"]
    st["clock"] += 1
    clk = st["clock"]
    p2s, s2p, lru = st["page2slot"][layer], st["slot2page"][layer], st["lru"][layer]
    miss = {}
    for r in range(n_req):                               # miss_diff, grid (n_req, n_kv)
        for kv in range(n_kv):
            n, s = int(cnt[r, kv]), int(sl[r])
            m = []
            for i in range(n):
                pt = int(tab[r, kv, i])
                blk = int(bt[r, pt])
                if (pt + 1) * page > s:
                    continue                             # partial tail: neither
                slot = int(p2s[kv, blk])
                if slot >= 0:
                    lru[kv, slot] = clk                  # hit: touched this step
                else:
                    m.append(blk)
            miss[(r, kv)] = m
    victims, fetch = {}, []
    for kv in range(n_kv):                               # select_victims, grid (n_kv,)
        for r in range(n_req):
            v = []
            for blk in miss[(r, kv)]:
                if p2s[kv, blk] >= 0:                    # installed earlier this pass
                    v.append(-1)
                    continue
                ck = np.where(lru[kv] >= clk, np.iinfo(np.int32).max, lru[kv])
                best = int(np.argmin(ck))                # first (lowest) slot on ties
                if ck[best] == np.iinfo(np.int32).max:
                    st["res_overflow"] = 1
                    v.append(-1)
                    continue
                old = int(s2p[kv, best])
                if old >= 0:
                    p2s[kv, old] = -1
                p2s[kv, blk] = best
                s2p[kv, best] = blk
                lru[kv, best] = clk
                v.append(best)
                fetch.append((kv, blk, best))
            victims[(r, kv)] = v
    return miss, victims, fetch


def gather_fetch(st, layer, fetch):
    """residency.py:216-268: each installed miss page's V (and K) into its hot
    slot: from the pinned pool when flushed, else from the staging pool via
    vbo with write-through to the pool (sets pool_valid), else the pool."""
    for kv, blk, slot in fetch:
        names = [("hot", "pool", "v_pool")]
        if st["offload_k"]:
            names.append(("hot_k", "pool_k", "k_pool"))
        if st["pool_valid"][layer, kv, blk] > 0:
            for h, p, _ in names:
                st[h][layer, kv, slot] = st[p][layer, blk, kv]
            continue
        vb = int(st["vbo"][blk])
        if vb >= 0:
            for h, p, sp in names:
                x = st[sp][layer, vb, :, kv, :]
                st[h][layer, kv, slot] = x
                st[p][layer, blk, kv] = x
            st["pool_valid"][layer, kv, blk] = 1
        else:
            for h, p, _ in names:
                st[h][layer, kv, slot] = st[p][layer, blk, kv]


def staging_begin_step(st, bt, sl, qsl, n_tokens, max_flush):
    """staging.py:373-442 in its fixed order: reset the slot mapping, clear
    the flushed latch of written pages, collect + free complete staged pages,
    copy the collected pages to the pinned pool, allocate staging blocks for
    written pages, fill the slot mapping.  Returns the flush list."""
    page = st["page"]
    if n_tokens > st["v_slot_mapping"].shape[0]:
        raise RuntimeError("n_tokens exceeds the slot mapping capacity")
    st["v_slot_mapping"][:] = -1
    vfl, vbo = st["v_flushed"], st["vbo"]
    for r, s, ql in _written(bt, sl, qsl, page):          # vflush_clear :125-138
        if ql <= 0:
            continue
        for p in range((s - ql) // page, (s - 1) // page + 1):
            vfl[int(bt[r, p])] = 0
    flush = []                                            # flush_collect :141-191
    for r, s, ql in _written(bt, sl, qsl, page):
        if ql <= 0:
            continue
        for p in range((s - ql) // page):
            blk = int(bt[r, p])
            vb = int(vbo[blk])
            if vb < 0:
                continue
            if vfl[blk] == 0:
                vfl[blk] = 1
                if len(flush) < max_flush:
                    flush.append((blk, vb))
                else:                                     # list full: stays staged
                    vfl[blk] = 0
                    continue
            vbo[blk] = -1                                 # free after the claim
            st["free_stack"][st["free_top"]] = vb
            st["free_top"] += 1
    for blk, vb in flush:                                 # flush_copy :247-277
        for l in range(st["L"]):
            for kv in range(st["n_kv"]):
                st["pool"][l, blk, kv] = st["v_pool"][l, vb, :, kv, :]
                if st["offload_k"]:
                    st["pool_k"][l, blk, kv] = st["k_pool"][l, vb, :, kv, :]
                st["pool_valid"][l, kv, blk] = 1
    for r, s, ql in _written(bt, sl, qsl, page):          # valloc :194-221
        if ql <= 0:
            continue
        for p in range((s - ql) // page, (s - 1) // page + 1):
            blk = int(bt[r, p])
            if vbo[blk] >= 0:
                continue
            if st["free_top"] <= 0:
                st["stg_overflow"] = 1
                continue
            st["free_top"] -= 1
            vbo[blk] = st["free_stack"][st["free_top"]]
    for r, s, ql in _written(bt, sl, qsl, page):          # vslot :224-244
        if ql <= 0:
            continue
        for i in range(ql):
            pos = s - ql + i
            vb = int(vbo[int(bt[r, pos // page])])
            st["v_slot_mapping"][int(qsl[r]) + i] = vb * page + pos % page if vb >= 0 else -1
    return flush


def scatter_kv(st, layer, value, key=None):
    """staging.py:57-82: token t's V (and K) (n_kv, d) into the staging pool at
    v_slot_mapping[t] (skipped when -1)."""
    page = st["page"]
    for t in range(value.shape[0]):
        vs = int(st["v_slot_mapping"][t])
        if vs < 0:
            continue
        st["v_pool"][layer, vs // page, vs % page] = value[t]
        if st["offload_k"]:
            st["k_pool"][layer, vs // page, vs % page] = key[t]
