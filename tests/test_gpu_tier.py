"""GPU parity of the DRAM-tier V source of the split decode (the mem tier's
data plane; reference attention/decode_cuda.py:178-222).  The reference's
invariant is that a tiered decode equals the resident one on tier-identical
bytes (torch.equal, tier/__init__.py:8-16); here the split partials and the
merged output must match the resident decode bit for bit.

Every (kv head, block) is given exactly one source holding its true bytes --
the one the select rule must pick (hot slot for a complete page, else the
staged block, else the pinned host pool) -- and every other copy, and the
cache's V half (and K half under mem-kv), is filled with NaN, so a read from
any wrong place shows up as NaN or a bit difference.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from tests.cases import make_case, to_dev

pytestmark = pytest.mark.gpu

LAYER, LAYERS, HOT_SLOTS, STAGE_BLOCKS = 1, 2, 8, 24


def say(*a):
    print("[tier]", *a, flush=True)


def _state(case, split):
    import torch
    from locks.attention import ensure_stage_b_buffers
    from locks.selection import Rki4State
    st = Rki4State("cuda", num_layers=1, num_blocks=case.NB, n_kv=case.n_kv, G=case.G,
                   head_dim=case.d, page=case.page, max_reqs=case.R, max_pages=case.MP,
                   budget=0.1, budget_pages=126, sink_pages=1, window_pages=1)
    ensure_stage_b_buffers(st, torch.device("cuda"), split)
    return st


def _tiered(case, d, tab, cnt, k_tier, seed):
    """A Tier with one true source per used (kv head, block); returns
    (tier, {(kh, blk): source}) and poisons the cache halves the tier replaces."""
    import torch
    from locks.tier import Tier
    rng = np.random.default_rng(seed)
    t = Tier("cuda", num_layers=LAYERS, num_blocks=case.NB, n_kv=case.n_kv,
             head_dim=case.d, page=case.page, hot_slots=HOT_SLOTS, v_blocks=STAGE_BLOCKS,
             max_tokens=case.page, offload_k=k_tier)
    t.offload(LAYER, d["kv"], np.arange(case.NB))
    # (row, page) of every selected page, its block and completeness
    used = {}
    for r in range(case.R):
        for kh in range(case.n_kv):
            for pt in tab[r, kh, :cnt[r, kh]].tolist():
                blk = int(case.bt[r, pt])
                used[(kh, blk)] = (pt + 1) * case.page <= case.seq_lens[r]
    blocks = sorted({b for (_, b) in used})
    staged = [b for b in blocks if rng.random() < 0.3][:STAGE_BLOCKS]
    for i, b in enumerate(staged):
        t.stage([d["kv"]] * LAYERS, b, i)
    nan = float("nan")
    src = {}
    next_slot = [0] * case.n_kv
    for (kh, blk), complete in sorted(used.items()):
        hot = next_slot[kh] < HOT_SLOTS and rng.random() < 0.35
        if hot:
            t.make_hot(LAYER, kh, blk, next_slot[kh])
            next_slot[kh] += 1
        s = "hot" if (hot and complete) else ("staged" if blk in staged else "pool")
        src[(kh, blk)] = s
        # poison every copy the rule must not read
        if hot and s != "hot":
            slot = int(t.page2slot[LAYER, kh, blk])
            t.hot[LAYER, kh, slot] = nan
            if k_tier:
                t.hot_k[LAYER, kh, slot] = nan
        if blk in staged and s != "staged":
            sb = int(t.vbo[blk])
            t.v_pool[LAYER, sb, :, kh] = nan
            if k_tier:
                t.k_pool[LAYER, sb, :, kh] = nan
        if s != "pool":
            t.pool[LAYER, blk, kh] = nan
            if k_tier:
                t.pool_k[LAYER, blk, kh] = nan
    # out-of-range keys on pages whose source is the pool: ignored by the select
    bogus = [(kh, blk) for (kh, blk), s in sorted(src.items())
             if s == "pool" and blk not in staged and int(t.page2slot[LAYER, kh, blk]) < 0][:6]
    for kh, blk in bogus:
        t.page2slot[LAYER, kh, blk] = HOT_SLOTS + 3
        t.vbo[blk] = STAGE_BLOCKS + 2
    d["kv"][:, 1] = nan
    if k_tier:
        d["kv"][:, 0] = nan
    torch.cuda.synchronize()
    return t, src


CASES = [
    (2, 4, [16 * 40 + 5, 16 * 9], 16, False, 128, 16),
    (4, 5, [1000, 7, 0, 4099], 32, False, 128, 16),
    (2, 16, [16 * 300 + 3], 64, True, 128, 16),
    (8, 4, [16384], 128, False, 128, 16),
    (8, 4, [16 * 500 + 1, 16 * 200], 128, True, 128, 16),
    (4, 4, [32 * 90 + 7, 32 * 20], 32, True, 64, 32),
    (2, 8, [16 * 200 + 9], 32, False, 256, 16),
    (2, 4, [64 * 40 + 5, 64 * 9], 16, False, 128, 64),
    (2, 4, [64 * 40 + 5, 64 * 9], 16, True, 128, 64),
]


@pytest.mark.parametrize("n_kv,G,seq_lens,split,k_tier,hd,page", CASES)
def test_tier_decode_equals_resident(n_kv, G, seq_lens, split, k_tier, hd, page):
    import torch
    from locks.attention import decode_merge, decode_splitk, decode_splitk_tier
    from locks.attention.decode import _pps_min, _split_kv
    say("tier", n_kv, G, seq_lens, split, "mem-kv" if k_tier else "mem-v", f"d={hd} page={page}")
    MP = max(1, max((s + page - 1) // page for s in seq_lens))
    case = make_case(31, n_kv, G, seq_lens, MP=MP, build=False, page=page, d=hd)
    rng = np.random.default_rng(32)
    npg, nsh, b = O.derive_page_params(seq_lens, page, 1, 1, 126, 0.1)
    sc = rng.random((case.R, n_kv, MP)).astype(np.float32)
    tab, cnt = O.topb_select(sc, npg, nsh, b, 1, MP)
    st = _state(case, split)
    d = to_dev(case)
    st.page_table.copy_(torch.from_numpy(tab))
    st.page_cnt.copy_(torch.from_numpy(cnt))
    pps = _pps_min(case.R)

    def run(tier_src, kv):
        k, v = _split_kv(kv)
        for t in (st.m_part, st.l_part, st.acc_part):
            t.fill_(7.0)                                  # inactive splits store nothing
        kw = dict(n_req=case.R, G=G, split=st.split, pps_min=pps, scale=case.scale)
        if tier_src is None:
            decode_splitk(d["q"], k, v, d["bt"], d["sl"], st.page_table, st.page_cnt, st.m_part,
                          st.l_part, st.acc_part, **kw)
        else:
            decode_splitk_tier(d["q"], k, v, d["bt"], d["sl"], st.page_table, st.page_cnt,
                               st.m_part, st.l_part, st.acc_part, tier_src, **kw)
        out = torch.full((case.R, n_kv * G, case.d), float("nan"), dtype=torch.float32, device="cuda")
        decode_merge(st.m_part, st.l_part, st.acc_part, st.page_cnt, out, n_req=case.R, n_kv=n_kv,
                     G=G, split=st.split, pps_min=pps, pt_cols=st.page_table.shape[2])
        torch.cuda.synchronize()
        return [t.clone() for t in (st.m_part, st.l_part, st.acc_part)], out

    ref_parts, ref_out = run(None, d["kv"])
    tier, src = _tiered(case, d, tab, cnt, k_tier, seed=33)
    n = {s: sum(1 for v in src.values() if v == s) for s in ("hot", "staged", "pool")}
    say(f"sources {n}")
    assert n["pool"] > 0 and (n["hot"] > 0 or sum(seq_lens) < 400)
    parts, out = run(tier.vsource(LAYER).tier_src(), d["kv"])
    for name, a, bb in zip(("m", "l", "acc"), ref_parts, parts):
        assert torch.equal(a, bb), f"{name} partials differ"
    assert torch.equal(ref_out, out)
    live = cnt.sum(axis=1) > 0
    assert torch.isfinite(out[torch.from_numpy(live).cuda()]).all()


def test_tier_through_the_reference_call_and_graph():
    """``decode_dispatch`` with a TierVSource (the reference's seam,
    _runtime.py:807) equals the resident call, eagerly and in a HIP graph
    replayed after the tier moved pages (hot -> evicted, pool -> staged):
    the baked pointers stay valid and only device-side keys change."""
    import torch
    from locks.backend._runtime import decode_dispatch
    say("tier via decode_dispatch + graph")
    n_kv, G, seq_lens = 4, 4, [16 * 120 + 7, 16 * 33]
    MP = max((s + 15) // 16 for s in seq_lens)
    case = make_case(41, n_kv, G, seq_lens, MP=MP, build=False)
    rng = np.random.default_rng(42)
    npg, nsh, b = O.derive_page_params(seq_lens, 16, 1, 1, 40, 0.1)
    sc = rng.random((case.R, n_kv, MP)).astype(np.float32)
    tab, cnt = O.topb_select(sc, npg, nsh, b, 1, MP)
    st = _state(case, 32)
    st.scale = case.scale
    d = to_dev(case)
    st.page_table.copy_(torch.from_numpy(tab))
    st.page_cnt.copy_(torch.from_numpy(cnt))
    H = n_kv * G
    ref = torch.empty(case.R, H, case.d, dtype=torch.bfloat16, device="cuda")
    decode_dispatch(d["q"], d["kv"], d["bt"], d["sl"], st, ref, None, case.scale, None)
    torch.cuda.synchronize()
    from locks.tier import Tier
    t = Tier("cuda", num_layers=1, num_blocks=case.NB, n_kv=n_kv, head_dim=case.d,
             hot_slots=HOT_SLOTS, v_blocks=STAGE_BLOCKS, max_tokens=16)
    t.offload(0, d["kv"], np.arange(case.NB))
    blk0 = [int(case.bt[0, p]) for p in tab[0, 0, :cnt[0, 0]].tolist()]
    for i, blk in enumerate(blk0[:HOT_SLOTS]):
        t.make_hot(0, 0, blk, i)
    kv_src = d["kv"].clone()
    d["kv"][:, 1] = float("nan")
    vs = t.vsource(0)
    out = torch.empty_like(ref)
    decode_dispatch(d["q"], d["kv"], d["bt"], d["sl"], st, out, vs, case.scale, None)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            decode_dispatch(d["q"], d["kv"], d["bt"], d["sl"], st, out, vs, case.scale, None)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        out.fill_(float("nan"))
        if rep == 1:                                  # evict two hot pages, stage another block
            t.evict(0, 0, blk0[0])
            t.evict(0, 0, blk0[1])
            t.stage([kv_src], blk0[-1], 0)
        if rep == 2:
            t.unstage(blk0[-1])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
