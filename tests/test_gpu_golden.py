"""The HIP hot path on the committed golden fixture
(tests/golden/locks_golden.npz): the stored inputs go through the kernels
and the results are compared with the stored oracle outputs, at the bars of
the parity tests:
  * score_h within 2e-5 on every scored page;
  * page tables and counts bit-exact for the "max" combine; for "nrm" the
    combined scores within 1e-5 x G and the kept sets equal up to near-ties
    of the b-th score (and bit-exact against the oracle's top-b of the GPU's
    own combined scores);
  * attention: fp32 output within 2e-3 max-abs, bf16 within 2e-2 max-abs
    and 1e-3 mean-rel of the stored float64 result.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import locks_oracle as O

pytestmark = pytest.mark.gpu

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "locks_golden.npz")
SLAB_KEYS = ("v4", "vs", "c8", "cs", "mu8", "mus")


def say(*a):
    print("[golden]", *a, flush=True)


@pytest.fixture(scope="module")
def gold():
    with np.load(PATH, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bf(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _state(n_kv, G, NB, R, MP, budget_pages, combine, split=32):
    import torch
    from locks.attention import ensure_stage_b_buffers
    from locks.selection import Rki4State
    st = Rki4State("cuda", num_layers=1, num_blocks=NB, n_kv=n_kv, G=G, head_dim=128, page=16,
                   max_reqs=R, max_pages=MP, budget=0.1, budget_pages=budget_pages,
                   sink_pages=1, window_pages=1, combine=combine)
    ensure_stage_b_buffers(st, torch.device("cuda"), split)
    return st


def _load_slabs(st, gold):
    import torch
    for name, attr in (("v4", "pp_v4"), ("c8", "pp_c8"), ("mu8", "pp_mu8")):
        getattr(st, attr)[0].copy_(torch.from_numpy(gold["pipe_slab_" + name]))
    for name, attr in (("vs", "pp_vs"), ("cs", "pp_cs"), ("mus", "pp_mus")):
        getattr(st, attr)[0].copy_(torch.from_numpy(gold["pipe_slab_" + name].view(np.int16)).view(torch.bfloat16))


def _set_scores(st, sh, nsh):
    """score_h and the per-chunk head maxima the scorer would publish."""
    import torch
    R, n_kv, G, MP = sh.shape
    pm = np.full((R, n_kv, 16, st.score_chunks), -np.inf, np.float32)
    for r in range(R):
        for z in range(st.score_chunks):
            lo, hi = z * st.score_chunk, min((z + 1) * st.score_chunk, int(nsh[r]))
            if hi > lo:
                pm[r, :, :G, z] = sh[r, :, :, lo:hi].max(axis=-1)
    st.score_h.copy_(torch.from_numpy(sh))
    st.page_max.copy_(torch.from_numpy(pm))


def _check_select(st, prefix, gold, combine, G):
    import torch
    torch.cuda.synchronize()
    R = st.page_cnt.shape[0]
    npg, nsh, b = gold[prefix + "npg"], gold[prefix + "nsh"], gold[prefix + "b"]
    assert np.array_equal(st.n_pages.cpu().numpy()[:R], npg)
    assert np.array_equal(st.n_sel_hi.cpu().numpy()[:R], nsh)
    assert np.array_equal(st.b_fix.cpu().numpy()[:R], b)
    gtab, gcnt = st.page_table.cpu().numpy(), st.page_cnt.cpu().numpy()
    gsc = st.score.cpu().numpy()
    tab, cnt = gold[prefix + "tab_" + combine], gold[prefix + "cnt_" + combine]
    comb = gold[prefix + "comb_" + combine]
    assert np.array_equal(gcnt, cnt)
    for r in range(R):
        P = int(nsh[r])
        if combine == "max":
            assert np.array_equal(gsc[r, :, :P], comb[r, :, :P])
        else:
            assert np.abs(gsc[r, :, :P] - comb[r, :, :P]).max(initial=0) <= 1e-5 * G
    if combine == "max":
        assert np.array_equal(gtab, tab)
    else:
        n_diff = 0
        for r in range(R):
            for kh in range(gcnt.shape[1]):
                a = set(gtab[r, kh, :gcnt[r, kh]].tolist())
                c = set(tab[r, kh, :cnt[r, kh]].tolist())
                if a == c:
                    continue
                sel = comb[r, kh, 1:nsh[r]]
                tau = np.sort(sel)[::-1][b[r] - 1]
                for p in a ^ c:
                    assert abs(comb[r, kh, p] - tau) <= 1e-5 * max(abs(tau), 1e-30), p
                    n_diff += 1
        say(prefix, combine, "near-tie differences:", n_diff)
    tab2, cnt2 = O.topb_select(gsc, npg, nsh, b, 1, gtab.shape[-1])
    assert np.array_equal(gtab, tab2) and np.array_equal(gcnt, cnt2)


def test_golden_score(gold):
    import torch
    from locks.selection import derive_page_params, rki4_score_only
    q, bt, sl = gold["pipe_q"], gold["pipe_bt"], gold["pipe_seq_lens"]
    R, H, _ = q.shape
    n_kv, G = gold["pipe_slab_mus"].shape[1], H // gold["pipe_slab_mus"].shape[1]
    say("score", R, n_kv, G, sl.tolist())
    st = _state(n_kv, G, gold["pipe_k"].shape[0], R, bt.shape[1], 8, "nrm")
    _load_slabs(st, gold)
    slt = torch.from_numpy(sl).cuda()
    derive_page_params(st, slt, R)
    rki4_score_only(st, 0, _bf(q), torch.from_numpy(bt).cuda(), slt, R, 1.0 / np.sqrt(128))
    torch.cuda.synchronize()
    got, ref = st.score_h.cpu().numpy(), gold["pipe_score_h"]
    for r in range(R):
        P = int(gold["pipe_nsh"][r])
        err = np.abs(got[r, ..., :P] - ref[r, ..., :P]).max()
        say(f"request {r}: {P} pages, max|gpu - golden| = {err:.3e}")
        assert err <= 2e-5


@pytest.mark.parametrize("combine", ["max", "nrm"])
@pytest.mark.parametrize("prefix", ["pipe_", "ties_"])
def test_golden_select(gold, prefix, combine):
    import torch
    from locks.selection import derive_page_params, rki4_select_only
    sh, sl = gold[prefix + "score_h"], gold[prefix + "seq_lens"]
    R, n_kv, G, MP = sh.shape
    bp = 8 if prefix == "pipe_" else 126
    say("select", prefix, combine, R, n_kv, G, MP, bp)
    st = _state(n_kv, G, 1, R, MP, bp, combine)
    derive_page_params(st, torch.from_numpy(sl).cuda(), R)
    _set_scores(st, sh, gold[prefix + "nsh"])
    st.page_table.fill_(7)
    rki4_select_only(st, R)
    _check_select(st, prefix, gold, combine, G)


def test_golden_mla(gold):
    """MLA path: derive + latent score + topb_middle, then the split decode
    and merge over the selection."""
    import torch
    from locks.attention import mla_decode
    from locks.selection import MlaState, mla_select_pages
    u16 = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    q, cache, bt, sl = gold["mla_q"], gold["mla_cache"], gold["mla_bt"], gold["mla_seq_lens"]
    R, H, _ = q.shape
    say("mla", R, H, sl.tolist())
    st = MlaState("cuda", num_layers=1, num_blocks=cache.shape[0], n_heads=H, max_reqs=R,
                  max_pages=bt.shape[1], budget_pages=14, sink_pages=1, window_pages=10, rope="exact")
    for k, name in (("v4", "pp_v4"), ("vs", "pp_vs"), ("c8", "pp_c8"), ("cs", "pp_cs"),
                    ("mu8", "pp_mu8"), ("mus", "pp_mus")):
        a = gold["mla_slab_" + k]
        t = getattr(st, name)[0]
        if a.dtype == np.uint16:
            t.copy_(torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(t.shape))
        else:
            t.copy_(torch.from_numpy(a.copy()).reshape(t.shape))
    dq, dc = u16(q), u16(cache)
    dbt, dsl = torch.from_numpy(bt).cuda(), torch.from_numpy(sl).cuda()
    mla_select_pages(st, 0, dq, dc, dbt, dsl, R, 0.07)
    torch.cuda.synchronize()
    ref = gold["mla_score"]
    got = st.score_h[:, 0, 0, :].cpu().numpy()
    for r in range(R):
        P = int(gold["mla_nsh"][r])
        err = np.abs(got[r, :P] - ref[r, :P]).max()
        say(f"score: {P} pages, max|gpu - golden| = {err:.3e}")
        assert err <= 2e-4 * max(1.0, np.abs(ref[r, :P]).max())
    assert np.array_equal(st.page_table[:, 0].cpu().numpy(), gold["mla_tab"])
    assert np.array_equal(st.page_cnt[:, 0].cpu().numpy(), gold["mla_cnt"])
    out = torch.empty(R, H, 512, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(R, H, dtype=torch.float32, device="cuda")
    mla_decode(st, dq, dc, dbt, dsl, R, 0.07, out, lse=lse)
    torch.cuda.synchronize()
    ro = O.bf16_round(gold["mla_out"].astype(np.float32)).astype(np.float64)
    go = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(go - ro)
    mr = err.sum() / np.abs(ro).sum()
    lerr = np.abs(lse.cpu().numpy() - gold["mla_lse"]).max()
    say(f"decode: max-abs {err.max():.3e} mean-rel {mr:.3e}; lse max-abs {lerr:.3e}")
    assert err.max() <= 2e-2 and mr <= 1e-3 and lerr <= 2e-3


def test_golden_decode(gold):
    import torch
    from locks.attention import decode_merge, decode_splitk
    from locks.attention.decode import _pps_min
    q, bt, sl = gold["pipe_q"], gold["pipe_bt"], gold["pipe_seq_lens"]
    R, H, D = q.shape
    n_kv = gold["pipe_slab_mus"].shape[1]
    G = H // n_kv
    say("decode", R, n_kv, G, sl.tolist())
    st = _state(n_kv, G, gold["pipe_k"].shape[0], R, bt.shape[1], 8, "max")
    st.page_table.copy_(torch.from_numpy(gold["pipe_tab_max"]))
    st.page_cnt.copy_(torch.from_numpy(gold["pipe_cnt_max"]))
    k, v = _bf(gold["pipe_k"]), _bf(gold["pipe_v"])
    ref = gold["pipe_out"]
    for dt in (torch.float32, torch.bfloat16):
        out = torch.full((R, H, D), float("nan"), dtype=dt, device="cuda")
        pps = _pps_min(R)
        decode_splitk(_bf(q), k, v, torch.from_numpy(bt).cuda(), torch.from_numpy(sl).cuda(),
                      st.page_table, st.page_cnt, st.m_part, st.l_part, st.acc_part, n_req=R, G=G,
                      split=st.split, pps_min=pps, scale=1.0 / np.sqrt(D), max_cnt=0)
        decode_merge(st.m_part, st.l_part, st.acc_part, st.page_cnt, out, n_req=R, n_kv=n_kv, G=G,
                     split=st.split, pps_min=pps, pt_cols=st.page_table.shape[2], max_cnt=0)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all()
        if dt == torch.float32:
            err = np.abs(got - ref).max()
            say(f"fp32 out: max|gpu - golden| = {err:.3e}")
            assert err <= 2e-3
        else:
            rb = O.bf16_round(ref.astype(np.float32)).astype(np.float64)
            err = np.abs(got - rb)
            mr = err.sum() / max(np.abs(rb).sum(), 1e-30)
            say(f"bf16 out: max-abs {err.max():.3e} mean-rel {mr:.3e}")
            assert err.max() <= 2e-2 and mr <= 1e-3
