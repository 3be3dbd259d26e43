"""GPU parity of the MLA path (config 5 shape: one latent head of 512 + 64
RoPE dims, 16 query heads, page 16) through the C ABI, against the numpy
MLA oracle (oracle/mla_oracle.py) on seeded inputs."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from oracle import mla_oracle as M

pytestmark = pytest.mark.gpu

LKV, DR, HS, PAGE = 512, 64, 576, 16


def say(*a):
    print("[mla]", *a, flush=True)


def _case(seed, seq_lens, H=16, extra=8):
    rng = np.random.default_rng(seed)
    npg = [(s + PAGE - 1) // PAGE for s in seq_lens]
    NB = sum(npg) + extra
    MP = max(npg)
    cache = M.synth_latent(rng, NB, PAGE, LKV, DR)
    bt = O.synth_block_table(rng, seq_lens, PAGE, NB, MP)
    q = O.f32_to_bf16(rng.standard_normal((len(seq_lens), H, HS)).astype(np.float32))
    return dict(cache=cache, bt=bt, q=q, sl=np.array(seq_lens, np.int32), NB=NB, MP=MP, H=H, R=len(seq_lens))


def _dev(c):
    import torch
    u16 = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    return dict(cache=u16(c["cache"]), q=u16(c["q"]), bt=torch.from_numpy(c["bt"]).cuda(),
                sl=torch.from_numpy(c["sl"]).cuda())


def _state(c, budget, L=1, window=10, sink=1, rope="exact"):
    from locks.selection import MlaState
    return MlaState("cuda", num_layers=L, num_blocks=c["NB"], n_heads=c["H"], max_reqs=c["R"],
                    max_pages=c["MP"], budget_pages=budget, sink_pages=sink, window_pages=window,
                    rope=rope)


def _copy(t, a):
    import torch
    if a.dtype == np.uint16:
        t.copy_(torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(t.shape))
    else:
        t.copy_(torch.from_numpy(a.copy()).reshape(t.shape))


def _upload_slabs(st, slabs, layer=0, rope=None):
    for k, name in (("v4", "pp_v4"), ("vs", "pp_vs"), ("c8", "pp_c8"), ("cs", "pp_cs"),
                    ("mu8", "pp_mu8"), ("mus", "pp_mus")):
        _copy(getattr(st, name)[layer], slabs[k])
    if st.rope == "int8":
        assert rope is not None, "an int8-RoPE state needs the oracle's RoPE summary"
        _copy(st.pp_rk8[layer], rope["rk8"])
        _copy(st.pp_rks[layer], rope["rks"])


def _oracle_summaries(c, st, layer=0):
    """Oracle latent slabs (+ int8 RoPE summary for an int8-RoPE state) of the
    case's full blocks, uploaded into st; returns (slabs, rope or None)."""
    blocks = _blocks_of(c)
    slabs = M.mla_build_summaries(c["cache"], blocks, c["NB"])
    rope = M.mla_build_rope(c["cache"], blocks, c["NB"]) if st.rope == "int8" else None
    _upload_slabs(st, slabs, layer, rope)
    return slabs, rope


def _blocks_of(c):
    out = []
    for r, s in enumerate(c["sl"]):
        out.extend(c["bt"][r, :int(s) // PAGE].tolist())
    return np.array(sorted(set(out)), np.int32)


@pytest.mark.parametrize("rope", ["int8", "exact"])
@pytest.mark.parametrize("seq_lens,H", [([16 * 40 + 5], 16), ([16 * 300, 16 * 77 + 9], 16), ([16 * 50 + 1], 5)])
def test_mla_score_matches_oracle(seq_lens, H, rope):
    import torch
    from locks.selection import mla_derive, mla_score_only
    say("score", seq_lens, H, rope)
    c = _case(11, seq_lens, H)
    d = _dev(c)
    st = _state(c, budget=32, rope=rope)
    slabs, rs = _oracle_summaries(c, st)
    mla_derive(st, d["sl"], c["R"])
    st.score_h.fill_(123.0)
    # the int8-RoPE scorer must not read the cache: hand it a cache whose
    # RoPE keys are garbage (the latent part is unused by the scorer too)
    cache_arg = d["cache"].clone().fill_(float("nan")) if rope == "int8" else d["cache"]
    mla_score_only(st, 0, d["q"], cache_arg, d["bt"], c["R"], 0.07)
    torch.cuda.synchronize()
    npg, nsh, b = M.mla_derive(c["sl"], PAGE, 10, 1, 32)
    ref = M.mla_score_rki4(c["q"], slabs, c["cache"], c["bt"], nsh, 0.07, c["MP"], rope=rs)
    got = st.score_h[:, 0, 0, :].cpu().numpy()
    for r in range(c["R"]):
        P = int(nsh[r])
        err = np.abs(got[r, :P] - ref[r, :P]).max()
        say(f"row {r}: {P} pages, max |d| {err:.2e}")
        assert err <= 2e-4 * max(1.0, np.abs(ref[r, :P]).max())
        assert np.all(got[r, P:] == 123.0)                       # never written past n_sel_hi


def test_mla_score_q_quantisation_ties():
    """q rows (latent and RoPE parts) whose q / qs quotients are exact
    half-integers (qs = 2^-4) must round to even like the reference's rint;
    rounding half away from zero would move the page scores ~50x past the
    tolerance (checked on the oracle).  Both quantisations are exercised:
    q_c, and q_rope of the int8-RoPE scorer."""
    import torch
    from locks.selection import mla_derive, mla_score_only
    say("score q ties")
    c = _case(13, [16 * 40 + 5], 16)
    rng = np.random.default_rng(14)
    k = rng.integers(-120, 120, size=(1, 16, HS))
    q = O.bf16_to_f32(c["q"]).copy()
    q_tie = (k + 0.5) / 16.0
    q_tie[:, :, 0] = q_tie[:, :, LKV] = 127.0 / 16.0         # row maxima -> qs = 2^-4
    c["q"] = O.f32_to_bf16(q_tie.astype(np.float32))
    assert np.array_equal(O.bf16_to_f32(c["q"]), q_tie.astype(np.float32))
    d = _dev(c)
    st = _state(c, budget=32, rope="int8")
    slabs, rs = _oracle_summaries(c, st)
    mla_derive(st, d["sl"], c["R"])
    mla_score_only(st, 0, d["q"], d["cache"], d["bt"], c["R"], 0.07)
    torch.cuda.synchronize()
    npg, nsh, b = M.mla_derive(c["sl"], PAGE, 10, 1, 32)
    P = int(nsh[0])
    ref = M.mla_score_rki4(c["q"], slabs, c["cache"], c["bt"], nsh, 0.07, c["MP"], rope=rs)[0, :P]
    tol = 2e-4 * max(1.0, np.abs(ref).max())
    for part in (slice(1, LKV), slice(LKV + 1, HS)):          # half away from zero, one part at a time
        q_away = q_tie.copy()
        q_away[:, :, part] = np.where(k[:, :, part] >= 0, k[:, :, part] + 1, k[:, :, part]) / 16.0
        away = M.mla_score_rki4(O.f32_to_bf16(q_away.astype(np.float32)), slabs, c["cache"], c["bt"],
                                nsh, 0.07, c["MP"], rope=rs)[0, :P]
        assert np.abs(away - ref).max() > 10 * tol, part
    got = st.score_h[0, 0, 0, :P].cpu().numpy()
    assert np.abs(got - ref).max() <= tol


def test_mla_build_matches_oracle_through_the_score():
    """Eigenvectors agree only up to sign/rotation, so the GPU-built latent
    summary is compared through the oracle score it produces."""
    import torch
    from locks.selection import mla_build_blocks
    say("build")
    c = _case(12, [16 * 64 + 3])
    d = _dev(c)
    st = _state(c, budget=32, rope="int8")
    blocks = _blocks_of(c)
    mla_build_blocks(st, 0, d["cache"], torch.from_numpy(blocks).cuda())
    torch.cuda.synchronize()
    gpu = dict(v4=st.pp_v4[0].cpu().numpy(), vs=st.pp_vs[0].view(torch.int16).cpu().numpy().view(np.uint16),
               c8=st.pp_c8[0].cpu().numpy(), cs=st.pp_cs[0].view(torch.int16).cpu().numpy().view(np.uint16),
               mu8=st.pp_mu8[0].cpu().numpy(), mus=st.pp_mus[0].view(torch.int16).cpu().numpy().view(np.uint16))
    ref = M.mla_build_summaries(c["cache"], blocks, c["NB"])
    rope = M.mla_build_rope(c["cache"], blocks, c["NB"])                   # int8 RoPE summary: bit-exact
    assert np.array_equal(st.pp_rk8[0].cpu().numpy(), rope["rk8"])
    assert np.array_equal(st.pp_rks[0].view(torch.int16).cpu().numpy().view(np.uint16), rope["rks"])
    assert np.array_equal(gpu["mu8"][blocks], ref["mu8"][blocks])          # mean path is exact
    assert np.array_equal(gpu["mus"][blocks], ref["mus"][blocks])
    npg, nsh, b = M.mla_derive(c["sl"], PAGE, 10, 1, 32)
    s_gpu = M.mla_score_rki4(c["q"], gpu, c["cache"], c["bt"], nsh, 0.07, c["MP"])[0, :int(nsh[0])]
    s_ref = M.mla_score_rki4(c["q"], ref, c["cache"], c["bt"], nsh, 0.07, c["MP"])[0, :int(nsh[0])]
    rel = np.abs(s_gpu - s_ref).max() / np.abs(s_ref).max()
    say(f"score from GPU vs oracle build: max rel {rel:.2e}")
    assert rel <= 5e-3


@pytest.mark.parametrize("seq_lens,budget", [([16 * 200 + 7], 32), ([16 * 100, 16 * 20 + 3, 16 * 9], 24),
                                             ([16 * 8192], 128)])
def test_mla_select_matches_topb_middle(seq_lens, budget):
    import torch
    from locks.selection import mla_select_pages
    say("select", seq_lens, budget)
    c = _case(13, seq_lens)
    d = _dev(c)
    st = _state(c, budget=budget)
    _oracle_summaries(c, st)
    mla_select_pages(st, 0, d["q"], d["cache"], d["bt"], d["sl"], c["R"], 0.07)
    torch.cuda.synchronize()
    tab, cnt = st.page_table[:, 0].cpu().numpy(), st.page_cnt[:, 0].cpu().numpy()
    gsc = st.score_h[:, 0, 0, :].cpu().numpy()
    for r in range(c["R"]):
        P = (int(c["sl"][r]) + PAGE - 1) // PAGE
        ps = np.full(P, -np.inf, np.float32)
        nfull = int(c["sl"][r]) // PAGE
        n_sc = max(min(nfull, P - 10), 0)
        ps[:n_sc] = gsc[r, :n_sc]
        keep = M.topb_middle(ps, budget, 1, 10)                  # reference rule on GPU scores
        assert np.array_equal(np.nonzero(keep)[0], tab[r, :cnt[r]]), f"row {r}"
        assert (tab[r, cnt[r]:] == -1).all()
        assert cnt[r] == min(P, budget)


@pytest.mark.parametrize("seq_lens,budget,H,rope", [([16 * 60 + 5], 24, 16, "exact"),
                                                    ([16 * 30, 16 * 7 + 2], 16, 16, "exact"),
                                                    ([16 * 2048], 128, 16, "exact"),
                                                    ([16 * 2048], 128, 16, "int8"),
                                                    ([16 * 90 + 3, 16 * 33], 20, 5, "int8"),
                                                    ([16 * 64], 32, 1, "exact")])
def test_mla_decode_matches_oracle(seq_lens, budget, H, rope):
    import torch
    from locks.backend.mla_attn import mla_forward_mqa
    say("decode", seq_lens, budget, H, rope)
    c = _case(14, seq_lens, H)
    d = _dev(c)
    st = _state(c, budget=budget, rope=rope)
    _oracle_summaries(c, st)
    out = torch.empty(c["R"], c["H"], LKV, dtype=torch.bfloat16, device="cuda")
    o, lse = mla_forward_mqa(d["q"], d["cache"], d["bt"], d["sl"], st, 0.07, out=out, layer=0)
    torch.cuda.synchronize()
    tab, cnt = st.page_table[:, 0].cpu().numpy(), st.page_cnt[:, 0].cpu().numpy()
    ref_o, ref_lse = M.mla_attention(c["q"], c["cache"], c["bt"], c["sl"], tab, cnt, 0.07)
    got = o.float().cpu().numpy()
    ref_b = O.bf16_round(ref_o.astype(np.float32))
    err = np.abs(got - ref_b)
    mr = err.sum() / np.abs(ref_b).sum()
    lerr = np.abs(lse.cpu().numpy() - ref_lse).max()
    say(f"o max-abs {err.max():.2e} mean-rel {mr:.2e}; lse max-abs {lerr:.2e}")
    assert err.max() <= 2e-2 and mr <= 1e-3 and lerr <= 2e-3


def test_mla_dense_equality():
    """Budget >= page count keeps every page: the sparse decode equals dense
    attention over the whole sequence."""
    import torch
    from locks.backend.mla_attn import mla_forward_mqa
    c = _case(15, [16 * 37 + 11])
    d = _dev(c)
    st = _state(c, budget=10_000)
    out = torch.empty(1, c["H"], LKV, dtype=torch.float32, device="cuda")
    o, lse = mla_forward_mqa(d["q"], d["cache"], d["bt"], d["sl"], st, 0.07, out=out, layer=0)
    torch.cuda.synchronize()
    P = (int(c["sl"][0]) + 15) // 16
    assert int(st.page_cnt[0, 0]) == P
    ref_o, ref_lse = M.mla_attention(c["q"], c["cache"], c["bt"], c["sl"],
                                     np.arange(P, dtype=np.int32)[None], np.array([P]), 0.07)
    assert np.abs(o.cpu().numpy() - ref_o).max() <= 2e-3
    assert np.abs(lse.cpu().numpy() - ref_lse).max() <= 1e-3


@pytest.mark.parametrize("seq_lens,split", [([16 * 37 + 11], 512), ([16 * 37 + 11], 3),
                                            ([9000, 1, 16 * 200, 333], 64), ([40000], 128)])
def test_mla_dense_comparator_matches_oracle(seq_lens, split):
    """locks_mla_decode_dense (every page of every row, three stages in
    flight, non-temporal DMA) equals the oracle's attention over all pages:
    ragged rows, a one-token row, more splits than pages, fewer."""
    import torch
    from locks.attention import mla_decode_dense
    say("mla dense comparator", seq_lens, split)
    c = _case(16, seq_lens)
    d = _dev(c)
    R = c["R"]
    mp = torch.empty(R, split, 16, device="cuda")
    lp = torch.empty_like(mp)
    ap = torch.empty(R, split, 16, LKV, device="cuda")
    for dt in (torch.float32, torch.bfloat16):
        out = torch.full((R, c["H"], LKV), float("nan"), dtype=dt, device="cuda")
        lse = torch.full((R, c["H"]), float("nan"), device="cuda")
        mla_decode_dense(d["q"], d["cache"], d["bt"], d["sl"], mp, lp, ap, out, n_req=R,
                         split=split, scale=0.07, num_blocks=c["NB"], lse=lse)
        torch.cuda.synchronize()
        P = [(s + 15) // 16 for s in seq_lens]
        tab = np.zeros((R, max(P)), np.int32)
        for r, n in enumerate(P):
            tab[r, :n] = np.arange(n)
        ref_o, ref_lse = M.mla_attention(c["q"], c["cache"], c["bt"], c["sl"], tab,
                                         np.array(P, np.int32), 0.07)
        got = out.float().cpu().numpy()
        if dt == torch.float32:
            err = np.abs(got - ref_o).max()
            say(f"fp32 max-abs {err:.2e}")
            assert err <= 2e-3
        else:
            rb = O.bf16_round(ref_o.astype(np.float32))
            e = np.abs(got - rb)
            assert e.max() <= 2e-2 and e.sum() / np.abs(rb).sum() <= 1e-3
        assert np.abs(lse.cpu().numpy() - ref_lse).max() <= 1e-3
