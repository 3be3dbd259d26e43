"""GPU parity at the reference's other geometries: head_dim 64 / 128 / 256
and page 16 / 32 / 64 (rki4_state.py:295-324), against the CPU oracle.

The oracle is shape-generic (its functions read page and head_dim from the
arrays); the bars are the north-star ones: bf16 attention output within
max-abs 2e-2 and mean-rel 1e-3 of the fp32 oracle, fp32 within 2e-3.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from tests.cases import make_case, to_dev

pytestmark = pytest.mark.gpu

GEOMS = [(64, 16), (256, 16), (128, 32), (128, 64), (64, 32), (256, 64)]


def say(*a):
    print("[case]", *a, flush=True)


def _tables(case, seed, budget_pages=40):
    """A top-b page table from random scores (sink + window kept)."""
    rng = np.random.default_rng(seed)
    npg, nsh, b = O.derive_page_params(case.seq_lens, case.page, 1, 1, budget_pages, 0.1)
    sc = rng.random((case.R, case.n_kv, case.MP)).astype(np.float32)
    return O.topb_select(sc, npg, nsh, b, 1, case.MP)


def _check(case, out, tab, cnt):
    import torch
    got = out.float().cpu().numpy()
    ref, _ = O.decode_attention(case.q, case.k, case.v, case.bt, case.seq_lens, tab, cnt,
                                case.G, case.scale)
    if out.dtype == torch.bfloat16:
        rb = O.bf16_round(ref.astype(np.float32))
        e = np.abs(got - rb)
        mr = e.sum() / max(np.abs(rb).sum(), 1e-30)
        say(f"bf16 out: max-abs {e.max():.3e} mean-rel {mr:.3e}")
        assert e.max() <= 2e-2 and mr <= 1e-3
    else:
        e = np.abs(got - ref)
        say(f"fp32 out: max-abs {e.max():.3e}")
        assert e.max() <= 2e-3
    assert np.isfinite(got).all()


@pytest.mark.parametrize("hd,page", GEOMS)
@pytest.mark.parametrize("n_kv,G,seq_lens,split", [
    (2, 4, [5000], 16), (2, 8, [3001, 40, 1, 777], 8)])
def test_decode_geometry(hd, page, n_kv, G, seq_lens, split):
    """Split + merge and the fused launch at each geometry; ragged rows
    (partial last page, one-token and one-page rows)."""
    import torch
    from locks.attention import decode_merge, decode_splitk
    from locks.attention.decode import decode_fused
    from locks.attention.decode import _split_kv
    say("decode geometry", hd, page, n_kv, G, seq_lens, split)
    MP = max(1, max((s + page - 1) // page for s in seq_lens))
    case = make_case(21, n_kv, G, seq_lens, MP=MP, build=False, page=page, d=hd)
    tab, cnt = _tables(case, 22)
    d = to_dev(case)
    k, v = _split_kv(d["kv"])
    R = case.R
    ptab = torch.from_numpy(tab).cuda()
    pcnt = torch.from_numpy(cnt).cuda()
    mp = torch.empty(R, n_kv, split, G, device="cuda")
    lp = torch.empty_like(mp)
    ap = torch.empty(R, n_kv, split, G, hd, device="cuda")
    ctr = torch.zeros(R, n_kv, 64, dtype=torch.int32, device="cuda")
    for dt in (torch.bfloat16, torch.float32):
        out = torch.full((R, n_kv * G, hd), float("nan"), dtype=dt, device="cuda")
        decode_splitk(d["q"], k, v, d["bt"], d["sl"], ptab, pcnt, mp, lp, ap, n_req=R, G=G,
                      split=split, pps_min=1, scale=case.scale)
        decode_merge(mp, lp, ap, pcnt, out, n_req=R, n_kv=n_kv, G=G, split=split, pps_min=1,
                     pt_cols=MP)
        torch.cuda.synchronize()
        _check(case, out, tab, cnt)
        out2 = torch.full_like(out, float("nan"))
        decode_fused(d["q"], k, v, d["bt"], d["sl"], ptab, pcnt, mp, lp, ap, ctr, out2, n_req=R,
                     G=G, split=split, pps_min=1, scale=case.scale)
        torch.cuda.synchronize()
        _check(case, out2, tab, cnt)


@pytest.mark.parametrize("hd,page", GEOMS)
def test_dense_geometry(hd, page):
    """The dense comparator (every page of every row) equals the oracle's
    attention over a page table holding all of the row's pages."""
    import torch
    from locks.attention import decode_dense
    from locks.attention.decode import _split_kv
    n_kv, G, seq_lens, split = 2, 4, [3000, 17, 1200], 8
    say("dense geometry", hd, page)
    MP = max((s + page - 1) // page for s in seq_lens)
    case = make_case(23, n_kv, G, seq_lens, MP=MP, build=False, page=page, d=hd)
    R = case.R
    tab = np.zeros((R, n_kv, MP), np.int32)
    cnt = np.zeros((R, n_kv), np.int32)
    for r, s in enumerate(seq_lens):
        n = (s + page - 1) // page
        tab[r, :, :n] = np.arange(n)
        cnt[r, :] = n
    d = to_dev(case)
    k, v = _split_kv(d["kv"])
    mp = torch.empty(R, n_kv, split, G, device="cuda")
    lp = torch.empty_like(mp)
    ap = torch.empty(R, n_kv, split, G, hd, device="cuda")
    out = torch.full((R, n_kv * G, hd), float("nan"), dtype=torch.float32, device="cuda")
    decode_dense(d["q"], k, v, d["bt"], d["sl"], mp, lp, ap, out, n_req=R, G=G, split=split,
                 scale=case.scale)
    torch.cuda.synchronize()
    _check(case, out, tab, cnt)
