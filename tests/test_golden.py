"""The committed golden fixture (tests/golden/locks_golden.npz, written by
tests/golden/make_golden.py) against the CPU oracle: every stored output is
recomputed from the stored inputs, so a change to the oracle that moves any
of them fails here.  Integer outputs (page tables, counts, derived
parameters) must match exactly; floating outputs to 1e-6 relative (the
same numpy code; only BLAS summation order may differ between machines)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import locks_oracle as O
from oracle import mla_oracle as M
from tests.golden import make_golden as MG

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "locks_golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(PATH, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _close(a, b, rtol=1e-6, atol=1e-7):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape
    same_inf = np.isinf(a) & np.isinf(b) & (np.sign(a) == np.sign(b))
    fin = ~same_inf
    assert np.isfinite(a[fin]).all() and np.isfinite(b[fin]).all()
    assert np.allclose(a[fin], b[fin], rtol=rtol, atol=atol)


def test_pipe_case(gold):
    p = MG.PIPE
    slabs = {k: gold["pipe_slab_" + k] for k in MG.SLAB_KEYS}
    MP = gold["pipe_bt"].shape[1]
    got = MG.pipe_outputs(gold["pipe_q"], gold["pipe_k"], gold["pipe_v"], gold["pipe_bt"], slabs,
                          gold["pipe_seq_lens"].tolist(), p["n_kv"], p["G"], MP,
                          p["budget_pages"], p["sink"], p["window"])
    for k in ("npg", "nsh", "b", "tab_nrm", "cnt_nrm", "tab_max", "cnt_max"):
        assert np.array_equal(got[k], gold["pipe_" + k]), k
    for k in ("score_h", "comb_nrm", "comb_max", "out", "lse"):
        _close(got[k], gold["pipe_" + k])
    # the case exercises what it is meant to: a selection below the row
    # length on the longer request, keep-all on the shorter one
    assert int(gold["pipe_b"][0]) < int(gold["pipe_nsh"][0]) - p["sink"]
    assert int(gold["pipe_b"][1]) == int(gold["pipe_nsh"][1]) - p["sink"]


def test_pipe_slabs_are_the_builders(gold):
    """The stored slabs are what the oracle builder makes of the stored K
    (the build itself goes through LAPACK's eigh, so codes are compared with
    the same boundary allowance as the GPU build tests: identical except for
    a few rounding-boundary flips of one code step)."""
    p = MG.PIPE
    bt, sl = gold["pipe_bt"], gold["pipe_seq_lens"]
    fin = sorted({int(bt[r, j]) for r in range(len(sl)) for j in range(int(sl[r]) // 16)})
    slabs = O.build_state_slabs(gold["pipe_k"], np.array(fin, np.int64), gold["pipe_k"].shape[0])
    for k in ("mu8", "mus"):
        assert np.array_equal(slabs[k][fin], gold["pipe_slab_" + k][fin]), k
    for k in ("c8", "v4"):
        a, b = slabs[k][fin], gold["pipe_slab_" + k][fin]
        if k == "v4":
            a, b = O.unpack_i4(a), O.unpack_i4(b)
        d = np.abs(a.astype(np.int32) - b.astype(np.int32))
        assert d.max() <= 1 and (d > 0).mean() < 0.01, k


def test_ties_case(gold):
    t = MG.TIES
    MP = gold["ties_score_h"].shape[-1]
    got = MG.ties_outputs(gold["ties_score_h"], gold["ties_seq_lens"].tolist(), MP,
                          t["budget_pages"], t["sink"], t["window"])
    for k in ("npg", "nsh", "b", "tab_nrm", "cnt_nrm", "tab_max", "cnt_max"):
        assert np.array_equal(got[k], gold["ties_" + k]), k
    for k in ("comb_nrm", "comb_max"):
        _close(got[k], gold["ties_" + k])
    # the tie rule decides: the b-th largest combined score is shared by
    # kept and dropped pages of the same row
    nsh, b, sink = int(gold["ties_nsh"][0]), int(gold["ties_b"][0]), t["sink"]
    for kh in range(t["n_kv"]):
        sel = gold["ties_comb_max"][0, kh, sink:nsh]
        tau = np.sort(sel)[::-1][b - 1]
        assert (sel == tau).sum() > (np.sort(sel)[::-1][:b] == tau).sum()


def test_mla_case(gold):
    m = MG.MLA
    slabs = {k: gold["mla_slab_" + k] for k in MG.SLAB_KEYS}
    got = MG.mla_outputs(gold["mla_q"], gold["mla_cache"], gold["mla_bt"], slabs,
                         gold["mla_seq_lens"].tolist(), m["budget_pages"], m["sink"], m["window"],
                         m["scale"])
    for k in ("npg", "nsh", "b", "tab", "cnt"):
        assert np.array_equal(got[k], gold["mla_" + k]), k
    for k in ("score", "out", "lse"):
        _close(got[k], gold["mla_" + k])
    # a real selection: fewer pages kept than the row has
    assert int(gold["mla_cnt"][0]) == m["budget_pages"] < int(gold["mla_npg"][0])


def test_mla_slabs_are_the_builders(gold):
    bt, sl = gold["mla_bt"], gold["mla_seq_lens"]
    fin = sorted({int(bt[r, j]) for r in range(len(sl)) for j in range(int(sl[r]) // 16)})
    slabs = M.mla_build_summaries(gold["mla_cache"], np.array(fin, np.int32), gold["mla_cache"].shape[0])
    for k in ("mu8", "mus"):
        assert np.array_equal(slabs[k][fin], gold["mla_slab_" + k][fin]), k
    for k in ("c8", "v4"):
        a, b = slabs[k][fin], gold["mla_slab_" + k][fin]
        if k == "v4":
            a, b = O.unpack_i4(a), O.unpack_i4(b)
        d = np.abs(a.astype(np.int32) - b.astype(np.int32))
        assert d.max() <= 1 and (d > 0).mean() < 0.01, k


def test_derive_table(gold):
    rows = [(int(sl), int(babs), float(bud)) for (sl, babs), bud in
            zip(gold["derive_in"], gold["derive_budget"])]
    assert np.array_equal(MG.derive_outputs(rows), gold["derive_out"])
