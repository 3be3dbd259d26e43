"""Write tests/golden/locks_golden.npz: seeded inputs of the decode hot path at
small shapes together with the CPU oracle's outputs for them.

The reference ships no tests, fixtures or golden vectors, so these are this
build's own: the oracle functions that produce them are pinned by closed
forms, invariants and brute force (tests/test_oracle_pins.py).  The file
anchors two things:
  * the oracle itself, against drift (tests/test_golden.py recomputes every
    output from the stored inputs on the CPU);
  * the HIP kernels, which tests/test_gpu_golden.py runs on the stored
    inputs and compares with the stored outputs directly.

Cases (page 16; head_dim 128 for the GQA cases):
  pipe   2 ragged requests (21 and 9 pages), 2 kv heads x 4 query heads:
         K/V cache, block table, q, the summary slabs built by the oracle
         builder, score_h, both combines' scores and page tables at a
         budget of 8 pages, and the decode output over the "max" table.
  ties   one 3000-page row, 2 kv heads x 8 query heads, score_h quantized
         to steps of 1/8 (many equal combined scores, so the exact-b tie
         rule decides), budget 126: combined scores and page tables.
  derive seq_len / budget edge cases -> (n_pages, n_sel_hi, b).
  mla    one 24-page request of the DeepSeek-V2-Lite latent cache (512 +
         64 dims, 16 query heads): cache, block table, q, the oracle's
         latent slabs, page scores (exact RoPE keys), the topb_middle keep
         set at a budget of 14 (sink 1, window 10: 3 of 13 middle pages;
         the generator checks a clear score gap at the boundary) and the
         attention output and LSE over it in float64.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import locks_oracle as O          # noqa: E402
from oracle import mla_oracle as M            # noqa: E402
from tests.cases import make_case             # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "locks_golden.npz")
SLAB_KEYS = ("v4", "vs", "c8", "cs", "mu8", "mus")

PIPE = dict(seed=11, n_kv=2, G=4, seq_lens=[20 * 16 + 5, 9 * 16], budget_pages=8, sink=1, window=1)
TIES = dict(seed=12, n_kv=2, G=8, seq_lens=[3000 * 16], budget_pages=126, sink=1, window=1)
MLA = dict(seed=21, seq_lens=[23 * 16 + 5], H=16, budget_pages=14, sink=1, window=10, scale=0.07,
           extra_blocks=2)
DERIVE = [  # (seq_len, budget_abs, budget)
    (0, 126, 0.1), (1, 126, 0.1), (15, 126, 0.1), (16, 126, 0.1), (17, 126, 0.1),
    (32, 126, 0.1), (33, 126, 0.1), (48, 126, 0.1), (2048, 126, 0.1), (2049, 126, 0.1),
    (131072, 126, 0.1), (1 << 20, 126, 0.1), (1 << 20, 0, 0.1), (131072, 0, 0.1),
    (16 * 31, 0, 0.1), (16 * 32, 0, 0.1), (16 * 33 + 1, 0, 0.1), (100000, 0, 0.3),
    (100000, 0, 1.0), (5, 0, 0.1), (40, 0, 0.5), (1000, 5, 0.1), (1000, 100000, 0.1),
]


def pipe_outputs(q, k, v, bt, slabs, seq_lens, n_kv, G, MP, budget_pages, sink, window):
    """Every oracle output of the pipe case from its inputs."""
    scale = 1.0 / np.sqrt(q.shape[-1])
    npg, nsh, b = O.derive_page_params(seq_lens, 16, window, sink, budget_pages, 0.1)
    score_h = O.score_rki4_twin(q, slabs, bt, nsh, n_kv, G, scale, MP)
    comb_nrm = O.combine_nrm(score_h, nsh)
    tab_nrm, cnt_nrm = O.topb_select(comb_nrm, npg, nsh, b, sink, MP)
    comb_max = O.combine_max(score_h, nsh)
    tab_max, cnt_max = O.topb_select(comb_max, npg, nsh, b, sink, MP)
    out, lse = O.decode_attention(q, k, v, bt, seq_lens, tab_max, cnt_max, G, scale,
                                  dtype=np.float64)
    return dict(npg=npg, nsh=nsh, b=b, score_h=score_h, comb_nrm=comb_nrm, tab_nrm=tab_nrm,
                cnt_nrm=cnt_nrm, comb_max=comb_max, tab_max=tab_max, cnt_max=cnt_max,
                out=out, lse=lse)


def ties_outputs(score_h, seq_lens, MP, budget_pages, sink, window):
    npg, nsh, b = O.derive_page_params(seq_lens, 16, window, sink, budget_pages, 0.1)
    comb_nrm = O.combine_nrm(score_h, nsh)
    tab_nrm, cnt_nrm = O.topb_select(comb_nrm, npg, nsh, b, sink, MP)
    comb_max = O.combine_max(score_h, nsh)
    tab_max, cnt_max = O.topb_select(comb_max, npg, nsh, b, sink, MP)
    return dict(npg=npg, nsh=nsh, b=b, comb_nrm=comb_nrm, tab_nrm=tab_nrm, cnt_nrm=cnt_nrm,
                comb_max=comb_max, tab_max=tab_max, cnt_max=cnt_max)


def mla_outputs(q, cache, bt, slabs, seq_lens, budget_pages, sink, window, scale):
    """Page scores, the topb_middle keep set and attention over it."""
    R, MP = bt.shape
    npg, nsh, b = M.mla_derive(seq_lens, 16, window, sink, budget_pages)
    score = M.mla_score_rki4(q, slabs, cache, bt, nsh, scale, MP)
    tab = np.full((R, MP), -1, np.int32)
    cnt = np.zeros(R, np.int32)
    for r in range(R):
        P = int(npg[r])
        ps = np.full(P, -np.inf, np.float32)
        n_sc = max(min(int(seq_lens[r]) // 16, P - window), 0)
        ps[:n_sc] = score[r, :n_sc]
        kept = np.nonzero(M.topb_middle(ps, budget_pages, sink, window))[0]
        tab[r, :kept.size] = kept
        cnt[r] = kept.size
    out, lse = M.mla_attention(q, cache, bt, seq_lens, tab, cnt, scale)
    return dict(npg=npg, nsh=nsh, b=b, score=score, tab=tab, cnt=cnt, out=out, lse=lse)


def mla_inputs():
    m = MLA
    rng = np.random.default_rng(m["seed"])
    npg = [(s + 15) // 16 for s in m["seq_lens"]]
    NB = sum(npg) + m["extra_blocks"]
    cache = M.synth_latent(rng, NB, 16, 512, 64)
    bt = O.synth_block_table(rng, m["seq_lens"], 16, NB, max(npg))
    q = O.f32_to_bf16(rng.standard_normal((len(m["seq_lens"]), m["H"], 576)).astype(np.float32))
    full = sorted({int(bt[r, j]) for r, s in enumerate(m["seq_lens"]) for j in range(s // 16)})
    slabs = M.mla_build_summaries(cache, np.array(full, np.int32), NB)
    return q, cache, bt, slabs


def derive_outputs(rows):
    res = []
    for sl, babs, bud in rows:
        npg, nsh, b = O.derive_page_params([sl], 16, 1, 1, babs, bud)
        res.append((int(npg[0]), int(nsh[0]), int(b[0])))
    return np.array(res, np.int32)


def ties_score_h(seed, n_kv, G, MP, P):
    """score_h in steps of 1/8 (equal combined scores are common); pages
    past P are never read by the selector and stay 0."""
    rng = np.random.default_rng(seed)
    sh = np.zeros((1, n_kv, G, MP), np.float32)
    sh[..., :P] = np.round(rng.standard_normal((1, n_kv, G, P)) * 8.0) / 8.0
    return sh


def main():
    p = PIPE
    case = make_case(p["seed"], p["n_kv"], p["G"], p["seq_lens"], build=True)
    arrs = {"pipe_q": case.q, "pipe_k": case.k, "pipe_v": case.v, "pipe_bt": case.bt,
            "pipe_seq_lens": np.array(case.seq_lens, np.int32)}
    for k in SLAB_KEYS:
        arrs["pipe_slab_" + k] = case.slabs[k]
    for k, val in pipe_outputs(case.q, case.k, case.v, case.bt, case.slabs, case.seq_lens,
                               p["n_kv"], p["G"], case.MP, p["budget_pages"], p["sink"],
                               p["window"]).items():
        arrs["pipe_" + k] = val

    t = TIES
    MP = (t["seq_lens"][0] + 15) // 16
    _, nsh, _ = O.derive_page_params(t["seq_lens"], 16, t["window"], t["sink"], t["budget_pages"], 0.1)
    sh = ties_score_h(t["seed"], t["n_kv"], t["G"], MP, int(nsh[0]))
    arrs["ties_score_h"] = sh
    arrs["ties_seq_lens"] = np.array(t["seq_lens"], np.int32)
    for k, val in ties_outputs(sh, t["seq_lens"], MP, t["budget_pages"], t["sink"], t["window"]).items():
        arrs["ties_" + k] = val

    m = MLA
    q, cache, bt, slabs = mla_inputs()
    arrs.update(mla_q=q, mla_cache=cache, mla_bt=bt, mla_seq_lens=np.array(m["seq_lens"], np.int32))
    for k in SLAB_KEYS:
        arrs["mla_slab_" + k] = slabs[k]
    mo = mla_outputs(q, cache, bt, slabs, m["seq_lens"], m["budget_pages"], m["sink"], m["window"],
                     m["scale"])
    # the keep set must not hinge on the scorer's tolerance: a clear gap
    # between the last kept and the first dropped middle page
    P = int(mo["npg"][0])
    mid = [p for p in range(m["sink"], P - m["window"])]
    kept = set(mo["tab"][0, :mo["cnt"][0]].tolist())
    sk = min(mo["score"][0, p] for p in mid if p in kept)
    sd = max(mo["score"][0, p] for p in mid if p not in kept)
    assert sk - sd > 1e-3 * np.abs(mo["score"][0, :P]).max(), (sk, sd)
    for k, val in mo.items():
        arrs["mla_" + k] = val

    arrs["derive_in"] = np.array([(sl, babs) for sl, babs, _ in DERIVE], np.int64)
    arrs["derive_budget"] = np.array([bud for _, _, bud in DERIVE], np.float64)
    arrs["derive_out"] = derive_outputs(DERIVE)
    np.savez_compressed(OUT, **arrs)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(arrs)} arrays")


if __name__ == "__main__":
    main()
