"""Pins of the MLA oracle (no GPU): every function is checked against an
independent formulation -- float64 SVD, brute-force loops, closed forms."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from oracle import mla_oracle as M


def _blk(rng, n, page=16, Lkv=64, rank=None):
    x = rng.standard_normal((n, page, Lkv)).astype(np.float32)
    if rank is not None:                      # exactly rank-`rank` pages
        a = rng.standard_normal((n, page, rank)).astype(np.float32)
        b = rng.standard_normal((n, rank, Lkv)).astype(np.float32)
        x = np.einsum("ntr,nrd->ntd", a, b).astype(np.float32)
    return x


# ---- factors (mla_select.py:26-108) -------------------------------------
def test_factor_product_is_truncated_svd():
    rng = np.random.default_rng(0)
    blk = _blk(rng, 6, Lkv=96)
    Lf, Rf = M.mla_factor_build(blk, rank=8)
    C8 = np.einsum("ntr,nrd->ntd", Lf, Rf)
    for i in range(blk.shape[0]):
        U, s, Vt = np.linalg.svd(blk[i].astype(np.float64), full_matrices=False)
        ref = (U[:, :8] * s[:8]) @ Vt[:8]
        assert np.abs(C8[i] - ref).max() <= 2e-4 * np.abs(ref).max()
    assert np.all(Lf[:, :, 8:] == 0) and np.all(Rf[:, 8:, :] == 0)      # rpad zeros


def test_factor_drops_null_modes_without_nan():
    rng = np.random.default_rng(1)
    blk = _blk(rng, 3, Lkv=64, rank=3)                 # rank 3 < r = 8
    Lf, Rf = M.mla_factor_build(blk, rank=8)
    assert np.isfinite(Lf).all() and np.isfinite(Rf).all()
    C8 = np.einsum("ntr,nrd->ntd", Lf, Rf)
    assert np.abs(C8 - blk).max() <= 1e-3 * np.abs(blk).max()          # exact rank-3 page
    assert np.count_nonzero(np.abs(Rf).sum(axis=-1) > 0, axis=-1).max() <= 3
    z = np.zeros((1, 16, 32), np.float32)                                # all-zero page
    Lz, Rz = M.mla_factor_build(z, rank=8)
    assert np.all(Lz == 0) and np.all(Rz == 0)


# ---- page score (mla_score_torch.py:27-48) -----------------------------
def test_page_score_brute_force():
    rng = np.random.default_rng(2)
    H, D, Dr, P, page = 3, 8, 4, 5, 4
    qc = rng.standard_normal((H, D)).astype(np.float32)
    qr = rng.standard_normal((H, Dr)).astype(np.float32)
    C8 = rng.standard_normal((P, page, D)).astype(np.float32)
    kr = rng.standard_normal((P, page, Dr)).astype(np.float32)
    valid = np.array([4, 1, 3, 4, 2])
    got = M.mla_page_score_ref(qc, qr, C8, kr, valid, 0.7)
    for p in range(P):
        best = -np.inf
        for h in range(H):
            for t in range(valid[p]):
                v = (sum(float(qc[h, d]) * float(C8[p, t, d]) for d in range(D))
                     + sum(float(qr[h, d]) * float(kr[p, t, d]) for d in range(Dr))) * 0.7
                best = max(best, v)
        assert abs(got[p] - best) <= 1e-5 * max(1.0, abs(best))


# ---- topb_middle (mla_score_torch.py:51-73) ----------------------------
@pytest.mark.parametrize("P,budget,sink,recent", [(12, 5, 1, 2), (12, 12, 1, 2), (7, 3, 1, 10),
                                                  (20, 8, 2, 3), (9, 4, 0, 1)])
def test_topb_middle_brute_force(P, budget, sink, recent):
    rng = np.random.default_rng(P * 7 + budget)
    for trial in range(20):
        ps = rng.integers(0, 4, P).astype(np.float32)          # tie-heavy
        keep = M.topb_middle(ps, budget, sink, recent)
        if P <= budget:
            assert keep.all()
            continue
        forced = set(range(min(sink, P))) | set(range(max(0, P - recent), P))
        assert all(keep[p] for p in forced)
        mid = [p for p in range(P) if p not in forced]
        n_mid = max(budget - len(forced), 0)
        want = sorted(mid, key=lambda p: (-ps[p], p))[:n_mid]
        assert set(np.nonzero(keep)[0].tolist()) == forced | set(want)


def test_topb_middle_equals_gqa_selector_with_derived_budget():
    """mla_derive maps topb_middle onto the GQA exact top-b (G = 1, max)."""
    rng = np.random.default_rng(5)
    for sl in (100, 16 * 40, 16 * 40 + 5, 16 * 128, 16 * 129 + 3, 16 * 300):
        P = (sl + 15) // 16
        ps = rng.integers(0, 6, P).astype(np.float32)
        ps[-1] = -np.inf if sl % 16 else ps[-1]
        keep = M.topb_middle(ps, 128, 1, 10)
        npg, nsh, b = M.mla_derive([sl], 16, 10, 1, 128)
        tab, cnt = O.topb_select(ps[None, None, :], npg, nsh, b, 1, P)
        assert np.array_equal(np.nonzero(keep)[0], tab[0, 0, :cnt[0, 0]])


# ---- latent rki4 score -------------------------------------------------
def _latent_case(seed, NB=24, Lkv=512, Dr=64, H=4, sl=16 * 20 + 3):
    rng = np.random.default_rng(seed)
    cache = M.synth_latent(rng, NB, 16, Lkv, Dr)
    bt = rng.permutation(NB).astype(np.int32)[None, :]
    q = O.f32_to_bf16(rng.standard_normal((1, H, Lkv + Dr)).astype(np.float32))
    return rng, cache, bt, q, sl


def test_latent_score_vs_explicit_reconstruction():
    _, cache, bt, q, sl = _latent_case(3)
    npg = (sl + 15) // 16
    nsh = np.array([npg - 1])
    slabs = M.mla_build_summaries(cache, bt[0, :npg - 1], cache.shape[0])
    got = M.mla_score_rki4(q, slabs, cache, bt, nsh, 0.1, npg)
    # independent: dequantize every token row by loops, dot in float64
    qf = O.bf16_to_f32(q[0]).astype(np.float64)
    q8, qs = O.quantize_q(q[0, :, :512])
    qc = q8.astype(np.float64) * qs[:, None]
    for p in range(int(nsh[0])):
        b = bt[0, p]
        V = O.unpack_i4(slabs["v4"][b, 0]).astype(np.float64) * O.bf16_to_f32(slabs["vs"][b, 0])[:, None]
        best = -np.inf
        for t in range(16):
            k = (slabs["mu8"][b, 0] * O.bf16_to_f32(slabs["mus"][b, 0:1])[0]).astype(np.float64)
            for c in range(8):
                k = k + float(slabs["c8"][b, 0, t, c]) * float(O.bf16_to_f32(slabs["cs"][b, 0, t:t + 1])[0]) * V[c]
            kr = O.bf16_to_f32(cache[b, t, 512:]).astype(np.float64)
            for h in range(q.shape[1]):
                best = max(best, (qc[h] @ k + qf[h, 512:] @ kr) * 0.1)
        assert abs(got[0, p] - best) <= 1e-5 * max(1.0, abs(best))
    assert np.all(got[0, int(nsh[0]):] == 0)


def test_latent_score_constant_page_closed_form():
    """A constant page has dc = 0: C hits the scale floor, so every token
    reconstructs to mu and the score is scale * max_h (q.mu + max_t rope)."""
    rng = np.random.default_rng(4)
    Lkv, Dr, H = 512, 64, 3
    row = rng.standard_normal(Lkv + Dr).astype(np.float32)
    cache = np.repeat(O.f32_to_bf16(row)[None, None, :], 16, axis=1)     # (1,16,576)
    rope = O.f32_to_bf16(rng.standard_normal((16, Dr)).astype(np.float32))
    cache[0, :, Lkv:] = rope
    q = O.f32_to_bf16(rng.standard_normal((1, H, Lkv + Dr)).astype(np.float32))
    slabs = M.mla_build_summaries(cache, np.array([0]), 1)
    got = M.mla_score_rki4(q, slabs, cache, np.zeros((1, 2), np.int32), np.array([1]), 0.5, 2)
    mu = slabs["mu8"][0, 0].astype(np.float64) * O.bf16_to_f32(slabs["mus"][0, 0])
    q8, qs = O.quantize_q(q[0, :, :Lkv])
    qc = q8.astype(np.float64) * qs[:, None]
    qr = O.bf16_to_f32(q[0, :, Lkv:]).astype(np.float64)
    kr = O.bf16_to_f32(rope).astype(np.float64)
    want = max(qc[h] @ mu + max(qr[h] @ kr[t] for t in range(16)) for h in range(H)) * 0.5
    assert abs(got[0, 0] - want) <= 1e-4 * max(1.0, abs(want))


# ---- int8 RoPE summary ---------------------------------------------------
def test_rope_summary_scale_rule_and_round_trip():
    """Per token: the stored scale is bf16(max(absmax/127, 1e-8)), the
    largest key maps to +-127, keys are quantized with that stored scale, so
    every key dequantizes within half a stored step (plus the clamp when bf16
    rounded the scale below absmax/127: <= 127 x that rounding),
    listed out-of-range ids are skipped and unlisted blocks stay zero."""
    rng = np.random.default_rng(21)
    cache = M.synth_latent(rng, 6, 16)
    cache[2, 5, 512:] = 0                                              # all-zero token
    rope = M.mla_build_rope(cache, np.array([0, 2, 3, 9, -1]), 6)
    k = O.bf16_to_f32(cache[:, :, 512:]).astype(np.float64)
    am = np.abs(k).max(axis=-1)
    sc_f32 = np.maximum(am / 127.0, 1e-8)
    sc = O.bf16_to_f32(rope["rks"]).astype(np.float64)
    for b in (0, 2, 3):
        assert np.allclose(sc[b], sc_f32[b], rtol=2.0 ** -8, atol=0)
        deq = rope["rk8"][b].astype(np.float64) * sc[b][:, None]
        bound = 0.5 * sc[b] + 127 * np.maximum(sc_f32[b] - sc[b], 0) + 1e-12
        assert np.all(np.abs(deq - k[b]) <= bound[:, None])
        nz = am[b] > 0
        assert np.all(np.abs(rope["rk8"][b]).max(axis=-1)[nz] == 127)
    assert np.all(rope["rk8"][2, 5] == 0)
    for b in (1, 4, 5):
        assert not rope["rk8"][b].any() and not rope["rks"][b].any()


def _representable_case(rng, H=4):
    """Keys = integers in [-127, 127] (one +-127 per token) x 2^-3 and q_rope
    = integers (one +-127 per head) x 2^-4: both int8 round trips are exact."""
    cache = M.synth_latent(rng, 3, 16)
    ki = rng.integers(-127, 128, size=(3, 16, 64))
    ki[:, :, 0] = 127 * np.where(rng.random((3, 16)) < 0.5, -1, 1)
    cache[:, :, 512:] = O.f32_to_bf16((ki * 2.0 ** -3).astype(np.float32))
    q = O.f32_to_bf16(rng.standard_normal((1, H, 576)).astype(np.float32))
    qi = rng.integers(-127, 128, size=(1, H, 64))
    qi[:, :, 3] = 127
    q[:, :, 512:] = O.f32_to_bf16((qi * 2.0 ** -4).astype(np.float32))
    return cache, q, ki


def test_int8_rope_score_equals_exact_on_representable_keys():
    rng = np.random.default_rng(22)
    cache, q, ki = _representable_case(rng)
    rope = M.mla_build_rope(cache, np.arange(3), 3)
    assert np.array_equal(rope["rk8"].astype(np.int64), ki)
    assert np.all(O.bf16_to_f32(rope["rks"]) == np.float32(2.0 ** -3))
    slabs = M.mla_build_summaries(cache, np.arange(3), 3)
    bt = np.array([[2, 0, 1]], np.int32)
    nsh = np.array([3])
    exact = M.mla_score_rki4(q, slabs, cache, bt, nsh, 0.3, 3)
    r8 = M.mla_score_rki4(q, slabs, cache, bt, nsh, 0.3, 3, rope=rope)
    assert np.array_equal(exact, r8)


def test_int8_rope_score_vs_explicit_loop():
    """The int8 RoPE term recomputed by loops from the summary bytes: integer
    dot of the int8 keys with the int8 q_rope, times both scales."""
    _, cache, bt, q, sl = _latent_case(5)
    npg = (sl + 15) // 16
    nsh = np.array([npg - 1])
    blocks = bt[0, :npg - 1]
    slabs = M.mla_build_summaries(cache, blocks, cache.shape[0])
    rope = M.mla_build_rope(cache, blocks, cache.shape[0])
    got = M.mla_score_rki4(q, slabs, cache, bt, nsh, 0.1, npg, rope=rope)
    base = M.mla_score_rki4(q, slabs, cache, bt, nsh, 0.1, npg)
    q8, qs = O.quantize_q(q[0, :, :512])
    qc = q8.astype(np.float64) * qs[:, None]
    qf = O.bf16_to_f32(q[0, :, 512:]).astype(np.float64)
    for p in range(int(nsh[0])):
        b = bt[0, p]
        V = O.unpack_i4(slabs["v4"][b, 0]).astype(np.float64) * O.bf16_to_f32(slabs["vs"][b, 0])[:, None]
        best = -np.inf
        for t in range(16):
            k = (slabs["mu8"][b, 0] * O.bf16_to_f32(slabs["mus"][b, 0:1])[0]).astype(np.float64)
            for c in range(8):
                k = k + float(slabs["c8"][b, 0, t, c]) * float(O.bf16_to_f32(slabs["cs"][b, 0, t:t + 1])[0]) * V[c]
            ks = float(O.bf16_to_f32(rope["rks"][b, t:t + 1])[0])
            for h in range(q.shape[1]):
                am = max(abs(float(x)) for x in qf[h])
                qsr = np.float32(max(am, 1e-8)) / np.float32(127.0)
                dot = sum(int(np.rint(np.float32(qf[h, d]) / qsr)) * int(rope["rk8"][b, t, d]) for d in range(64))
                best = max(best, (qc[h] @ k + dot * float(qsr) * ks) * 0.1)
        assert abs(got[0, p] - best) <= 1e-5 * max(1.0, abs(best))
    # the summary moves the scores by about the keys' quantisation step only
    assert np.abs(got - base).max() <= 0.02 * np.abs(base).max()


@pytest.mark.parametrize("rope", [False, True])
def test_latent_summary_tracks_reference_selection(rope):
    """Quality link to the reference: on the BASELINE-shaped distribution
    with planted query-matching tokens, the int4 latent summary keeps every
    planted page (as the reference's fp32 factors do) and its recall of the
    exact top pages (max logit over the full-precision page) is within 0.1
    of the reference estimator's.  Informative bound, not bit parity: the two
    estimators differ (rank-8 about the mean, quantized, vs uncentred fp32).
    With ``rope`` the RoPE term comes from the int8 RoPE summary."""
    rng = np.random.default_rng(7)
    Lkv, Dr, H = 512, 64, 16
    NB, sl, budget = 200, 16 * 190 + 7, 40
    cache = M.synth_latent(rng, NB, 16, Lkv, Dr)
    q = rng.standard_normal((H, Lkv + Dr)).astype(np.float32)
    bt = rng.permutation(NB).astype(np.int32)[None, :]
    planted = rng.choice(np.arange(1, 150), 12, replace=False)
    for p in planted:
        lat = O.bf16_to_f32(cache[bt[0, p]])
        lat[rng.integers(0, 16)] += 0.5 * q[rng.integers(0, H)]
        cache[bt[0, p]] = O.f32_to_bf16(lat)
    qb = O.f32_to_bf16(q)[None]
    qf = O.bf16_to_f32(qb[0]).astype(np.float64)
    cf = O.bf16_to_f32(cache)
    npg, nsh, b = M.mla_derive([sl], 16, 10, 1, budget)
    P = int(npg[0])
    exact = np.full(P, -np.inf)
    for p in range(sl // 16):
        exact[p] = (qf @ cf[bt[0, p]].astype(np.float64).T).max()
    keep_true = M.topb_middle(exact.astype(np.float32), budget, 1, 10)
    keep_ref = M.mla_select_pages_ref(O.bf16_to_f32(qb[0, :, :Lkv]), O.bf16_to_f32(qb[0, :, Lkv:]),
                                      cf, bt[0], sl, 0.07, 8, budget, 1, 10)
    slabs = M.mla_build_summaries(cache, bt[0, :int(nsh[0])], NB)
    rs = M.mla_build_rope(cache, bt[0, :int(nsh[0])], NB) if rope else None
    sc = M.mla_score_rki4(qb, slabs, cache, bt, nsh, 0.07, P, rope=rs)
    tab, cnt = O.topb_select(sc[:, None, :], npg, nsh, b, 1, P)
    ours = set(tab[0, 0, :cnt[0, 0]].tolist())
    ref = set(np.nonzero(keep_ref)[0].tolist())
    true = set(np.nonzero(keep_true)[0].tolist())
    assert len(ours) == len(ref) == budget
    assert set(planted.tolist()) <= ours and set(planted.tolist()) <= ref
    rec_ours, rec_ref = len(ours & true) / budget, len(ref & true) / budget
    assert rec_ours >= rec_ref - 0.1, (rec_ours, rec_ref)


# ---- attention (mla_attn.py:178-201) -----------------------------------
def test_mla_attention_matches_direct_softmax():
    rng = np.random.default_rng(6)
    NB, H, Lkv, Dr = 10, 3, 32, 8
    cache = M.synth_latent(rng, NB, 16, Lkv, Dr)
    bt = rng.permutation(NB).astype(np.int32)[None, :]
    q = O.f32_to_bf16(rng.standard_normal((1, H, Lkv + Dr)).astype(np.float32))
    sl = 16 * 7 + 5
    tab = np.array([[0, 2, 7, -1]], np.int32)
    o, lse = M.mla_attention(q, cache, bt, [sl], tab, np.array([3]), 0.3, Lkv=Lkv)
    toks = [(pg, t) for pg in (0, 2, 7) for t in range(16) if pg * 16 + t < sl]
    kv = np.stack([O.bf16_to_f32(cache[bt[0, pg], t]).astype(np.float64) for pg, t in toks])
    qf = O.bf16_to_f32(q[0]).astype(np.float64)
    for h in range(H):
        s = np.array([qf[h] @ k for k in kv]) * 0.3
        w = np.exp(s - s.max())
        assert np.allclose(o[0, h], (w @ kv[:, :Lkv]) / w.sum(), rtol=1e-12, atol=1e-12)
        assert abs(lse[0, h] - (s.max() + np.log(w.sum()))) < 1e-12
