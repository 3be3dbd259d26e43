"""Pins of the CPU oracle (no GPU).  Each check compares an oracle function
with an independent formulation -- brute force, float64 linear algebra, a
closed form or a library routine -- chosen so that a plausible mistake
(dropped term, wrong sign/index, transposed operand) fails."""
from __future__ import annotations

import itertools
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import locks_oracle as O


# ---- int4 pack / unpack (rki4_build.py:161-175, rki4_score_torch.py:41-55) --
def test_unpack_every_byte():
    b = np.arange(256, dtype=np.uint8)[None, :]
    u = O.unpack_i4(b)[0]
    for x in range(256):
        lo, hi = x & 15, x >> 4
        assert u[2 * x] == (lo - 16 if lo >= 8 else lo)
        assert u[2 * x + 1] == (hi - 16 if hi >= 8 else hi)


def test_pack_roundtrip_all_pairs():
    vals = np.array(list(itertools.product(range(-8, 8), repeat=2)), np.int8).reshape(-1)
    p = O.pack_i4(vals[None, :])
    assert p.shape[-1] == vals.size // 2
    assert np.array_equal(O.unpack_i4(p)[0], vals)
    # low nibble holds the even index
    assert O.pack_i4(np.array([[3, -1]], np.int8))[0, 0] == (3 | (0xF << 4))


def test_bf16_round_matches_torch():
    import torch
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 1e3
    x[:4] = [0.0, -0.0, np.inf, 1e-40]
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), t)


# ---- summary build (rki4_build.py:147-225) -----------------------------------
def _pages(seed, N=64, n_kv=2, page=16, d=128):
    rng = np.random.default_rng(seed)
    k, _, _ = O.synth_kv(rng, N, page, n_kv, d)
    return k


def test_eigh_identity():
    k = _pages(0)
    _, _, _, gram = O.summary_pre(k)
    S2, U = O.summary_eigh(gram)
    g64 = gram.astype(np.float64)
    lhs = g64 @ U.astype(np.float64)
    rhs = U.astype(np.float64) * S2.astype(np.float64)[..., None, :]
    assert np.abs(lhs - rhs).max() <= 1e-3 * np.abs(g64).max()
    assert (np.diff(S2, axis=-1) >= -1e-3).all()            # ascending


def test_pre_matches_float64():
    k = _pages(1)
    tag, mu, dc, gram = O.summary_pre(k)
    K = O.bf16_to_f32(k).astype(np.float64).transpose(0, 2, 1, 3)
    assert np.abs(mu - K.mean(2)).max() < 1e-5
    assert np.abs(dc - (K - K.mean(2, keepdims=True))).max() < 1e-4
    assert np.array_equal(tag, k[:, 15, :, :8])


def test_summary_codes_vs_float64_svd():
    """Basis/coefficient codes equal an independent float64 SVD of the centred
    page pushed through the quantization formula (columns matched by singular
    value, eigenvector sign aligned).  Only fp rounding at exact .5 code
    boundaries may differ."""
    k = _pages(2, N=32)
    s = O.build_summaries(k)
    _, mu, dc, _ = O.summary_pre(k)
    U_, S_, Vt = np.linalg.svd(dc.astype(np.float64), full_matrices=False)
    vq = O.unpack_i4(s["v4"]).astype(np.float64)             # (N,k,R,d), col 0 = 8th largest
    mism = tot = 0
    for r in range(8):
        j = 7 - r                                               # SVD index (descending)
        v = Vt[..., j, :]                                       # (N,k,d) unit right vector
        sign = np.sign(np.einsum("nkd,nkd->nk", vq[:, :, r], v))[..., None]
        v = v * sign
        sc = np.abs(v).max(-1, keepdims=True) / 7.0
        code = np.clip(np.rint(v / sc), -8, 7)
        mism += (code != vq[:, :, r]).sum()
        tot += code.size
        c = U_[..., :, j] * S_[..., None, j] * sign             # (N,k,t)
        # per-token scale uses all 8 columns: check the reconstruction C*cs instead
        cdeq = s["c8"][..., r].astype(np.float64) * O.bf16_to_f32(s["cs"]).astype(np.float64)
        assert np.abs(cdeq - c).max() <= np.abs(c).max() * 0.02 + 1e-3
    assert mism / tot < 0.01, (mism, tot)
    mu_d = s["mu8"].astype(np.float64) * O.bf16_to_f32(s["mus"])[..., None]
    assert np.abs(mu_d - mu).max() <= np.abs(mu).max() / 127 * 0.6 + 1e-6


def test_summary_exact_low_rank_page():
    """A page of exact rank <= 8 around its mean is reproduced to quant error."""
    rng = np.random.default_rng(3)
    A = rng.standard_normal((4, 2, 16, 5)) @ rng.standard_normal((4, 2, 5, 128))
    A += rng.standard_normal((4, 2, 1, 128))
    kp = O.f32_to_bf16(A.transpose(0, 2, 1, 3).astype(np.float32))
    s = O.build_summaries(kp)
    _, mu, dc, _ = O.summary_pre(kp)
    V = O.unpack_i4(s["v4"]).astype(np.float64) * O.bf16_to_f32(s["vs"])[..., None]
    C = s["c8"].astype(np.float64) * O.bf16_to_f32(s["cs"])[..., None]
    rec = np.einsum("nktr,nkrd->nktd", C, V)
    assert np.linalg.norm(rec - dc) / np.linalg.norm(dc) < 0.2     # int4 floor only


def test_summary_constant_page_hits_floors():
    kp = np.full((1, 16, 1, 128), O.f32_to_bf16(np.float32(0.0)), np.uint16)
    s = O.build_summaries(kp)
    # dc = 0: V = dc^T U8 / S8 = 0 -> all codes 0 at the 1e-8 scale floor;
    # mu = 0 likewise; C = U8 * sqrt(1e-10) is tiny but nonzero (its own scale)
    assert (O.unpack_i4(s["v4"]) == 0).all() and (s["mu8"] == 0).all()
    floor = O.bf16_round(np.float32(1e-8))
    assert (O.bf16_to_f32(s["vs"]) == floor).all() and (O.bf16_to_f32(s["mus"]) == floor).all()
    cdeq = s["c8"].astype(np.float64) * O.bf16_to_f32(s["cs"])[..., None]
    assert np.abs(cdeq).max() <= 1.01e-5


def test_quant_invariants():
    s = O.build_summaries(_pages(4, N=16))
    vq = O.unpack_i4(s["v4"])
    assert vq.min() >= -8 and vq.max() <= 7
    assert np.abs(s["c8"]).max() <= 127 and np.abs(s["mu8"]).max() <= 127
    # every column / token / page reaches its absmax code (scale = absmax/Q)
    assert (np.abs(vq).max(axis=-1) >= 7).all()
    assert (np.abs(s["c8"]).max(axis=-1) == 127).all()


# ---- scorer (rki4_score_torch.py:111-160) -------------------------------------
def _score_case(seed, n_kv=2, G=4, npages=40):
    rng = np.random.default_rng(seed)
    NB = npages + 3
    k, _, _ = O.synth_kv(rng, NB, 16, n_kv, 128)
    slabs = O.build_state_slabs(k, np.arange(NB), NB)
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, 128)).astype(np.float32))
    bt = rng.permutation(NB)[None, :npages].astype(np.int32)
    return slabs, q, bt


def _score_reconstructed_keys(q, slabs, bt, P, n_kv, G, s):
    """float64: rebuild every key of every page from the dequantized summary
    (k_t = mu + sum_r C[t,r] V[:,r]) and take LSE_t of s * q8dq . k_t."""
    q8, qs = O.quantize_q(q.reshape(1, n_kv, G, 128))
    qd = q8.astype(np.float64) * qs[..., None]
    out = np.zeros((n_kv, G, P))
    for p in range(P):
        b = bt[0, p]
        for kh in range(n_kv):
            V = O.unpack_i4(slabs["v4"][b, kh]).astype(np.float64) * \
                O.bf16_to_f32(slabs["vs"][b, kh])[:, None]                 # (R, d)
            C = slabs["c8"][b, kh].astype(np.float64) * O.bf16_to_f32(slabs["cs"][b, kh])[:, None]
            mu = slabs["mu8"][b, kh].astype(np.float64) * float(O.bf16_to_f32(slabs["mus"][b, kh:kh + 1])[0])
            keys = mu[None, :] + C @ V                                      # (t, d)
            for g in range(G):
                x = s * (keys @ qd[0, kh, g])
                out[kh, g, p] = O.log_sum_exp(list(x))
    return out


@pytest.mark.parametrize("G", [1, 4, 16])
def test_score_twin_vs_reconstructed_keys(G):
    slabs, q, bt = _score_case(5, G=G)
    P, s = 37, 1 / math.sqrt(128)
    twin = O.score_rki4_twin(q, slabs, bt, np.array([P]), 2, G, s, 40)
    intp = O.score_rki4_intpath(q, slabs, bt, np.array([P]), 2, G, s, 40)
    ref = _score_reconstructed_keys(q, slabs, bt, P, 2, G, s)
    assert np.abs(twin[0, :, :, :P] - ref).max() < 1e-5
    assert np.abs(intp[0, :, :, :P] - ref).max() < 1e-5
    assert (twin[0, :, :, P:] == 0).all()


def test_score_rank0_closed_form():
    """V = 0 -> every token logit is s*mud, so LSE = s*mud + log 16."""
    slabs, q, bt = _score_case(6, G=4)
    slabs = dict(slabs)
    slabs["v4"] = np.full_like(slabs["v4"], 0)      # nibble 0 -> V = 0
    s = 0.5
    out = O.score_rki4_twin(q, slabs, bt, np.array([10]), 2, 4, s, 40)
    q8, qs = O.quantize_q(q.reshape(1, 2, 4, 128))
    for p in range(10):
        b = bt[0, p]
        for kh in range(2):
            mud = (slabs["mu8"][b, kh].astype(np.float64) @ q8[0, kh].T.astype(np.float64)) \
                * qs[0, kh] * float(O.bf16_to_f32(slabs["mus"][b, kh:kh + 1])[0])
            assert np.allclose(out[0, kh, :, p], s * mud + math.log(16), atol=1e-5)


def test_score_zero_q_floor():
    slabs, q, bt = _score_case(7, G=2)
    q = np.zeros_like(q)
    out = O.score_rki4_twin(q, slabs, bt, np.array([5]), 2, 2, 0.1, 40)
    assert np.allclose(out[0, :, :, :5], math.log(16), atol=1e-6)


# ---- derive (select.py:28-58) ---------------------------------------------------
@pytest.mark.parametrize("sl", [0, 1, 15, 16, 17, 33, 4096, 16384, 1 << 20])
@pytest.mark.parametrize("babs,budget", [(126, 0.1), (0, 0.1), (0, 1.0), (5000, 0.1)])
def test_derive_closed_form(sl, babs, budget):
    npg, nsh, b = O.derive_page_params([sl], 16, 1, 1, babs, budget)
    n = -(-sl // 16)
    S = n - 1 - 1
    if babs > 0:
        exp_b = max(min(babs, max(S, 1)), 1)
    else:
        exp_b = min(max(math.ceil(Fraction(S) * Fraction(budget)), 1), max(S, 1))
    assert (int(npg[0]), int(nsh[0]), int(b[0])) == (n, n - 1, exp_b)


# ---- combine + top-b (select_cuda.py:547-658, select.py:123-180) --------------
def test_combine_nrm_closed_form():
    rng = np.random.default_rng(8)
    sh = rng.standard_normal((1, 2, 3, 20)).astype(np.float32)
    out = O.combine_nrm(sh, np.array([17]))
    for kh in range(2):
        for p in range(17):
            exp = sum(math.exp(float(sh[0, kh, g, p]) - float(sh[0, kh, g, :17].max()))
                      for g in range(3))
            assert abs(out[0, kh, p] - exp) < 1e-5
    g1 = O.combine_nrm(sh[:, :, :1], np.array([17]))
    assert np.allclose(g1[0, :, :17], np.exp(sh[0, :, 0, :17] - sh[0, :, 0, :17].max(-1, keepdims=True)))
    assert (out[0, :, 17:] == 0).all()


def _brute_topb(score, npg, nsh, b, sink):
    keep = set()
    if nsh - sink <= 1:
        return list(range(max(npg, 0)))
    keep |= set(range(sink)) | set(range(nsh, npg))
    sel = sorted(range(sink, nsh), key=lambda p: (-score[p], p))
    keep |= set(sel[:min(b, nsh - sink)])
    return sorted(keep)


@pytest.mark.parametrize("seed", range(30))
def test_topb_vs_bruteforce(seed):
    rng = np.random.default_rng(seed)
    P = int(rng.integers(1, 13))
    MP = 14
    sl = int(rng.integers(0, 16 * P + 1))
    babs = int(rng.integers(1, 8))
    sink = int(rng.integers(0, 3))
    npg, nsh, b = O.derive_page_params([sl], 16, 1, sink, babs, 0.1)
    vals = rng.integers(0, 4, size=(1, 2, MP)).astype(np.float32)   # many ties
    tab, cnt = O.topb_select(vals, npg, nsh, b, sink, MP)
    for kh in range(2):
        exp = _brute_topb(vals[0, kh], int(npg[0]), int(nsh[0]), int(b[0]), sink)
        assert tab[0, kh, :cnt[0, kh]].tolist() == exp
        assert (tab[0, kh, cnt[0, kh]:] == -1).all()


def test_topb_batteries():
    MP = 1024
    npg, nsh, b = O.derive_page_params([16 * 1000], 16, 1, 1, 126, 0.1)
    for vals in (np.ones((1, 1, MP), np.float32),                       # all equal
                 np.zeros((1, 1, MP), np.float32),                      # +0 underflow
                 np.repeat(np.arange(8, dtype=np.float32), MP // 8)[None, None]):
        tab, cnt = O.topb_select(vals, npg, nsh, b, 1, MP)
        assert cnt[0, 0] == 1 + 126 + 1
        exp = _brute_topb(vals[0, 0], 1000, 999, 126, 1)
        assert tab[0, 0, :cnt[0, 0]].tolist() == exp


# ---- decode / merge (decode.py:209-322, merge.py:105-152) ---------------------
def test_decode_dense_matches_sdpa():
    import torch
    rng = np.random.default_rng(9)
    n_kv, G, sl = 2, 4, 300
    NB = 25
    k, v, _ = O.synth_kv(rng, NB, 16, n_kv, 128)
    bt = rng.permutation(NB)[None, :].astype(np.int32)
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, 128)).astype(np.float32))
    npg = -(-sl // 16)
    tab = np.full((1, n_kv, NB), -1, np.int32)
    tab[..., :npg] = np.arange(npg)
    cnt = np.full((1, n_kv), npg, np.int32)
    out, lse = O.decode_attention(q, k, v, bt, [sl], tab, cnt, G, 0.088, dtype=np.float64)
    K = torch.from_numpy(O.bf16_to_f32(k[bt[0, :npg]]).reshape(-1, n_kv, 128)[:sl]).double()
    V = torch.from_numpy(O.bf16_to_f32(v[bt[0, :npg]]).reshape(-1, n_kv, 128)[:sl]).double()
    Q = torch.from_numpy(O.bf16_to_f32(q[0])).double().reshape(n_kv, G, 128)
    ref = torch.nn.functional.scaled_dot_product_attention(
        Q[:, :, None], K.permute(1, 0, 2)[:, None].expand(-1, G, -1, -1),
        V.permute(1, 0, 2)[:, None].expand(-1, G, -1, -1), scale=0.088)[:, :, 0]
    assert np.abs(out[0] - ref.reshape(-1, 128).numpy()).max() < 1e-10
    lse_ref = torch.logsumexp(0.088 * torch.einsum("kgd,tkd->kgt", Q, K), -1).reshape(-1)
    assert np.abs(lse[0] - lse_ref.numpy()).max() < 1e-10


def test_merge_split_invariance():
    """Flash-decode partials over any contiguous split merge to the direct
    softmax; empty splits (l=0) get weight 0; cnt=0 rows give 0."""
    rng = np.random.default_rng(10)
    G, D, T = 3, 8, 50
    s = rng.standard_normal((G, T)) * 3
    v = rng.standard_normal((T, D))
    direct = (np.exp(s - s.max(1, keepdims=True)) @ v) / np.exp(s - s.max(1, keepdims=True)).sum(1, keepdims=True)
    for split in (1, 3, 8):
        cnt = T  # one "page" per token for this check
        pps = max(-(-cnt // split), 1)
        m = np.full((1, 2, split, G), -np.inf, np.float32)
        l = np.zeros((1, 2, split, G), np.float32)
        acc = np.zeros((1, 2, split, G, D), np.float32)
        for sp in range(split):
            j0, j1 = sp * pps, min(sp * pps + pps, cnt)
            if j0 >= cnt:
                continue
            mm = s[:, j0:j1].max(1)
            p = np.exp(s[:, j0:j1] - mm[:, None])
            m[0, 0, sp], l[0, 0, sp], acc[0, 0, sp] = mm, p.sum(1), p @ v[j0:j1]
        out = O.merge_partials(m, l, acc, np.array([[cnt, 0]]), split, 1)
        assert np.abs(out[0, :G] - direct).max() < 1e-5
        assert (out[0, G:] == 0).all()


# ---- the other geometries (rki4_state.py:295-324: d 64/128/256, page 16/32) ----
GEOMS = [(64, 16), (256, 16), (128, 32), (64, 32), (256, 32), (128, 64), (256, 64)]


@pytest.mark.parametrize("d,page", GEOMS)
def test_geometry_pre_and_low_rank(d, page):
    """Centre / tag at float64, and an exact rank-5 page reproduced to the
    int4/int8 quantization floor (the build's eigh + pack at this shape)."""
    rng = np.random.default_rng(40)
    A = rng.standard_normal((3, 2, page, 5)) @ rng.standard_normal((3, 2, 5, d))
    A += rng.standard_normal((3, 2, 1, d))
    kp = O.f32_to_bf16(A.transpose(0, 2, 1, 3).astype(np.float32))
    tag, mu, dc, _ = O.summary_pre(kp)
    K = O.bf16_to_f32(kp).astype(np.float64).transpose(0, 2, 1, 3)
    assert np.abs(mu - K.mean(2)).max() < 1e-5
    assert np.array_equal(tag, kp[:, page - 1, :, :8])
    s = O.build_summaries(kp)
    assert s["v4"].shape[-2:] == (8, d // 2) and s["c8"].shape[-2:] == (page, 8)
    V = O.unpack_i4(s["v4"]).astype(np.float64) * O.bf16_to_f32(s["vs"])[..., None]
    C = s["c8"].astype(np.float64) * O.bf16_to_f32(s["cs"])[..., None]
    rec = np.einsum("nktr,nkrd->nktd", C, V)
    assert np.linalg.norm(rec - dc) / np.linalg.norm(dc) < 0.2


@pytest.mark.parametrize("d,page", GEOMS)
@pytest.mark.parametrize("G", [1, 8])
def test_geometry_score_vs_reconstructed_keys(d, page, G):
    """Twin and integer-path scores equal the float64 LSE over the page's
    keys rebuilt from the dequantized summary, at each geometry."""
    rng = np.random.default_rng(41)
    n_kv, npages = 2, 12
    NB = npages + 2
    k, _, _ = O.synth_kv(rng, NB, page, n_kv, d)
    slabs = O.build_state_slabs(k, np.arange(NB), NB)
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, d)).astype(np.float32))
    bt = rng.permutation(NB)[None, :npages].astype(np.int32)
    P, s = 11, 1 / math.sqrt(d)
    twin = O.score_rki4_twin(q, slabs, bt, np.array([P]), n_kv, G, s, npages)
    intp = O.score_rki4_intpath(q, slabs, bt, np.array([P]), n_kv, G, s, npages)
    q8, qs = O.quantize_q(q.reshape(1, n_kv, G, d))
    qd = q8.astype(np.float64) * qs[..., None]
    for p in range(P):
        b = bt[0, p]
        for kh in range(n_kv):
            V = O.unpack_i4(slabs["v4"][b, kh]).astype(np.float64) * O.bf16_to_f32(slabs["vs"][b, kh])[:, None]
            C = slabs["c8"][b, kh].astype(np.float64) * O.bf16_to_f32(slabs["cs"][b, kh])[:, None]
            mu = slabs["mu8"][b, kh].astype(np.float64) * float(O.bf16_to_f32(slabs["mus"][b, kh:kh + 1])[0])
            keys = mu[None, :] + C @ V                                   # (page, d)
            assert keys.shape == (page, d)
            for g in range(G):
                ref = O.log_sum_exp(list(s * (keys @ qd[0, kh, g])))
                assert abs(twin[0, kh, g, p] - ref) < 1e-5 and abs(intp[0, kh, g, p] - ref) < 1e-5


@pytest.mark.parametrize("d,page", GEOMS)
def test_geometry_rank0_closed_form(d, page):
    """V = 0 -> every token logit is s*mud, so LSE = s*mud + log(page)."""
    rng = np.random.default_rng(42)
    NB, n_kv, G = 6, 2, 4
    k, _, _ = O.synth_kv(rng, NB, page, n_kv, d)
    slabs = dict(O.build_state_slabs(k, np.arange(NB), NB))
    slabs["v4"] = np.zeros_like(slabs["v4"])
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, d)).astype(np.float32))
    bt = np.arange(NB, dtype=np.int32)[None]
    s = 0.3
    out = O.score_rki4_twin(q, slabs, bt, np.array([NB]), n_kv, G, s, NB)
    q8, qs = O.quantize_q(q.reshape(1, n_kv, G, d))
    for p in range(NB):
        for kh in range(n_kv):
            mud = (slabs["mu8"][p, kh].astype(np.float64) @ q8[0, kh].T.astype(np.float64)) \
                * qs[0, kh] * float(O.bf16_to_f32(slabs["mus"][p, kh:kh + 1])[0])
            assert np.allclose(out[0, kh, :, p], s * mud + math.log(page), atol=1e-5)


@pytest.mark.parametrize("d,page", GEOMS)
def test_geometry_decode_matches_sdpa(d, page):
    """decode_attention over every page of a ragged row equals float64 SDPA."""
    import torch
    rng = np.random.default_rng(43)
    n_kv, G, sl = 2, 3, 5 * page + 7
    npg = -(-sl // page)
    NB = npg + 2
    k, v, _ = O.synth_kv(rng, NB, page, n_kv, d)
    bt = rng.permutation(NB)[None, :npg].astype(np.int32)
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, d)).astype(np.float32))
    tab = np.full((1, n_kv, npg), -1, np.int32)
    tab[..., :npg] = np.arange(npg)
    cnt = np.full((1, n_kv), npg, np.int32)
    sc = 1 / math.sqrt(d)
    out, _ = O.decode_attention(q, k, v, bt, [sl], tab, cnt, G, sc, dtype=np.float64)
    K = torch.from_numpy(O.bf16_to_f32(k[bt[0]]).reshape(-1, n_kv, d)[:sl]).double()
    V = torch.from_numpy(O.bf16_to_f32(v[bt[0]]).reshape(-1, n_kv, d)[:sl]).double()
    Q = torch.from_numpy(O.bf16_to_f32(q[0])).double().reshape(n_kv, G, d)
    ref = torch.nn.functional.scaled_dot_product_attention(
        Q[:, :, None], K.permute(1, 0, 2)[:, None].expand(-1, G, -1, -1),
        V.permute(1, 0, 2)[:, None].expand(-1, G, -1, -1), scale=sc)[:, :, 0]
    assert np.abs(out[0] - ref.reshape(-1, d).numpy()).max() < 1e-10
