"""CPU oracle for the LOCKS MLA (latent) decode path -- TEST INFRASTRUCTURE ONLY.

Like ``locks_oracle`` this module is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
may import it.

Two things are restated here (paths relative to the reference package
``src/locks/``):

1. The reference's MLA selection, as it runs there (fp32 factors):
     mla_factor_build     selection/mla_select.py:26-53 (_page_basis: top-r
                          eigenpairs of the page Gram, spectral floor) and
                          :69-108 (build_page_factors: Lf = W sig,
                          Rf = W^T blk / sig, dropped modes exactly zero)
     mla_page_score_ref   selection/mla_score_torch.py:27-48 (max over heads
                          and valid tokens of (q_c.C8 + q_rope.k_rope) * scale)
     topb_middle          selection/mla_score_torch.py:51-73 (sink + recent
                          forced inside the budget, top-scored middle fills)
     mla_attention        backend/mla_attn.py:178-201 (fp32 softmax over the
                          gathered selected tokens; o = attn @ latent[:, :Lkv],
                          lse = logsumexp)
2. This build's latent summary -- the rki4 record (``locks_oracle``'s
   summary build, rki4_build.py:147-225, at d = kv_lora_rank) plus the exact
   bf16 RoPE keys read from the cache -- and its page score:
     mla_build_summaries  locks_oracle.build_summaries on (N, page, 1, Lkv)
     mla_score_rki4       tok[h][t] = (q8.mu8)qs mus + cs_t sum_c c8[t][c]
                          (sum_d V4[c][d] q8[h][d]) qs vs_c + q_rope[h].k_rope[t]
                          page score = scale * max_{h, t} tok[h][t]
     mla_build_rope       int8 RoPE summary: per token scale max(absmax/127,
                          1e-8) (the rki4 token-scale rule, rki4_build.py's
                          C8 quantisation), keys rint(k / scale) clipped to
                          +-127, scale stored as bf16
     mla_score_rki4(rope=) RoPE term (qr8[h].rk8[t]) qrs[h] rks[t] with
                          q_rope int8-quantized per head like q_c
   The reference ships no latent rki4 format and no RoPE summary (these
   layouts are new: the reference scores with fp32 factors and the exact
   keys, mla_select.py:69-108, mla_score_torch.py:41); the max-union score,
   the budget rule and the attention are the reference's.

Ties: the reference's ``topb_middle`` uses ``torch.topk``, whose order among
equal scores is unspecified; ``topb_middle`` here breaks ties by the lowest
page index (the total order the GPU selector implements).
"""
from __future__ import annotations

import numpy as np

from . import locks_oracle as O

NEG_REF = -1e30                      # mla_score_torch.py:24


# --------------------------------------------------------------------------- #
# reference semantics: fp32 factors (mla_select.py:26-108)
# --------------------------------------------------------------------------- #
def mla_page_basis(blk: np.ndarray, r: int):
    """_page_basis (mla_select.py:26-53): top-r eigenpairs of the page Gram
    blk blk^T, descending; modes with sig <= sig_max * sqrt(eps) get sig 0.
    blk (n, page, Lkv) fp32.  Returns W (n, page, r), sig (n, r)."""
    G = np.einsum("ntd,nsd->nts", blk, blk).astype(np.float32)
    lam, W = np.linalg.eigh(G)                                  # ascending
    lam = lam[:, -r:][:, ::-1]
    W = W[:, :, -r:][:, :, ::-1]
    sig = np.sqrt(np.maximum(lam, 0)).astype(np.float32)
    tol = sig[:, :1] * np.float32(np.sqrt(np.finfo(np.float32).eps))
    return W.astype(np.float32), np.where(sig > tol, sig, 0).astype(np.float32)


def mla_factor_build(blk: np.ndarray, rank: int, rpad: int = 16):
    """build_page_factors (mla_select.py:69-108).  blk (n, page, Lkv) fp32.
    Returns Lf (n, page, rpad), Rf (n, rpad, Lkv); Lf @ Rf = W W^T blk."""
    n, page, Lkv = blk.shape
    r = min(rank, page, Lkv, rpad)
    W, sig = mla_page_basis(blk, r)
    Lf = np.zeros((n, page, rpad), np.float32)
    Rf = np.zeros((n, rpad, Lkv), np.float32)
    Lf[:, :, :r] = W * sig[:, None, :]
    inv = np.where(sig > 0, 1.0 / np.maximum(sig, np.finfo(np.float32).tiny), 0).astype(np.float32)
    Rf[:, :r, :] = np.einsum("ntr,ntd->nrd", W, blk) * inv[:, :, None]
    return Lf, Rf


def mla_page_score_ref(q_c, q_rope, C8, k_rope, valid, scale):
    """mla_score_torch.py:27-48.  q_c (H, D), q_rope (H, Dr), C8 (P, page, D),
    k_rope (P, page, Dr), valid (P,).  Returns page_score (P,) fp32."""
    s_nope = np.einsum("hD,ptD->hpt", q_c.astype(np.float32), C8.astype(np.float32))
    s_rope = np.einsum("hd,ptd->hpt", q_rope.astype(np.float32), k_rope.astype(np.float32))
    approx = ((s_nope + s_rope) * np.float32(scale)).astype(np.float32)
    page = C8.shape[1]
    vmask = np.arange(page)[None, :] < np.asarray(valid)[:, None]
    approx = np.where(vmask[None], approx, np.float32(NEG_REF))
    return approx.max(axis=2).max(axis=0).astype(np.float32)


def topb_middle(page_score, budget_pages, n_sink, n_recent):
    """mla_score_torch.py:51-73 keep mask (P,) bool; ties -> lowest page."""
    ps = np.asarray(page_score, np.float32)
    P = ps.shape[0]
    keep = np.zeros(P, bool)
    if P <= budget_pages:
        keep[:] = True
        return keep
    forced = set(range(min(n_sink, P))) | set(range(max(0, P - n_recent), P))
    for p in forced:
        keep[p] = True
    n_mid = budget_pages - len(forced)
    if n_mid > 0:
        idx = np.array([p for p in range(P) if p not in forced], np.int64)
        if idx.size:
            k = min(n_mid, idx.size)
            order = sorted(idx.tolist(), key=lambda p: (-float(ps[p]), p))
            keep[np.array(order[:k], np.int64)] = True
    return keep


def mla_select_pages_ref(q_c, q_rope, cache_f32, blocks, seq_len, scale, rank,
                         budget_pages, n_sink, n_recent, Lkv=512):
    """One row of the reference's selection (mla_attn.py:126-164 +
    mla_select.py:111-130): factors over the FULL prompt pages, -inf for the
    partial page, topb_middle.  cache_f32 (NB, page, Lkv + Dr)."""
    page = cache_f32.shape[1]
    n_pages = (seq_len + page - 1) // page
    n_cache = seq_len // page
    ps = np.full(n_pages, -np.inf, np.float32)
    if n_cache > 0:
        blk = cache_f32[np.asarray(blocks[:n_cache])]
        Lf, Rf = mla_factor_build(blk[:, :, :Lkv], rank)
        C8 = np.einsum("ntr,nrd->ntd", Lf, Rf).astype(np.float32)
        kr = blk[:, :, Lkv:]
        ps[:n_cache] = mla_page_score_ref(q_c, q_rope, C8, kr, np.full(n_cache, page), scale)
    return topb_middle(ps, budget_pages, n_sink, n_recent)


# --------------------------------------------------------------------------- #
# this build's latent summary (rki4 record at d = Lkv) and its score
# --------------------------------------------------------------------------- #
def mla_build_summaries(cache_bf16: np.ndarray, blocks, n_blocks: int, Lkv: int = 512):
    """rki4 slabs (n_kv = 1, d = Lkv) of the latent part of the listed
    physical blocks; cache_bf16 (NB, page, Lkv + Dr) bf16 bits."""
    lat = np.ascontiguousarray(cache_bf16[:, :, None, :Lkv])      # (NB, page, 1, Lkv)
    return O.build_state_slabs(lat, np.asarray(blocks), n_blocks)


def mla_build_rope(cache_bf16: np.ndarray, blocks, n_blocks: int, Lkv: int = 512):
    """int8 RoPE summary of the listed physical blocks (ids outside
    [0, n_blocks) skipped; unlisted blocks stay zero).  cache_bf16
    (NB, page, Lkv + Dr) bf16 bits.  Returns dict rk8 (NB, page, Dr) int8,
    rks (NB, page) bf16 bits."""
    f32 = np.float32
    NB, page, HS = cache_bf16.shape
    Dr = HS - Lkv
    rk8 = np.zeros((n_blocks, page, Dr), np.int8)
    rks = np.zeros((n_blocks, page), np.uint16)
    blk = np.array([b for b in np.asarray(blocks).tolist() if 0 <= b < n_blocks], np.int64)
    if blk.size:
        k = O.bf16_to_f32(cache_bf16[blk, :, Lkv:])                      # (n, page, Dr)
        sc = np.maximum((np.abs(k).max(axis=-1) / f32(127.0)).astype(f32), f32(1e-8))
        rks[blk] = O.f32_to_bf16(sc)
        sc = O.bf16_to_f32(rks[blk])             # quantize with the stored scale
        rk8[blk] = np.clip(np.rint(k / sc[..., None]), -127, 127).astype(np.int8)
    return dict(rk8=rk8, rks=rks)


def mla_score_rki4(q_bf16, slabs, cache_bf16, bt, nsh, scale, MP, Lkv=512, rope=None):
    """Page score from the latent rki4 summary + RoPE keys.

    q (R, H, Lkv + Dr) bf16 bits: q_c = q[..., :Lkv] is int8-quantized per
    head (absmax / 127, as the GQA scorer).  rope None: q_rope = q[..., Lkv:]
    as bf16 against the exact keys of the cache; rope = mla_build_rope(...):
    q_rope int8-quantized per head the same way, against rk8 * rks.  Returns
    (R, MP) fp32 for p < nsh[r] (0 elsewhere): scale * max_{h, t}
    (q_c8[h] . khat[t] + q_rope[h] . k_rope[t]), khat = mu + C V^T."""
    R, H, HS = q_bf16.shape
    NB = slabs["v4"].shape[0]
    q8, qs = O.quantize_q(q_bf16[:, :, :Lkv])
    qc = (q8.astype(np.float64) * qs[..., None].astype(np.float64))     # (R,H,Lkv)
    if rope is None:
        qr = O.bf16_to_f32(q_bf16[:, :, Lkv:]).astype(np.float64)      # (R,H,Dr)
    else:
        qr8, qrs = O.quantize_q(q_bf16[:, :, Lkv:])
        qr = qr8.astype(np.float64) * qrs[..., None].astype(np.float64)
    out = np.zeros((R, MP), np.float32)
    for r in range(R):
        P = int(nsh[r])
        if P <= 0:
            continue
        blk = np.clip(bt[r, :P].astype(np.int64), 0, NB - 1)
        Vq = O.unpack_i4(slabs["v4"][blk, 0]).astype(np.float64)        # (P,R8,Lkv)
        Vref = Vq * O.bf16_to_f32(slabs["vs"][blk, 0])[..., None]
        Cref = slabs["c8"][blk, 0].astype(np.float64) * O.bf16_to_f32(slabs["cs"][blk, 0])[..., None]
        muref = slabs["mu8"][blk, 0].astype(np.float64) * O.bf16_to_f32(slabs["mus"][blk, 0])[..., None]
        khat = muref[:, None, :] + np.einsum("ptc,pcd->ptd", Cref, Vref)  # (P,page,Lkv)
        if rope is None:
            kr = O.bf16_to_f32(cache_bf16[blk, :, Lkv:]).astype(np.float64)  # (P,page,Dr)
        else:
            kr = rope["rk8"][blk].astype(np.float64) * O.bf16_to_f32(rope["rks"][blk])[..., None]
        s = np.einsum("hd,ptd->hpt", qc[r], khat) + np.einsum("hd,ptd->hpt", qr[r], kr)
        out[r, :P] = (s.max(axis=2).max(axis=0) * scale).astype(np.float32)
    return out


def mla_derive(seq_lens, page, window, sink, budget_pages):
    """The selector parameters that make the GQA exact top-b equal
    topb_middle: n_pages, n_sel_hi = n_pages - window, and b = the middle
    budget (budget_pages minus the forced sink + window pages, inside the
    budget as in mla_score_torch.py:63); rows with n_pages <= budget keep
    everything (b >= selectable count)."""
    b_mid = max(int(budget_pages) - int(sink) - int(window), 1)
    return O.derive_page_params(seq_lens, page, window, sink, budget_abs=b_mid)


def mla_attention(q_bf16, cache_bf16, bt, seq_lens, page_table, page_cnt, scale, Lkv=512):
    """mla_attn.py:178-201 in float64: per row, softmax over the tokens of the
    selected pages (position < seq_len) of q . [latent | rope]; o = attn @
    latent.  q (R, H, HS) bits, cache (NB, page, HS) bits, page_table (R, MP),
    page_cnt (R,).  Returns o (R, H, Lkv) fp64 and lse (R, H) fp64."""
    R, H, HS = q_bf16.shape
    page = cache_bf16.shape[1]
    o = np.zeros((R, H, Lkv))
    lse = np.full((R, H), -np.inf)
    for r in range(R):
        c = int(page_cnt[r])
        if c <= 0:
            continue
        pts = page_table[r, :c].astype(np.int64)
        blks = bt[r, pts].astype(np.int64)
        pos = (pts[:, None] * page + np.arange(page)[None, :]).reshape(-1)
        ok = pos < int(seq_lens[r])
        kv = O.bf16_to_f32(cache_bf16[blks]).astype(np.float64).reshape(-1, HS)[ok]
        qv = O.bf16_to_f32(q_bf16[r]).astype(np.float64)
        s = qv @ kv.T * scale
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(axis=-1, keepdims=True)
        o[r] = (p @ kv[:, :Lkv]) / l
        lse[r] = (m + np.log(l))[:, 0]
    return o, lse


def synth_latent(rng: np.random.Generator, n_blocks, page, Lkv=512, Dr=64):
    """Latent cache ~ N(0, 1) times seeded per-dim scales (log-normal,
    sigma 0.5), bf16 bits (NB, page, Lkv + Dr)."""
    sc = np.exp(rng.standard_normal(Lkv + Dr).astype(np.float32) * np.float32(0.5))
    x = rng.standard_normal((n_blocks, page, Lkv + Dr), dtype=np.float32) * sc
    return O.f32_to_bf16(x)
