"""CPU oracle for the LOCKS sparse-decode hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``locks`` package + ``liblocks_hip.so``) never
routes through it and raises if the HIP library is missing.

It restates, in numpy, the reference's algorithm for each stage of the path
(paths relative to the reference package ``src/locks/``):

  pack_i4 / unpack_i4      selection/rki4_build.py:161-175 (_pack_ibit) and
                           selection/rki4_score_torch.py:41-55 (_unpack_ibit)
  summary_pre              selection/rki4_build.py:147-158 (_write_pre)
  summary_eigh             selection/rki4_build.py:93-129  (_eigh_chunked;
                           third-party LAPACK eigh -> "parity unpinned" at the
                           eigen boundary, gated by reconstruction instead)
  summary_post             selection/rki4_build.py:178-225 (_write_post)
  score_rki4_twin          selection/rki4_score_torch.py:111-160 (fp32 twin)
  score_rki4_intpath       selection/rki4_score_cuda.py:436-466,648-722 (the
                           integer-dot op order of the deployed CUDA kernel)
  derive_page_params       selection/select.py:28-58
  combine_nrm/combine_max  selection/select_cuda.py:547-658 ("nrm"),
                           selection/rki4_score_cuda.py:3494-3497 ("max")
  topb_select              selection/select.py:123-180 (exact-b torch twin)
  decode_attention         attention/decode.py:209-322 + attention/merge.py:
                           105-152 (split-K online softmax + LSE merge,
                           restated as one fp32 softmax per (req, head))

Every function works on host numpy arrays.  bf16 values are carried as their
raw uint16 bit patterns (``bf16_to_f32`` / ``f32_to_bf16``) so byte-level
checks are exact.

Pinning: every function here is checked by ``tests/test_oracle_*.py`` against
closed forms, brute force in float64 or an independent formulation; see the
test files for which check pins which function.  ``summary_eigh`` is the one
third-party boundary (LAPACK); its output is pinned by the eigen identity
``G U = U diag(S2)`` and the reconstruction identity, not bit-for-bit.
"""
from __future__ import annotations

import math

import numpy as np

IBITS = 4
RNK = 8
QMAX = (1 << (IBITS - 1)) - 1      # 7
QMIN = -(1 << (IBITS - 1))         # -8
TAGW = 8


# --------------------------------------------------------------------------- #
# bf16 helpers (round-to-nearest-even, the rounding torch's .to(bfloat16) uses)
# --------------------------------------------------------------------------- #
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round-to-nearest-even; NaN kept."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> fp32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 value, returned as fp32."""
    return bf16_to_f32(f32_to_bf16(x))


# --------------------------------------------------------------------------- #
# int4 column-major pack / unpack (rki4_build.py:161-175, rki4_score_torch.py:41-55)
# --------------------------------------------------------------------------- #
def pack_i4(vc: np.ndarray) -> np.ndarray:
    """int8 (..., d) with values in [-8, 7] -> uint8 (..., d/2).
    byte k = (v[2k] & 0xF) | ((v[2k+1] & 0xF) << 4): low nibble = even d."""
    v = np.asarray(vc).astype(np.int16)
    lo = (v[..., 0::2] & 0xF).astype(np.uint8)
    hi = (v[..., 1::2] & 0xF).astype(np.uint8)
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_i4(vb: np.ndarray) -> np.ndarray:
    """uint8 (..., d/2) -> int8 (..., d): two's-complement nibble extension
    ((n ^ 8) - 8), even d from the low nibble."""
    b = np.asarray(vb).astype(np.int16)
    lo = ((b & 0xF) ^ 8) - 8
    hi = (((b >> 4) & 0xF) ^ 8) - 8
    out = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


# --------------------------------------------------------------------------- #
# summary build (rki4_build.py:147-225)
# --------------------------------------------------------------------------- #
def summary_pre(kp_bf16: np.ndarray):
    """_write_pre (rki4_build.py:147-158).

    kp_bf16: (N, page, n_kv, d) bf16 bit patterns (one finalized page each).
    Returns (tag bf16 (N, n_kv, TAGW), mu (N, n_kv, d) f32,
             dc (N, n_kv, page, d) f32, gram (N, n_kv, page, page) f32).
    The mean and gram sums run sequentially over the token / d axis in fp32
    (the order the HIP build kernel uses)."""
    page = kp_bf16.shape[1]
    tag = np.ascontiguousarray(kp_bf16[:, page - 1, :, :TAGW])
    K = bf16_to_f32(kp_bf16).transpose(0, 2, 1, 3)          # (N, n_kv, page, d)
    acc = np.zeros(K.shape[:2] + (K.shape[3],), np.float32)
    for t in range(page):
        acc = (acc + K[:, :, t, :]).astype(np.float32)
    mu = (acc / np.float32(page)).astype(np.float32)
    dc = (K - mu[:, :, None, :]).astype(np.float32)
    gram = np.einsum("nktd,nksd->nkts", dc.astype(np.float64),
                     dc.astype(np.float64)).astype(np.float32)
    return tag, mu, dc, gram


def summary_eigh(gram: np.ndarray):
    """Batched symmetric eigh, eigenvalues ascending (third-party LAPACK;
    the reference calls torch.linalg.eigh, rki4_build.py:115-122)."""
    S2, U = np.linalg.eigh(gram.astype(np.float32))
    return S2.astype(np.float32), U.astype(np.float32)


def summary_post(mu: np.ndarray, dc: np.ndarray, S2: np.ndarray, U: np.ndarray):
    """_write_post (rki4_build.py:178-225): eigenpairs -> quantized, packed slabs.

    mu (N, n_kv, d), dc (N, n_kv, page, d), S2 (N, n_kv, page), U (N, n_kv,
    page, page), all fp32.  Reductions that feed bytes (V = dc^T U8 / S8) are
    evaluated as a sequential fp32 sum over the page axis with separately
    rounded multiply and add, the order the HIP pack kernel reproduces.

    Returns dict of v4 (N,n_kv,RNK,d/2) u8, vs (N,n_kv,RNK) bf16 bits,
    c8 (N,n_kv,page,RNK) i8, cs (N,n_kv,page) bf16 bits, mu8 (N,n_kv,d) i8,
    mus (N,n_kv) bf16 bits."""
    f32 = np.float32
    page = dc.shape[2]
    S8 = np.sqrt(np.maximum(S2[..., -RNK:], f32(1e-10))).astype(f32)   # (N,k,R)
    U8 = U[..., -RNK:].astype(f32)                                      # (N,k,page,R)
    C = (U8 * S8[..., None, :]).astype(f32)                             # (N,k,page,R)
    V = np.zeros(dc.shape[:2] + (dc.shape[3], RNK), f32)                # (N,k,d,R)
    for t in range(page):
        V = (V + (dc[:, :, t, :, None] * U8[:, :, t, None, :]).astype(f32)).astype(f32)
    V = (V / S8[:, :, None, :]).astype(f32)
    vsc = np.maximum((np.abs(V).max(axis=2) / f32(QMAX)).astype(f32), f32(1e-8))
    Vq = np.clip(np.rint(V / vsc[:, :, None, :]), QMIN, QMAX)
    Vc = np.ascontiguousarray(Vq.transpose(0, 1, 3, 2)).astype(np.int8)  # (N,k,R,d)
    v4 = pack_i4(Vc)
    csc = np.maximum((np.abs(C).max(axis=-1) / f32(127.0)).astype(f32), f32(1e-8))
    Cq = np.clip(np.rint(C / csc[..., None]), -127, 127).astype(np.int8)
    msc = np.maximum((np.abs(mu).max(axis=-1) / f32(127.0)).astype(f32), f32(1e-8))
    muq = np.clip(np.rint(mu / msc[..., None]), -127, 127).astype(np.int8)
    return dict(v4=v4, vs=f32_to_bf16(vsc), c8=Cq, cs=f32_to_bf16(csc),
                mu8=muq, mus=f32_to_bf16(msc))


def build_summaries(kp_bf16: np.ndarray):
    """Full build for N pages: pre -> eigh -> post (+ the content tag)."""
    tag, mu, dc, gram = summary_pre(kp_bf16)
    S2, U = summary_eigh(gram)
    out = summary_post(mu, dc, S2, U)
    out["tag"] = tag
    return out


def build_state_slabs(k_cache_bf16: np.ndarray, blocks: np.ndarray, n_blocks: int):
    """Build six-slab summaries (rki4_state.py:7-16 layout, one layer) for the
    physical blocks ``blocks`` of a K cache (NB, page, n_kv, d) bf16 bits.
    Unbuilt blocks stay zero (the reference zero-inits the slabs)."""
    NB, page, n_kv, d = k_cache_bf16.shape
    slabs = dict(
        v4=np.zeros((n_blocks, n_kv, RNK, d // 2), np.uint8),
        vs=np.zeros((n_blocks, n_kv, RNK), np.uint16),
        c8=np.zeros((n_blocks, n_kv, page, RNK), np.int8),
        cs=np.zeros((n_blocks, n_kv, page), np.uint16),
        mu8=np.zeros((n_blocks, n_kv, d), np.int8),
        mus=np.zeros((n_blocks, n_kv), np.uint16),
    )
    blocks = np.asarray(blocks, np.int64)
    if blocks.size:
        s = build_summaries(k_cache_bf16[blocks])
        for k in slabs:
            slabs[k][blocks] = s[k]
    return slabs


# --------------------------------------------------------------------------- #
# scorer (rki4_score_torch.py:111-160 and rki4_score_cuda.py:436-466,648-722)
# --------------------------------------------------------------------------- #
def quantize_q(q_bf16: np.ndarray):
    """Per-(req, head) int8 round trip of q (rki4_score_torch.py:138-140;
    kernel rki4_score_cuda.py:440-466).  q (..., d) bf16 bits.
    Returns (q8 int8 (..., d), qs fp32 (...,))."""
    qv = bf16_to_f32(q_bf16)
    qs = (np.maximum(np.abs(qv).max(axis=-1), np.float32(1e-8))
          / np.float32(127.0)).astype(np.float32)
    q8 = np.rint(qv / qs[..., None]).astype(np.int32)
    return q8.astype(np.int8), qs


def score_rki4_twin(q_bf16, slabs, bt, nsh, n_kv, G, sm_scale, MP):
    """fp32 torch-twin restatement (rki4_score_torch.py:111-160).

    q_bf16 (R, n_kv*G, d) bf16 bits; slabs: one layer's six slabs indexed by
    physical block; bt (R, MB) int32 logical page -> block; nsh (R,) n_sel_hi.
    Returns score_h (R, n_kv, G, MP) fp32, zero outside [0, nsh[r])."""
    R = q_bf16.shape[0]
    d = q_bf16.shape[-1]
    NB = slabs["v4"].shape[0]
    q8, qs = quantize_q(q_bf16[:R].reshape(R, n_kv, G, d))
    qref = (q8.astype(np.float32) * qs[..., None]).astype(np.float32)
    out = np.zeros((R, n_kv, G, MP), np.float32)
    s = np.float32(sm_scale)
    for r in range(R):
        P = int(nsh[r])
        if P <= 0:
            continue
        blk = np.clip(bt[r, :P].astype(np.int64), 0, NB - 1)
        Vq = unpack_i4(slabs["v4"][blk]).astype(np.float32)           # (P,k,R,d)
        vsb = bf16_to_f32(slabs["vs"][blk])                           # (P,k,R)
        Vref = (Vq * vsb[..., None]).astype(np.float32)
        Cref = (slabs["c8"][blk].astype(np.float32)
                * bf16_to_f32(slabs["cs"][blk])[..., None]).astype(np.float32)
        muref = (slabs["mu8"][blk].astype(np.float32)
                 * bf16_to_f32(slabs["mus"][blk])[..., None]).astype(np.float32)
        qt = np.einsum("pknd,kgd->pkgn", Vref, qref[r]).astype(np.float32)
        tok = np.einsum("pktn,pkgn->pkgt", Cref, qt).astype(np.float32)
        mud = np.einsum("pkd,kgd->pkg", muref, qref[r]).astype(np.float32)
        x = ((tok + mud[..., None]) * s).astype(np.float32)
        m = x.max(axis=-1)
        S = (m + np.log(np.exp(x - m[..., None]).sum(axis=-1))).astype(np.float32)
        out[r, :, :, :P] = S.transpose(1, 2, 0)
    return out


def score_rki4_intpath(q_bf16, slabs, bt, nsh, n_kv, G, sm_scale, MP,
                       dtype=np.float32):
    """Integer-dot formulation of the same score, in the op order of the
    deployed kernel (rki4_score_cuda.py:653-722): exact int32 V.q8 and mu.q8
    dots, then qt = acci*qs*vs, mud = mui*qs*mus, tok = s*(cs*sum_j c8*qt + mud),
    LSE over the page's tokens.  dtype=float64 gives the exact-arithmetic
    value used to pin both this and the twin."""
    R = q_bf16.shape[0]
    d = q_bf16.shape[-1]
    NB = slabs["v4"].shape[0]
    q8, qs = quantize_q(q_bf16[:R].reshape(R, n_kv, G, d))
    out = np.zeros((R, n_kv, G, MP), np.float32)
    for r in range(R):
        P = int(nsh[r])
        if P <= 0:
            continue
        blk = np.clip(bt[r, :P].astype(np.int64), 0, NB - 1)
        Vq = unpack_i4(slabs["v4"][blk]).astype(np.int64)              # (P,k,R,d)
        acci = np.einsum("pknd,kgd->pkgn", Vq, q8[r].astype(np.int64))
        mui = np.einsum("pkd,kgd->pkg", slabs["mu8"][blk].astype(np.int64),
                        q8[r].astype(np.int64))
        qsr = qs[r].astype(dtype)                                      # (k,g)
        vs = bf16_to_f32(slabs["vs"][blk]).astype(dtype)               # (P,k,R)
        qt = acci.astype(dtype) * qsr[None, :, :, None] * vs[:, :, None, :]
        mud = (mui.astype(dtype) * qsr[None]
               * bf16_to_f32(slabs["mus"][blk]).astype(dtype)[:, :, None])
        c8 = slabs["c8"][blk].astype(dtype)                            # (P,k,t,R)
        cs = bf16_to_f32(slabs["cs"][blk]).astype(dtype)               # (P,k,t)
        dt = np.einsum("pktn,pkgn->pkgt", c8, qt)
        tok = dtype(sm_scale) * (dt * cs[:, :, None, :] + mud[..., None])
        m = tok.max(axis=-1)
        S = m + np.log(np.exp(tok - m[..., None]).sum(axis=-1))
        out[r, :, :, :P] = S.astype(np.float32).transpose(1, 2, 0)
    return out


# --------------------------------------------------------------------------- #
# selection (select.py:28-58, select_cuda.py:547-658, select.py:123-180)
# --------------------------------------------------------------------------- #
def derive_page_params(seq_lens, page, window, sink, budget_abs=0, budget=0.1):
    """select.py:28-58.  Returns (n_pages, n_sel_hi, b) int32 arrays."""
    sl = np.asarray(seq_lens, np.int64)
    npg = (sl + page - 1) // page
    nsh = npg - window
    s = nsh - sink
    if budget_abs > 0:
        b = np.maximum(np.minimum(budget_abs, np.maximum(s, 1)), 1)
    else:
        bf = np.ceil(s.astype(np.float64) * float(budget))
        b = np.minimum(np.maximum(bf.astype(np.int64), 1), np.maximum(s, 1))
    return npg.astype(np.int32), nsh.astype(np.int32), b.astype(np.int32)


def combine_nrm(score_h, nsh):
    """GQA "nrm" combine (select_cuda.py:547-658): per (r, kh)
    hm[g] = max_{0<=p<nsh} score_h[g,p];
    score[p] = sum_{g ascending} exp(score_h[g,p] - hm[g])  for p < nsh.
    Entries at p >= nsh are left 0 (never consumed)."""
    R, n_kv, G, MP = score_h.shape
    out = np.zeros((R, n_kv, MP), np.float32)
    for r in range(R):
        P = int(nsh[r])
        if P <= 0:
            continue
        sh = score_h[r, :, :, :P]
        hm = sh.max(axis=-1)                                           # (k,g)
        acc = np.zeros((n_kv, P), np.float32)
        for g in range(G):
            acc = (acc + np.exp((sh[:, g] - hm[:, g, None]).astype(np.float32))
                   .astype(np.float32)).astype(np.float32)
        out[r, :, :P] = acc
    return out


def combine_max(score_h, nsh):
    """GQA "max" combine (rki4_score_cuda.py:3494-3497: amax over g)."""
    R, n_kv, G, MP = score_h.shape
    out = np.zeros((R, n_kv, MP), np.float32)
    for r in range(R):
        P = int(nsh[r])
        if P > 0:
            out[r, :, :P] = score_h[r, :, :, :P].max(axis=1)
    return out


def topb_select(score, npg, nsh, bfix, sink, MP):
    """Exact-b top-b (select.py:123-180 semantics; also the CUDA kernel's
    count-and-demote rule select_cuda.py:729-752).

    tau  = b-th largest score over the selectable slice [sink, nsh)
    keep = {> tau} U {== tau, lowest page index first, up to b total}
           U [0, sink) U [nsh, npg);  (nsh - sink) <= 1 -> keep [0, npg).
    Returns page_table (R, n_kv, MP) int32 ascending, -1 padded, and
    page_cnt (R, n_kv) int32."""
    R, n_kv = score.shape[0], score.shape[1]
    table = np.full((R, n_kv, MP), -1, np.int32)
    cnt = np.zeros((R, n_kv), np.int32)
    for r in range(R):
        n_pages, n_sel_hi, b = int(npg[r]), int(nsh[r]), int(bfix[r])
        lo = min(sink, max(n_pages, 0))
        hi = max(min(n_sel_hi, n_pages), lo)
        L = hi - lo
        for kh in range(n_kv):
            keep = np.zeros(max(n_pages, 0), bool)
            if L <= 1:
                keep[:] = True
            else:
                keep[:lo] = True
                keep[hi:n_pages] = True
                sel = score[r, kh, lo:hi]
                if b >= L:
                    keep[lo:hi] = True
                else:
                    tau = np.sort(sel)[::-1][b - 1]
                    gt = sel > tau
                    quota = max(b - int(gt.sum()), 0)
                    eq = sel == tau
                    eqrank = np.cumsum(eq)
                    keep[lo:hi] = gt | (eq & (eqrank <= quota))
            idx = np.nonzero(keep)[0].astype(np.int32)
            cnt[r, kh] = idx.size
            table[r, kh, :idx.size] = idx
    return table, cnt


# --------------------------------------------------------------------------- #
# sparse paged decode + LSE merge (decode.py:209-322, merge.py:105-152)
# --------------------------------------------------------------------------- #
def decode_attention(q_bf16, k_cache_bf16, v_cache_bf16, bt, seq_lens,
                     page_table, page_cnt, G, sm_scale, dtype=np.float32):
    """Attention of each (req, query head) over the tokens of its kv-head's
    selected pages: token t of logical page pt is attended iff
    pt*page + t < seq_len.  One fp32 softmax per (req, head) -- the value the
    split-K partials + LSE merge compute up to fp summation order.

    q (R, H, d) bf16 bits; k/v caches (NB, page, n_kv, d) bf16 bits.
    Returns out (R, H, d) in ``dtype`` and lse (R, H); rows with page_cnt 0
    give 0 (merge.py:141-150)."""
    R, H, d = q_bf16.shape
    NB, page, n_kv, _ = k_cache_bf16.shape
    out = np.zeros((R, H, d), dtype)
    lse = np.full((R, H), -np.inf, dtype)
    for r in range(R):
        for kh in range(n_kv):
            c = int(page_cnt[r, kh])
            if c <= 0:
                continue
            pts = page_table[r, kh, :c].astype(np.int64)
            blks = bt[r, pts].astype(np.int64)
            pos = (pts[:, None] * page + np.arange(page)[None, :]).reshape(-1)
            valid = pos < int(seq_lens[r])
            if not valid.any():
                continue
            K = bf16_to_f32(k_cache_bf16[blks, :, kh, :]).reshape(-1, d)[valid]
            V = bf16_to_f32(v_cache_bf16[blks, :, kh, :]).reshape(-1, d)[valid]
            qh = bf16_to_f32(q_bf16[r, kh * G:(kh + 1) * G, :])
            s = (qh.astype(dtype) @ K.T.astype(dtype)) * dtype(sm_scale)
            m = s.max(axis=-1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=-1, keepdims=True)
            out[r, kh * G:(kh + 1) * G] = (p @ V.astype(dtype)) / l
            lse[r, kh * G:(kh + 1) * G] = (m + np.log(l))[:, 0]
    return out, lse


def merge_partials(m_part, l_part, acc_part, page_cnt, split, pps_min):
    """LSE merge of split-K partials (merge.py:105-152).  m/l (R,n_kv,split,G),
    acc (R,n_kv,split,G,D) fp32.  Only the first n_act = cdiv(cnt, pps) splits
    are read, pps = max(cdiv(cnt, split), pps_min)."""
    R, n_kv, S, G = m_part.shape
    D = acc_part.shape[-1]
    out = np.zeros((R, n_kv * G, D), np.float32)
    for r in range(R):
        for kh in range(n_kv):
            cnt = int(page_cnt[r, kh])
            pps = max(-(-cnt // split), pps_min)
            n_act = -(-cnt // pps) if cnt > 0 else 0
            if n_act == 0:
                continue
            m = m_part[r, kh, :n_act]
            l = l_part[r, kh, :n_act]
            acc = acc_part[r, kh, :n_act]
            mx = m.max(axis=0)
            w = np.where(l > 0, np.exp(m - mx[None]), 0.0).astype(np.float32)
            lt = (l * w).sum(axis=0)
            o = (acc * w[..., None]).sum(axis=0)
            o = np.where(lt[:, None] > 0, o / np.where(lt > 0, lt, 1)[:, None], 0.0)
            out[r, kh * G:(kh + 1) * G] = o
    return out


# --------------------------------------------------------------------------- #
# synthetic inputs (the BASELINE input distribution)
# --------------------------------------------------------------------------- #
def synth_kv(rng: np.random.Generator, n_blocks, page, n_kv, d, n_outlier=4,
             outlier_scale=8.0):
    """K/V ~ N(0,1) with ``n_outlier`` fixed channels per kv head scaled x8,
    returned as bf16 bit patterns (NB, page, n_kv, d)."""
    ch = np.stack([rng.choice(d, n_outlier, replace=False) for _ in range(n_kv)])
    scale = np.ones((n_kv, d), np.float32)
    for h in range(n_kv):
        scale[h, ch[h]] = outlier_scale
    K = rng.standard_normal((n_blocks, page, n_kv, d), dtype=np.float32) * scale
    V = rng.standard_normal((n_blocks, page, n_kv, d), dtype=np.float32) * scale
    return f32_to_bf16(K), f32_to_bf16(V), ch


def synth_block_table(rng: np.random.Generator, seq_lens, page, pool_blocks, MB):
    """Per-request block tables drawn as disjoint slices of ONE shuffled pool."""
    perm = rng.permutation(pool_blocks).astype(np.int32)
    R = len(seq_lens)
    bt = np.zeros((R, MB), np.int32)
    off = 0
    for r, sl in enumerate(seq_lens):
        n = (int(sl) + page - 1) // page
        assert off + n <= pool_blocks, "page pool too small"
        bt[r, :n] = perm[off:off + n]
        off += n
    return bt


def cdiv(a, b):
    return -(-a // b)


def next_pow2(x: int) -> int:
    return 1 if x <= 1 else 1 << (int(x) - 1).bit_length()


def log_sum_exp(x):
    m = max(x)
    return m + math.log(sum(math.exp(v - m) for v in x))
