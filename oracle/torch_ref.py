"""PyTorch (CPU, fp32) restatement of the reference's CPU decode path.

TEST / MEASUREMENT INFRASTRUCTURE ONLY.  Imported by `tests/` (pinned against
the numpy oracle `oracle/locks_oracle.py`) and by `bench.py`'s
`cpu_baseline` leg, which times it on the host cores as the reported CPU
baseline.  Nothing in the product path imports it.

It follows the reference's own torch code paths, op for op where one exists:
  * scorer: `_rki4_score_torch_fp32` (selection/rki4_score_torch.py:111-160):
    int8 round trip of q per (kv head, group) with torch.round, unpack of the
    int4 column-major basis (`_unpack_ibit`, :41-55), dequantised V / C / mu,
    three einsums, logsumexp over the page's tokens; pages at or past
    n_sel_hi are zero;
  * nrm GQA combine: score[p] = sum_g exp(score_h[g, p] - max_{p < nsh} score_h[g])
    (selection/select_cuda.py:547-658 semantics);
  * exact top-b: `_topb_select_torch` (selection/select.py:123-180): the b-th
    largest selectable score by torch.topk, strictly-greater pages plus ties
    at tau lowest page first, sink + window + tail always kept, keep-all when
    the selectable slice has <= 1 page, ascending page table padded with -1;
  * attention: gather of the selected pages' K/V through the block table,
    fp32 softmax over the tokens below seq_len, fp16-rounded P times fp16 V
    accumulated in fp32 (attention/decode.py:209-322 with the split-K merge
    of attention/merge.py:105-152 being exact in real arithmetic, so one
    softmax over all selected tokens).
"""
from __future__ import annotations

import torch


def unpack_i4(vb: torch.Tensor, d: int) -> torch.Tensor:
    """uint8 (..., d/2) -> fp32 (..., d): low nibble -> even d, high -> odd d,
    4-bit two's complement (rki4_score_torch.py:41-55 with IBITS = 4)."""
    v = vb.to(torch.int16)
    out = torch.empty(*vb.shape[:-1], d, dtype=torch.float32)
    out[..., 0::2] = (((v & 0xF) ^ 8) - 8).float()
    out[..., 1::2] = ((((v >> 4) & 0xF) ^ 8) - 8).float()
    return out


def score_rki4(q: torch.Tensor, slabs: dict, bt: torch.Tensor, nsh: torch.Tensor, n_kv: int,
               G: int, scale: float, MP: int) -> torch.Tensor:
    """score_h (R, n_kv, G, MP) fp32.  q (R, n_kv*G, d) bf16; slabs: torch
    tensors v4 u8 (NB,n_kv,8,d/2), vs bf16 (NB,n_kv,8), c8 i8 (NB,n_kv,16,8),
    cs bf16 (NB,n_kv,16), mu8 i8 (NB,n_kv,d), mus bf16 (NB,n_kv)."""
    R, _, d = q.shape
    NB = slabs["v4"].shape[0]
    qv = q[:R].reshape(R, n_kv, G, d).float()
    qs = qv.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 127.0
    qref = torch.round(qv / qs) * qs
    out = torch.zeros(R, n_kv, G, MP, dtype=torch.float32)
    max_hi = int(nsh.max().item()) if R else 0
    if max_hi <= 0:
        return out
    blk = bt[:R, :max_hi].to(torch.int64).clamp(0, NB - 1)
    Vq = unpack_i4(slabs["v4"][blk], d)                                 # (R,P,k,n,d)
    Vref = (Vq * slabs["vs"][blk].float()[..., None]).transpose(-1, -2)  # (R,P,k,d,n)
    Cref = slabs["c8"][blk].float() * slabs["cs"][blk].float()[..., None]
    muref = slabs["mu8"][blk].float() * slabs["mus"][blk].float()[..., None]
    qt = torch.einsum("rpkdn,rkgd->rpkgn", Vref, qref)
    tok = torch.einsum("rpktn,rpkgn->rpkgt", Cref, qt)
    mud = torch.einsum("rpkd,rkgd->rpkg", muref, qref)
    S = torch.logsumexp((tok + mud[..., None]) * float(scale), dim=-1)
    out[:, :, :, :max_hi] = S.permute(0, 2, 3, 1)
    for r in range(R):
        hr = int(nsh[r])
        if hr < max_hi:
            out[r, :, :, max(hr, 0):max_hi] = 0.0
    return out


def combine_nrm(score_h: torch.Tensor, nsh: torch.Tensor) -> torch.Tensor:
    """score (R, n_kv, MP): sum_g exp(score_h - per-head max over [0, nsh))."""
    R, n_kv, G, MP = score_h.shape
    out = torch.zeros(R, n_kv, MP, dtype=torch.float32)
    for r in range(R):
        P = int(nsh[r])
        if P <= 0:
            continue
        sh = score_h[r, :, :, :P]
        hm = sh.amax(-1, keepdim=True)
        out[r, :, :P] = torch.exp(sh - hm).sum(1)
    return out


def topb_select(score: torch.Tensor, npg, nsh, bfix, sink: int, MP: int):
    """(page_table (R, n_kv, MP) i32, page_cnt (R, n_kv) i32), the exact-b
    rule of select.py:123-180."""
    R, n_kv, _ = score.shape
    tab = torch.full((R, n_kv, MP), -1, dtype=torch.int32)
    cnt = torch.zeros(R, n_kv, dtype=torch.int32)
    idx = torch.arange(MP, dtype=torch.int32)
    for r in range(R):
        n, hi_, b = int(npg[r]), int(nsh[r]), int(bfix[r])
        keep = torch.zeros(n_kv, MP, dtype=torch.bool)
        lo = min(sink, max(n, 0))
        hi = max(min(hi_, n), lo)
        L = hi - lo
        if L <= 1:
            if n > 0:
                keep[:, :n] = True
        else:
            if lo > 0:
                keep[:, :lo] = True
            if hi < n:
                keep[:, hi:n] = True
            sel = score[r, :, lo:hi]
            if b >= L:
                keep[:, lo:hi] = True
            else:
                tau = torch.topk(sel, b, dim=-1, largest=True, sorted=True).values[:, -1]
                gt = sel > tau[:, None]
                quota = (b - gt.sum(-1)).clamp_min(0)
                eq = sel == tau[:, None]
                eqrank = eq.to(torch.int32).cumsum(-1)
                keep[:, lo:hi] = gt | (eq & (eqrank <= quota[:, None]))
        keep[:, max(n, 0):] = False
        for kh in range(n_kv):
            kept = idx[keep[kh]]
            tab[r, kh, :kept.numel()] = kept
            cnt[r, kh] = kept.numel()
    return tab, cnt


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     bt: torch.Tensor, seq_lens, page_table: torch.Tensor,
                     page_cnt: torch.Tensor, G: int, scale: float) -> torch.Tensor:
    """out (R, n_kv*G, d) fp32 over the selected pages.  k/v_cache (NB, page,
    n_kv, d) bf16; masked tokens are those at or past seq_len."""
    R, H, d = q.shape
    NB, page, n_kv, _ = k_cache.shape
    out = torch.zeros(R, H, d, dtype=torch.float32)
    for r in range(R):
        sl = int(seq_lens[r])
        for kh in range(n_kv):
            c = int(page_cnt[r, kh])
            if c <= 0:
                continue
            pages = page_table[r, kh, :c].to(torch.int64)
            blk = bt[r, pages].to(torch.int64).clamp(0, NB - 1)
            K = k_cache[blk, :, kh, :].float().reshape(-1, d)                # (c*page, d)
            V = v_cache[blk, :, kh, :].float().reshape(-1, d)
            pos = (pages[:, None] * page + torch.arange(page)[None, :]).reshape(-1)
            qg = q[r, kh * G:(kh + 1) * G].float()                            # (G, d)
            s = (qg @ K.T) * float(scale)
            s = s.masked_fill((pos >= sl)[None, :], float("-inf"))
            m = s.amax(-1, keepdim=True)
            p = torch.exp(s - m)
            l = p.sum(-1, keepdim=True)
            o = p.half().float() @ V.half().float()
            out[r, kh * G:(kh + 1) * G] = o / l
    return out
