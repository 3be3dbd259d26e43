"""rki4 summary build (off the hot path): finalized K pages -> six slabs.

Op sequence of the reference builder (src/locks/selection/rki4_build.py:
147-158 _write_pre, :93-129 chunked eigh, :178-225 _write_post, :161-175
int4 pack), per (block, kv head):
    mu = mean_t K; dc = K - mu; Gm = dc dc^T (page x page)
    S2, U = eigh(Gm) (ascending); S8 = sqrt(max(S2[-8:], 1e-10)); U8 = U[:, -8:]
    C = U8 * S8; V = dc^T U8 / S8
    vs = max(|V|_d / 7, 1e-8); Vq = clamp(round(V / vs), -8, 7)   (int4, packed)
    cs = max(|C|_r / 127, 1e-8); Cq = clamp(round(C / cs), +-127)  (int8)
    ms = max(|mu| / 127, 1e-8);  muq = clamp(round(mu / ms), +-127) (int8)
Scales are stored as bf16; the tag is K[page-1, :, :8].
Runs with torch on the state's device (eigh: rocSOLVER on ROCm), chunked.
"""
from __future__ import annotations

import torch

from .rki4_state import QMAX, QMIN, RNK

EIGH_CHUNK = 8192


def pack_i4(vc: torch.Tensor) -> torch.Tensor:
    """int8 (..., d) in [-8, 7] -> uint8 (..., d/2), low nibble = even d."""
    lo = (vc[..., 0::2] & 0xF).to(torch.uint8)
    hi = (vc[..., 1::2] & 0xF).to(torch.uint8)
    return (lo | (hi << 4)).contiguous()


def _eigh_chunked(Gf: torch.Tensor):
    n = Gf.shape[-1]
    S2 = torch.empty(Gf.shape[0], n, device=Gf.device, dtype=torch.float32)
    U = torch.empty_like(Gf)
    for i in range(0, Gf.shape[0], EIGH_CHUNK):
        S2[i:i + EIGH_CHUNK], U[i:i + EIGH_CHUNK] = torch.linalg.eigh(Gf[i:i + EIGH_CHUNK])
    return S2, U


def summarize_pages(kp: torch.Tensor):
    """kp (N, page, n_kv, d) bf16 -> dict of slab tensors for those N blocks."""
    N, page, n_kv, d = kp.shape
    tag = kp[:, page - 1, :, :8]
    K = kp.permute(0, 2, 1, 3).float().contiguous()          # (N, n_kv, page, d)
    mu = K.mean(2)
    dc = K - mu[:, :, None]
    Gm = dc @ dc.transpose(-1, -2)
    S2, U = _eigh_chunked(Gm.reshape(-1, page, page))
    S2 = S2.reshape(N, n_kv, page)
    U = U.reshape(N, n_kv, page, page)
    S8 = S2[..., -RNK:].clamp_min(1e-10).sqrt()
    U8 = U[..., -RNK:]
    C = U8 * S8[..., None, :]
    V = dc.transpose(-1, -2) @ U8 / S8[..., None, :]
    vsc = (V.abs().amax(2) / float(QMAX)).clamp_min(1e-8)
    Vq = torch.round(V / vsc[:, :, None]).clamp(QMIN, QMAX)
    v4 = pack_i4(Vq.permute(0, 1, 3, 2).contiguous().to(torch.int8))
    csc = (C.abs().amax(-1) / 127.0).clamp_min(1e-8)
    Cq = torch.round(C / csc[..., None]).clamp(-127, 127)
    msc = (mu.abs().amax(-1) / 127.0).clamp_min(1e-8)
    muq = torch.round(mu / msc[..., None]).clamp(-127, 127)
    return dict(v4=v4, vs=vsc.to(torch.bfloat16), c8=Cq.to(torch.int8),
                cs=csc.to(torch.bfloat16), mu8=muq.to(torch.int8),
                mus=msc.to(torch.bfloat16), tag=tag.to(torch.bfloat16))


@torch.no_grad()
def rki4_build_blocks(st, layer: int, K: torch.Tensor, blocks: torch.Tensor,
                      chunk: int = 8192) -> int:
    """(Re)build the summaries of physical ``blocks`` of one layer from the K
    half ``K`` (NB, page, n_kv, d).  Out-of-range block ids are dropped
    (rki4_build.py:133-144)."""
    nb = min(int(st.NB), int(K.shape[0]))
    blocks = blocks.to(device=K.device, dtype=torch.int64)
    blocks = blocks[(blocks >= 0) & (blocks < nb)]
    n = int(blocks.numel())
    for i in range(0, n, chunk):
        b = blocks[i:i + chunk]
        s = summarize_pages(K[b])
        st.pp_v4[layer, b] = s["v4"]
        st.pp_vs[layer, b] = s["vs"]
        st.pp_c8[layer, b] = s["c8"]
        st.pp_cs[layer, b] = s["cs"]
        st.pp_mu8[layer, b] = s["mu8"]
        st.pp_mus[layer, b] = s["mus"]
        st.pp_tag[layer, b] = s["tag"]
    return n


@torch.no_grad()
def rki4_build_refresh(st, layer: int, K: torch.Tensor, block_table: torch.Tensor,
                       seq_lens: torch.Tensor, n_req: int, *, force: bool = False) -> int:
    """Rebuild every stale FINALIZED page of the batch (rki4_build.py:318-364):
    a page is stale when its content tag (first 8 channels of the page's last
    key) differs from the stored tag (NaN-initialised -> always stale)."""
    if n_req == 0:
        return 0
    page, tagw = st.page, st.tagw
    sl = seq_lens[:n_req].to(torch.int64)
    n_fin = sl // page
    max_fin = int(n_fin.max().item())
    if max_fin == 0:
        return 0
    pidx = torch.arange(max_fin, device=K.device)
    fin = pidx[None, :] < n_fin[:, None]
    blocks = block_table[:n_req, :max_fin].to(torch.int64)[fin]
    nb = min(int(st.NB), int(K.shape[0]))
    blocks = blocks[(blocks >= 0) & (blocks < nb)]
    if blocks.numel() == 0:
        return 0
    if not force:
        cur = K[blocks, page - 1, :, :tagw].float()
        old = st.pp_tag[layer, blocks].float()
        blocks = blocks[(cur != old).any(dim=(1, 2))]
    sb = torch.unique(blocks)
    if sb.numel() == 0:
        return 0
    return rki4_build_blocks(st, layer, K, sb)
