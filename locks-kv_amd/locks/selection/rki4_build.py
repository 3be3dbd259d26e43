"""rki4 summary build (off the hot path): finalized K pages -> six slabs.

Runs on the GPU through ``locks_build_rki4`` (gram on the matrix core,
16x16 parallel Jacobi eigensolver, quantize/pack), following the reference
builder's op sequence (src/locks/selection/rki4_build.py:147-158 _write_pre,
:93-129 eigh, :178-225 _write_post, :161-175 int4 pack).  The lifecycle
entry ``rki4_build_refresh`` mirrors rki4_build.py:318-364 (content-tag
staleness); ``rki4_pack`` exposes the quantize/pack half for callers that
bring their own eigen decomposition.
"""
from __future__ import annotations

import torch

from .. import _lib


def _slabs(st, layer):
    return (st.pp_v4[layer], st.pp_vs[layer], st.pp_c8[layer], st.pp_cs[layer],
            st.pp_mu8[layer], st.pp_mus[layer], st.pp_tag[layer])


@torch.no_grad()
def rki4_build_blocks(st, layer: int, K: torch.Tensor, blocks: torch.Tensor) -> int:
    """(Re)build the summaries of physical ``blocks`` of one layer from the K
    half ``K`` (NB, page, n_kv, d) view.  Ids outside [0, NB) are skipped."""
    if K.dtype != torch.bfloat16 or K.stride(-1) != 1:
        raise TypeError("K must be bf16 with a contiguous head dim")
    b = blocks.to(device=K.device, dtype=torch.int32).contiguous()
    n = int(b.numel())
    if n == 0:
        return 0
    v4, vs, c8, cs, mu8, mus, tag = _slabs(st, layer)
    nb = min(int(st.NB), int(K.shape[0]))
    lib = _lib.load()
    _lib.check(lib.locks_build_rki4(
        _lib.ptr(K), K.stride(0), K.stride(1), K.stride(2), nb, _lib.ptr(b), n, int(st.n_kv),
        int(st.d), int(st.page), _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8), _lib.ptr(cs),
        _lib.ptr(mu8), _lib.ptr(mus), _lib.ptr(tag), _lib.stream_ptr(K.device)), "build_rki4")
    return n


@torch.no_grad()
def rki4_pack(st, layer: int, mu, dc, S2, U, rows) -> None:
    """Quantize + pack from a given eigen decomposition (fp32 device tensors
    mu (n, d), dc (n, page, d), S2 (n, page) ascending, U (n, page, page);
    rows (n,) int32 = block * n_kv + kv head)."""
    v4, vs, c8, cs, mu8, mus, _ = _slabs(st, layer)
    ts = [t.contiguous() for t in (mu, dc, S2, U)]
    rows = rows.to(torch.int32).contiguous()
    lib = _lib.load()
    _lib.check(lib.locks_pack_rki4(
        *[_lib.ptr(t) for t in ts], _lib.ptr(rows), int(rows.numel()), int(st.d), int(st.page),
        _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8), _lib.ptr(cs), _lib.ptr(mu8), _lib.ptr(mus),
        _lib.stream_ptr(rows.device)), "pack_rki4")


@torch.no_grad()
def rki4_build_refresh(st, layer: int, K: torch.Tensor, block_table: torch.Tensor,
                       seq_lens: torch.Tensor, n_req: int, *, force: bool = False) -> int:
    """Rebuild every stale FINALIZED page of the batch: a page is stale when
    its content tag (first 8 channels of the page's last key) differs from
    the stored tag (NaN-initialised -> always stale).  Host-side gather of
    the finalized block list (not graph-safe, like the reference)."""
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
