"""rki4 summary build (off the hot path): finalized K pages -> six slabs.

Runs on the GPU through ``locks_build_rki4`` (gram on the matrix core,
page x page parallel Jacobi eigensolver, quantize/pack), following the reference
builder's op sequence (src/locks/selection/rki4_build.py:147-158 _write_pre,
:93-129 eigh, :178-225 _write_post, :161-175 int4 pack).  The lifecycle
entry ``rki4_build_refresh`` mirrors rki4_build.py:318-364 (content-tag
staleness, one layer); the batched all-layer producers ``rki4_build_tail``,
``rki4_build_bulk`` and ``rki4_build_delta`` (rki4_build.py:264-315) pick
their blocks on the device (``locks_refresh_blocks``) and build every layer
in one launch (``locks_build_rki4_layers``) with no host sync, except the
delta's returned count; ``rki4_pack`` exposes the quantize/pack half for
callers that bring their own eigen decomposition.
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
        _lib.ptr(mu8), _lib.ptr(mus), _lib.rows_arg(st), _lib.ptr(tag), _lib.stream_ptr(K.device)),
        "build_rki4")
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
        _lib.rows_arg(st), _lib.stream_ptr(rows.device)), "pack_rki4")


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


# ---- batched all-layer refresh (rki4_build.py:264-315) ----------------------
_MODE = {"tail": 0, "bulk": 1, "delta": 2}


def _k_layers(st, K_layers):
    """Device array of the per-layer K base addresses (cached on the state:
    the engine's KV tensors do not move) and their common geometry."""
    if len(K_layers) != st.L:
        raise ValueError(f"K_layers has {len(K_layers)} layers, state has {st.L}")
    K0 = K_layers[0]
    for K in K_layers:
        if (K.dtype != torch.bfloat16 or K.stride() != K0.stride() or K.shape != K0.shape
                or K.device != K0.device or K.stride(-1) != 1):
            raise TypeError("K_layers must be bf16 views of one shape and stride "
                            "with a contiguous head dim")
    key = tuple(int(K.data_ptr()) for K in K_layers)
    if getattr(st, "_k_layers_key", None) != key:
        st._k_layers_dev = torch.tensor(key, dtype=torch.int64).to(K0.device)
        st._k_layers_key = key
    if getattr(st, "refresh_mark", None) is None:
        st.refresh_mark = torch.zeros(st.NB, device=K0.device, dtype=torch.uint8)
        st.refresh_blocks = torch.zeros(st.NB, device=K0.device, dtype=torch.int32)
        st.refresh_count = torch.zeros(1, device=K0.device, dtype=torch.int32)
    return st._k_layers_dev, K0


def _refresh(st, mode: str, K_layers, block_table, seq_lens, n_req: int, rows=None,
             max_fin: int = 0) -> int:
    """Pick the blocks on the device, then build them in every layer.
    Returns the host-known upper bound of blocks built."""
    kptr, K0 = _k_layers(st, K_layers)
    dev = K0.device
    nb = min(int(st.NB), int(K0.shape[0]))
    bt = block_table
    if bt.dtype != torch.int32 or bt.stride(-1) != 1:
        bt = bt.to(torch.int32).contiguous()
    if n_req > bt.shape[0] or n_req > seq_lens.shape[0]:
        raise ValueError(f"n_req {n_req} exceeds block_table / seq_lens rows")
    sl = seq_lens[:n_req].to(device=dev, dtype=torch.int32).contiguous()
    if mode == "tail":
        if rows is None:
            r, n_rows = None, n_req
        else:
            r = torch.as_tensor(rows).to(device=dev, dtype=torch.int32).contiguous()
            n_rows = int(r.numel())
        bound = min(n_rows, nb)
    else:
        r, n_rows = None, 0
        max_fin = min(int(max_fin), int(bt.shape[1]))
        bound = min(n_req * max_fin, nb)
    if bound == 0:
        return 0
    lib = _lib.load()
    v4, vs, c8, cs, mu8, mus, tag = (st.pp_v4, st.pp_vs, st.pp_c8, st.pp_cs, st.pp_mu8,
                                     st.pp_mus, st.pp_tag)
    stream = _lib.stream_ptr(dev)
    _lib.check(lib.locks_refresh_blocks(
        _MODE[mode], _lib.ptr(bt), bt.stride(0), _lib.ptr(sl), n_req,
        _lib.ptr(r) if r is not None else None, n_rows, max_fin, int(st.page), nb,
        _lib.ptr(kptr), int(st.L), K0.stride(0), K0.stride(1), K0.stride(2), int(st.n_kv),
        _lib.ptr(tag), int(st.NB), _lib.ptr(st.refresh_mark), _lib.ptr(st.refresh_blocks),
        _lib.ptr(st.refresh_count), stream), "refresh_blocks")
    _lib.check(lib.locks_build_rki4_layers(
        _lib.ptr(kptr), int(st.L), K0.stride(0), K0.stride(1), K0.stride(2), nb,
        _lib.ptr(st.refresh_blocks), _lib.ptr(st.refresh_count), bound, int(st.n_kv),
        int(st.d), int(st.page), int(st.NB), _lib.ptr(v4), _lib.ptr(vs), _lib.ptr(c8),
        _lib.ptr(cs), _lib.ptr(mu8), _lib.ptr(mus), _lib.rows_arg(st), _lib.ptr(tag), stream),
        "build_rki4_layers")
    if getattr(st, "pp_rk8", None) is not None:
        # MLA state with the int8 RoPE summary: the latent views start at the
        # cache rows, whose RoPE keys follow the latent ([kv_c | k_pe] rows,
        # backend/mla_attn.py:100-101); same device block list and count
        if K0.shape[-1] != st.D or K0.stride(1) < st.D + st.Dr:
            raise TypeError("MLA K_layers must be the (NB, page, 1, kv_lora_rank) latent views "
                            "of (NB, page, kv_lora_rank + rope_dim) cache rows")
        for layer, K in enumerate(K_layers):
            _lib.check(lib.locks_mla_build_rope(
                _lib.ptr(K), K.stride(0), K.stride(1), nb, _lib.ptr(st.refresh_blocks), bound,
                _lib.ptr(st.refresh_count), _lib.ptr(st.pp_rk8[layer]), _lib.ptr(st.pp_rks[layer]),
                stream), "mla_build_rope")
    return bound


@torch.no_grad()
def rki4_build_tail(st, K_layers, block_table: torch.Tensor, seq_lens: torch.Tensor,
                    n_req: int, rows=None) -> int:
    """Rebuild, in every layer, the last finalized page (max(sl // page - 1, 0))
    of ``rows`` (or of every request); rki4_build.py:264-290.  Sync-free,
    idempotent.  Returns layers x rows."""
    if n_req == 0:
        return 0
    n = _refresh(st, "tail", K_layers, block_table, seq_lens, n_req, rows=rows)
    return st.L * n


@torch.no_grad()
def rki4_build_bulk(st, K_layers, block_table: torch.Tensor, seq_lens: torch.Tensor,
                    n_req: int, max_fin: int, chunk_pairs: int = 8192) -> int:
    """Rebuild every finalized page (p < seq_lens // page, p < max_fin) of the
    batch in every layer; rki4_build.py:293-303.  Sync-free.  ``chunk_pairs``
    is accepted for call compatibility: the build has no fp32 transient to
    bound.  Returns layers x candidate pages (an upper bound)."""
    if n_req == 0 or max_fin <= 0:
        return 0
    return st.L * _refresh(st, "bulk", K_layers, block_table, seq_lens, n_req,
                           max_fin=max_fin)


@torch.no_grad()
def rki4_build_delta(st, K_layers, block_table: torch.Tensor, seq_lens: torch.Tensor,
                     n_req: int, max_fin: int, chunk_pairs: int = 8192) -> int:
    """Rebuild, in every layer, only the finalized blocks whose content tag is
    stale in ANY layer (rki4_build.py:306-315, build.py:472-488).  The block
    choice and the build stay on the device; the returned count (layers x
    stale blocks) is read back, the one sync of this path, as in the
    reference."""
    if n_req == 0 or max_fin <= 0:
        return 0
    if _refresh(st, "delta", K_layers, block_table, seq_lens, n_req, max_fin=max_fin) == 0:
        return 0
    return st.L * int(st.refresh_count.item())
