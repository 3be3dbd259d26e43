"""Rki4State: persistent per-model summary state + per-step selection buffers.

Tensor names, shapes and dtypes follow the reference's six-slab layout
(src/locks/selection/rki4_state.py:7-16, allocation :229-273):

    pp_v4  (L, NB, n_kv, 8, d/2) uint8  int4 basis V, column-major, low nibble = even d
    pp_vs  (L, NB, n_kv, 8)      bf16   per-column scales (absmax/7)
    pp_c8  (L, NB, n_kv, page, 8) int8  coefficients C = U8*S8
    pp_cs  (L, NB, n_kv, page)   bf16   per-token scales (absmax/127)
    pp_mu8 (L, NB, n_kv, d)      int8   page centroid
    pp_mus (L, NB, n_kv)         bf16   centroid scale (absmax/127)
    pp_tag (L, NB, n_kv, 8)      bf16   content tag, NaN-initialised

Per-step outputs: score (R, n_kv, MP) f32, page_table (R, n_kv, MP) i32,
page_cnt (R, n_kv) i32, score_h (R, n_kv, G, MP) f32, n_pages / n_sel_hi /
b_fix (R,) i32.  Added for the MI355X kernels (all persistent, allocated here
so no call allocates): page_max (R, n_kv, 16, chunks) f32 -- the scorer's
per-chunk maxima, head-major -- and sel_ws, the selector's candidate workspace.

Footprint per (page, kv head): 5d + 10*page + 18 bytes of summary (818 B at
d=128, page 16) + 16 B tag (rki4_state.py:18-22, record_bytes :124-141).
Geometry: d in {64, 128, 256}, page 16, 32 or 64, G <= 16.

Memory layout (this build): the six summary fields of one (block, kv head)
are stored together in one record of ``pp_rows`` (L, NB, n_kv, row_bytes)
u8, row_bytes = 5d + 10*page + 18 rounded up to 64 (832 B at d=128, page
16), fields in the order v4 | mu8 | c8 | cs | vs | mus -- the reference's
AoS record (rki4_state.py:93-110, 198-219; the reference builds it for
d=128 / page 16 under RKI4_MMA_AOS, this build for every geometry).  The
scorer reads a page's summary as one contiguous ~0.8 KB row instead of six
rows in six arrays (16-, 32- and 2-byte rows each costing a cache line of
their own).
``pp_v4`` .. ``pp_mus`` are strided views with the reference's shapes and
dtypes, so every tensor-level use (copies, comparisons) is unchanged; the
kernels take each slab's row stride (``slab_row_bytes``).  The tag stays a
separate slab (read only by the refresh lifecycle).
"""
from __future__ import annotations

import ctypes
import math

import torch

from .. import _lib

TAGW = 8
RNK = 8
IBITS = 4
QMAX = (1 << (IBITS - 1)) - 1
QMIN = -(1 << (IBITS - 1))


def packed_row_bytes(d: int, page: int) -> int:
    """Bytes of one packed (block, kv head) summary record: 5d + 10*page + 18
    rounded up to 64 (the reference's _rec_bytes_aos, rki4_state.py:106-109)."""
    return -(-(5 * d + 10 * page + 18) // 64) * 64


def packed_slab_views(rows: torch.Tensor, d: int, page: int):
    """(v4, vs, c8, cs, mu8, mus) views of packed rows (..., row_bytes) u8,
    with the reference's slab shapes and dtypes."""
    P, i8, bf16 = page, torch.int8, torch.bfloat16
    o_mu = RNK * d // 2
    o_c8 = o_mu + d
    o_cs = o_c8 + RNK * P
    o_vs = o_cs + 2 * P
    o_mus = o_vs + 2 * RNK
    v4 = rows[..., 0:o_mu].unflatten(-1, (RNK, d // 2))
    mu8 = rows[..., o_mu:o_c8].view(i8)
    c8 = rows[..., o_c8:o_cs].view(i8).unflatten(-1, (P, RNK))
    cs = rows[..., o_cs:o_vs].view(bf16)
    vs = rows[..., o_vs:o_mus].view(bf16)
    mus = rows[..., o_mus:o_mus + 2].view(bf16)[..., 0]
    return v4, vs, c8, cs, mu8, mus


def slab_row_bytes(slabs) -> "ctypes.Array":
    """The C ABI's slab_row_bytes argument for (v4, vs, c8, cs, mu8, mus)
    tensors shaped (..., NB, n_kv, field...): each slab's byte stride between
    consecutive (block, kv head) rows."""
    vals = []
    for t, tail in zip(slabs, (2, 1, 2, 1, 1, 0)):    # field dims after (NB, n_kv)
        kv_dim = t.dim() - tail - 1
        rb = t.stride(kv_dim) * t.element_size()
        assert t.stride(kv_dim - 1) * t.element_size() == rb * t.shape[kv_dim], \
            "slab rows of one block must be consecutive over kv heads"
        vals.append(rb)
    return (ctypes.c_int64 * 6)(*vals)


def record_bytes(d: int, page: int, tagw: int = TAGW) -> int:
    """Per-(page, kv head) slab bytes including the tag (rki4_state.py:124-141)."""
    return RNK * (d * IBITS // 8) + RNK * 2 + page * RNK + page * 2 + d + 2 + tagw * 2


class Rki4State:
    """Allocated once from engine maxima; every address is stable across
    decode steps, so the per-layer chain can be captured in a HIP graph."""

    def __init__(self, device, *, num_layers: int, num_blocks: int, n_kv: int, G: int,
                 head_dim: int, page: int, max_reqs: int, max_pages: int, rank: int = RNK,
                 budget: float = 0.1, budget_pages=None, sink_pages: int = 1,
                 window_pages: int = 1, tagw: int = TAGW, combine: str = "nrm",
                 zsplit=None):
        assert window_pages >= 1, "window_pages>=1: the partial tail must live inside " \
            "the always-attended window"
        self.validate_geometry(head_dim=head_dim, G=G, page=page, rank=rank)
        assert combine in ("max", "nrm")
        L, NB, D, MP, R = num_layers, num_blocks, head_dim, max_pages, max_reqs
        self.L, self.NB, self.n_kv, self.G, self.d = L, NB, n_kv, G, D
        self.D = D
        self.page, self.r, self.tagw = page, RNK, tagw
        self.v_bits = IBITS
        self.max_reqs, self.max_pages = R, MP
        self.budget = float(budget)
        self.budget_abs = int(budget_pages or 0)
        # upper bound of the per-row budget b (derive_page_params), passed to
        # the selector so that large budgets take its histogram route
        self.b_max = self.budget_abs if self.budget_abs > 0 else \
            int(math.ceil(self.budget * max_pages))
        self.sink_pages, self.window_pages = int(sink_pages), int(window_pages)
        self.combine = combine
        self.device = torch.device(device)
        u8, i8, bf16 = torch.uint8, torch.int8, torch.bfloat16
        i32, f32 = torch.int32, torch.float32
        dev = self.device

        self.row_bytes = packed_row_bytes(D, page)
        self.pp_rows = torch.zeros(L, NB, n_kv, self.row_bytes, device=dev, dtype=u8)
        (self.pp_v4, self.pp_vs, self.pp_c8, self.pp_cs, self.pp_mu8,
         self.pp_mus) = packed_slab_views(self.pp_rows, D, page)
        self.slab_row_bytes = slab_row_bytes(
            (self.pp_v4, self.pp_vs, self.pp_c8, self.pp_cs, self.pp_mu8, self.pp_mus))
        self.pp_tag = torch.full((L, NB, n_kv, tagw), float("nan"), device=dev, dtype=bf16)

        self.score = torch.zeros(R, n_kv, MP, device=dev, dtype=f32)
        self.page_table = torch.full((R, n_kv, MP), -1, device=dev, dtype=i32)
        self.page_cnt = torch.zeros(R, n_kv, device=dev, dtype=i32)
        self.score_h = torch.zeros(R, n_kv, G, MP, device=dev, dtype=f32)

        self.n_pages = torch.zeros(R, device=dev, dtype=i32)
        self.n_sel_hi = torch.zeros(R, device=dev, dtype=i32)
        self.b_fix = torch.ones(R, device=dev, dtype=i32)

        lib = _lib.load()
        # scorer launch shape: pages per workgroup (explicit zsplit = chunks)
        if zsplit:
            chunk = max(8, -(-MP // int(zsplit)))
            chunk = min(1024, -(-chunk // 8) * 8)
        else:
            chunk = int(lib.locks_score_auto_chunk(R, n_kv, MP))
        self.score_chunk = chunk
        self.score_chunks = int(lib.locks_score_num_chunks(MP, chunk))
        self.zsplit = self.score_chunks
        self.page_max = torch.full((R, n_kv, 16, self.score_chunks), float("-inf"),
                                   device=dev, dtype=f32)
        ws = int(lib.locks_select_workspace_bytes(R, n_kv, MP))
        self.sel_ws = torch.zeros(max(ws, 256), device=dev, dtype=torch.uint8)

        assert self.bytes_per_layer() == record_bytes(D, page, tagw) * n_kv * NB

    @staticmethod
    def validate_geometry(*, head_dim: int, G: int, page: int, rank: int = RNK) -> None:
        """Supported set of the gfx950 kernels, checked at wiring time: the
        reference's d in {64, 128, 256} and page in {16, 32, 64}
        (rki4_state.py:295-324), G up to 16."""
        assert head_dim in (64, 128, 256), \
            f"rki4 supports d in {{64, 128, 256}}, model has d={head_dim}"
        assert 1 <= G <= 16, f"this build supports 1 <= G <= 16 query heads per kv head, got {G}"
        assert page in (16, 32, 64), \
            f"rki4 supports page in {{16, 32, 64}}, engine block_size={page}"
        assert rank == RNK, f"rki4 rank is fixed at {RNK} in this build, got {rank}"

    @classmethod
    def record_bytes(cls, d: int, page: int, tagw: int = TAGW) -> int:
        return record_bytes(d, page, tagw)

    def bytes_per_layer(self) -> int:
        return (self.pp_v4[0].numel() + self.pp_vs[0].numel() * 2 + self.pp_c8[0].numel()
                + self.pp_cs[0].numel() * 2 + self.pp_mu8[0].numel()
                + self.pp_mus[0].numel() * 2 + self.pp_tag[0].numel() * 2)

    def layer_state(self, layer: int):
        """(v4, vs, c8, cs, mu8, mus, tag) views of one layer."""
        return (self.pp_v4[layer], self.pp_vs[layer], self.pp_c8[layer], self.pp_cs[layer],
                self.pp_mu8[layer], self.pp_mus[layer], self.pp_tag[layer])
