"""MlaState: persistent per-model latent-summary state + per-step selection
and decode buffers for MLA models (one latent KV head shared by all query
heads; DeepSeek-V2-Lite: kv_lora_rank 512 + 64 RoPE dims, 16 heads).

The summary of a (layer, physical block) is the rki4 record of the page's
latent block at d = kv_lora_rank (slab names and layouts as Rki4State with
n_kv = 1): 2738 B per page.  The RoPE term of the score reads either the
exact bf16 keys of the latent cache itself (``rope="exact"``, the default,
2048 B per page) or the int8 RoPE summary (``rope="int8"``: per token 64 int8
keys and a bf16 scale, 1056 B per page; q_rope is then int8-quantized per
head).  The int8 form cuts the scorer's bytes by 21 % but its time by only
~2 % at 128K (the scorer is latency-bound there), and the decode that
follows loses the cache hits the exact scorer leaves on the selected pages'
RoPE rows, so the exact keys are the default.  The reference keeps per-page fp32 factors Lf (page, 16) and
Rf (16, 512) in a host-side dict keyed by the first block
(backend/mla_attn.py:41-43, :203-232); here the summaries live in
block-keyed device slabs like the GQA state, so a refresh is a block-list
rebuild and every address is stable for graph capture.
"""
from __future__ import annotations

import math

import torch

from .. import _lib

RNK = 8
TAGW = 8


class MlaState:
    def __init__(self, device, *, num_layers: int, num_blocks: int, n_heads: int,
                 kv_lora_rank: int = 512, rope_dim: int = 64, page: int = 16,
                 max_reqs: int, max_pages: int, budget_pages: int = 128, sink_pages: int = 1,
                 window_pages: int = 10, split: int | None = None, rope: str = "exact"):
        assert kv_lora_rank == 512 and rope_dim == 64, \
            f"this MI355X build supports kv_lora_rank 512 + rope 64, got {kv_lora_rank} + {rope_dim}"
        assert page == 16, f"this MI355X build supports page 16, got {page}"
        assert 1 <= n_heads <= 16, f"this build supports <= 16 query heads on MLA, got {n_heads}"
        assert window_pages >= 1 and sink_pages >= 0 and budget_pages >= 1
        if rope not in ("int8", "exact"):
            raise ValueError(f"rope must be 'int8' or 'exact', got {rope!r}")
        self.rope = rope
        L, NB, D, MP, R = num_layers, num_blocks, kv_lora_rank, max_pages, max_reqs
        self.L, self.NB, self.H, self.D, self.Dr = L, NB, n_heads, D, rope_dim
        self.n_kv, self.G, self.d = 1, 1, D
        self.page, self.max_reqs, self.max_pages = page, R, MP
        self.budget_pages = int(budget_pages)
        self.sink_pages, self.window_pages = int(sink_pages), int(window_pages)
        # topb_middle counts the forced sink + window pages inside the budget
        # (selection/mla_score_torch.py:63): the selector's middle budget
        self.budget_abs = max(self.budget_pages - self.sink_pages - self.window_pages, 1)
        self.device = torch.device(device)
        dev = self.device
        u8, i8, bf16, i32, f32 = torch.uint8, torch.int8, torch.bfloat16, torch.int32, torch.float32
        self.pp_v4 = torch.zeros(L, NB, 1, RNK, D // 2, device=dev, dtype=u8)
        self.pp_vs = torch.zeros(L, NB, 1, RNK, device=dev, dtype=bf16)
        self.pp_c8 = torch.zeros(L, NB, 1, page, RNK, device=dev, dtype=i8)
        self.pp_cs = torch.zeros(L, NB, 1, page, device=dev, dtype=bf16)
        self.pp_mu8 = torch.zeros(L, NB, 1, D, device=dev, dtype=i8)
        self.pp_mus = torch.zeros(L, NB, 1, device=dev, dtype=bf16)
        self.pp_tag = torch.full((L, NB, 1, TAGW), float("nan"), device=dev, dtype=bf16)
        if rope == "int8":
            self.pp_rk8 = torch.zeros(L, NB, page, rope_dim, device=dev, dtype=i8)
            self.pp_rks = torch.zeros(L, NB, page, device=dev, dtype=bf16)
        else:
            self.pp_rk8 = self.pp_rks = None

        self.score_h = torch.zeros(R, 1, 1, MP, device=dev, dtype=f32)   # page scores
        self.score = torch.zeros(R, 1, MP, device=dev, dtype=f32)
        self.page_table = torch.full((R, 1, MP), -1, device=dev, dtype=i32)
        self.page_cnt = torch.zeros(R, 1, device=dev, dtype=i32)
        self.n_pages = torch.zeros(R, device=dev, dtype=i32)
        self.n_sel_hi = torch.zeros(R, device=dev, dtype=i32)
        self.b_fix = torch.ones(R, device=dev, dtype=i32)

        lib = _lib.load()
        self.score_chunk = int(lib.locks_mla_score_auto_chunk(R, MP))
        ws = int(lib.locks_select_workspace_bytes(R, 1, MP))
        self.sel_ws = torch.zeros(max(ws, 256), device=dev, dtype=torch.uint8)
        # split-K partials: ~4 attended pages per split at the expected budget
        if split is None:
            split = min(512, max(8, math.ceil(self.budget_pages / 4)))
        self.split = int(split)
        self.m_part = torch.empty(R, self.split, 16, device=dev, dtype=f32)
        self.l_part = torch.empty(R, self.split, 16, device=dev, dtype=f32)
        self.acc_part = torch.empty(R, self.split, 16, D, device=dev, dtype=f32)
        self.lse = torch.empty(R, 16, device=dev, dtype=f32)

    def layer_state(self, layer: int):
        """(v4, vs, c8, cs, mu8, mus, tag) views of one layer."""
        return (self.pp_v4[layer], self.pp_vs[layer], self.pp_c8[layer], self.pp_cs[layer],
                self.pp_mu8[layer], self.pp_mus[layer], self.pp_tag[layer])

    def rope_state(self, layer: int):
        """(rk8, rks) views of one layer's int8 RoPE summary, or (None, None)
        when the scorer reads the exact keys from the cache."""
        if self.pp_rk8 is None:
            return None, None
        return self.pp_rk8[layer], self.pp_rks[layer]

    def summary_bytes_per_page(self) -> int:
        """Bytes the scorer reads per page: latent summary + RoPE keys (int8
        keys + bf16 token scales, or the exact bf16 keys)."""
        rope = self.page * (self.Dr + 2) if self.rope == "int8" else self.page * self.Dr * 2
        return RNK * self.D // 2 + RNK * 2 + self.page * RNK + self.page * 2 + self.D + 2 + rope
