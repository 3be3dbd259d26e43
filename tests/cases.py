"""Seeded synthetic decode cases shared by the GPU parity tests.

Inputs follow the BASELINE distribution: K, V ~ N(0, 1) bf16 with 4 fixed
outlier channels per kv head scaled x8, q ~ N(0, 1) bf16, block tables drawn
from one shuffled page pool.  Summaries are built by the CPU oracle builder
so the kernels and the oracle score identical slab bytes.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from oracle import locks_oracle as O


@dataclasses.dataclass
class Case:
    n_kv: int
    G: int
    seq_lens: list
    MP: int
    NB: int
    k: np.ndarray          # (NB, page, n_kv, d) bf16 bits
    v: np.ndarray
    q: np.ndarray          # (R, n_kv*G, d) bf16 bits
    bt: np.ndarray         # (R, MB) int32
    slabs: dict
    page: int = 16
    d: int = 128

    @property
    def R(self):
        return len(self.seq_lens)

    @property
    def scale(self):
        return 1.0 / np.sqrt(self.d)


def make_case(seed, n_kv, G, seq_lens, MP=None, extra_blocks=3, build=True,
              page=16, d=128, kv=True) -> Case:
    rng = np.random.default_rng(seed)
    npg = [(s + page - 1) // page for s in seq_lens]
    MP = MP or max(max(npg), 1)
    NB = sum(npg) + extra_blocks
    if kv:
        k, v, _ = O.synth_kv(rng, NB, page, n_kv, d)
    else:                      # selection-only cases: a one-block dummy cache
        k = v = np.zeros((1, page, n_kv, d), np.uint16)
        build = False
    q = O.f32_to_bf16(rng.standard_normal((len(seq_lens), n_kv * G, d), dtype=np.float32))
    bt = O.synth_block_table(rng, seq_lens, page, NB, MP)
    slabs = None
    if build:
        fin = []
        for r, s in enumerate(seq_lens):
            fin.extend(bt[r, : s // page].tolist())
        slabs = O.build_state_slabs(k, np.array(sorted(set(fin)), np.int64), NB)
    return Case(n_kv, G, list(seq_lens), MP, NB, k, v, q, bt, slabs, page, d)


def to_dev(case: Case, device="cuda"):
    """Upload the case: returns dict of torch tensors."""
    import torch

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)

    out = dict(
        q=bf(case.q),
        kv=torch.stack([bf(case.k), bf(case.v)], dim=1),   # (NB', 2, page, n_kv, d)
        bt=torch.from_numpy(case.bt).to(device),
        sl=torch.tensor(case.seq_lens, dtype=torch.int32, device=device),
    )
    return out


def load_slabs(st, layer, slabs):
    import torch
    for name, attr in (("v4", "pp_v4"), ("c8", "pp_c8"), ("mu8", "pp_mu8")):
        getattr(st, attr)[layer].copy_(torch.from_numpy(slabs[name]))
    for name, attr in (("vs", "pp_vs"), ("cs", "pp_cs"), ("mus", "pp_mus")):
        getattr(st, attr)[layer].copy_(
            torch.from_numpy(slabs[name].view(np.int16)).view(torch.bfloat16))
