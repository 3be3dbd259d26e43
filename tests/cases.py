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


def random_slabs(rng: np.random.Generator, NB: int, n_kv: int, d: int = 128, page: int = 16,
                 rank: int = 8) -> dict:
    """Seeded rki4 slab bytes for scorer-only cases at full row lengths.

    The scorer is a function of the slab bytes alone, so long rows (128K,
    1M) are covered without running the O(pages) eigen build: every int4
    nibble and int8 code value is drawn uniformly over its full range, and
    the bf16 scales over the magnitudes a build of N(0, 1) keys with x8
    outlier channels produces (vs ~ |V|max/7, cs ~ |C|max/127, mus ~
    |mu|max/127)."""
    bf = lambda lo, hi, shape: O.f32_to_bf16(rng.uniform(lo, hi, shape).astype(np.float32))
    return dict(
        v4=rng.integers(0, 256, (NB, n_kv, rank, d // 2), dtype=np.uint8),
        vs=bf(0.005, 0.06, (NB, n_kv, rank)),
        c8=rng.integers(-127, 128, (NB, n_kv, page, rank), dtype=np.int8),
        cs=bf(0.01, 0.3, (NB, n_kv, page)),
        mu8=rng.integers(-127, 128, (NB, n_kv, d), dtype=np.int8),
        mus=bf(0.005, 0.08, (NB, n_kv)),
    )


def score_oracle_chunked(q, slabs, bt, nsh, n_kv, G, scale, MP, chunk=8192, dtype=None):
    """O.score_rki4_twin (or, with dtype, O.score_rki4_intpath) over page
    slices of at most `chunk` pages: a page's score depends on that page
    alone, so the slices concatenate to the full row's result."""
    R = q.shape[0]
    out = np.zeros((R, n_kv, G, MP), np.float32)
    for r in range(R):
        P = int(nsh[r])
        for lo in range(0, max(P, 0), chunk):
            hi = min(lo + chunk, P)
            sub_bt = np.ascontiguousarray(bt[r:r + 1, lo:hi])
            args = (q[r:r + 1], slabs, sub_bt, np.array([hi - lo]), n_kv, G, scale, hi - lo)
            if dtype is None:
                s = O.score_rki4_twin(*args)
            else:
                s = O.score_rki4_intpath(*args, dtype=dtype)
            out[r, :, :, lo:hi] = s[0]
    return out
