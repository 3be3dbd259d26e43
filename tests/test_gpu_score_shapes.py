"""GPU parity of the rki4 scorer at the launch shapes the decode step uses.

The scorer's workgroup scores `chunk` pages of one kv head as 8-page units,
4 waves each taking every 4th unit: with chunk >= 64 a wave scores several
units, DMA'ing the next unit's summary records into its other LDS stage
while it scores the current one, and folding each unit's per-head maxima
into the chunk's `page_max`.  These cases force those paths (explicit zsplit on the
16K Llama-shaped row: chunk 64 / 128 / 256 / 1024) and run the full rows of
the benchmarked configurations at their automatic chunking: Llama 128K
(8 kv x 8191 pages), GLM 1M (2 kv x 65535 pages, G = 16), the ragged GLM
batch {256K, 192K, 128K, 64K}, and the MLA latent scorer at 8182 pages.

Oracle: `score_rki4_twin` (rki4_score_torch.py:111-160) and the float64
integer path, evaluated over page slices (a page's score depends on that
page alone).  Bar: |score_h - oracle| <= 2e-5 on every scored page,
page_max[r, kh, z, g] equal to the max of the chunk's scored pages, and no
write past n_sel_hi.  Slab bytes are seeded random draws over the full
code ranges (tests/cases.random_slabs): the scorer reads bytes, not keys.
The same bytes as the reference's six separate contiguous slabs (C ABI,
slab_row_bytes NULL) must score bit-identically to the state's AoS records.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from tests.cases import random_slabs, score_oracle_chunked

pytestmark = pytest.mark.gpu

SENTINEL = 123.0


def say(*a):
    print("[score-shape]", *a, flush=True)


def _run(seed, n_kv, G, seq_lens, zsplit=None, expect_chunk=None, check64=True):
    import torch
    from locks.selection import Rki4State, derive_page_params, rki4_score_only
    from tests.cases import load_slabs
    rng = np.random.default_rng(seed)
    R = len(seq_lens)
    npg = [(s + 15) // 16 for s in seq_lens]
    MP = max(npg)
    NB = sum(npg) + 5
    bt = O.synth_block_table(rng, seq_lens, 16, NB, MP)
    slabs = random_slabs(rng, NB, n_kv)
    q = O.f32_to_bf16(rng.standard_normal((R, n_kv * G, 128), dtype=np.float32))
    scale = 1.0 / np.sqrt(128.0)
    st = Rki4State("cuda", num_layers=1, num_blocks=NB, n_kv=n_kv, G=G, head_dim=128, page=16,
                   max_reqs=R, max_pages=MP, budget_pages=126, zsplit=zsplit)
    say(f"n_kv={n_kv} G={G} seq_lens={seq_lens} zsplit={zsplit} -> chunk={st.score_chunk} "
        f"chunks={st.score_chunks}")
    if expect_chunk is not None:
        assert st.score_chunk == expect_chunk
    load_slabs(st, 0, slabs)
    dq = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).cuda()
    dbt = torch.from_numpy(bt).cuda()
    dsl = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    derive_page_params(st, dsl, R)
    st.score_h.fill_(SENTINEL)
    st.page_max.fill_(float("nan"))
    rki4_score_only(st, 0, dq, dbt, dsl, R, scale)
    torch.cuda.synchronize()
    got = st.score_h.cpu().numpy()
    pm = st.page_max.cpu().numpy().transpose(0, 1, 3, 2)   # (R, n_kv, chunks, 16)
    nsh = st.n_sel_hi.cpu().numpy()
    ref = score_oracle_chunked(q, slabs, bt, nsh, n_kv, G, scale, MP)
    ref64 = score_oracle_chunked(q, slabs, bt, nsh, n_kv, G, scale, MP,
                                 dtype=np.float64) if check64 else None
    C = st.score_chunk
    for r in range(R):
        P = int(nsh[r])
        err = np.abs(got[r, ..., :P] - ref[r, ..., :P]).max()
        msg = f"row {r}: {P} pages, max|gpu-twin| {err:.2e}"
        if ref64 is not None:
            err64 = np.abs(got[r, ..., :P] - ref64[r, ..., :P]).max()
            msg += f", max|gpu-exact| {err64:.2e}"
            assert err64 <= 2e-5, msg
        say(msg)
        assert err <= 2e-5, msg
        assert np.all(got[r, ..., P:] == SENTINEL), "score_h written past n_sel_hi"
        for z in range(st.score_chunks):
            lo, hi = z * C, min((z + 1) * C, P)
            if hi > lo:
                exp = got[r, :, :, lo:hi].max(axis=-1)            # (n_kv, G)
            else:
                exp = np.full((n_kv, G), -np.inf, np.float32)
            assert np.array_equal(pm[r, :, z, :G], exp), f"page_max row {r} chunk {z}"
            assert np.all(pm[r, :, z, G:] == -np.inf)
    return st


@pytest.mark.parametrize("zsplit,chunk", [(16, 64), (8, 128), (4, 256), (1, 1024)])
def test_score_forced_chunks_16k(zsplit, chunk):
    """Llama-shaped 16K row (8 kv x 4 heads) with 1, 2, 4 and 32 units per
    wave (chunk 64..1024)."""
    _run(21, 8, 4, [16384], zsplit=zsplit, expect_chunk=chunk)


@pytest.mark.parametrize("zsplit,chunk", [(4, 64), (1, 256)])
def test_score_forced_chunks_g16(zsplit, chunk):
    """GLM-shaped group (G = 16: one page per token-stage MFMA) over several
    units per wave, with a ragged last tile (4000 tokens -> 249 pages)."""
    _run(22, 2, 16, [4000], zsplit=zsplit, expect_chunk=chunk)


@pytest.mark.parametrize("n_kv,G", [(8, 4), (4, 8), (2, 16)])
def test_score_uneven_unit_counts(n_kv, G):
    """One request (the software-pipelined unit loop): chunk 72 = 9 units,
    so wave 0 scores 3 units and the others 2, and the last chunk's 19 pages
    are 3 units with one wave idle; for each token-stage form (G = 4: 4x4
    blocks, 8 and 16: 16x16 blocks)."""
    _run(27 + G, n_kv, G, [1100 * 16], zsplit=16, expect_chunk=72)


def test_score_llama_128k_full_row():
    """BASELINE configs[1] row: 8 kv heads x 8191 scored pages at the auto
    chunking (128 pages per workgroup) and at the engine's zsplit 64."""
    _run(23, 8, 4, [131072], expect_chunk=128)
    _run(24, 8, 4, [131072], zsplit=64, expect_chunk=128, check64=False)


def test_score_glm_1m_full_row():
    """BASELINE configs[2] row: 2 kv heads x 65535 pages, G = 16, auto chunk
    (256 pages per workgroup) and the engine's zsplit 64 (1024 pages)."""
    _run(25, 2, 16, [1 << 20], expect_chunk=256, check64=False)
    _run(26, 2, 16, [1 << 20], zsplit=64, expect_chunk=1024, check64=False)


def test_score_ragged_glm_batch():
    """{256K, 192K, 128K, 64K}, one grid sized for the
    longest row; the shorter rows' tail chunks score nothing."""
    _run(27, 2, 16, [262144, 196608, 131072, 65536], check64=False)


@pytest.mark.parametrize("d,page,n_kv,G,seq,zsplit", [
    (128, 16, 8, 4, 16384, 8),       # Llama shape, 2 units per wave
    (128, 16, 2, 16, 4000, 1),       # G = 16, ragged last tile
    (64, 32, 4, 8, 6000, 2),         # another geometry
])
def test_score_six_slabs_equal_records(d, page, n_kv, G, seq, zsplit):
    """locks_score_rki4 over six separate contiguous slabs (the reference's
    tensors; slab_row_bytes NULL: each row's fields gathered from six arrays)
    returns bit-identical score_h and page_max to the state's AoS records
    (one stream per record)."""
    import ctypes
    import torch
    from locks import _lib
    from locks.selection import Rki4State, derive_page_params, rki4_score_only
    from tests.cases import load_slabs
    rng = np.random.default_rng(31)
    npg = (seq + page - 1) // page
    MP, NB = npg, npg + 3
    bt = O.synth_block_table(rng, [seq], page, NB, MP)
    slabs = random_slabs(rng, NB, n_kv, d, page)
    q = O.f32_to_bf16(rng.standard_normal((1, n_kv * G, d), dtype=np.float32))
    scale = 1.0 / np.sqrt(d)
    st = Rki4State("cuda", num_layers=1, num_blocks=NB, n_kv=n_kv, G=G, head_dim=d, page=page,
                   max_reqs=1, max_pages=MP, budget_pages=16, zsplit=zsplit)
    say(f"six slabs vs records: d={d} page={page} n_kv={n_kv} G={G} seq={seq} chunk={st.score_chunk}")
    load_slabs(st, 0, slabs)
    dq = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).cuda()
    dbt = torch.from_numpy(bt).cuda()
    dsl = torch.tensor([seq], dtype=torch.int32, device="cuda")
    derive_page_params(st, dsl, 1)
    st.score_h.fill_(SENTINEL)
    rki4_score_only(st, 0, dq, dbt, dsl, 1, scale)
    torch.cuda.synchronize()
    rec_sh, rec_pm = st.score_h.clone(), st.page_max.clone()
    six = [t[0].contiguous() for t in (st.pp_v4, st.pp_vs, st.pp_c8, st.pp_cs, st.pp_mu8, st.pp_mus)]
    assert all(t.is_contiguous() for t in six)
    sh = torch.full_like(st.score_h, SENTINEL)
    pm = torch.full_like(st.page_max, float("nan"))
    lib = _lib.load()
    _lib.check(lib.locks_score_rki4(
        _lib.ptr(dq), dq.stride(0), dq.stride(1), *[_lib.ptr(t) for t in six], None,
        NB, _lib.ptr(dbt), dbt.stride(0), int(dbt.shape[1]), _lib.ptr(st.n_sel_hi), _lib.ptr(sh), MP,
        _lib.ptr(pm), st.score_chunk, 1, n_kv, G, d, page, ctypes.c_float(scale).value,
        _lib.stream_ptr()), "score (six slabs)")
    torch.cuda.synchronize()
    assert torch.equal(sh, rec_sh), "score_h differs between six slabs and records"
    assert torch.equal(pm, rec_pm), "page_max differs between six slabs and records"


@pytest.mark.parametrize("rope", ["int8", "exact"])
def test_mla_score_8k_pages(rope):
    """MLA latent scorer over the config-5 row (128K tokens, window 10:
    8182 scored pages) at its automatic chunking, with the int8 RoPE summary
    and with the exact keys."""
    import torch
    from oracle import mla_oracle as M
    from locks.selection import MlaState, mla_derive, mla_score_only
    from tests.cases import random_slabs as rs
    rng = np.random.default_rng(28)
    seq = 131072
    MP = seq // 16
    NB = MP + 4
    cache = M.synth_latent(rng, NB, 16, 512, 64)
    bt = O.synth_block_table(rng, [seq], 16, NB, MP)
    slabs = rs(rng, NB, 1, d=512)
    q = O.f32_to_bf16(rng.standard_normal((1, 16, 576)).astype(np.float32))
    st = MlaState("cuda", num_layers=1, num_blocks=NB, n_heads=16, max_reqs=1, max_pages=MP,
                  budget_pages=128, sink_pages=1, window_pages=10, rope=rope)
    say(f"mla chunk={st.score_chunk} rope={rope}")
    rsum = M.mla_build_rope(cache, np.arange(NB), NB) if rope == "int8" else None
    if rsum is not None:
        st.pp_rk8[0].copy_(torch.from_numpy(rsum["rk8"]))
        st.pp_rks[0].copy_(torch.from_numpy(rsum["rks"].view(np.int16)).view(torch.bfloat16))
    for k, name in (("v4", "pp_v4"), ("vs", "pp_vs"), ("c8", "pp_c8"), ("cs", "pp_cs"),
                    ("mu8", "pp_mu8"), ("mus", "pp_mus")):
        a = slabs[k]
        t = getattr(st, name)[0]
        if a.dtype == np.uint16:
            t.copy_(torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(t.shape))
        else:
            t.copy_(torch.from_numpy(a.copy()).reshape(t.shape))
    u16 = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    dsl = torch.tensor([seq], dtype=torch.int32, device="cuda")
    mla_derive(st, dsl, 1)
    st.score_h.fill_(SENTINEL)
    scale = 1.0 / np.sqrt(192.0)
    mla_score_only(st, 0, u16(q), u16(cache), torch.from_numpy(bt).cuda(), 1, scale)
    torch.cuda.synchronize()
    npg, nsh, b = M.mla_derive([seq], 16, 10, 1, 128)
    P = int(nsh[0])
    assert P == 8182
    got = st.score_h[0, 0, 0, :].cpu().numpy()
    ref = np.zeros(P, np.float32)
    for lo in range(0, P, 1024):
        hi = min(lo + 1024, P)
        ref[lo:hi] = M.mla_score_rki4(q, slabs, cache, np.ascontiguousarray(bt[:, lo:hi]),
                                      np.array([hi - lo]), scale, hi - lo, rope=rsum)[0]
    err = np.abs(got[:P] - ref).max()
    say(f"mla 8182 pages: max |d| {err:.2e}")
    assert err <= 2e-4 * max(1.0, np.abs(ref).max())
    assert np.all(got[P:] == SENTINEL)
