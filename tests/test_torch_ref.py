"""Pins of the torch CPU restatement (oracle/torch_ref.py, timed as the
bench's CPU baseline) against the numpy oracle, which is itself pinned in
test_oracle_pins.py.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import locks_oracle as O
from oracle import torch_ref as T
from tests.cases import make_case, random_slabs


def _t(slabs):
    out = {}
    for k, a in slabs.items():
        if a.dtype == np.uint16:
            out[k] = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        else:
            out[k] = torch.from_numpy(a.copy())
    return out


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def test_unpack_every_byte():
    b = np.arange(256, dtype=np.uint8)[None, :]
    assert np.array_equal(T.unpack_i4(torch.from_numpy(b), 512).numpy(),
                          O.unpack_i4(b).astype(np.float32))


@pytest.mark.parametrize("n_kv,G,seq_lens", [(2, 4, [3000]), (2, 16, [1200, 700]),
                                             (4, 8, [2000, 16, 33])])
def test_score_matches_oracle(n_kv, G, seq_lens):
    rng = np.random.default_rng(3)
    MP = max((s + 15) // 16 for s in seq_lens)
    NB = sum((s + 15) // 16 for s in seq_lens) + 3
    slabs = random_slabs(rng, NB, n_kv)
    bt = O.synth_block_table(rng, seq_lens, 16, NB, MP)
    q = O.f32_to_bf16(rng.standard_normal((len(seq_lens), n_kv * G, 128), dtype=np.float32))
    npg, nsh, b = O.derive_page_params(seq_lens, 16, 1, 1, 126)
    scale = 1 / np.sqrt(128)
    ref = O.score_rki4_intpath(q, slabs, bt, nsh, n_kv, G, scale, MP, dtype=np.float64)
    got = T.score_rki4(_bf(q), _t(slabs), torch.from_numpy(bt), torch.from_numpy(nsh), n_kv, G,
                       scale, MP).numpy()
    assert np.abs(got - ref).max() <= 2e-5


def test_score_on_built_summaries():
    case = make_case(4, 2, 4, [2500])
    npg, nsh, b = O.derive_page_params(case.seq_lens, 16, 1, 1, 126)
    ref = O.score_rki4_twin(case.q, case.slabs, case.bt, nsh, 2, 4, case.scale, case.MP)
    got = T.score_rki4(_bf(case.q), _t(case.slabs), torch.from_numpy(case.bt),
                       torch.from_numpy(nsh), 2, 4, case.scale, case.MP).numpy()
    assert np.abs(got - ref).max() <= 2e-5


def test_combine_and_topb_match_oracle():
    rng = np.random.default_rng(5)
    seq_lens = [40000, 17, 0, 9000]
    MP = 2500
    sh = (rng.standard_normal((4, 2, 8, MP)) * 3).astype(np.float32)
    sh[1, :, :, ::3] = np.round(sh[1, :, :, ::3])                 # ties
    npg, nsh, b = O.derive_page_params(seq_lens, 16, 1, 1, 126)
    c_ref = O.combine_nrm(sh, nsh)
    c_got = T.combine_nrm(torch.from_numpy(sh), torch.from_numpy(nsh)).numpy()
    assert np.abs(c_got - c_ref).max() <= 1e-5 * 8
    for score in (c_ref, np.round(c_ref * 4) / 4):                 # plus a tie-heavy copy
        tab, cnt = O.topb_select(score, npg, nsh, b, 1, MP)
        tt, tc = T.topb_select(torch.from_numpy(score.astype(np.float32)), npg, nsh, b, 1, MP)
        assert np.array_equal(tt.numpy(), tab) and np.array_equal(tc.numpy(), cnt)


def test_decode_matches_oracle():
    case = make_case(6, 2, 4, [5000, 300], build=False)
    rng = np.random.default_rng(7)
    MP = case.MP
    npg, nsh, b = O.derive_page_params(case.seq_lens, 16, 1, 1, 40)
    score = rng.standard_normal((2, 2, MP)).astype(np.float32)
    tab, cnt = O.topb_select(score, npg, nsh, b, 1, MP)
    ref, _ = O.decode_attention(case.q, case.k, case.v, case.bt, case.seq_lens, tab, cnt,
                                case.G, case.scale)
    got = T.decode_attention(_bf(case.q), _bf(case.k), _bf(case.v), torch.from_numpy(case.bt),
                             case.seq_lens, torch.from_numpy(tab), torch.from_numpy(cnt),
                             case.G, case.scale).numpy()
    # fp16 rounding of P and V in the restatement (the kernels' P.V precision)
    assert np.abs(got - ref).max() <= 2e-3
