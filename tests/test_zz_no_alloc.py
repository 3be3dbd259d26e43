"""locks_decode_fused_noalloc (the entry point that allocates nothing) against
locks_decode_fused with caller-owned partials, through the C ABI: two calls
in a row, the second on a smaller input, each bit-identical to the
caller-buffer entry point; oversized calls are rejected with a message."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import locks_oracle as O
from tests.cases import make_case, to_dev

pytestmark = pytest.mark.gpu


def say(*a):
    print("[noalloc]", *a, flush=True)


def _inputs(seed, n_kv, G, seq_lens, budget):
    import torch
    case = make_case(seed, n_kv, G, seq_lens, build=False)
    rng = np.random.default_rng(seed + 100)
    npg, nsh, b = O.derive_page_params(case.seq_lens, 16, 1, 1, budget)
    score = rng.standard_normal((case.R, n_kv, case.MP)).astype(np.float32)
    tab, cnt = O.topb_select(score, npg, nsh, b, 1, case.MP)
    d = to_dev(case)
    d["tab"] = torch.from_numpy(tab).cuda()
    d["cnt"] = torch.from_numpy(cnt).cuda()
    return case, d


def _pair(case, d, split, pps_min, dtype):
    """(reference out from locks_decode_fused, out from the no-alloc entry)."""
    import torch
    from locks.attention import decode as D
    k, v = D._split_kv(d["kv"])
    R, n_kv, G = case.R, case.n_kv, case.G
    mp = torch.empty(R, n_kv, split, G, device="cuda")
    lp = torch.empty_like(mp)
    ap = torch.empty(R, n_kv, split, G, 128, device="cuda")
    ctr = torch.zeros(R, n_kv, D.COUNTER_STRIDE, dtype=torch.int32, device="cuda")
    ref = torch.full((R, n_kv * G, 128), float("nan"), dtype=dtype, device="cuda")
    out = torch.full_like(ref, float("nan"))
    D.decode_fused(d["q"], k, v, d["bt"], d["sl"], d["tab"], d["cnt"], mp, lp, ap, ctr, ref,
                   n_req=R, G=G, split=split, pps_min=pps_min, scale=case.scale)
    D.decode_fused_noalloc(d["q"], k, v, d["bt"], d["sl"], d["tab"], d["cnt"], out, n_req=R,
                           G=G, split=split, pps_min=pps_min, scale=case.scale)
    torch.cuda.synchronize()
    return ref, out


def _same(a, b):
    import torch
    iv = torch.int16 if a.dtype == torch.bfloat16 else torch.int32
    return torch.equal(a.view(iv), b.view(iv))


@pytest.mark.parametrize("dtype_name", ["bf16", "f32"])
def test_noalloc_matches_fused_two_calls(dtype_name):
    import torch
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float32
    # first call: a ragged batch of three rows on GLM-shaped groups
    say("call 1: n_kv=2 G=16 seq_lens=[20000, 9000, 4000] split=64", dtype_name)
    case, d = _inputs(31, 2, 16, [20000, 9000, 4000], 126)
    ref, out = _pair(case, d, 64, 4, dtype)
    assert _same(ref, out)
    assert torch.isfinite(out.float()).all()
    # second call, smaller input: one shorter row, fewer splits
    say("call 2: n_kv=2 G=16 seq_lens=[3000] split=16", dtype_name)
    case2, d2 = _inputs(32, 2, 16, [3000], 60)
    ref2, out2 = _pair(case2, d2, 16, 4, dtype)
    assert _same(ref2, out2)
    # and the output is the attention the oracle computes
    got = out2.float().cpu().numpy()
    exp, _ = O.decode_attention(case2.q, case2.k, case2.v, case2.bt, case2.seq_lens,
                                d2["tab"].cpu().numpy(), d2["cnt"].cpu().numpy(), 16, case2.scale)
    rb = exp if dtype == torch.float32 else O.bf16_round(exp.astype(np.float32))
    e = np.abs(got - rb)
    assert e.max() <= 2e-2 and e.sum() / np.abs(rb).sum() <= 1e-3


def test_noalloc_llama_shape_then_smaller():
    import torch
    say("llama shape: n_kv=8 G=4 seq_lens=[131072] split=128")
    case, d = _inputs(33, 8, 4, [131072], 126)
    ref, out = _pair(case, d, 128, 4, torch.bfloat16)
    assert _same(ref, out)
    say("smaller: n_kv=8 G=4 seq_lens=[5000, 700] split=32")
    case2, d2 = _inputs(34, 8, 4, [5000, 700], 126)
    ref2, out2 = _pair(case2, d2, 32, 4, torch.bfloat16)
    assert _same(ref2, out2)


def test_noalloc_rejects_oversized_call():
    """n_req 64 x n_kv 8 x split 128 x G 4 needs ~136 MB of partials: refused
    on the host before any launch, with the limit in the message."""
    import torch
    from locks.attention import decode as D
    say("oversized call")
    case, d = _inputs(35, 8, 4, [4096], 126)
    k, v = D._split_kv(d["kv"])
    # every buffer sized for 64 requests (empty rows), so even a launch
    # would stay in bounds
    R = 64
    q = torch.zeros(R, 32, 128, dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros(R, d["bt"].shape[1], dtype=torch.int32, device="cuda")
    sl = torch.ones(R, dtype=torch.int32, device="cuda")
    tab = torch.full((R, 8, case.MP), -1, dtype=torch.int32, device="cuda")
    cnt = torch.zeros(R, 8, dtype=torch.int32, device="cuda")
    out = torch.empty(R, 32, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="scratch"):
        D.decode_fused_noalloc(q, k, v, bt, sl, tab, cnt, out, n_req=R, G=4, split=128,
                               pps_min=4, scale=case.scale)


def test_noalloc_odd_partial_counts():
    """n_req x n_kv x split x G odd (3, then 9): each scratch region still
    starts 256-byte aligned, so the 16-byte partial stores and merge loads
    stay aligned; bit-identical to the caller-buffer entry point."""
    import torch
    say("odd: n_kv=1 G=1 seq_lens=[3000] split=3")
    case, d = _inputs(36, 1, 1, [3000], 60)
    ref, out = _pair(case, d, 3, 4, torch.bfloat16)
    assert _same(ref, out) and torch.isfinite(out.float()).all()
    say("odd: n_kv=1 G=3 seq_lens=[1500] split=3")
    case2, d2 = _inputs(37, 1, 3, [1500], 40)
    ref2, out2 = _pair(case2, d2, 3, 2, torch.float32)
    assert _same(ref2, out2) and torch.isfinite(out2).all()
