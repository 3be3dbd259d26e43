"""Batched all-layer summary refresh (tail / bulk / delta) on the GPU.

The producers pick their blocks on the device and build every layer in one
launch; they run the same per-(block, kv head) build as locks_build_rki4, so
every slab byte must equal a per-layer ``rki4_build_blocks`` over the block
set the reference's producers choose (selection/build.py:372-384 tail,
:415-427 bulk, :472-488 delta), restated here in numpy from the block table.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.cases import make_case, to_dev

pytestmark = pytest.mark.gpu

PAGE = 16
SLABS = ("pp_v4", "pp_vs", "pp_c8", "pp_cs", "pp_mu8", "pp_mus", "pp_tag")


def _state(NB, L, n_kv, R, MP):
    from locks.selection import Rki4State
    return Rki4State("cuda", num_layers=L, num_blocks=NB, n_kv=n_kv, G=4, head_dim=128,
                     page=PAGE, max_reqs=R, max_pages=MP, budget_pages=126)


def _layers(case, L, seed):
    """L K views of one shape: layer 0 is the case's K, the others fresh bf16."""
    import torch
    d = to_dev(case)
    g = torch.Generator().manual_seed(seed)
    ks = [d["kv"][:, 0]]
    for _ in range(1, L):
        kv = torch.randn(d["kv"].shape, generator=g).to(torch.bfloat16).cuda()
        ks.append(kv[:, 0])
    return d, ks


def _slab_bytes(st):
    import torch
    torch.cuda.synchronize()
    return {n: getattr(st, n).contiguous().view(torch.uint8).cpu().numpy() for n in SLABS}


def _assert_same(a, b):
    for n in SLABS:
        np.testing.assert_array_equal(a[n], b[n], err_msg=n)


def _assert_same_rope(a, b):
    """int8 RoPE summaries of two MLA states, byte for byte."""
    import torch
    torch.cuda.synchronize()
    for n in ("pp_rk8", "pp_rks"):
        np.testing.assert_array_equal(getattr(a, n).contiguous().view(torch.uint8).cpu().numpy(),
                                      getattr(b, n).contiguous().view(torch.uint8).cpu().numpy(), err_msg=n)


def _per_layer(st, ks, blocks):
    import torch
    from locks.selection import rki4_build_blocks
    b = torch.tensor(sorted(set(int(x) for x in blocks)), dtype=torch.int32)
    for layer, K in enumerate(ks):
        rki4_build_blocks(st, layer, K, b)


def _finalized(bt, sl, max_fin=None):
    out = set()
    for r, s in enumerate(sl):
        nf = s // PAGE if max_fin is None else min(s // PAGE, max_fin)
        out.update(int(x) for x in bt[r, :nf])
    return out


def _case(seed, n_kv=2):
    # row 1 shares row 0's first two blocks (prefix sharing); row 2 has no
    # finalized page
    case = make_case(seed, n_kv, 4, [16 * 40 + 3, 16 * 25, 7], build=False)
    case.bt[1, :2] = case.bt[0, :2]
    return case


def test_bulk_equals_per_layer_build():
    from locks.selection import rki4_build_bulk
    case = _case(21)
    L = 3
    d, ks = _layers(case, L, 1)
    sl = np.array(case.seq_lens)
    max_fin = int((sl // PAGE).max())
    print(f"[case] bulk L={L} NB={case.NB} sl={case.seq_lens}", flush=True)
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    n = rki4_build_bulk(a, ks, d["bt"], d["sl"], 3, max_fin)
    b = _state(case.NB, L, case.n_kv, 3, case.MP)
    _per_layer(b, ks, _finalized(case.bt, sl))
    _assert_same(_slab_bytes(a), _slab_bytes(b))
    assert n >= L * len(_finalized(case.bt, sl))
    assert int(a.refresh_mark.sum().item()) == 0
    assert int(a.refresh_count.item()) == len(_finalized(case.bt, sl))
    # never-finalized blocks keep the NaN tag
    tag = a.pp_tag.float().cpu().numpy()
    unfin = sorted(set(range(case.NB)) - _finalized(case.bt, sl))
    assert np.isnan(tag[:, unfin]).all()


def test_bulk_respects_max_fin():
    from locks.selection import rki4_build_bulk
    case = _case(22)
    L = 2
    d, ks = _layers(case, L, 2)
    sl = np.array(case.seq_lens)
    print("[case] bulk max_fin=10", flush=True)
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    rki4_build_bulk(a, ks, d["bt"], d["sl"], 3, 10)
    b = _state(case.NB, L, case.n_kv, 3, case.MP)
    _per_layer(b, ks, _finalized(case.bt, sl, max_fin=10))
    _assert_same(_slab_bytes(a), _slab_bytes(b))


@pytest.mark.parametrize("rows", [None, [1], [2, 0]])
def test_tail_builds_last_finalized_page(rows):
    import torch
    from locks.selection import rki4_build_tail
    case = _case(23)
    L = 3
    d, ks = _layers(case, L, 3)
    print(f"[case] tail rows={rows}", flush=True)
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    rr = None if rows is None else torch.tensor(rows, device="cuda")
    n = rki4_build_tail(a, ks, d["bt"], d["sl"], 3, rr)
    want = set()
    for r in (range(3) if rows is None else rows):
        want.add(int(case.bt[r, max(case.seq_lens[r] // PAGE - 1, 0)]))
    b = _state(case.NB, L, case.n_kv, 3, case.MP)
    _per_layer(b, ks, want)
    _assert_same(_slab_bytes(a), _slab_bytes(b))
    assert n == L * (3 if rows is None else len(rows))


def test_delta_rebuilds_only_stale_blocks():
    import torch
    from locks.selection import rki4_build_bulk, rki4_build_delta
    case = _case(24)
    L = 3
    d, ks = _layers(case, L, 4)
    sl = np.array(case.seq_lens)
    max_fin = int((sl // PAGE).max())
    fin = sorted(_finalized(case.bt, sl))
    x, y, z = fin[3], fin[7], fin[11]
    # a zero in the tag window, later flipped to -0 (equal as numbers)
    ks[1][z, PAGE - 1, 0, 0] = 0.0
    print(f"[case] delta stale={x} untagged={y} signed-zero={z}", flush=True)
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    rki4_build_bulk(a, ks, d["bt"], d["sl"], 3, max_fin)
    assert rki4_build_delta(a, ks, d["bt"], d["sl"], 3, max_fin) == 0

    y_orig = ks[0][y, PAGE - 1, 0, 100].clone()
    ks[2][x, PAGE - 1, 1, 3] += 1.0                  # inside the tag: stale
    ks[0][y, PAGE - 1, 0, 100] += 1.0                # outside the tag: not seen
    ks[1][z, PAGE - 1, 0, 0] = -0.0                  # -0 == +0: not stale
    n = rki4_build_delta(a, ks, d["bt"], d["sl"], 3, max_fin)
    assert n == L * 1
    # b: every block built from the content a's summaries were built from
    b = _state(case.NB, L, case.n_kv, 3, case.MP)
    ks[0][y, PAGE - 1, 0, 100] = y_orig
    ks[1][z, PAGE - 1, 0, 0] = 0.0
    _per_layer(b, ks, fin)
    _assert_same(_slab_bytes(a), _slab_bytes(b))

    # a longer settled length finalizes one more page of row 0: never built
    # (NaN tag) -> stale by construction
    sl2 = d["sl"].clone()
    sl2[0] += PAGE
    n = rki4_build_delta(a, ks, d["bt"], sl2, 3, max_fin + 1)
    assert n == L * 1
    assert int(a.refresh_mark.sum().item()) == 0


def test_tail_replays_in_a_graph():
    """The tail producer is capturable: every replay rebuilds from the live K."""
    import torch
    from locks.selection import rki4_build_tail
    case = _case(25)
    L = 2
    d, ks = _layers(case, L, 5)
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    rows = torch.tensor([0, 1], device="cuda")
    rki4_build_tail(a, ks, d["bt"], d["sl"], 3, rows)          # allocates the buffers
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rki4_build_tail(a, ks, d["bt"], d["sl"], 3, rows)
    torch.cuda.synchronize()
    blk = int(case.bt[0, case.seq_lens[0] // PAGE - 1])
    for rep in range(3):
        print(f"[case] tail graph replay {rep}", flush=True)
        ks[rep % L][blk, 2, 0, :] += 0.5
        g.replay()
        torch.cuda.synchronize()
        b = _state(case.NB, L, case.n_kv, 3, case.MP)
        _per_layer(b, ks, {blk, int(case.bt[1, case.seq_lens[1] // PAGE - 1])})
        _assert_same(_slab_bytes(a), _slab_bytes(b))


def test_gate_keeps_every_finalized_page_fresh():
    """Decode steps through the host gate: the forward writes each step's key
    AFTER the refresh, so a page's last key lands one step after it
    finalizes.  After every step, every page below settled // page must hold
    the summary a fresh build of the current K gives (and nothing else is
    required); an arrival and a frozen drain step are included."""
    import torch
    from locks.backend.refresh import RefreshGate
    n_kv, L, MP = 2, 2, 12
    NB = 2 * MP + 2
    g = torch.Generator().manual_seed(7)
    kvs = [torch.randn(NB, 2, PAGE, n_kv, 128, generator=g).to(torch.bfloat16).cuda()
           for _ in range(L)]
    ks = [kv[:, 0] for kv in kvs]
    perm = torch.randperm(NB, generator=g)[:2 * MP].view(2, MP).to(torch.int32)
    bt = perm.cuda()
    st = _state(NB, L, n_kv, 2, MP)
    gate = RefreshGate(PAGE)

    def write_token(r, pos):                     # the forward writes K of token pos
        blk = int(perm[r, pos // PAGE])
        for K in ks:
            K[blk, pos % PAGE] = torch.randn(n_kv, 128, generator=g).to(torch.bfloat16).cuda()

    lens = [37]                                  # row 0 prefilled 36 tokens + 1 in flight
    qlen = [37]
    for step in range(40):
        if step == 12:                           # arrival of row 1 (prefill 20 tokens)
            lens, qlen = lens + [20], [1, 20]
        elif step == 25:                         # drain replay: nothing moves
            qlen = [1] * len(lens)
        n = len(lens)
        qs = np.concatenate([[0], np.cumsum(qlen)])
        sl_dev = torch.tensor(lens, dtype=torch.int32, device="cuda")
        qs_dev = torch.tensor(qs, dtype=torch.int32, device="cuda")
        gate.refresh(st, ks, bt, sl_dev, qs_dev, n, np.array(lens), qs)
        # check every settled page against a fresh build
        settled = [lens[r] - qlen[r] for r in range(n)]
        fin = set()
        for r in range(n):
            fin.update(int(x) for x in perm[r, :settled[r] // PAGE])
        ref = _state(NB, L, n_kv, 2, MP)
        if fin:
            _per_layer(ref, ks, fin)
        a, b = _slab_bytes(st), _slab_bytes(ref)
        rows_ = [blk * n_kv + kh for blk in sorted(fin) for kh in range(n_kv)]
        for name in SLABS:
            x = a[name].reshape(L, NB * n_kv, -1)[:, rows_]
            y = b[name].reshape(L, NB * n_kv, -1)[:, rows_]
            np.testing.assert_array_equal(x, y, err_msg=f"step {step} {name}")
        # the forward of this step writes its query tokens' keys
        for r in range(n):
            for pos in range(lens[r] - qlen[r], lens[r]):
                write_token(r, pos)
        if step != 24:                           # step 25 replays step 24's lengths
            lens = [x + 1 for x in lens]
        qlen = [1] * n
    print(f"[case] gate steps ok, built_once={gate.built_once}", flush=True)


def test_mla_latent_refresh_equals_per_layer_build():
    """The batched producers serve the MLA latent summaries too (head_dim 512,
    one latent head): bulk and delta over the latent views of the cache give
    the bytes of the per-layer latent build, int8 RoPE summary included."""
    import torch
    from locks.selection import MlaState, mla_build_blocks, rki4_build_bulk, rki4_build_delta
    L, NB, MP = 2, 40, 16
    g = torch.Generator().manual_seed(11)
    caches = [torch.randn(NB, PAGE, 576, generator=g).to(torch.bfloat16).cuda() for _ in range(L)]
    lat = [c[:, :, None, :512] for c in caches]            # (NB, page, 1, 512) views
    perm = torch.randperm(NB, generator=g)[:2 * MP].view(2, MP).to(torch.int32)
    bt = perm.cuda()
    sl = torch.tensor([16 * 11 + 4, 16 * 6], dtype=torch.int32, device="cuda")

    def state():
        return MlaState("cuda", num_layers=L, num_blocks=NB, n_heads=16, max_reqs=2,
                        max_pages=MP, budget_pages=8, sink_pages=1, window_pages=2, rope="int8")

    print("[case] mla latent bulk/delta", flush=True)
    a = state()
    rki4_build_bulk(a, lat, bt, sl, 2, 11)
    fin = sorted(set(perm[0, :11].tolist()) | set(perm[1, :6].tolist()))
    b = state()
    for layer in range(L):
        mla_build_blocks(b, layer, caches[layer], torch.tensor(fin, dtype=torch.int32))
    _assert_same(_slab_bytes(a), _slab_bytes(b))
    _assert_same_rope(a, b)
    assert a.pp_rk8.abs().sum() > 0                       # the int8 RoPE summary was built
    assert rki4_build_delta(a, lat, bt, sl, 2, 11) == 0
    caches[1][fin[2], PAGE - 1, 5] += 1.0                  # latent tag channel
    caches[1][fin[2], PAGE - 1, 512 + 7] += 3.0            # and a RoPE key of the same token
    assert rki4_build_delta(a, lat, bt, sl, 2, 11) == L
    for layer in range(L):
        mla_build_blocks(b, layer, caches[layer], torch.tensor([fin[2]], dtype=torch.int32))
    _assert_same(_slab_bytes(a), _slab_bytes(b))
    _assert_same_rope(a, b)


def test_bulk_replays_in_a_graph():
    """The bulk producer is capturable too (no host sync): each replay
    rebuilds every finalized page from the live K, which changes between
    replays."""
    import torch
    from locks.selection import rki4_build_bulk
    case = _case(26)
    L = 2
    d, ks = _layers(case, L, 6)
    sl = np.array(case.seq_lens)
    max_fin = int((sl // PAGE).max())
    a = _state(case.NB, L, case.n_kv, 3, case.MP)
    rki4_build_bulk(a, ks, d["bt"], d["sl"], 3, max_fin)      # allocates the buffers
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rki4_build_bulk(a, ks, d["bt"], d["sl"], 3, max_fin)
    torch.cuda.synchronize()
    fin = _finalized(case.bt, sl)
    some = sorted(fin)[:5]
    for rep in range(3):
        print(f"[case] bulk graph replay {rep}", flush=True)
        for blk in some:
            ks[rep % L][blk, 3, 1, :] -= 0.25
        g.replay()
        torch.cuda.synchronize()
        b = _state(case.NB, L, case.n_kv, 3, case.MP)
        _per_layer(b, ks, fin)
        _assert_same(_slab_bytes(a), _slab_bytes(b))
        assert int(a.refresh_mark.sum().item()) == 0
