"""LOCKS sparse decode step on one MI355X: ms/step + achieved HBM GB/s.

A "step" is one bs=1 decode step of the LOCKS attention hot path over every
layer of the model: derive (once) and, per layer, rki4 score -> GQA combine +
exact top-b -> split-K sparse paged decode -> LSE merge, captured in one HIP
graph and replayed.  Inputs (K/V cache, summaries, q, block table) are
resident in HBM before the timed region.  Synthetic data: K/V ~ N(0,1) bf16
with 4 outlier channels x8 per kv head, q ~ N(0,1), block tables shuffled in
a page pool, rki4 summaries built on the GPU from that K.

Also measured in the same run: dense full-KV decode (same kernels, every
page selected) on the same GPU, the scorer's live roofline, and the CPU
oracle on a bounded sample (rank 0, N=1 only).

    python bench.py [--workload llama8b-128k|glm9b-1m|glm9b-batch|dsv2lite-mla-128k]
                    [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "locks-kv_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0
SUMMARY_BYTES = 818          # rki4 bytes per (page, kv head) read by the scorer
PAGE = 16
D = 128

WORKLOADS = {
    # Llama-3.1-8B shape, 128K, bs=1, b=2048
    "llama8b-128k": dict(layers=32, n_kv=8, G=4, seq_lens=[131072]),
    # GLM-4-9B-1M shape, 1M context
    "glm9b-1m": dict(layers=40, n_kv=2, G=16, seq_lens=[1 << 20]),
    # batched ragged GLM
    "glm9b-batch": dict(layers=40, n_kv=2, G=16, seq_lens=[262144, 196608, 131072, 65536]),
    # small smoke-size workload
    "tiny": dict(layers=2, n_kv=2, G=4, seq_lens=[16384]),
    # DeepSeek-V2-Lite MLA, 27 layers, 16 heads over one
    # latent of 512 + 64 RoPE dims, 128K, b=2048 tokens (128 pages incl. the
    # sink and the 10-page window)
    "dsv2lite-mla-128k": dict(layers=27, heads=16, seq_lens=[131072], mla=True,
                              budget_pages=128, window_pages=10),
}
MLA_LKV, MLA_DR = 512, 64
MLA_SCALE = 1.0 / math.sqrt(128 + 64)        # softmax scale over the q/k head dim (nope + rope)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def make_model(wl, budget_pages, seed=0, summaries="build", zsplit=None):
    import torch
    from locks.attention import ensure_stage_b_buffers
    from locks.selection import Rki4State
    from locks.selection.rki4_build import rki4_build_blocks

    dev = torch.device("cuda")
    L, n_kv, G, sls = wl["layers"], wl["n_kv"], wl["G"], wl["seq_lens"]
    R = len(sls)
    npg = [(s + PAGE - 1) // PAGE for s in sls]
    MP = max(npg)
    NB = sum(npg) + 64                                   # shared page pool
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    perm = torch.randperm(NB, generator=g, device=dev).to(torch.int32)
    bt = torch.zeros(R, MP, dtype=torch.int32, device=dev)
    off = 0
    for r, n in enumerate(npg):
        bt[r, :n] = perm[off:off + n]
        off += n
    st = Rki4State(dev, num_layers=L, num_blocks=NB, n_kv=n_kv, G=G, head_dim=D, page=PAGE,
                   max_reqs=R, max_pages=MP, budget=0.1, budget_pages=budget_pages,
                   zsplit=zsplit)
    ensure_stage_b_buffers(st, dev, 128)
    kv_layers = []
    t_build = 0.0
    fin = torch.cat([bt[r, : sls[r] // PAGE] for r in range(R)]).to(torch.int64)
    for layer in range(L):
        scale = torch.ones(n_kv, D, device=dev)
        for h in range(n_kv):
            ch = torch.randperm(D, generator=g, device=dev)[:4]
            scale[h, ch] = 8.0
        kv = torch.empty(NB, 2, PAGE, n_kv, D, dtype=torch.bfloat16, device=dev)
        for half in range(2):
            x = torch.randn(NB, PAGE, n_kv, D, generator=g, device=dev) * scale
            kv[:, half].copy_(x)
            del x
        kv_layers.append(kv)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if summaries == "build" or layer == 0:
            rki4_build_blocks(st, layer, kv[:, 0], fin)
        else:                                            # reuse layer 0's slab bytes
            for a in ("pp_v4", "pp_vs", "pp_c8", "pp_cs", "pp_mu8", "pp_mus", "pp_tag"):
                getattr(st, a)[layer].copy_(getattr(st, a)[0])
        torch.cuda.synchronize()
        t_build += time.perf_counter() - t0
        if layer == 0:
            log(f"layer 0 summary build: {t_build:.2f}s for {fin.numel() * n_kv} grams")
    st._layer_of = {kv.data_ptr(): i for i, kv in enumerate(kv_layers)}
    q = [torch.randn(R, n_kv * G, D, generator=g, device=dev).to(torch.bfloat16)
         for _ in range(L)]
    sl = torch.tensor(sls, dtype=torch.int32, device=dev)
    return dict(st=st, kv=kv_layers, q=q, bt=bt, sl=sl, R=R, L=L, n_kv=n_kv, G=G, MP=MP,
                NB=NB, build_s=t_build, scale=1.0 / math.sqrt(D))


def sparse_step(m, out, vsources=None, tier=None):
    """One decode step; with ``tier`` (a locks.tier.Tier) each layer runs the
    tier's residency step (plan + fetch) between selection and the decode."""
    from locks.backend import _runtime
    from locks.selection import derive_page_params
    st = m["st"]
    derive_page_params(st, m["sl"], m["R"])
    for layer in range(m["L"]):
        kv = m["kv"][layer]
        _runtime._rki4_select_adapter(m["q"][layer], kv, m["bt"], m["sl"], st, m["R"],
                                      m["scale"], None)
        if tier is not None:
            tier.step(layer, st.page_table, st.page_cnt, m["bt"], m["sl"], m["R"])
        _runtime.decode_dispatch(m["q"][layer], kv, m["bt"], m["sl"], st, out[layer],
                                 vsources[layer] if vsources else None, m["scale"], None)


def make_tier(m, mode):
    """DRAM-tier V source for every layer (mem-v): ``pool`` = every page's V
    in the pinned host pool; ``hot`` = every complete page in a hot slot of
    its own (slot = block id), partial pages from the pool; ``lru`` = every
    page's V in the pinned pool and an empty exact-LRU hot buffer of the
    reference's default size (6 x the 10 % budget's pages + sink + window per
    (layer, kv head)), filled by the tier's own residency step."""
    import torch
    from locks.tier import Tier
    L, NB, n_kv = m["L"], m["NB"], m["n_kv"]
    hot = {"hot": NB, "pool": 1}.get(mode) or Tier.recommend_hot_slots(0.1, m["MP"], n_seqs=m["R"])
    t = Tier("cuda", num_layers=L, num_blocks=NB, n_kv=n_kv, head_dim=D, page=PAGE,
             hot_slots=hot, max_reqs=m["R"], max_pages=m["MP"], max_tokens=PAGE)
    sls = m["sl"].tolist()
    partial = [int(m["bt"][r, s // PAGE]) for r, s in enumerate(sls) if s % PAGE]
    for layer in range(L):
        kv = m["kv"][layer]
        if mode == "hot":
            t.hot[layer].copy_(kv[:, 1].permute(2, 0, 1, 3))
            t.page2slot[layer].copy_(torch.arange(NB, dtype=torch.int32, device="cuda").expand(n_kv, NB))
            if partial:
                t.offload(layer, kv, partial)
        else:
            t.offload(layer, kv, list(range(NB)))
    torch.cuda.synchronize()
    return t


def dense_split(m, split=0):
    """Dense comparator split count (the dense kernel holds two workgroups
    per CU).  Measured on MI355X: 512 workgroups for the 2-row GLM 1M step
    (split 256: 5.97 TB/s; 512: 5.62), 1024 for the 8-row Llama 128K step
    (split 128 beat 64)."""
    if split:
        return int(split)
    rows = m["R"] * m["n_kv"]
    target = 512 if rows <= 2 else 1024
    return max(1, min(512, -(-target // rows)))


def make_dense(m, split=0):
    import torch
    R, n_kv, G = m["R"], m["n_kv"], m["G"]
    split = dense_split(m, split)
    mp = torch.empty(R, n_kv, split, G, device="cuda")
    lp = torch.empty_like(mp)
    ap = torch.empty(R, n_kv, split, G, D, device="cuda")
    return dict(m=mp, l=lp, acc=ap, split=split)


def dense_step(m, dn, out):
    """Dense full-KV decode of every layer: every page of every row, through
    the dense kernel (block table only, four page stages per wave)."""
    from locks.attention import decode_dense
    from locks.attention.decode import _split_kv
    for layer in range(m["L"]):
        k, v = _split_kv(m["kv"][layer])
        decode_dense(m["q"][layer], k, v, m["bt"], m["sl"], dn["m"], dn["l"], dn["acc"],
                     out[layer], n_req=m["R"], G=m["G"], split=dn["split"], scale=m["scale"])


def capture(fn):
    import torch
    fn()                                  # eager warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, steps, warmup):
    import torch
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def step_bytes(m):
    """Algorithmic HBM bytes of one sparse step (per-stage formulas)."""
    st = m["st"]
    npg = [(s + PAGE - 1) // PAGE for s in m["sl"].tolist()]
    nsc = [n - st.window_pages for n in npg]
    L, n_kv, G = m["L"], m["n_kv"], m["G"]
    cnt = st.page_cnt.cpu().numpy()
    score = sum(n_kv * P * (SUMMARY_BYTES + G * 4) for P in nsc)
    select = sum(n_kv * P * (G * 4 + 4) + n_kv * m["MP"] * 4 for P in nsc)
    decode = int(cnt.sum()) * PAGE * D * 2 * 2
    dense = sum(n_kv * n * PAGE * D * 2 * 2 for n in npg)
    return dict(score=L * score, select=L * select, decode=L * decode, dense=L * dense,
                score_per_launch=score)


def scorer_traffic(workload):
    """HBM bytes per scorer launch measured with rocprofv3 PMC (FETCH_SIZE,
    WRITE_SIZE, KiB per dispatch) and scaled by the counters' reading of a
    plain 1 GiB copy; the commands and raw counts are in profiles/."""
    path = os.path.join(ROOT, "profiles", "rki4_score_traffic.json")
    if not os.path.isfile(path):
        return None
    with open(path) as f:
        t = json.load(f)
    w = t.get(workload)
    if not w:
        return None
    return int((w["fetch_kib"] * t["fetch_factor"] + w["write_kib"] * t["write_factor"]) * 1024)


def scorer_roofline(m, reps=3):
    """Average scorer launch duration over every layer's slabs (cold across
    layers): the launches are captured in one HIP graph and its replays are
    timed with HIP events on the capture stream, so host-side launch latency
    does not starve the GPU between launches."""
    import torch
    from locks.selection import rki4_score_only
    st = m["st"]

    def launches():
        for layer in range(m["L"]):
            rki4_score_only(st, layer, m["q"][layer], m["bt"], m["sl"], m["R"], m["scale"])

    g = capture(launches)
    s = torch.cuda.current_stream()
    g.replay()                                  # warm-up replay
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * m["L"])       # us per launch


def stream_read_us(nbytes, layers, reps=3):
    """Practical read ceiling for a launch of `nbytes`: a plain streaming read
    (`locks_calib_read`) over `layers` distinct buffers, captured and timed
    like the scorer (so each launch is cold in the 256 MB Infinity Cache when
    layers x nbytes exceeds it).  Returns us per launch."""
    import torch
    from locks import _lib
    lib = _lib.load()
    nb = (int(nbytes) + 15) // 16 * 16
    buf = torch.ones(layers * nb, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def launches():
        st = _lib.stream_ptr()
        for layer in range(layers):
            _lib.check(lib.locks_calib_read(buf.data_ptr() + layer * nb, nb, sink.data_ptr(), st),
                       "calib_read")

    g = capture(launches)
    s = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * layers)
    del g, buf
    torch.cuda.empty_cache()
    return us


def host_cores():
    """Host threads this process may use: its CPU affinity, capped by
    OMP_NUM_THREADS (the GPU box's per-GPU CPU share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(a, runs=10, warmup=2):
    """BASELINE configs[0] (one GQA layer, 32 q / 8 kv heads, d 128, 16K
    context, bs=1, b = 126 + sink + window pages) through the torch CPU
    restatement of the reference's CPU path (oracle/torch_ref.py: twin
    scorer, nrm combine, torch.topk exact top-b, fp32 gather attention), at
    full size, on the host cores: median of `runs` timed runs after `warmup`
    untimed ones, per stage.  The same config's sparse step is timed on the
    GPU (HIP graph) for the ratio."""
    import statistics

    import torch

    from oracle import torch_ref as T
    wl = dict(layers=1, n_kv=8, G=4, seq_lens=[16384])
    m = make_model(wl, a.budget_pages, seed=0)
    st = m["st"]
    out = [torch.empty(1, 32, D, dtype=torch.bfloat16, device="cuda")]
    g = capture(lambda: sparse_step(m, out))
    gpu_ms = time_graph(g, 200, 20)
    cpu = lambda t: t.detach().cpu()
    slabs = {k: cpu(getattr(st, "pp_" + k)[0]) for k in ("v4", "vs", "c8", "cs", "mu8", "mus")}
    kv = cpu(m["kv"][0])
    k, v = kv[:, 0].contiguous(), kv[:, 1].contiguous()
    q, bt, sl = cpu(m["q"][0]), cpu(m["bt"]), [int(x) for x in m["sl"].tolist()]
    npg = torch.tensor([(x + PAGE - 1) // PAGE for x in sl], dtype=torch.int32)
    nsh = npg - st.window_pages
    b = torch.clamp(torch.clamp(nsh - st.sink_pages, min=1), max=st.budget_abs)
    threads = host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    stages = {"score": [], "select": [], "decode": []}
    try:
        for it in range(warmup + runs):
            t0 = time.perf_counter()
            sh = T.score_rki4(q, slabs, bt, nsh, 8, 4, m["scale"], m["MP"])
            t1 = time.perf_counter()
            comb = T.combine_nrm(sh, nsh)
            tab, cnt = T.topb_select(comb, npg, nsh, b, st.sink_pages, m["MP"])
            t2 = time.perf_counter()
            T.decode_attention(q, k, v, bt, sl, tab, cnt, 4, m["scale"])
            t3 = time.perf_counter()
            if it >= warmup:
                stages["score"].append(t1 - t0)
                stages["select"].append(t2 - t1)
                stages["decode"].append(t3 - t2)
    finally:
        torch.set_num_threads(prev)
    # the CPU path's selection must equal the GPU's on this config up to the
    # documented fp32 near-ties; report how many kept pages differ
    gtab = st.page_table.cpu()
    diff = sum(len(set(gtab[0, h, :int(st.page_cnt[0, h])].tolist())
                   ^ set(tab[0, h, :int(cnt[0, h])].tolist())) for h in range(8))
    tot = [sum(x) for x in zip(stages["score"], stages["select"], stages["decode"])]
    med = lambda xs: round(statistics.median(xs) * 1e3, 3)
    cpu_ms = med(tot)
    del g, m, out
    torch.cuda.empty_cache()
    return dict(value=cpu_ms, unit="ms/step", cores=threads, kind="port",
                sample=("BASELINE configs[0] at full size: one layer, 8 kv x 4 q heads, 16K "
                        "tokens, 1023 scored pages, b=126+2; torch CPU restatement of the "
                        f"reference CPU path; median of {runs} runs after {warmup} warm-ups"),
                cpu_model=cpu_model(), torch_threads=threads,
                stages_ms={k_: med(v_) for k_, v_ in stages.items()},
                gpu_ms_same_config=round(gpu_ms, 4),
                cpu_over_gpu=round(cpu_ms / gpu_ms, 1),
                selection_pages_differing=int(diff))


# --------------------------------------------------------------------------- #
# MLA (config 5)
# --------------------------------------------------------------------------- #
def make_mla_model(wl, seed=0, rope="exact", split=None, zsplit=None):
    import torch
    from locks.selection import MlaState, mla_build_blocks
    dev = torch.device("cuda")
    L, H, sls = wl["layers"], wl["heads"], wl["seq_lens"]
    R = len(sls)
    npg = [(s + PAGE - 1) // PAGE for s in sls]
    MP, NB = max(npg), sum(npg) + 64
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    perm = torch.randperm(NB, generator=g, device=dev).to(torch.int32)
    bt = torch.zeros(R, MP, dtype=torch.int32, device=dev)
    off = 0
    for r, n in enumerate(npg):
        bt[r, :n] = perm[off:off + n]
        off += n
    st = MlaState(dev, num_layers=L, num_blocks=NB, n_heads=H, max_reqs=R, max_pages=MP,
                  budget_pages=wl["budget_pages"], sink_pages=1, window_pages=wl["window_pages"],
                  rope=rope, split=split)
    fin = torch.cat([bt[r, : sls[r] // PAGE] for r in range(R)])
    caches, t_build = [], 0.0
    for layer in range(L):
        sc = torch.exp(torch.randn(MLA_LKV + MLA_DR, generator=g, device=dev) * 0.5)
        x = torch.randn(NB, PAGE, MLA_LKV + MLA_DR, generator=g, device=dev) * sc
        cache = x.to(torch.bfloat16)
        del x
        caches.append(cache)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        mla_build_blocks(st, layer, cache, fin)
        torch.cuda.synchronize()
        t_build += time.perf_counter() - t0
    st._layer_of = {c.data_ptr(): i for i, c in enumerate(caches)}
    if zsplit:                                   # scorer chunks per request (sweeps)
        st.score_chunk = max(2, 2 * ((MP + 2 * zsplit - 1) // (2 * zsplit)))
    q = [torch.randn(R, H, MLA_LKV + MLA_DR, generator=g, device=dev).to(torch.bfloat16)
         for _ in range(L)]
    sl = torch.tensor(sls, dtype=torch.int32, device=dev)
    return dict(st=st, cache=caches, q=q, bt=bt, sl=sl, R=R, L=L, H=H, MP=MP, NB=NB,
                build_s=t_build, scale=MLA_SCALE)


def mla_sparse_step(m, out, lse):
    from locks.backend.mla_attn import mla_forward_mqa
    for layer in range(m["L"]):                    # derive once per step (layer 0)
        mla_forward_mqa(m["q"][layer], m["cache"][layer], m["bt"], m["sl"], m["st"], m["scale"],
                        out=out[layer], lse=lse[layer], layer=layer, derive=(layer == 0))


def make_mla_dense(m, split=0):
    """Partials of the dense MLA comparator (locks_mla_decode_dense): about
    two workgroups per CU over the batch's rows."""
    import torch
    R = m["R"]
    split = split or max(1, min(512, 512 // R))
    return dict(split=split,
                m=torch.empty(R, split, 16, device="cuda"),
                l=torch.empty(R, split, 16, device="cuda"),
                acc=torch.empty(R, split, 16, MLA_LKV, device="cuda"))


def mla_dense_step(m, dn, out, lse):
    from locks.attention import mla_decode_dense
    for layer in range(m["L"]):
        mla_decode_dense(m["q"][layer], m["cache"][layer], m["bt"], m["sl"], dn["m"], dn["l"],
                         dn["acc"], out[layer], n_req=m["R"], split=dn["split"],
                         scale=m["scale"], num_blocks=m["NB"], lse=lse[layer])


def mla_step_bytes(m):
    st = m["st"]
    npg = [(s + PAGE - 1) // PAGE for s in m["sl"].tolist()]
    nsc = [n - st.window_pages for n in npg]
    cnt = int(st.page_cnt.sum().item())
    page_b = PAGE * (MLA_LKV + MLA_DR) * 2
    score = sum(P * (st.summary_bytes_per_page() + 4) for P in nsc)
    select = sum(P * 8 + m["MP"] * 4 for P in nsc)
    decode = cnt * page_b
    dense = sum(n * page_b for n in npg)
    L = m["L"]
    return dict(score=L * score, select=L * select, decode=L * decode, dense=L * dense,
                score_per_launch=score)


def mla_scorer_us(m, reps=3):
    import torch
    from locks.selection import mla_derive, mla_score_only
    st = m["st"]
    mla_derive(st, m["sl"], m["R"])

    def launches():
        for layer in range(m["L"]):
            mla_score_only(st, layer, m["q"][layer], m["cache"][layer], m["bt"], m["R"], m["scale"])

    g = capture(launches)                       # timed as graph replays, like scorer_roofline
    s = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * m["L"])


def mla_cpu_baseline(m, sample_pages=1024):
    """MLA oracle on the host: layer 0's latent score + topb_middle over a
    sample of `sample_pages` pages (scaled to the row) + attention over the
    selected pages, x layers."""
    import numpy as np
    import torch

    from oracle import locks_oracle as O
    from oracle import mla_oracle as M
    st = m["st"]
    P = min(sample_pages, int(m["sl"][0].item()) // PAGE - st.window_pages)
    to_np = lambda t: t.cpu().numpy()
    slabs = {}
    for name, attr, bf in (("v4", "pp_v4", 0), ("vs", "pp_vs", 1), ("c8", "pp_c8", 0),
                           ("cs", "pp_cs", 1), ("mu8", "pp_mu8", 0), ("mus", "pp_mus", 1)):
        t = getattr(st, attr)[0]
        a = to_np(t.view(torch.int16) if bf else t)
        slabs[name] = a.view(np.uint16) if bf else a
    cache = to_np(m["cache"][0].view(torch.int16)).view(np.uint16)
    q = to_np(m["q"][0][:1].view(torch.int16)).view(np.uint16)
    sl = [(P + st.window_pages) * PAGE]
    bt = m["bt"][:1, :P + st.window_pages].cpu().numpy()
    t0 = time.perf_counter()
    npg, nsh, b = M.mla_derive(sl, PAGE, st.window_pages, st.sink_pages, st.budget_pages)
    sc = M.mla_score_rki4(q, slabs, cache, bt, nsh, m["scale"], int(npg[0]))
    tab, cnt = O.topb_select(sc[:, None, :], npg, nsh, b, st.sink_pages, int(npg[0]))
    t1 = time.perf_counter()
    M.mla_attention(q, cache, bt, sl, tab[:, 0], cnt[:, 0], m["scale"])
    t2 = time.perf_counter()
    full_P = int(m["sl"][0].item()) // PAGE - st.window_pages
    f = full_P / P
    per_layer = (t1 - t0) * f + (t2 - t1)
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:
        cores = 1
    return dict(value=round(per_layer * m["L"] * 1e3, 3), unit="ms/step", cores=cores,
                kind="port",
                sample=(f"numpy MLA oracle, layer 0, latent score + topb_middle over {P} of "
                        f"{full_P} selectable pages (scaled x{f:.1f}), attention over the "
                        f"selected pages, x{m['L']} layers"))


def run_mla(a, wl):
    print(json.dumps(measure_mla(a, wl, a.workload)), flush=True)


def measure_mla(a, wl, workload, cpu=True):
    """The MLA workload: captured sparse step, dense
    latent comparator, scorer roofline; returns the JSON line."""
    import torch
    t0 = time.perf_counter()
    m = make_mla_model(wl, rope=a.mla_rope, split=a.mla_split or None, zsplit=a.zsplit or None)
    log(f"MLA model ready in {time.perf_counter() - t0:.1f}s (latent summary build {m['build_s']:.1f}s)")
    R, H, L = m["R"], m["H"], m["L"]
    out = [torch.empty(R, H, MLA_LKV, dtype=torch.bfloat16, device="cuda") for _ in range(L)]
    lse = [torch.empty(R, H, dtype=torch.float32, device="cuda") for _ in range(L)]
    mla_sparse_step(m, out, lse)
    torch.cuda.synchronize()
    ref_tab, ref_out = m["st"].page_table.clone(), out[-1].clone()
    g = capture(lambda: mla_sparse_step(m, out, lse))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(m["st"].page_table, ref_tab), "graph replay changed the selection"
        assert torch.equal(out[-1], ref_out), "graph replay changed the output"
    ms = time_graph(g, a.steps, a.warmup)
    by = mla_step_bytes(m)
    score_us = mla_scorer_us(m)
    score_gbps = by["score_per_launch"] / (score_us * 1e-6) / 1e9
    stream_us = stream_read_us(by["score_per_launch"], L)
    res = {}
    if not a.no_dense:
        dn = make_mla_dense(m, a.dense_split)
        outd = [torch.empty_like(o) for o in out]
        lsed = [torch.empty_like(x) for x in lse]
        gd = capture(lambda: mla_dense_step(m, dn, outd, lsed))
        ms_dense = time_graph(gd, max(3, a.steps // 5), 2)
        res = dict(dense_ms_per_step=round(ms_dense, 4),
                   dense_achieved_GBps=round(by["dense"] / (ms_dense * 1e-3) / 1e9, 1),
                   speedup_vs_dense=round(ms_dense / ms, 3))
    cpu = None if (a.no_cpu or not cpu) else mla_cpu_baseline(m)
    sparse_bytes = by["score"] + by["select"] + by["decode"]
    if "dense_ms_per_step" in res:
        ideal = by["dense"] / (HBM_PEAK_GBPS * 1e9) * 1e3
        res.update(dense_ideal_ms_per_step=round(ideal, 4), speedup_vs_ideal_dense=round(ideal / ms, 3))
    line = {
        "metric": "decode ms/step + achieved HBM GB/s, bs=1 @128K/1M ctx, b=2048",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": workload, "layers": L, "heads": H, "kv_lora_rank": MLA_LKV,
                   "rope_dim": MLA_DR, "seq_lens": wl["seq_lens"], "page": PAGE,
                   "budget_pages": wl["budget_pages"], "window_pages": wl["window_pages"],
                   "attended_pages": int(m["st"].page_cnt[0, 0].item()),
                   "mla_rope": a.mla_rope, "parallelism": "single-gpu"},
        "tokens_per_s": round(R * 1e3 / ms, 2),
        "achieved_GBps": round(sparse_bytes / (ms * 1e-3) / 1e9, 1),
        "step_algorithmic_bytes": sparse_bytes,
        **res,
        "roofline": {"bound": "hbm", "kernel": "mla_score_kernel", "achieved": round(score_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(score_gbps / HBM_PEAK_GBPS, 4),
                     "avg_launch_us": round(score_us, 3),
                     "bytes_per_launch": by["score_per_launch"],
                     # the committed PMC traffic is the default (exact-key) scorer's
                     "traffic": scorer_traffic(workload) if a.mla_rope == "exact" else None,
                     "stream_read_same_bytes_us": round(stream_us, 3),
                     "frac_of_stream_read": round(stream_us / score_us, 4)},
        "cpu_baseline": cpu,
    }
    del g, m, out, lse
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return line


def run_refresh(a, m):
    """Summary refresh lifecycle on the bench model (one JSON line): bulk
    rebuild of every finalized page in every layer, the delta tag scan with
    nothing stale, the one-row tail of a page-crossing decode step alone, and
    what the tail adds to a captured decode step (tail + step vs step)."""
    import torch
    from locks.selection import rki4_build_bulk, rki4_build_delta, rki4_build_tail

    st, ks, R = m["st"], [kv[:, 0] for kv in m["kv"]], m["R"]
    sl = (m["sl"] - 1).clamp(min=0)                      # settled lengths
    max_fin = int(sl.max().item()) // PAGE
    rows = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()

    def ms(fn, reps):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    bulk = ms(lambda: rki4_build_bulk(st, ks, m["bt"], sl, R, max_fin), 2)
    delta = ms(lambda: rki4_build_delta(st, ks, m["bt"], sl, R, max_fin), 10)
    tail = ms(lambda: rki4_build_tail(st, ks, m["bt"], sl, R, rows), 20)
    # in situ: a page-crossing decode step (tail + the sparse step) against
    # the sparse step alone, both as graph replays on a busy GPU
    out = [torch.empty(m["R"], m["n_kv"] * m["G"], D, dtype=torch.bfloat16, device="cuda")
           for _ in range(m["L"])]
    g_step = capture(lambda: sparse_step(m, out))
    g_cross = capture(lambda: (rki4_build_tail(st, ks, m["bt"], sl, R, rows), sparse_step(m, out)))
    t_step = time_graph(g_step, 30, 3)
    t_cross = time_graph(g_cross, 30, 3)
    pages = int((sl // PAGE).sum().item())
    print(json.dumps({
        "metric": "summary refresh ms", "unit": "ms", "higher_is_better": False,
        "config": {"workload": a.workload, "layers": m["L"], "n_kv": m["n_kv"],
                   "finalized_pages": pages},
        "bulk_ms": round(bulk, 3), "delta_nothing_stale_ms": round(delta, 4),
        "tail_one_row_ms": round(tail, 4),
        "step_ms": round(t_step, 4), "step_with_tail_ms": round(t_cross, 4),
        "tail_in_step_ms": round(t_cross - t_step, 4),
        "bulk_us_per_gram": round(bulk * 1e3 / (pages * m["L"] * m["n_kv"]), 4)}), flush=True)


def run_ladder(a, wl):
    """Sparse vs dense decode step over a context ladder (BASELINE configs[2]'s
    dense comparison at 16K..1M): one JSON line per context, same model shape."""
    import torch
    for ctx in [int(c) for c in a.ladder.split(",") if c]:
        w = dict(wl, seq_lens=[ctx])
        m = make_model(w, a.budget_pages, summaries=a.summaries, zsplit=a.zsplit or None)
        out = [torch.empty(m["R"], m["n_kv"] * m["G"], D, dtype=torch.bfloat16, device="cuda")
               for _ in range(m["L"])]
        g_sparse = capture(lambda: sparse_step(m, out))
        ms = time_graph(g_sparse, a.steps, a.warmup)
        dn = make_dense(m)
        outd = [torch.empty_like(o) for o in out]
        g_dense = capture(lambda: dense_step(m, dn, outd))
        ms_dense = time_graph(g_dense, max(3, a.steps // 5), 2)
        by = step_bytes(m)
        print(json.dumps({"ladder": a.workload, "ctx": ctx, "layers": m["L"],
                          "attended_pages_per_kv_head": int(m["st"].page_cnt[0, 0].item()),
                          "sparse_ms_per_step": round(ms, 4), "dense_ms_per_step": round(ms_dense, 4),
                          "speedup_vs_dense": round(ms_dense / ms, 3),
                          "dense_achieved_GBps": round(by["dense"] / (ms_dense * 1e-3) / 1e9, 1)}),
              flush=True)
        del g_sparse, g_dense, dn, outd, out, m
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama8b-128k", choices=sorted(WORKLOADS))
    ap.add_argument("--budget-pages", type=int, default=126)
    ap.add_argument("--summaries", default="build", choices=["build", "copy"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mla-rope", default="exact", choices=["exact", "int8"],
                    help="MLA scorer RoPE term: int8 RoPE summary or the exact cache keys")
    ap.add_argument("--mla-split", type=int, default=0,
                    help="MLA sparse decode split count (0: the state's default, ~4 pages per split)")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--tier", default="", choices=["", "pool", "hot", "lru"],
                    help="also time the step with V through the DRAM tier (pinned host pool, "
                         "every complete page in a hot slot, or the tier's own LRU residency)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the ragged GLM batch and MLA points of the default run")
    ap.add_argument("--no-1m", action="store_true",
                    help="default workload only: skip the GLM-4-9B 1M north-star point")
    ap.add_argument("--dense-split", type=int, default=0,
                    help="dense comparator split count (0: about two workgroups per CU)")
    ap.add_argument("--zsplit", type=int, default=0, help="scorer chunks per (req, kv head)")
    ap.add_argument("--pps-min", type=int, default=0, help="override the decode pps_min table")
    ap.add_argument("--fused-decode", type=int, default=-1,
                    help="1: one-launch decode (last split merges), 0: split + merge launches")
    ap.add_argument("--calib-copy", type=int, default=0,
                    help="only run N device copies of 1 GiB (PMC byte-counter calibration)")
    ap.add_argument("--ladder", default="",
                    help="comma-separated contexts (tokens): one sparse + dense line per context, "
                         "e.g. 16384,131072,262144,524288,1048576 (single-request GQA workloads)")
    ap.add_argument("--refresh", action="store_true",
                    help="time the summary refresh lifecycle (bulk / delta / tail) instead")
    ap.add_argument("--profile-scorer", type=int, default=0,
                    help="only launch the scorer N times per layer (for rocprof)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1"}))
        sys.exit(2)
    import torch
    if a.calib_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(a.calib_copy):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {a.calib_copy} x {src.numel() * 4} B (read + write each)")
        return
    wl = WORKLOADS[a.workload]
    if wl.get("mla"):
        if a.pps_min:
            from locks.attention import mla_decode as _mdec
            _mdec.PPS_MIN_OVERRIDE = a.pps_min
        run_mla(a, wl)
        return
    from locks.attention import decode as _dec
    if a.pps_min:
        _dec.PPS_MIN_OVERRIDE = a.pps_min
    if a.fused_decode >= 0:
        _dec.FUSED_MERGE = bool(a.fused_decode)
    if a.ladder:
        run_ladder(a, wl)
        return
    # the default run also times the Llama step through the DRAM tier's own
    # LRU residency (the `tier` object of the line); the other workloads run
    # resident
    default_tier = a.workload == "llama8b-128k" and not a.no_extra and not a.tier
    if default_tier:
        a.tier = "lru"
    res = measure_gqa(a, wl, a.workload, quickstart=(a.workload == "llama8b-128k"))
    if default_tier:
        a.tier = ""
    if res is None:
        return
    line, ms = res
    if a.workload == "llama8b-128k" and not a.no_1m:
        # the north-star target point (1M, bs=1, b=2048)
        # in the same JSON line: sparse and dense steps, scorer roofline
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        g1m, _ = measure_gqa(a, WORKLOADS["glm9b-1m"], "glm9b-1m", summaries="copy",
                             quickstart=False)
        keep = ("ms_per_step", "tokens_per_s", "achieved_GBps", "step_algorithmic_bytes",
                "dense_ms_per_step", "dense_achieved_GBps", "dense_ideal_ms_per_step",
                "speedup_vs_dense", "speedup_vs_ideal_dense", "roofline", "config")
        line["glm9b_1m"] = {k: g1m[k] for k in keep if k in g1m}
    if a.workload == "llama8b-128k" and not a.no_extra:
        # BASELINE configs[3] (ragged GLM batch) and configs[4] (MLA) in the
        # same line, each with its dense leg and scorer roofline
        keep = ("ms_per_step", "tokens_per_s", "achieved_GBps", "step_algorithmic_bytes",
                "dense_ms_per_step", "dense_achieved_GBps", "dense_ideal_ms_per_step",
                "speedup_vs_dense", "speedup_vs_ideal_dense", "roofline", "config")
        gb, _ = measure_gqa(a, WORKLOADS["glm9b-batch"], "glm9b-batch", summaries="copy",
                            quickstart=False)
        line["glm9b_batch"] = {k: gb[k] for k in keep if k in gb}
        ml = measure_mla(a, WORKLOADS["dsv2lite-mla-128k"], "dsv2lite-mla-128k", cpu=False)
        line["dsv2lite_mla_128k"] = {k: ml[k] for k in keep if k in ml}
    line["cpu_baseline"] = None if a.no_cpu else cpu_baseline(a)
    print(json.dumps(line), flush=True)


def measure_gqa(a, wl, workload, summaries=None, quickstart=False):
    """One GQA workload: the captured sparse step (value), the dense
    comparator, the scorer roofline and, for the quickstart, the README
    budget_pages=128 point.  Returns (line, ms) or None (special modes)."""
    import torch
    t0 = time.perf_counter()
    m = make_model(wl, a.budget_pages, summaries=summaries or a.summaries, zsplit=a.zsplit or None)
    log(f"{workload}: model ready in {time.perf_counter() - t0:.1f}s (summary build {m['build_s']:.1f}s)")
    if a.refresh:
        run_refresh(a, m)
        return None
    if a.profile_scorer:
        from locks.selection import derive_page_params
        derive_page_params(m["st"], m["sl"], m["R"])
        us = scorer_roofline(m, reps=a.profile_scorer)
        log(f"scorer avg {us:.2f} us/launch")
        return None
    out = [torch.empty(m["R"], m["n_kv"] * m["G"], D, dtype=torch.bfloat16, device="cuda")
           for _ in range(m["L"])]
    # eager vs graph consistency (graph replays must reproduce the eager step)
    sparse_step(m, out)
    torch.cuda.synchronize()
    ref_tab = m["st"].page_table.clone()
    ref_out = out[-1].clone()
    g_sparse = capture(lambda: sparse_step(m, out))
    for _ in range(3):
        g_sparse.replay()
        torch.cuda.synchronize()
        assert torch.equal(m["st"].page_table, ref_tab), "graph replay changed the selection"
        assert torch.equal(out[-1], ref_out), "graph replay changed the output"
    ms = time_graph(g_sparse, a.steps, a.warmup)
    by = step_bytes(m)
    sparse_bytes = by["score"] + by["select"] + by["decode"]
    log(f"{workload}: sparse step {ms:.3f} ms")
    attended = int(m["st"].page_cnt[0, 0].item())
    del g_sparse
    res = {}
    if quickstart and a.budget_pages != 128:
        # README quickstart budget (budget_pages=128: 130 attended pages)
        st = m["st"]
        keep_b = st.budget_abs
        st.budget_abs = 128
        gq = capture(lambda: sparse_step(m, out))
        ms128 = time_graph(gq, a.steps, a.warmup)
        res["budget_pages_128"] = dict(ms_per_step=round(ms128, 4),
                                       attended_pages_per_kv_head=int(st.page_cnt[0, 0].item()))
        log(f"{workload}: budget_pages=128 step {ms128:.3f} ms")
        st.budget_abs = keep_b
        del gq
        sparse_step(m, out)                  # restore the headline budget's page tables
        torch.cuda.synchronize()
    if a.tier:
        # the same step with V through the DRAM tier: bit-identical output
        t0 = time.perf_counter()
        tier = make_tier(m, a.tier)
        log(f"{workload}: tier ({a.tier}) ready in {time.perf_counter() - t0:.1f}s")
        vs = [tier.vsource(layer) for layer in range(m["L"])]
        lru = tier if a.tier == "lru" else None
        out_t = [torch.empty_like(o) for o in out]
        sparse_step(m, out_t, vs, lru)
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(out, out_t)), "tiered step differs from resident"
        gt = capture(lambda: sparse_step(m, out_t, vs, lru))
        ms_t = time_graph(gt, a.steps, a.warmup)
        v_bytes = by["decode"] // 2                           # V half of the decode bytes
        res["tier"] = dict(source=a.tier, ms_per_step=round(ms_t, 4),
                           decode_v_bytes_per_step=v_bytes,
                           v_GBps_if_all_extra_time=round(v_bytes / max((ms_t - ms) * 1e-3, 1e-9) / 1e9, 1)
                           if a.tier == "pool" else None)
        if lru is not None:
            # steady state above: the selection repeats, every page hits.  Cold:
            # empty hot buffers before each replay, every selected page misses
            # and is fetched from the pinned pool over the host link
            s_ = torch.cuda.current_stream()
            tot = 0.0
            for _ in range(5):
                tier.page2slot.fill_(-1)
                tier.slot2page.fill_(-1)
                tier.lru.zero_()
                tier.clock.zero_()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s_)
                gt.replay()
                e1.record(s_)
                torch.cuda.synchronize()
                tot += e0.elapsed_time(e1)
                assert all(torch.equal(x, y) for x, y in zip(out, out_t)), "cold tiered step differs"
            res["tier"].update(hot_slots=tier.S, cold_ms_per_step=round(tot / 5, 4),
                               selected_pages_per_step=int(attended * m["n_kv"] * m["L"] * m["R"]))
            log(f"{workload}: tier (lru) cold step {tot / 5:.3f} ms")
        log(f"{workload}: tier ({a.tier}) step {ms_t:.3f} ms vs resident {ms:.3f} ms")
        del gt, tier, vs, out_t
        torch.cuda.synchronize()
    score_us = scorer_roofline(m)
    score_gbps = by["score_per_launch"] / (score_us * 1e-6) / 1e9
    stream_us = stream_read_us(by["score_per_launch"], m["L"])
    if not a.no_dense:
        dn = make_dense(m, a.dense_split)
        outd = [torch.empty_like(o) for o in out]
        g_dense = capture(lambda: dense_step(m, dn, outd))
        ms_dense = time_graph(g_dense, max(3, a.steps // 5), 2)
        ideal = by["dense"] / (HBM_PEAK_GBPS * 1e9) * 1e3
        res.update(dense_ms_per_step=round(ms_dense, 4),
                   dense_achieved_GBps=round(by["dense"] / (ms_dense * 1e-3) / 1e9, 1),
                   dense_split=dn["split"],
                   dense_ideal_ms_per_step=round(ideal, 4),
                   speedup_vs_dense=round(ms_dense / ms, 3),
                   speedup_vs_ideal_dense=round(ideal / ms, 3))
        log(f"{workload}: dense step {ms_dense:.3f} ms (split {dn['split']})")
        del g_dense, dn, outd
    line = {
        "metric": "decode ms/step + achieved HBM GB/s, bs=1 @128K/1M ctx, b=2048",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": workload, "layers": m["L"], "n_kv": m["n_kv"], "G": m["G"],
                   "seq_lens": wl["seq_lens"], "page": PAGE, "head_dim": D,
                   "budget_pages": a.budget_pages, "attended_pages_per_kv_head": attended,
                   "summaries": summaries or a.summaries, "parallelism": "single-gpu"},
        "tokens_per_s": round(m["R"] * 1e3 / ms, 2),
        "achieved_GBps": round(sparse_bytes / (ms * 1e-3) / 1e9, 1),
        "step_algorithmic_bytes": sparse_bytes,
        **res,
        "roofline": {"bound": "hbm", "kernel": "rki4_score_kernel",
                     "achieved": round(score_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(score_gbps / HBM_PEAK_GBPS, 4),
                     "avg_launch_us": round(score_us, 3),
                     "bytes_per_launch": by["score_per_launch"],
                     "traffic": scorer_traffic(workload),
                     "stream_read_same_bytes_us": round(stream_us, 3),
                     "frac_of_stream_read": round(stream_us / score_us, 4)},
    }
    del m, out
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return line, ms

if __name__ == "__main__":
    main()
