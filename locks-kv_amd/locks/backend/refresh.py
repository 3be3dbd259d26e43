"""Summary refresh gate: which rebuild a decode step needs, decided on the host.

Mirrors the builder's refresh-skip gate (src/locks/backend/builder.py:
1138-1282 ``_maybe_refresh``, helpers :1284-1392).  Summaries change only
when a page finalizes or a request slot is reused; both show in the
runner's HOST copies of ``seq_lens`` and ``query_start_loc``, so the gate
needs no device sync:

* steady batch (every row decoded exactly one token this step and the last
  one, or is a padded row at 0, or is frozen), no page boundary crossed:
  nothing to do;
* steady batch, some rows' SETTLED length (seq_len - query_len) reached a
  multiple of the page: ``rki4_build_tail`` for exactly those rows;
* anything else (first step, shape change, prefill -> decode, arrival, slot
  reuse, drain shuffle): ``rki4_build_bulk`` the first time, afterwards
  ``rki4_build_delta`` (content-tag scan);
* no host lengths: the per-layer tag-gated ``rki4_build_refresh``.

``need_derive`` tells the caller whether ``derive_page_params`` must run:
the page counts move only on steps that crossed a boundary or on full steps.
The device side of every branch is the batched producers in
``locks.selection.rki4_build``; this module holds only host logic and the
pinned row buffers that carry the tail rows to the device without a sync.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class RefreshPlan:
    kind: str                       # "skip" | "tail" | "bulk" | "delta" | "legacy"
    need_derive: bool
    rows: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int64))
    max_fin: int = 0


def _host_lens(x, n):
    if x is None:
        return None
    a = x.numpy() if hasattr(x, "numpy") else np.asarray(x)
    return np.asarray(a[:n], dtype=np.int64)


class RefreshGate:
    """Per-engine refresh state (one per model runner).

    ``plan`` is pure host logic; ``refresh`` runs the chosen producer."""

    def __init__(self, page: int):
        self.page = int(page)
        self._prev = None           # seq_lens of the previous step
        self._prev_st = None        # settled lengths of the previous step
        self.built_once = False
        self._pin = None
        self._rows_dev = None
        self._par = 0

    def reset(self):
        self._prev = self._prev_st = None
        self.built_once = False

    def plan(self, seq_lens_cpu, query_start_loc_cpu, n_req: int) -> RefreshPlan:
        """Decide this step's refresh from the host lengths
        (builder.py:1200-1270).  ``seq_lens_cpu`` counts this step's
        in-flight tokens; ``query_start_loc_cpu`` has n_req + 1 entries."""
        page = self.page
        cur = _host_lens(seq_lens_cpu, n_req)
        qs = _host_lens(query_start_loc_cpu, n_req + 1)
        if cur is None or qs is None or qs.shape[0] < n_req + 1:
            self._prev = self._prev_st = None
            return RefreshPlan("legacy", True)
        # settled = tokens whose K earlier steps already wrote
        cur_st = np.maximum(cur - (qs[1:n_req + 1] - qs[:n_req]), 0)
        prev, prev_st = self._prev, self._prev_st
        full, crossed = True, None
        if (prev is not None and prev.shape == cur.shape and prev_st is not None
                and prev_st.shape == cur_st.shape):
            # one token this step AND one token last step (a row leaving a
            # chunked prefill advances seq_len by one but settled by a chunk)
            adv = (cur == prev + 1) & (cur_st == prev_st + 1)
            pad = (cur == 0) & (prev == 0)                    # padded decode rows
            frozen = (cur == prev) & (cur_st == prev_st)      # drain replays
            if bool(np.all(adv | pad | frozen)):
                full = False
                # fires one step after the boundary, when the page's last
                # key is written (settled % page == 0)
                crossed = (cur_st % page == 0) & adv
        self._prev, self._prev_st = cur.copy(), cur_st.copy()
        if full:
            max_fin = int(cur_st.max()) // page if cur_st.size else 0
            kind = "delta" if self.built_once else "bulk"
            return RefreshPlan(kind, True, max_fin=max_fin)
        rows = np.nonzero(crossed)[0].astype(np.int64)
        if rows.size:
            return RefreshPlan("tail", True, rows=rows)
        return RefreshPlan("skip", False)

    def _rows_to_device(self, rows: np.ndarray, device, cap: int):
        """Host rows -> device through pinned ping-pong buffers: the copy is
        stream-ordered before the build and never blocks the host
        (builder.py:1284-1312)."""
        import torch
        k = rows.shape[0]
        if self._pin is None or self._pin[0].shape[0] < k:
            n = max(k, cap)
            self._pin = [torch.empty(n, dtype=torch.int32, pin_memory=True) for _ in range(2)]
            self._rows_dev = [torch.empty(n, dtype=torch.int32, device=device) for _ in range(2)]
        p = self._par = self._par ^ 1
        self._pin[p][:k].copy_(torch.from_numpy(rows.astype(np.int32)))
        self._rows_dev[p][:k].copy_(self._pin[p][:k], non_blocking=True)
        return self._rows_dev[p][:k]

    def refresh(self, st, K_layers, block_table, seq_lens, query_start_loc, n_req: int,
                seq_lens_cpu=None, query_start_loc_cpu=None) -> bool:
        """Plan and run this step's refresh; returns ``need_derive``.

        ``seq_lens`` / ``query_start_loc`` are the device tensors of the step
        (builder.py:1354-1392 use settled lengths on the device for bulk,
        delta and the legacy path, and ``seq_lens - 1`` for the tail)."""
        from ..selection import (rki4_build_bulk, rki4_build_delta, rki4_build_refresh,
                                 rki4_build_tail)
        plan = self.plan(seq_lens_cpu, query_start_loc_cpu, n_req)
        if plan.kind == "skip":
            return False
        if plan.kind == "tail":
            rows = self._rows_to_device(plan.rows, block_table.device, max(n_req, 1))
            rki4_build_tail(st, K_layers, block_table, (seq_lens[:n_req] - 1).clamp(min=0),
                            n_req, rows)
            return True
        ql = query_start_loc[1:n_req + 1] - query_start_loc[:n_req]
        settled = (seq_lens[:n_req] - ql).clamp(min=0)
        if plan.kind == "legacy":
            for layer, K in enumerate(K_layers):
                rki4_build_refresh(st, layer, K, block_table, settled, n_req)
            return True
        if plan.kind == "delta":
            rki4_build_delta(st, K_layers, block_table, settled, n_req, plan.max_fin)
        else:
            rki4_build_bulk(st, K_layers, block_table, settled, n_req, plan.max_fin)
            self.built_once = True      # later full steps scan tags (NaN = never built)
        return True
