"""Host refresh gate (builder.py:1138-1282): hand-worked step sequences.

Every expectation below is worked out by hand from the vLLM step semantics
(seq_lens counts the in-flight token, settled = seq_lens - query_len), not
recomputed with the gate's own expressions.
"""
from __future__ import annotations

import numpy as np

from locks.backend.refresh import RefreshGate


def _qs(*qlens):
    return np.concatenate([[0], np.cumsum(qlens)])


def test_first_step_is_bulk_then_steady_skips():
    g = RefreshGate(16)
    p = g.plan([33], _qs(1), 1)                 # 32 settled tokens = 2 pages
    assert (p.kind, p.max_fin, p.need_derive) == ("bulk", 2, True)
    g.built_once = True
    for sl in range(34, 49):                   # settled 33 .. 47: inside page 2
        p = g.plan([sl], _qs(1), 1)
        assert p.kind == "skip" and not p.need_derive, sl
    p = g.plan([49], _qs(1), 1)                 # settled 48: page 2 just finished
    assert p.kind == "tail" and p.rows.tolist() == [0] and p.need_derive
    p = g.plan([50], _qs(1), 1)
    assert p.kind == "skip"


def test_tail_only_for_rows_that_crossed():
    g = RefreshGate(16)
    g.plan([20, 100, 0], _qs(1, 1, 0), 3)
    g.built_once = True
    # row 0 settled 20, row 1 settled 100, padded row 2 stays at 0
    p = g.plan([21, 101, 0], _qs(1, 1, 0), 3)   # settled 20 -> no; 100 -> no
    assert p.kind == "skip"
    # rows 0 and 1 advance to settled 21 and 101; none at a multiple of 16
    for k in range(2, 12):
        p = g.plan([20 + k, 100 + k, 0], _qs(1, 1, 0), 3)
        want = [1] if (99 + k) % 16 == 0 else []
        want = ([0] if (19 + k) % 16 == 0 else []) + want
        assert p.rows.tolist() == want, k
        assert p.kind == ("tail" if want else "skip")


def test_prefill_to_decode_transition_is_a_full_step():
    g = RefreshGate(16)
    g.plan([512], _qs(512), 1)                  # prefill chunk: settled 0
    g.built_once = True
    # first decode: seq_len +1, but settled jumps by the whole chunk
    p = g.plan([513], _qs(1), 1)
    assert p.kind == "delta" and p.max_fin == 32
    p = g.plan([514], _qs(1), 1)
    assert p.kind == "skip"


def test_frozen_and_padded_rows_are_steady():
    g = RefreshGate(16)
    g.plan([40, 0], _qs(1, 0), 2)
    g.built_once = True
    g.plan([41, 0], _qs(1, 0), 2)
    p = g.plan([41, 0], _qs(1, 0), 2)           # drain replay: nothing moved
    assert p.kind == "skip"


def test_composition_changes_are_full():
    g = RefreshGate(16)
    g.plan([40], _qs(1), 1)
    g.built_once = True
    p = g.plan([41, 7], _qs(1, 7), 2)           # arrival: shape change
    assert p.kind == "delta" and p.max_fin == 2
    p = g.plan([42, 8], _qs(1, 1), 2)           # row 1 left prefill: settled 0 -> 7
    assert p.kind == "delta"
    p = g.plan([44, 9], _qs(1, 1), 2)           # row 0 jumped by two
    assert p.kind == "delta"
    p = g.plan([45, 10], _qs(1, 1), 2)
    assert p.kind == "skip"


def test_without_host_lengths_the_legacy_path_runs():
    g = RefreshGate(16)
    assert g.plan(None, None, 1).kind == "legacy"
    assert g.plan([5], [0], 1).kind == "legacy"     # too short query_start_loc
    # the next step with lengths is a full one again
    assert g.plan([5], _qs(1), 1).kind == "bulk"


def test_mixed_step_counts_only_settled_tokens():
    g = RefreshGate(16)
    # row 0 decodes, row 1 prefills a 300-token chunk on top of 100 settled
    p = g.plan([65, 400], _qs(1, 300), 2)
    assert p.kind == "bulk" and p.max_fin == 100 // 16


# ---- property test: the gate keeps every finalized page fresh ---------------
# A model of the cache and the summaries under the producers' semantics
# (rki4_build_tail / _bulk / _delta, selection/rki4_build.py:264-315):
#   bulk   rebuilds every finalized page of the batch;
#   delta  rebuilds the finalized pages whose last key changed since their
#          build (the content tag is that key's first channels);
#   tail   rebuilds page max((seq_len - 1) // page - 1, 0) of each given row.
# Keys of a step's query tokens are written after the prologue.  Invariant
# after every prologue: each finalized page (p < settled // page) was built
# after its last key write.

from hypothesis import given, settings, strategies as hst  # noqa: E402

PG = 16


class _Model:
    def __init__(self):
        self.rows = []              # [row id, seq_len incl. in-flight, query_len]
        self.next_id = 0
        self.write_step = {}        # (row id, token) -> step of the last write
        self.built = {}             # (row id, page) -> step of the last build
        self.step = 0

    def settled(self, row):
        return max(row[1] - row[2], 0)

    def page_last_write(self, rid, p):
        return max(self.write_step.get((rid, p * PG + t), -1) for t in range(PG))

    def run(self, plan):
        n = len(self.rows)
        if plan.kind == "skip":
            return
        if plan.kind == "tail":
            for r in plan.rows:
                rid, sl, _ = self.rows[int(r)]
                self.built[(rid, max((sl - 1) // PG - 1, 0))] = self.step
            return
        for i in range(n):
            rid = self.rows[i][0]
            nf = self.settled(self.rows[i]) // PG
            if plan.kind in ("bulk", "legacy"):
                nf = min(nf, plan.max_fin) if plan.kind == "bulk" else nf
            for p in range(nf):
                key_step = self.write_step.get((rid, p * PG + PG - 1), -1)
                if plan.kind == "delta" or plan.kind == "legacy":
                    if self.built.get((rid, p), -2) > key_step:
                        continue
                self.built[(rid, p)] = self.step

    def check(self):
        for rid, sl, ql in self.rows:
            for p in range(max(sl - ql, 0) // PG):
                assert self.built.get((rid, p), -2) > self.page_last_write(rid, p), (rid, p, self.step)

    def write(self):
        for rid, sl, ql in self.rows:
            for t in range(sl - ql, sl):
                self.write_step[(rid, t)] = self.step


_ACTIONS = hst.lists(hst.tuples(hst.sampled_from(
    ["decode", "decode", "decode", "arrive", "prefill", "drop", "shuffle", "frozen", "pad"]),
    hst.integers(1, 70)), min_size=1, max_size=60)


@settings(max_examples=150, deadline=None)
@given(_ACTIONS)
def test_gate_keeps_finalized_pages_fresh(actions):
    g = RefreshGate(PG)
    m = _Model()
    prev_lens = None
    for act, k in actions:
        if act == "arrive" or not m.rows:
            m.rows.append([m.next_id, k, k])                 # prefill of k tokens
            m.next_id += 1
        elif act == "prefill":                               # a row continues a chunked prefill
            r = m.rows[k % len(m.rows)]
            r[1], r[2] = r[1] + k, k
        elif act == "drop" and len(m.rows) > 1:
            m.rows.pop(k % len(m.rows))
        elif act == "shuffle":
            m.rows = m.rows[k % len(m.rows):] + m.rows[:k % len(m.rows)]
        elif act == "frozen" and prev_lens is not None and len(prev_lens) == len(m.rows):
            for r, pl in zip(m.rows, prev_lens):             # drain replay: last step's lengths
                r[1], r[2] = pl, (1 if pl > 0 else 0)
        elif act == "pad":
            m.rows.append([m.next_id, 0, 0])                 # padded uniform-decode row
            m.next_id += 1
        lens = [r[1] for r in m.rows]
        qs = np.concatenate([[0], np.cumsum([r[2] for r in m.rows])])
        plan = g.plan(np.array(lens), qs, len(m.rows))
        if plan.kind == "bulk":
            g.built_once = True
        m.run(plan)
        m.check()
        m.write()
        m.step += 1
        prev_lens = lens
        for r in m.rows:                                     # the next step decodes by default
            if r[1] > 0:
                r[1], r[2] = r[1] + 1, 1
