"""ORACLE — test infrastructure only. Restatement of the recurrent-state checkpoint store and policy of zerollm's hybrid
(Gated DeltaNet) models, src/model/state-checkpoints.js:18-85, used by the oracle model (oracle.OracleModel) and the
tests that check the library's own policy against it. A snapshot is a pair of numpy arrays (conv, ssm).
"""
from __future__ import annotations

# RECURRENT_CHECKPOINTS (src/model/config.js:9)
RECURRENT_CHECKPOINTS = 6


class StateCheckpoints:
    """StateCheckpoints (src/model/state-checkpoints.js:18-85)."""

    def __init__(self, max_checkpoints=None, checkpoint_every=0, boundary_ids=()):
        self.max = RECURRENT_CHECKPOINTS if max_checkpoints is None else max_checkpoints
        self.every = checkpoint_every or 0
        self.boundary_ids = set(boundary_ids or ())
        self.list = []          # [(pos, (conv, ssm))] sorted by pos
        self.rollback = None    # (pos, (conv, ssm)) or None

    @property
    def positions(self):
        return [p for p, _ in self.list]

    def wants_before(self, pos, token, want_logits, prev_no_logits):
        """wantsBefore (:37-39)."""
        return pos > 0 and ((want_logits and prev_no_logits) or token in self.boundary_ids
                            or (self.every > 0 and pos % self.every == 0))

    def save(self, pos, live):
        """save (:42-50): drop the smallest position when full."""
        if pos == 0 or self.max <= 0 or any(p == pos for p, _ in self.list):
            return
        if len(self.list) >= self.max:
            self.list.pop(0)
        self.list.append((pos, (live[0].copy(), live[1].copy())))
        self.list.sort(key=lambda c: c[0])

    def mark(self, pos, live):
        """mark (:53-58): the single rollback slot; skipped when a checkpoint already holds pos."""
        if pos == 0 or any(p == pos for p, _ in self.list):
            self.rollback = None
            return
        self.rollback = (pos, (live[0].copy(), live[1].copy()))

    def plan(self, n, pos):
        """plan (:61-67): (from, replay)."""
        if n >= pos:
            return pos, 0
        frm = 0
        for p, _ in self.list:
            if p <= n and p > frm:
                frm = p
        if self.rollback and self.rollback[0] <= n and self.rollback[0] > frm:
            frm = self.rollback[0]
        return frm, n - frm

    def drop_after(self, n):
        """dropAfter (:70-73)."""
        self.list = [c for c in self.list if c[0] <= n]
        if self.rollback and self.rollback[0] > n:
            self.rollback = None

    def restore(self, live, frm):
        """restore (:76-81): copy the snapshot at frm into the live arrays (zeros for 0)."""
        if frm == 0:
            live[0][:] = 0
            live[1][:] = 0
            return
        for p, st in self.list:
            if p == frm:
                break
        else:
            if self.rollback and self.rollback[0] == frm:
                st = self.rollback[1]
            else:
                raise RuntimeError(f"no recurrent-state snapshot at position {frm}")
        live[0][:] = st[0]
        live[1][:] = st[1]

    def clear(self):
        self.list = []
        self.rollback = None
