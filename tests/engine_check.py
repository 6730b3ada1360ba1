"""Teacher-forced layer checks of engine steps against the oracle (helper for
the engine parity tests).

A traced engine step records each layer's input and the Q8_K activation of
each quantization point (attention input, O input, FFN input, PLE inp_gate
and proj inputs).  The oracle then runs every layer from the engine's input
twice:

* with its own quantize_row_q8_K ("plain"): differences come from the fp32
  summation order of norms and attention and, through them, from Q8_K codes
  that round the other way when an input moved by an ulp across a .5
  boundary, or from a block scale d that moved by an ulp with its maximum
  ("flips"; the dot's scale and min terms can cancel to well below their
  sizes, so an ulp of d can move an output by 1e-5 of its maximum);
* with the engine's Q8_K injected ("q8"): only the fp32 order remains, so the
  bar is tight.

A plain excursion above the q8 bar must coincide with a Q8_K difference in
its layer, and the first quantization point of the layer whose Q8_K differ
(in the order the layer runs them) must differ by single code steps (+-1)
and block scales within D_REL of each other (a scale follows its block's
maximum, which carries the fp32-order difference of the quantized vector:
up to ~1e-4 of itself after the attention or FFN sums; a wrong element or a
wrongly rounded scale would move it much further):
the flip is then shown, not assumed.  Later points of the same layer quantize
vectors that the flip already moved, so their codes may differ by more.  A
shared-KV layer also reads the K/V its donor layer computed at this position,
so a flip at the donor's attention input explains it too.
The q8 run goes second, so the oracle's
KV cache ends up holding the rows computed from the engine's Q8_K, which the
next position reads.
"""
from __future__ import annotations

import numpy as np

from oracle import Q8K_DTYPE, Q8_SLOT_BLOCKS, Q8_SLOT_NAMES, Q8_SLOTS


def rel(a, b) -> float:
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def as_q8(raw: np.ndarray) -> np.ndarray:
    """raw BlockQ8_K bytes (n_layers, slots, blocks, 292) -> (n_layers,
    slots, Q8_SLOT_BLOCKS) of Q8K_DTYPE"""
    raw = np.ascontiguousarray(raw[:, :, :Q8_SLOT_BLOCKS, :])
    return raw.view(Q8K_DTYPE).reshape(raw.shape[0], Q8_SLOTS, Q8_SLOT_BLOCKS)


D_REL = 1e-3   # block scales at the first differing quantization point of a layer


def q8_diff(a: np.ndarray, b: np.ndarray):
    """per (layer, slot): number of differing codes and block scales, the
    largest |code step| and the largest relative block-scale difference"""
    dq = np.abs(a["qs"].astype(np.int32) - b["qs"].astype(np.int32))      # (L, S, B, 256)
    da, db = a["d"].astype(np.float64), b["d"].astype(np.float64)
    dd = a["d"].view(np.uint32) != b["d"].view(np.uint32)
    drel = np.where(dd, np.abs(da - db) / np.maximum(np.abs(db), 1e-38), 0.0)     # (L, S, B)
    n = (dq > 0).sum(axis=(2, 3)) + dd.sum(axis=2)
    return n, dq.max(axis=(2, 3)), drel.max(axis=2)


class StepCheck:
    """Per-layer errors of one engine step, given its traced layer inputs X
    ((n_layers + 1, dim)) and Q8_K (as_q8 layout)."""

    def __init__(self, om, X: np.ndarray, Qe: np.ndarray, token: int, pos: int, lm_mode: int):
        X = np.ascontiguousarray(X, np.float32)
        out = om.forward_inject(token, pos, lm_mode, X)
        Qo = om.q8_rec()
        self.logits_plain = om.logits() if lm_mode else None
        outq = om.forward_inject_q8(token, pos, lm_mode, X, Qe)
        self.logits_q8 = om.logits() if lm_mode else None
        L = om.n_layers
        self.err_plain = np.array([rel(X[l + 1], out[l]) for l in range(L)])
        self.err_q8 = np.array([rel(X[l + 1], outq[l]) for l in range(L)])
        self.n_codes, self.max_step, self.max_drel = q8_diff(Qe, Qo)
        # per layer: the code step and scale difference at the first slot whose Q8_K differ
        root = [int(np.flatnonzero(self.n_codes[l])[0]) if self.n_codes[l].any() else -1 for l in range(L)]
        self.root_step = np.array([int(self.max_step[l][r]) if r >= 0 else 0 for l, r in enumerate(root)])
        self.root_drel = np.array([float(self.max_drel[l][r]) if r >= 0 else 0.0 for l, r in enumerate(root)])
        # the slots the oracle quantized are the ones the engine traced (a
        # used slot has a positive scale unless its vector is all zero)
        self.slots_match = bool(np.array_equal(np.abs(Qo["d"]).sum(axis=2) > 0, np.abs(Qe["d"]).sum(axis=2) > 0))
        self.src = [om.kv_source(l) for l in range(L)]
        self.pos = pos

    @classmethod
    def engine(cls, em, om, token: int, pos: int, lm_mode: int) -> "StepCheck":
        """the engine's last traced step (g4e_forward / g4e_decode_steps)"""
        return cls(om, em.layer_x(), as_q8(em.layer_q8()), token, pos, lm_mode)

    def flipped(self, l: int) -> bool:
        """a Q8_K difference (codes or block scales) in layer l, or at the
        attention input of the donor whose K/V it reads"""
        return bool(self.n_codes[l].sum() > 0 or (self.src[l] != l and self.n_codes[self.src[l], 0] > 0))

    def unexplained(self, tol: float) -> list[int]:
        """layers whose plain error exceeds tol with no Q8_K difference to
        account for it"""
        return [l for l in range(len(self.err_plain)) if self.err_plain[l] > tol and not self.flipped(l)]

    def summary(self) -> str:
        flips = {Q8_SLOT_NAMES[s]: int(self.n_codes[:, s].sum()) for s in range(Q8_SLOTS)}
        return (f"pos {self.pos}: plain median {np.median(self.err_plain):.1e} max {self.err_plain.max():.1e}; "
                f"q8-injected max {self.err_q8.max():.1e}; Q8_K codes differing {flips}, "
                f"first-slot step {int(self.root_step.max())}, scale diff {self.root_drel.max():.1e}")


def prefill_checks(om, toks, tr: np.ndarray, qt: np.ndarray, pos0: int = 0) -> list[StepCheck]:
    """StepCheck of every prompt position of an engine prefill trace
    (tr (n_layers + 1, n, dim), qt raw Q8_K rows (n_layers, n, slots, blocks,
    292)), in position order"""
    return [StepCheck(om, tr[:, i, :], as_q8(qt[:, i]), int(t), pos0 + i, 0) for i, t in enumerate(toks)]


def assert_bars(checks: list[StepCheck], what: str, median_tol: float, q8_tol: float) -> None:
    """plain median, q8-injected maximum, and every plain excursion above
    q8_tol explained by single-step Q8_K flips in its layer"""
    plain = np.concatenate([c.err_plain for c in checks])
    q8 = np.concatenate([c.err_q8 for c in checks])
    codes = sum(int(c.n_codes.sum()) for c in checks)
    print(f"{what}: plain median {np.median(plain):.2e} p90 {np.percentile(plain, 90):.2e} max {plain.max():.2e}; "
          f"q8-injected median {np.median(q8):.2e} max {q8.max():.2e}; {codes} Q8_K codes differ "
          f"(first differing slot per layer: code step {max(int(c.root_step.max()) for c in checks)}, scale "
          f"diff {max(float(c.root_drel.max()) for c in checks):.1e}; any slot: code step "
          f"{max(int(c.max_step.max()) for c in checks)})")
    assert all(c.slots_match for c in checks)
    assert np.median(plain) < median_tol
    assert q8.max() < q8_tol, [c.summary() for c in checks if c.err_q8.max() >= q8_tol][:3]
    bad = [(c.pos, c.unexplained(q8_tol)) for c in checks if c.unexplained(q8_tol)]
    assert not bad, bad
    assert max(int(c.root_step.max()) for c in checks) <= 1
    assert max(float(c.root_drel.max()) for c in checks) <= D_REL
