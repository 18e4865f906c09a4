"""ORACLE -- test infrastructure, not product code.

Greedy GPT-2 decoding on the CPU through the oracle interpreter
(oracle/interp.py), one batch row at a time. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.

Protocol (reference ``bench/g0_bench.py:166-180``, ``vesta/gpt2.py:27-55``):
  * a row's state is the residue dict: token ``x``, position ``t``, the
    stacked weights and the row's ``keys``/``vals`` cache ``[L, tmax, H, E]``;
  * one step runs the whole program once: it emits row ``t`` of the cache and
    answers ``logit`` and ``next``; feedback then sets ``x <- next`` and
    ``t <- t + 1`` (reference ``vesta/lower.py:1300-1307``);
  * prefill feeds the prompt one token per step; the token chosen after the
    last prompt token is the first generated one.

Inputs match the GPU's rounding points: weights are fp32 arrays holding the
fp16 values, the cache is fp16 so an emit rounds exactly as the kernel's
fp32->fp16 store does, and all arithmetic is fp32.
"""
from __future__ import annotations

import numpy as np

from . import interp


def _aligned_f32(a):
    """fp32 copy of ``a`` whose data starts on a 64-byte boundary."""
    a = np.asarray(a)
    buf = np.empty(a.size + 16, np.float32)
    off = (-buf.ctypes.data % 64) // 4
    out = buf[off:off + a.size].reshape(a.shape)
    out[...] = a
    return out


def oracle_weights(stacked_fp16: dict) -> dict:
    """fp16 residue arrays -> fp32 arrays holding the same values (64-byte
    aligned, so the interpreter's fast path can read per-layer slabs in place)."""
    return {k: _aligned_f32(v) for k, v in stacked_fp16.items()}


def program_extents(text: str) -> dict:
    """Constant axis extents a program declares (``axis NAME = NUMBER``)."""
    out = {}
    for s in interp.parse(text):
        if s[0] == 'axis' and s[2][0] == 'num':
            out[s[1]] = s[2][1]
    return out


class Row:
    """One sequence's decode state, advanced by the oracle interpreter."""

    def __init__(self, text: str, weights32: dict, tmax: int, fast: bool = True):
        ext = program_extents(text)
        self.fast = fast
        self.text = text
        self.prog = interp.parse(text)
        self.W = weights32
        L, H, E = ext['l'], ext['h'], ext['e']
        self.keys = np.zeros((L, tmax, H, E), np.float16)
        self.vals = np.zeros_like(self.keys)
        self.x, self.t = 0, 0

    def step(self):
        """One program run; returns (logit fp32 [V], next token, top-2 margin)."""
        res = {'x': self.x, 't': self.t, **self.W, 'keys': self.keys, 'vals': self.vals}
        m = interp.Machine(res, fast=self.fast)
        m.run_block(self.prog)
        logit = np.asarray(m.env['logit'][0])
        nxt = int(m.env['next'][0])
        top2 = np.partition(logit, -2)[-2:]
        margin = float(top2[1] - top2[0])
        self.x, self.t = nxt, self.t + 1
        return logit, nxt, margin


def greedy(text: str, weights32: dict, prompt: np.ndarray, gen: int, tmax: int,
           keep_logits: bool = False, fast: bool = True):
    """Greedy decode of one row: ``gen`` tokens after ``prompt``.

    Returns dict(tokens [gen], margins [gen], logits [gen, V] if asked), where
    token k is the ``next`` answered by step ``len(prompt) - 1 + k`` and
    ``margins[k]`` is that step's top-2 logit gap.
    """
    row = Row(text, weights32, tmax, fast)
    toks, margins, logits = [], [], []
    P = len(prompt)
    for i in range(P + gen - 1):
        if i < P:
            row.x = int(prompt[i])
        logit, nxt, margin = row.step()
        if i >= P - 1:
            toks.append(nxt)
            margins.append(margin)
            if keep_logits:
                logits.append(logit.copy())
    out = dict(tokens=np.array(toks, np.int64), margins=np.array(margins))
    if keep_logits:
        out['logits'] = np.stack(logits)
    return out


def teacher_forced(text: str, weights32: dict, inputs: np.ndarray, tmax: int, fast: bool = True):
    """Run the steps for a fixed input token sequence (the GPU's own inputs).

    Returns (next tokens [n], logits [n, V], margins [n]): step i sees token
    ``inputs[i]`` at position i.
    """
    row = Row(text, weights32, tmax, fast)
    nexts, logits, margins = [], [], []
    for i, tok in enumerate(inputs):
        row.x, row.t = int(tok), i
        logit, nxt, margin = row.step()
        nexts.append(nxt)
        logits.append(logit.copy())
        margins.append(margin)
    return np.array(nexts, np.int64), np.stack(logits), np.array(margins)
