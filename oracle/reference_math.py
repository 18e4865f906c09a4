"""ORACLE -- test infrastructure, not product code.

Two independent restatements of one GPT-2 decode step, used to pin the
oracle interpreter (oracle/interp.py) against what the mathematics fixes:

  * ``textbook_step``: plain NumPy matrix products, following the question
    definitions (reference ``QUESTIONS.md:13-88``): embed; per layer
    LayerNorm (biased variance, eps 1e-5), QKV, cache row t, causal scores
    divided by sqrt(head_dim), max-subtracted softmax, weighted values,
    projection + residual, LayerNorm, tanh-GELU MLP + residual; final
    LayerNorm, tied head, argmax with the lowest id on a tie.
  * ``brute_step``: the same with explicit Python loops and float64
    accumulation, for tiny shapes only.

Neither follows the interpreter's operation order, so they agree with it
within a floating-point tolerance, not bit for bit. Only ``tests/`` imports this.
"""
from __future__ import annotations

import math

import numpy as np


def _ln(x, w, b, eps=1e-5):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def _gelu(u):
    return 0.5 * u * (1.0 + np.tanh(0.7978845608028654 * (u + 0.044715 * u ** 3)))


def textbook_step(W, x, t, keys, vals, n_head):
    """One decode step for one row; keys/vals [L, tmax, H, E] are updated at row t."""
    L = W['qkvw'].shape[0]
    d = W['wte'].shape[1]
    E = d // n_head
    z = W['wte'][x].astype(np.float64) + W['wpe'][t].astype(np.float64)
    for l in range(L):
        a = _ln(z, W['ln1w'][l], W['ln1b'][l])
        qkv = a @ W['qkvw'][l] + W['qkvb'][l]
        q = qkv[:d].reshape(n_head, E)
        keys[l, t] = qkv[d:2 * d].reshape(n_head, E)
        vals[l, t] = qkv[2 * d:].reshape(n_head, E)
        K = keys[l, :t + 1].astype(np.float64)           # [s, H, E]
        V = vals[l, :t + 1].astype(np.float64)
        sc = np.einsum('he,she->hs', q, K) / math.sqrt(E)
        sc = sc - sc.max(-1, keepdims=True)
        p = np.exp(sc)
        p = p / p.sum(-1, keepdims=True)
        o = np.einsum('hs,she->he', p, V).reshape(d)
        z = z + o @ W['ow'][l] + W['ob'][l]
        bb = _ln(z, W['ln2w'][l], W['ln2b'][l])
        z = z + _gelu(bb @ W['fcw'][l] + W['fcb'][l]) @ W['pw'][l] + W['pb'][l]
    c = _ln(z, W['lnfw'], W['lnfb'])
    logit = W['wte'].astype(np.float64) @ c
    return logit, int(np.argmax(logit))


def brute_step(W, x, t, keys, vals, n_head):
    """Explicit loops (tiny shapes). keys/vals are float64 lists-of-arrays updated in place."""
    L = len(W['qkvw'])
    V_, d = W['wte'].shape
    E = d // n_head

    def ln(vec, w, b):
        m = sum(vec) / d
        var = sum((v - m) * (v - m) for v in vec) / d
        return [(vec[i] - m) / math.sqrt(var + 1e-5) * float(w[i]) + float(b[i]) for i in range(d)]

    z = [float(W['wte'][x][i]) + float(W['wpe'][t][i]) for i in range(d)]
    for l in range(L):
        a = ln(z, W['ln1w'][l], W['ln1b'][l])
        qkv = [sum(a[i] * float(W['qkvw'][l][i][j]) for i in range(d)) + float(W['qkvb'][l][j])
               for j in range(3 * d)]
        for hh in range(n_head):
            for e in range(E):
                keys[l][t][hh][e] = qkv[d + hh * E + e]
                vals[l][t][hh][e] = qkv[2 * d + hh * E + e]
        o = [0.0] * d
        for hh in range(n_head):
            sc = [sum(qkv[hh * E + e] * float(keys[l][s][hh][e]) for e in range(E)) / math.sqrt(E)
                  for s in range(t + 1)]
            mx = max(sc)
            ex = [math.exp(v - mx) for v in sc]
            tot = sum(ex)
            for e in range(E):
                o[hh * E + e] = sum(ex[s] / tot * float(vals[l][s][hh][e]) for s in range(t + 1))
        z = [z[k] + sum(o[i] * float(W['ow'][l][i][k]) for i in range(d)) + float(W['ob'][l][k]) for k in range(d)]
        b = ln(z, W['ln2w'][l], W['ln2b'][l])
        f = len(W['fcb'][l])
        u = [sum(b[i] * float(W['fcw'][l][i][k]) for i in range(d)) + float(W['fcb'][l][k]) for k in range(f)]
        g = [0.5 * v * (1 + math.tanh(0.7978845608028654 * (v + 0.044715 * v * v * v))) for v in u]
        z = [z[k] + sum(g[i] * float(W['pw'][l][i][k]) for i in range(f)) + float(W['pb'][l][k]) for k in range(d)]
    c = ln(z, W['lnfw'], W['lnfb'])
    logit = [sum(c[i] * float(W['wte'][n][i]) for i in range(d)) for n in range(V_)]
    best = max(logit)
    return logit, min(n for n in range(V_) if logit[n] == best)
