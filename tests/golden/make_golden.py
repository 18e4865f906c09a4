"""Write golden vectors by running the reference NumPy interpreter.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py [/root/reference]

Why an import: the reference interpreter's exact fp32 results (its einsum
contraction order and dtype promotion, reference ``vesta/interp.py:183-198``)
decide greedy tokens on near-ties, and nothing else pins them. The script
loads ``vesta/interp.py`` from the reference tree by path, runs it on small
seeded inputs and stores inputs and outputs as data. Nothing of the reference
is copied: the fixtures hold numbers only.

Fixtures (tests/golden/*.npz, *.json):
  grammar_cases.npz  small programs (text in grammar_cases.json) and the
                     values they produce, one case per language form
  tiny_gpt2.npz      a 2-layer d=16 GPT-2 program, greedy tokens, logits and
                     the final cache, seeded weights from vesta.weights
  small_gpt2.npz     GPT-2-small shape, seed 0: an 8-token prompt and 8
                     greedy tokens, with per-step top-5 logits and margins
"""
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, 'vesta-gpu_amd'))

from vesta.gpt2_program import gpt2_program  # noqa: E402
from vesta.weights import GPT2Shape, random_prompts, random_state, stacked  # noqa: E402

# Each case: program text, residue inputs (name -> (list, dtype) or scalar), names to record.
GRAMMAR_CASES = {
    'law_broadcast': ('''residue a[i]
residue b[j]
axis i = 3
axis j = 4
c[i, j] = a[i] * 2 + b[j] - i * j
d[j, i] = c[i, j] / (1 + exp(-c[i, j]))
''', {'a': ([0.5, -1.25, 2.0], 'f32'), 'b': ([1.0, 2.0, -3.0, 0.25], 'f32')}, ['c', 'd']),
    'folds': ('''residue a[i, k]
axis i = 3
axis k = 5
s[i] = fold sum k: a[i, k] * a[i, k]
m[k] = fold max i: a[i, k]
n[k] = fold min i: a[i, k] - k
lo = fold min i: fold min k: a[i, k]
w[i] = fold sum k: sqrt(a[i, k] * a[i, k] + 1)
''', {'a': ([[0.1, -2.0, 3.5, 0.7, -0.3], [1.5, 0.25, -1.0, 2.0, 0.0], [-0.5, 4.0, 0.125, -2.5, 1.0]], 'f32')},
        ['s', 'm', 'n', 'lo', 'w']),
    'fork_argmin': ('''residue v[n]
axis n = 7
best = fold max n: v[n]
first = fold min n: fork v[n] == best ? n : 7
pos[n] = fork v[n] > 0 ? v[n] : 0 - v[n]
''', {'v': ([0.5, 3.0, -1.0, 3.0, 2.0, -4.0, 3.0], 'f32')}, ['best', 'first', 'pos']),
    'index_affine_emit': ('''residue x
residue t
residue tab[r, c]
residue out[r, c]
axis r = 4
axis c = 6
axis h = 2
axis e = 3
row[c] = tab[x, c] + t
q[h, e] = row[h * 3 + e] * 10
residue out[t, h * 3 + e] <- q[h, e] + 0.5
back[e] = out[t, 3 + e]
''', {'x': 2, 't': 1, 'tab': (np.arange(24, dtype=np.float32).reshape(4, 6).tolist(), 'f32'),
      'out': (np.zeros((4, 6)).tolist(), 'f16')}, ['row', 'q', 'back', 'out']),
    'step_carry': ('''residue wts[l, d]
axis l = 3
axis d = 4
z0[d] = d + 1
zl[d] = fold step l: z0 as z
    m = fold sum d: z[d] / 4
    y[d] = z[d] * wts[l, d] - m
    -> y
end
tot = fold sum d: zl[d]
''', {'wts': ([[1.0, 0.5, -1.0, 2.0], [0.25, 1.0, 1.5, -0.5], [2.0, -1.0, 0.5, 1.0]], 'f32')}, ['zl', 'tot']),
    'nested_sum_contract': ('''residue o[h, e]
residue ow[k, d]
axis h = 2
axis e = 3
axis k = 6
axis d = 4
oo[d] = fold sum h: (fold sum e: o[h, e] * ow[h * 3 + e, d])
''', {'o': (np.linspace(-1, 1, 6, dtype=np.float32).reshape(2, 3).tolist(), 'f32'),
      'ow': (np.linspace(-2, 3, 24, dtype=np.float32).reshape(6, 4).tolist(), 'f32')}, ['oo']),
}

TINY = dict(n_layer=2, d=16, n_head=4, f=64, vocab=37)


def load_reference(root):
    path = os.path.join(root, 'vesta', 'interp.py')
    spec = importlib.util.spec_from_file_location('reference_vesta_interp', path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def residues(spec):
    out = {}
    for k, v in spec.items():
        if isinstance(v, tuple):
            vals, dt = v
            out[k] = np.array(vals, dtype={'f32': np.float32, 'f16': np.float16}[dt])
        else:
            out[k] = v
    return out


def greedy_ref(ref, text, W32, prompt, gen, tmax, L, H, E, keep_logits):
    keys = np.zeros((L, tmax, H, E), np.float16)
    vals = np.zeros_like(keys)
    toks, margins, logits, top5i, top5v = [], [], [], [], []
    x = 0
    P = len(prompt)
    for i in range(P + gen - 1):
        if i < P:
            x = int(prompt[i])
        env = ref.run(text, {'x': x, 't': i, **W32, 'keys': keys, 'vals': vals})
        logit = np.asarray(env['logit'][0])
        nxt = int(env['next'][0])
        if i >= P - 1:
            toks.append(nxt)
            srt = np.argsort(-logit, kind='stable')[:5]
            top5i.append(srt)
            top5v.append(logit[srt])
            margins.append(float(logit[srt[0]] - logit[srt[1]]))
            if keep_logits:
                logits.append(logit.copy())
        x = nxt
    return dict(tokens=np.array(toks), margins=np.array(margins), top5_ids=np.array(top5i),
                top5_vals=np.array(top5v), logits=np.array(logits) if keep_logits else None,
                keys=keys, vals=vals)


def main(root='/root/reference'):
    ref = load_reference(root)
    # 1. grammar cases
    texts, arrays = {}, {}
    for name, (text, spec, record) in GRAMMAR_CASES.items():
        res = residues(spec)
        env = ref.run(text, res)
        texts[name] = {'text': text, 'record': record,
                       'inputs': {k: (v if not isinstance(v, tuple) else {'values': v[0], 'dtype': v[1]})
                                  for k, v in spec.items()}}
        for r in record:
            if r in env:
                val, axes = env[r]
                arrays[f'{name}/{r}'] = np.asarray(val)
                texts[name].setdefault('axes', {})[r] = list(axes)
            else:
                arrays[f'{name}/{r}'] = np.asarray(res[r])
    np.savez(os.path.join(HERE, 'grammar_cases.npz'), **arrays)
    with open(os.path.join(HERE, 'grammar_cases.json'), 'w') as fh:
        json.dump(texts, fh, indent=1)

    # 2. tiny GPT-2
    cfg = GPT2Shape(TINY['n_layer'], TINY['d'], TINY['n_head'], TINY['f'], vocab=TINY['vocab'], n_positions=32)
    text = gpt2_program(TINY['n_layer'], TINY['d'], TINY['n_head'], TINY['f'], TINY['vocab'], 'tiny')
    W32 = {k: v.astype(np.float32) for k, v in stacked(random_state(cfg, 3), cfg.n_layer).items()}
    prompt = random_prompts(1, 4, cfg.vocab, seed=5)[0]
    g = greedy_ref(ref, text, W32, prompt, 12, 20, cfg.n_layer, cfg.n_head, cfg.head_dim, True)
    np.savez(os.path.join(HERE, 'tiny_gpt2.npz'), prompt=prompt, tokens=g['tokens'], logits=g['logits'],
             margins=g['margins'], keys=g['keys'], vals=g['vals'], seed=3, tmax=20)

    # 3. GPT-2-small shape, short
    cfg = GPT2Shape(12, 768, 12, 3072)
    text = gpt2_program(12, 768, 12, 3072, 50257, 'small')
    W32 = {k: v.astype(np.float32) for k, v in stacked(random_state(cfg, 0), cfg.n_layer).items()}
    prompt = random_prompts(1, 8, cfg.vocab, seed=1)[0]
    g = greedy_ref(ref, text, W32, prompt, 8, 384, 12, 12, 64, False)
    np.savez(os.path.join(HERE, 'small_gpt2.npz'), prompt=prompt, tokens=g['tokens'], margins=g['margins'],
             top5_ids=g['top5_ids'], top5_vals=g['top5_vals'], seed=0, prompt_seed=1, tmax=384,
             keys_row_sum=g['keys'].astype(np.float64).sum(axis=(0, 2, 3))[:16])
    print('tiny tokens', g['tokens'])


if __name__ == '__main__':
    main(*sys.argv[1:])
