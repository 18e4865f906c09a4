"""Write oracle fixtures for the full-size benchmark configurations.

    python tests/golden/make_configs.py [KEY ...]     (keys: c1 c2 c3 c4 c4b1 c5; default all)

The GPU parity tests run the exact kernels ``bench.py`` times, at the
configurations' real sizes, and compare them with these fixtures. A fixture
is this repository's CPU oracle (``oracle/decode.py`` over ``oracle/interp.py``)
run once here, because the full runs take minutes of CPU per row:

  * weights: ``vesta.weights.RandomGPT2(model, 0)``; prompts:
    ``random_prompts(B, P, 50257, seed=1)`` (the benchmark's inputs);
  * for each checked row, greedy decode of ``gen`` tokens; per generated token
    the oracle's token, its top-2 logit margin, and at the signature steps the
    logits at a fixed id set (the step's top-16 ids plus 48 ids drawn once
    from ``default_rng(7)``).

``tests/test_oracle.py`` re-derives the start of a fixture with the live
oracle, so a fixture cannot drift from the oracle it caches.
"""
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(REPO, 'vesta-gpu_amd'), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

N_TOP, N_FIXED = 16, 48
# key: (model, rows B, prompt P, generated tokens checked, rows checked, signature steps)
CONFIGS = {
    'c1': ('small', 1, 128, 256, (0,), None),
    'c2': ('small', 8, 128, 256, tuple(range(8)), None),
    'c3': ('small', 32, 768, 12, (0, 1, 7, 15, 16, 24, 30, 31), None),
    'c4': ('medium', 8, 256, 8, tuple(range(8)), None),
    'c4b1': ('medium', 1, 256, 8, (0,), None),
    'c5': ('xl', 64, 128, 8, (0, 1, 15, 31, 32, 47, 62, 63), None),
}
N_LAYER = {'small': 12, 'medium': 24, 'xl': 48}


def fixed_ids(vocab=50257):
    return np.sort(np.random.default_rng(7).choice(vocab, N_FIXED, replace=False)).astype(np.int32)


def signature_steps(gen):
    """Generated-token indices whose logits the fixture keeps (all of a short
    run; the first four and every 16th of a long one)."""
    if gen <= 8:
        return list(range(gen))
    return sorted(set(range(4)) | set(range(15, gen, 16)))


def program_text(model):
    from vesta import PROGRAMS
    name = {'small': 'gpt2.vst', 'medium': 'gpt2_medium.vst', 'xl': 'gpt2_xl.vst'}[model]
    return (PROGRAMS / name).read_text(encoding='utf-8')


def _row(args):
    model, prompt, gen, sig_steps = args
    from oracle import decode
    from vesta.weights import RandomGPT2, stacked
    hf = RandomGPT2(model, 0)
    W = decode.oracle_weights(stacked(hf.numpy_state(), N_LAYER[model]))
    del hf
    text = program_text(model)
    row = decode.Row(text, W, len(prompt) + gen)
    fid = fixed_ids()
    toks, margins, sids, svals = [], [], [], []
    P = len(prompt)
    for i in range(P + gen - 1):
        if i < P:
            row.x = int(prompt[i])
        logit, nxt, margin = row.step()
        if i >= P - 1:
            k = i - (P - 1)
            toks.append(nxt)
            margins.append(margin)
            if k in sig_steps:
                top = np.argsort(-logit, kind='stable')[:N_TOP].astype(np.int32)
                ids = np.concatenate([top, fid])
                sids.append(ids)
                svals.append(logit[ids].astype(np.float32))
    return (np.array(toks, np.int32), np.array(margins, np.float32), np.stack(sids), np.stack(svals))


def make(key, workers):
    from vesta.weights import random_prompts
    model, B, P, gen, rows, _ = CONFIGS[key]
    prompts = random_prompts(B, P, 50257, seed=1)
    sig = signature_steps(gen)
    t0 = time.time()
    with ProcessPoolExecutor(min(workers, len(rows))) as ex:
        res = list(ex.map(_row, [(model, prompts[r], gen, sig) for r in rows]))
    out = dict(model=model, B=B, P=P, gen=gen, rows=np.array(rows, np.int32), sig_steps=np.array(sig, np.int32),
               tokens=np.stack([r[0] for r in res]), margins=np.stack([r[1] for r in res]),
               sig_ids=np.stack([r[2] for r in res]), sig_vals=np.stack([r[3] for r in res]),
               weights_seed=0, prompt_seed=1)
    path = os.path.join(HERE, f'config_{key}.npz')
    np.savez_compressed(path, **out)
    print(f'{key}: {len(rows)} rows x {gen} tokens in {time.time() - t0:.0f} s -> {path}', flush=True)


if __name__ == '__main__':
    keys = sys.argv[1:] or list(CONFIGS)
    workers = int(os.environ.get('WORKERS', '8'))
    for key in keys:
        make(key, min(workers, 4) if CONFIGS[key][0] == 'xl' else workers)   # XL: ~7 GB per worker
