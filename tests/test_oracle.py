"""The CPU oracle (oracle/) pinned three ways:

1. golden vectors written by the reference interpreter (tests/golden), bit-exact;
2. independent restatements of the mathematics (textbook NumPy GPT-2 and a
   float64 brute-force loop version on tiny shapes), within tolerance;
3. invariants: softmax rows sum to 1, fold-min-id equals np.argmax, emits
   write only row t, the fast slice path equals the faithful gather bit for bit.
"""
import json
import os

import numpy as np
import pytest

from oracle import decode, interp, reference_math
from vesta.gpt2_program import gpt2_program
from vesta.weights import GPT2Shape, random_prompts, random_state, stacked

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def _inputs(spec):
    out = {}
    for k, v in spec.items():
        if isinstance(v, dict):
            out[k] = np.array(v['values'], dtype={'f32': np.float32, 'f16': np.float16}[v['dtype']])
        else:
            out[k] = v
    return out


CASES = json.load(open(os.path.join(GOLD, 'grammar_cases.json')))


@pytest.mark.parametrize('name', sorted(CASES))
@pytest.mark.parametrize('fast', [False, True])
def test_grammar_cases_match_reference_bits(name, fast):
    case = CASES[name]
    gold = np.load(os.path.join(GOLD, 'grammar_cases.npz'))
    res = _inputs(case['inputs'])
    env = interp.run(case['text'], res, fast=fast)
    for r in case['record']:
        got = np.asarray(env[r][0]) if r in env else res[r]
        want = gold[f'{name}/{r}']
        assert got.dtype == want.dtype and got.shape == want.shape, r
        assert np.array_equal(got, want), (name, r)
        if r in env:
            assert list(env[r][1]) == case['axes'][r]


def _tiny():
    cfg = GPT2Shape(2, 16, 4, 64, vocab=37, n_positions=32)
    text = gpt2_program(2, 16, 4, 64, 37, 'tiny')
    W = decode.oracle_weights(stacked(random_state(cfg, 3), 2))
    return cfg, text, W


@pytest.mark.parametrize('fast', [False, True])
def test_tiny_gpt2_matches_reference_bits(fast):
    cfg, text, W = _tiny()
    g = np.load(os.path.join(GOLD, 'tiny_gpt2.npz'))
    out = decode.greedy(text, W, g['prompt'], len(g['tokens']), int(g['tmax']), keep_logits=True, fast=fast)
    assert np.array_equal(out['tokens'], g['tokens'])
    assert np.array_equal(out['logits'], g['logits'])


def test_small_gpt2_matches_reference_bits():
    g = np.load(os.path.join(GOLD, 'small_gpt2.npz'))
    cfg = GPT2Shape(12, 768, 12, 3072)
    W = decode.oracle_weights(stacked(random_state(cfg, int(g['seed'])), 12))
    text = gpt2_program(12, 768, 12, 3072, 50257, 'small')
    out = decode.greedy(text, W, g['prompt'], len(g['tokens']), int(g['tmax']), keep_logits=True)
    assert np.array_equal(out['tokens'], g['tokens'])
    for k in range(len(g['tokens'])):
        assert np.array_equal(out['logits'][k][g['top5_ids'][k]], g['top5_vals'][k])


def test_prompts_are_seeded():
    p = random_prompts(2, 5, 50257, seed=1)
    assert p.shape == (2, 5) and np.array_equal(p, random_prompts(2, 5, 50257, seed=1))


def test_tiny_gpt2_agrees_with_textbook_and_brute_force():
    cfg, text, W = _tiny()
    tmax = 10
    row = decode.Row(text, W, tmax)
    kt = np.zeros((2, tmax, 4, 4))
    vt = np.zeros_like(kt)
    kb = [[[[0.0] * 4 for _ in range(4)] for _ in range(tmax)] for _ in range(2)]
    vb = [[[[0.0] * 4 for _ in range(4)] for _ in range(tmax)] for _ in range(2)]
    for i, tok in enumerate([5, 9, 3, 30, 1, 36]):
        row.x, row.t = tok, i
        lo, nx, _ = row.step()
        lt, nt = reference_math.textbook_step(W, tok, i, kt, vt, 4)
        lb, nb = reference_math.brute_step(W, tok, i, kb, vb, 4)
        assert np.abs(np.asarray(lb) - lt).max() < 1e-9
        assert np.abs(lo - lt).max() < 1e-4      # fp16 cache rounding in the oracle only
        assert nx == nt == nb
        # emits wrote row i only
        assert np.array_equal(row.keys[:, i + 1:], np.zeros_like(row.keys[:, i + 1:]))
        assert np.abs(row.keys[:, i] - kt[:, i]).max() < 2e-3


def test_small_gpt2_agrees_with_textbook():
    cfg = GPT2Shape(12, 768, 12, 3072)
    W = decode.oracle_weights(stacked(random_state(cfg, 0), 12))
    text = gpt2_program(12, 768, 12, 3072, 50257, 'small')
    row = decode.Row(text, W, 16)
    kt = np.zeros((12, 16, 12, 64))
    vt = np.zeros_like(kt)
    for i, tok in enumerate([464, 3290, 50256]):
        row.x, row.t = tok, i
        lo, nx, margin = row.step()
        lt, nt = reference_math.textbook_step(W, tok, i, kt, vt, 12)
        assert np.abs(lo - lt).max() < 2e-3
        if margin > 1e-2:
            assert nx == nt


def test_softmax_weights_sum_to_one_and_argmin_is_argmax():
    text = '''residue sc[h, s]
axis h = 3
axis s = 9
mx[h] = fold max s: sc[h, s]
ex[h, s] = exp(sc[h, s] - mx[h])
w[h, s] = ex[h, s] / (fold sum s: ex[h, s])
tot[h] = fold sum s: w[h, s]
best = fold max s: sc[0, s]
first = fold min s: fork sc[0, s] == best ? s : 9
'''
    rng = np.random.default_rng(0)
    sc = rng.standard_normal((3, 9)).astype(np.float32)
    sc[0, 6] = sc[0, 2] = sc[0].max() + 1           # a tie: the lowest index wins
    env = interp.run(text, {'sc': sc})
    assert np.allclose(env['tot'][0], 1.0, atol=1e-6)
    assert int(env['first'][0]) == int(np.argmax(sc[0])) == 2


def test_errors_raised():
    with pytest.raises(NameError):
        interp.run('residue q[i]\naxis i = 2\n', {})
    with pytest.raises(ValueError):
        interp.run('residue a[i]\naxis i = 2\naxis k = 3\nb = fold sum k: a[i]\n', {'a': np.ones(2, np.float32)})
    with pytest.raises(ValueError):
        interp.run('residue a[i]\naxis i = 2\nb = a[i] * 2\n', {'a': np.ones(2, np.float32)})
    with pytest.raises(SyntaxError):
        interp.run('residue a[i]\naxis i = 2\nz[i] = fold step k: a as c\n  y[i] = c[i]\nend\n',
                   {'a': np.ones(2, np.float32)})


# ---------------------------------------------------------------- full-size fixtures
CONFIG_KEYS = ('c1', 'c2', 'c3', 'c4', 'c4b1', 'c5')


@pytest.mark.parametrize('key', CONFIG_KEYS)
def test_config_fixture_is_consistent(key):
    """Each fixture records the configuration it caches (tests/golden/make_configs.py)
    and holds plausible decode output: ids inside the vocabulary, top-2
    margins >= 0, the signature's first id the argmax (its value the largest)."""
    import importlib.util
    path = os.path.join(GOLD, f'config_{key}.npz')
    if not os.path.exists(path):
        pytest.fail(f'{path} is missing: run tests/golden/make_configs.py {key}')
    spec = importlib.util.spec_from_file_location('make_configs', os.path.join(GOLD, 'make_configs.py'))
    mc = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mc)
    g = np.load(path)
    model, B, P, gen, rows, _ = mc.CONFIGS[key]
    assert (str(g['model']), int(g['B']), int(g['P']), int(g['gen'])) == (model, B, P, gen)
    assert g['rows'].tolist() == list(rows)
    assert g['tokens'].shape == (len(rows), gen) and g['margins'].shape == (len(rows), gen)
    assert ((g['tokens'] >= 0) & (g['tokens'] < 50257)).all() and (g['margins'] >= 0).all()
    steps = g['sig_steps'].tolist()
    assert steps == mc.signature_steps(gen)
    assert g['sig_ids'].shape[:2] == (len(rows), len(steps))
    # the first signature id of a step is its argmax, i.e. the step's token
    for i in range(len(rows)):
        for j, k in enumerate(steps):
            assert g['sig_ids'][i, j, 0] == g['tokens'][i, k]
            assert g['sig_vals'][i, j, 0] == g['sig_vals'][i, j].max()
    assert (g['sig_ids'][..., mc.N_TOP:] == mc.fixed_ids()).all()


def test_config1_fixture_is_row0_of_config2():
    """Same weights and the same prompt generator: config 1's single row is
    config 2's first."""
    a, b = np.load(os.path.join(GOLD, 'config_c1.npz')), np.load(os.path.join(GOLD, 'config_c2.npz'))
    assert (a['tokens'][0] == b['tokens'][0]).all() and (a['margins'][0] == b['margins'][0]).all()


def test_config2_fixture_matches_the_live_oracle():
    """Re-derive the start of config 2's first row with the oracle (128 prompt
    steps and 4 generated tokens): tokens, margins and signature logits bit
    for bit."""
    from vesta import PROGRAMS
    from vesta.weights import RandomGPT2
    g = np.load(os.path.join(GOLD, 'config_c2.npz'))
    W = decode.oracle_weights(stacked(RandomGPT2('small', 0).numpy_state(), 12))
    text = (PROGRAMS / 'gpt2.vst').read_text()
    prompt = random_prompts(8, 128, 50257, seed=1)[0]
    out = decode.greedy(text, W, prompt, 4, 132, keep_logits=True)
    assert out['tokens'].tolist() == g['tokens'][0, :4].tolist()
    assert np.array_equal(out['margins'].astype(np.float32), g['margins'][0, :4])
    for j in range(4):
        assert np.array_equal(out['logits'][j][g['sig_ids'][0, j]], g['sig_vals'][0, j])
