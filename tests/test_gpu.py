"""GPU parity: the generated gfx950 kernel against the CPU oracle and the
reference interpreter's golden vectors (run on an MI355X with -m gpu).

Bar (north star): greedy tokens identical to the interpreter; per-step logits
within max-abs 2e-2 (fp16 weights and cache, fp32 arithmetic). Comparisons
that follow the GPU's own trajectory feed the oracle the GPU's inputs
(teacher forcing), so one near-tie cannot hide every later step.
"""
import json
import os

import numpy as np
import pytest

from conftest import PKG, REPO

pytestmark = pytest.mark.gpu
GOLD = os.path.join(REPO, 'tests', 'golden')
LOGIT_TOL = 2e-2


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('no GPU visible: -m gpu tests need an MI355X')
    return torch


def _tokens_match(label, got, want, margins, err):
    """Greedy tokens against the oracle's: a token may differ only at a step
    whose oracle top-2 margin is below twice the measured logit error `err`
    (a near-tie the tolerance itself allows); prints how many were waived."""
    got, want, margins = np.asarray(got), np.asarray(want), np.asarray(margins)
    diff = [k for k in range(len(want)) if got[k] != want[k]]
    waived = [(k, float(margins[k])) for k in diff if margins[k] < 2 * err]
    bad = [(k, float(margins[k])) for k in diff if margins[k] >= 2 * err]
    print(f'{label}: {len(want)} tokens, logit error {err:.2e}, {len(waived)} near-tie steps waived {waived}')
    assert not bad, f'{label}: tokens differ from the oracle at (step, margin) {bad}'
    assert len(waived) <= max(1, len(want) // 32), f'{label}: {len(waived)} near-tie steps waived'


@pytest.fixture(scope='module')
def small():
    from oracle import decode
    from vesta.weights import RandomGPT2, stacked
    hf = RandomGPT2('small', 0)
    W = decode.oracle_weights(stacked(hf.numpy_state(), 12))
    text = open(os.path.join(PKG, 'vesta', 'programs', 'gpt2.vst')).read()
    return hf, W, text


def _run_steps(m, feed, n_steps):
    """Reference protocol: feed[i] (or the fed-back token) then one launch per step.
    Returns inputs [n, B], logits [n, B, V], next [n, B]."""
    torch = _torch()
    ins, lg, nx = [], [], []
    for i in range(n_steps):
        if i < len(feed):
            m.x.copy_(torch.as_tensor(feed[i], dtype=torch.int32, device='cuda'))
        ins.append(m.x.cpu().numpy().copy())
        m.step()
        torch.cuda.synchronize()
        lg.append(m.logits().float().cpu().numpy().copy())
        nx.append(m.x.cpu().numpy().copy())
    return np.array(ins), np.array(lg), np.array(nx)


def test_small_gpt2_matches_reference_golden(small):
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    hf, W, text = small
    g = np.load(os.path.join(GOLD, 'small_gpt2.npz'))
    m = VestaGPT2(hf, batch=1, tmax=int(g['tmax']))
    m.reset()
    prompt, want = g['prompt'], g['tokens']
    n = len(prompt) + len(want) - 1
    ins, lg, nx = _run_steps(m, [[int(p)] for p in prompt], n)
    got = nx[len(prompt) - 1:, 0].tolist()
    assert got == want.tolist()
    # logits at the golden top-5 ids, and all logits against the oracle
    for k in range(len(want)):
        assert np.abs(lg[len(prompt) - 1 + k, 0][g['top5_ids'][k]] - g['top5_vals'][k]).max() < LOGIT_TOL
    _, olog, _ = decode.teacher_forced(text, W, ins[:, 0], int(g['tmax']))
    assert np.abs(lg[:, 0] - olog).max() < LOGIT_TOL


def test_tiny_gpt2_matches_reference_golden():
    """A 2-layer d=16 GPT-2: other tile widths, thread placements, 37-word vocab."""
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import GPT2Shape, RandomGPT2
    g = np.load(os.path.join(GOLD, 'tiny_gpt2.npz'))
    hf = RandomGPT2(GPT2Shape(2, 16, 4, 64, vocab=37, n_positions=32), int(g['seed']))
    m = VestaGPT2(hf, batch=1, tmax=int(g['tmax']))
    m.reset()
    prompt, want = g['prompt'], g['tokens']
    ins, lg, nx = _run_steps(m, [[int(p)] for p in prompt], len(prompt) + len(want) - 1)
    assert nx[len(prompt) - 1:, 0].tolist() == want.tolist()
    assert np.abs(lg[len(prompt) - 1:, 0] - g['logits']).max() < 1e-4
    keys = m.keys[0].float().cpu().numpy()
    used = len(prompt) + len(want) - 1
    assert np.abs(keys[:, :used] - g['keys'][:, :used].astype(np.float32)).max() < 2e-3


def test_local_checkpoint_matches_oracle(tmp_path):
    """A transformers GPT-2 saved with save_pretrained (safetensors + config.json),
    read back through LocalGPT2 into the decode API, two rows."""
    pytest.importorskip('transformers')
    from oracle import decode
    from test_weights import _hf_tiny
    from vesta.gpt2 import VestaGPT2
    from vesta.gpt2_program import gpt2_program
    from vesta.weights import LocalGPT2, stacked
    hf = _hf_tiny(3, wscale=5.0)
    hf.save_pretrained(tmp_path, safe_serialization=True)
    local = LocalGPT2(tmp_path)
    m = VestaGPT2(local, batch=2, tmax=16)
    m.reset()
    feed = [[5, 30], [9, 1], [3, 36], [30, 0]]
    ins, lg, nx = _run_steps(m, feed, 12)
    sd = {k: v.numpy().astype(np.float16) for k, v in local.state_dict().items()}
    W = decode.oracle_weights(stacked(sd, 2))
    text = gpt2_program(2, 16, 4, 64, 37, 'tiny')
    for r in range(2):
        onx, olog, marg = decode.teacher_forced(text, W, ins[:, r], 16)
        err = np.abs(lg[:, r] - olog).max()
        assert err < 1e-3, r
        _tokens_match(f'local checkpoint row {r}', nx[:, r], onx, marg, err)


@pytest.mark.parametrize('B', [8, 6])
def test_batch_rows_match_oracle(small, B):
    """Rows on the matrix cores: 8, and 6 (a 16-row tile with 6 rows); the
    down-projection's fold split in point groups of two column tiles."""
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    P, G = 6, 5
    m = VestaGPT2(hf, batch=B, tmax=64)
    m.reset()
    pr = random_prompts(B, P, 50257, seed=7)
    ins, lg, nx = _run_steps(m, [pr[:, i] for i in range(P)], P + G - 1)
    for r in (0, B - 1):
        onx, olog, marg = decode.teacher_forced(text, W, ins[:, r], 64)
        err = np.abs(lg[:, r] - olog).max()
        assert err < LOGIT_TOL, r
        _tokens_match(f'B={B} row {r}', nx[:, r], onx, marg, err)


@pytest.mark.parametrize('B', [2, 3])
def test_few_rows_match_oracle(small, B):
    """Two and three rows: the grid of twelve replica blocks per head, the
    LayerNorm statistics one row per wave, and the down-projection's local
    fold with its fixed-point adds started apart by block. Every row against
    the oracle, teacher-forced."""
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    P, G = 6, 5
    m = VestaGPT2(hf, batch=B, tmax=64)
    assert m.engine == 'persistent' and m.k.grid == 144
    m.reset()
    pr = random_prompts(B, P, 50257, seed=11 + B)
    ins, lg, nx = _run_steps(m, [pr[:, i] for i in range(P)], P + G - 1)
    for r in range(B):
        onx, olog, marg = decode.teacher_forced(text, W, ins[:, r], 64)
        err = np.abs(lg[:, r] - olog).max()
        assert err < LOGIT_TOL, (B, r, err)
        _tokens_match(f'B={B} row {r}', nx[:, r], onx, marg, err)


def test_medium_two_rows_match_oracle():
    """GPT-2 medium at 2 rows: the local fold at width 1024 and 16 heads, on
    twelve replica blocks per head (192 blocks). Both rows against the oracle,
    teacher-forced."""
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts, stacked
    hf = RandomGPT2('medium', 0)
    W = decode.oracle_weights(stacked(hf.numpy_state(), 24))
    text = open(os.path.join(PKG, 'vesta', 'programs', 'gpt2_medium.vst')).read()
    B, P, G = 2, 6, 5
    m = VestaGPT2(hf, batch=B, tmax=64)
    assert m.engine == 'persistent' and m.k.grid == 192
    m.reset()
    pr = random_prompts(B, P, 50257, seed=13)
    ins, lg, nx = _run_steps(m, [pr[:, i] for i in range(P)], P + G - 1)
    for r in range(B):
        onx, olog, marg = decode.teacher_forced(text, W, ins[:, r], 64)
        err = np.abs(lg[:, r] - olog).max()
        assert err < LOGIT_TOL, (r, err)
        _tokens_match(f'medium B=2 row {r}', nx[:, r], onx, marg, err)


@pytest.mark.parametrize('B', [4, 8])
def test_matrix_core_rows_long_context_match_oracle(small, B):
    """Batches on the matrix-core streams (B >= 4: MFMA tiles, the feed-forward
    down-projection split over its fold into a fixed-point residual) with the
    context past two attention slots of 56 positions: prompt and generated
    tokens in one-launch prefill and one multi-step launch, logits of the
    last step and every token against the oracle run on the GPU's inputs."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    P, G, T = 100, 24, 128
    m = VestaGPT2(hf, batch=B, tmax=T)
    m.reset()
    pr = random_prompts(B, P, 50257, seed=11 + B)
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32), mode='steps')
    torch.cuda.synchronize()
    first = m.x.cpu().numpy().copy()
    hist = torch.zeros((G - 1) * B, dtype=torch.int32, device='cuda')
    m.step(G - 1, hist)
    torch.cuda.synchronize()
    gen = np.concatenate([first[None], hist.view(G - 1, B).cpu().numpy()])     # [G, B]
    last = m.logits().float().cpu().numpy()                                       # after step P + G - 2
    for r in range(B):
        inputs = np.concatenate([pr[r], gen[:-1, r]])                             # what step i saw
        onx, olog, marg = decode.teacher_forced(text, W, inputs, T)
        err = np.abs(last[r] - olog[-1]).max()
        assert err < LOGIT_TOL, r
        _tokens_match(f'B={B} long context row {r}', gen[:, r], onx[P - 1:], marg[P - 1:], err)


def _prefill_and_generate(m, pr, G):
    """Prompt in one launch, G - 1 more steps in one launch: generated tokens
    [G, B] and the logits of the last step."""
    torch = _torch()
    B = pr.shape[0]
    m.reset()
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32), mode='steps')
    torch.cuda.synchronize()
    first = m.x.cpu().numpy().copy()
    hist = torch.zeros((G - 1) * B, dtype=torch.int32, device='cuda')
    m.step(G - 1, hist)
    torch.cuda.synchronize()
    return np.concatenate([first[None], hist.view(G - 1, B).cpu().numpy()]), m.logits().float().cpu().numpy()


def _check_rows(text, W, pr, gen, last, T, rows):
    from oracle import decode
    P, G = pr.shape[1], gen.shape[0]
    for r in rows:
        inputs = np.concatenate([pr[r], gen[:-1, r]])
        onx, olog, marg = decode.teacher_forced(text, W, inputs, T)
        err = np.abs(last[r] - olog[-1]).max()
        assert err < LOGIT_TOL, r
        _tokens_match(f'row {r}', gen[:, r], onx[P - 1:P - 1 + G], marg[P - 1:P - 1 + G], err)


@pytest.mark.slow
def test_medium_long_context_matches_oracle():
    """GPT-2 medium (configs[3] shape, 24 layers, d 1024, 16 heads) at B=1 with
    a 512-position cache: more attention slots than registers hold, so the
    softmax runs over chunks of positions (running maximum and sum)."""
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts, stacked
    hf = RandomGPT2('medium', 0)
    W = decode.oracle_weights(stacked(hf.numpy_state(), 24))
    text = open(os.path.join(PKG, 'vesta', 'programs', 'gpt2_medium.vst')).read()
    T = 512
    m = VestaGPT2(hf, batch=1, tmax=T)
    pr = random_prompts(1, 70, 50257, seed=21)
    gen, last = _prefill_and_generate(m, pr, 6)
    _check_rows(text, W, pr, gen, last, T, [0])


@pytest.mark.slow
def test_batch32_long_cache_matches_oracle(small):
    """configs[2]'s batch (32 rows: more (row, head) points than blocks, the
    out-projection as its own stream, contractions on VALU row chunks) with a
    512-position cache (chunked softmax), rows checked against the oracle;
    the persistent kernel asked for (at 32 rows 'auto' takes the layered
    engine)."""
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    T = 512
    m = VestaGPT2(hf, batch=32, tmax=T, engine='persistent')
    assert m.engine == 'persistent'
    pr = random_prompts(32, 60, 50257, seed=23)
    gen, last = _prefill_and_generate(m, pr, 5)
    _check_rows(text, W, pr, gen, last, T, [0, 13, 31])


def test_batch8_launches_are_bit_reproducible(small):
    """Values several blocks add into are exact fixed-point sums, so two runs
    of the same launch give the same bits (logits and cache)."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, _, _ = small
    B = 8
    m = VestaGPT2(hf, batch=B, tmax=64)
    pr = torch.from_numpy(random_prompts(B, 20, 50257, seed=5)).to('cuda', torch.int32)
    outs = []
    for _ in range(2):
        m.reset()
        m.prefill(pr)
        m.step(8)
        torch.cuda.synchronize()
        outs.append((m.logits().clone(), m.keys.clone(), m.x.clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])


def test_multistep_launch_and_prefill_match_single_steps(small):
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, _, _ = small
    B, P, G = 2, 9, 7
    m = VestaGPT2(hf, batch=B, tmax=64)
    pr = random_prompts(B, P, 50257, seed=3)
    m.reset()
    _, _, nx = _run_steps(m, [pr[:, i] for i in range(P)], P + G - 1)
    ref = nx[P - 1:]                                           # [G, B]
    keys_ref = m.keys.clone()
    # prefill in one launch, then G-1 steps in one launch with the token history
    m.reset()
    hist = torch.zeros((G - 1) * B, dtype=torch.int32, device='cuda')
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32), mode='steps')
    torch.cuda.synchronize()
    first = m.x.cpu().numpy().copy()
    m.step(G - 1, hist)
    torch.cuda.synchronize()
    got = np.concatenate([first[None], hist.view(G - 1, B).cpu().numpy()])
    assert (got == ref).all()
    assert int(m.t.item()) == P + G - 1
    assert torch.equal(m.keys, keys_ref)


def _prefill_both(m, prompt):
    """The model state after prefilling ``prompt`` step by step, then batched:
    (keys, vals, x, logits) of each."""
    torch = _torch()
    out = []
    for mode in ('steps', 'batched'):
        m.reset()
        m.prefill(prompt, mode=mode)
        torch.cuda.synchronize()
        assert int(m.t.item()) == prompt.shape[1]
        out.append((m.keys.float().clone(), m.vals.float().clone(), m.x.cpu().numpy().copy(),
                    m.logits().float().cpu().numpy().copy()))
    return out


@pytest.mark.parametrize('B,P', [(1, 37), (8, 128)])
def test_batched_prefill_matches_step_prefill(small, B, P):
    """All prompt positions through each layer together (matrix-core products)
    against P decode steps: the cache rows, the next token and its logits."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, _, _ = small
    m = VestaGPT2(hf, batch=B, tmax=160)
    prompt = torch.from_numpy(random_prompts(B, P, 50257, seed=11)).to('cuda', torch.int32)
    (k0, v0, x0, l0), (k1, v1, x1, l1) = _prefill_both(m, prompt)
    for a, b in ((k0, k1), (v0, v1)):
        assert (a[:, :, P:] == 0).all() and (b[:, :, P:] == 0).all()
        d = (a[:, :, :P] - b[:, :, :P]).abs()
        print(f'cache rows: max diff {d.max().item():.3g}, mean {d.mean().item():.3g}, '
              f'differing {(d > 0).float().mean().item():.4f}, mean magnitude {a[:, :, :P].abs().mean().item():.3g}')
        assert d.max().item() < 2e-2, d.max().item()
        assert d.mean().item() < 1e-4
    assert np.abs(l0 - l1).max() < LOGIT_TOL
    top2 = np.sort(l0, axis=-1)[:, -2:]
    sure = (top2[:, 1] - top2[:, 0]) > 1e-3
    assert (x0[sure] == x1[sure]).all()


def test_batched_prefill_matches_oracle_and_continues(small):
    """Batched prefill at a nonzero start position (a second prompt after a
    first), then decode steps, against the oracle fed the same tokens."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    B, P1, P2, G = 2, 5, 7, 4
    m = VestaGPT2(hf, batch=B, tmax=32)
    pr = random_prompts(B, P1 + P2, 50257, seed=12)
    m.reset()
    m.prefill(torch.from_numpy(pr[:, :P1]).to('cuda', torch.int32), mode='batched')
    m.prefill(torch.from_numpy(pr[:, P1:]).to('cuda', torch.int32), mode='batched')
    torch.cuda.synchronize()
    assert int(m.t.item()) == P1 + P2
    lg = [m.logits().float().cpu().numpy().copy()]
    ins = [m.x.cpu().numpy().copy()]
    for _ in range(G):
        m.step()
        torch.cuda.synchronize()
        lg.append(m.logits().float().cpu().numpy().copy())
        ins.append(m.x.cpu().numpy().copy())
    for r in range(B):
        seq = np.concatenate([pr[r], [ins[k][r] for k in range(G)]])
        onx, olog, marg = decode.teacher_forced(text, W, seq, 32)
        got = np.stack([lg[k][r] for k in range(G + 1)])
        err = np.abs(got - olog[P1 + P2 - 1:]).max()
        assert err < LOGIT_TOL, r
        nxt = np.array([ins[k][r] for k in range(G + 1)])
        _tokens_match(f'prefill continued row {r}', nxt, onx[P1 + P2 - 1:], marg[P1 + P2 - 1:], err)
        keys = m.keys[r].float().cpu().numpy()
        row = decode.Row(text, W, 32)
        for i, tok in enumerate(seq[:P1 + P2]):
            row.x, row.t = int(tok), i
            row.step()
        assert np.abs(keys[:, :P1 + P2] - row.keys[:, :P1 + P2].astype(np.float32)).max() < 2e-2


def test_layered_engine_matches_persistent(small):
    """The per-layer launch sequence as a decode engine against the persistent
    kernel: the same prompt, then decode steps with tokens recorded."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, _, _ = small
    B, P, G = 8, 9, 6
    prompt = torch.from_numpy(random_prompts(B, P, 50257, seed=21)).to('cuda', torch.int32)
    out = []
    for engine in ('persistent', 'layered'):
        m = VestaGPT2(hf, batch=B, tmax=32, engine=engine)
        assert m.engine == engine
        m.reset()
        m.prefill(prompt)
        toks = torch.zeros(G * B, dtype=torch.int32, device='cuda')
        first = m.x.clone()
        m.step(G, toks)
        torch.cuda.synchronize()
        assert int(m.t.item()) == P + G
        out.append((first.cpu().numpy(), toks.view(G, B).cpu().numpy(), m.logits().float().cpu().numpy().copy(),
                    m.keys.float().clone()))
        del m
    (f0, t0, l0, k0), (f1, t1, l1, k1) = out
    assert (f0 == f1).all()
    same = (t0 == t1).all(axis=0)
    assert same.sum() >= B - 1, (t0, t1)
    assert np.abs(l0[same] - l1[same]).max() < LOGIT_TOL
    assert (k0[same] - k1[same]).abs().max().item() < 2e-2


def test_layered_graph_replays_match_launches(small):
    """Layered decode steps replayed from a captured HIP graph against the
    same steps launched kernel by kernel: bit-identical tokens, logits and
    cache rows at every step, with eager work and synchronizations between
    the replays."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, _, _ = small
    B, P, G = 4, 6, 5
    prompt = torch.from_numpy(random_prompts(B, P, 50257, seed=31)).to('cuda', torch.int32)
    runs = []
    for graphs in (False, True):
        m = VestaGPT2(hf, batch=B, tmax=32, engine='layered')
        m._pf.graphs = graphs
        m.reset()
        m.prefill(prompt)
        seen = []
        for _ in range(G):
            m.step()
            torch.cuda.synchronize()
            seen.append((m.x.cpu().numpy().copy(), m.logits().float().cpu().numpy().copy()))
            _ = (m.keys.float().sum() + 1).item()      # eager work between replays
        runs.append((seen, m.keys.clone(), int(m.t.item())))
        del m
    (s0, k0, t0), (s1, k1, t1) = runs
    assert t0 == t1 == P + G
    for (x0, l0), (x1, l1) in zip(s0, s1):
        assert (x0 == x1).all() and np.array_equal(l0, l1)
    assert torch.equal(k0, k1)


@pytest.mark.parametrize('B', [13, 40])
def test_layered_ragged_rows_match_oracle(small, B):
    """The layered decode with a row count that is not a multiple of the
    decode products' 16-row tiles (13 rows: one tile, 40 rows: four tiles,
    the last 24 rows of the fragment-order activations never written):
    the first and last rows against the oracle on the GPU's own inputs."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    P, G, T = 7, 4, 32
    m = VestaGPT2(hf, batch=B, tmax=T, engine='layered')
    pr = random_prompts(B, P, 50257, seed=50 + B)
    m.reset()
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32))
    lg, ins = [m.logits().float().cpu().numpy().copy()], [m.x.cpu().numpy().copy()]
    for _ in range(G):
        m.step()
        torch.cuda.synchronize()
        lg.append(m.logits().float().cpu().numpy().copy())
        ins.append(m.x.cpu().numpy().copy())
    m.check()
    for r in (0, B - 1):
        seq = np.concatenate([pr[r], [ins[k][r] for k in range(G)]])
        onx, olog, marg = decode.teacher_forced(text, W, seq, T)
        got = np.stack([lg[k][r] for k in range(G + 1)])
        err = np.abs(got - olog[P - 1:]).max()
        assert err < LOGIT_TOL, r
        nxt = np.array([ins[k][r] for k in range(G + 1)])
        _tokens_match(f'layered B={B} row {r}', nxt, onx[P - 1:], marg[P - 1:], err)


def test_layered_one_pass_attention_matches_oracle(small):
    """The layered decode on the one-pass attention (pf_attn1s: 5 rows x 12
    heads) over a 600-position cache at positions 140-143, where the first
    16 of a block's 32 lane groups take two batches of positions and the
    others one: rows 0 and 4 against the oracle on the GPU's own inputs."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    B, P, G, T = 5, 140, 3, 600
    m = VestaGPT2(hf, batch=B, tmax=T, engine='layered')
    assert m._pf._attn1() == 'pf_attn1s'
    pr = random_prompts(B, P, 50257, seed=77)
    m.reset()
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32))
    lg, ins = [m.logits().float().cpu().numpy().copy()], [m.x.cpu().numpy().copy()]
    for _ in range(G):
        m.step()
        torch.cuda.synchronize()
        lg.append(m.logits().float().cpu().numpy().copy())
        ins.append(m.x.cpu().numpy().copy())
    m.check()
    for r in (0, B - 1):
        seq = np.concatenate([pr[r], [ins[k][r] for k in range(G)]])
        onx, olog, marg = decode.teacher_forced(text, W, seq, T)
        got = np.stack([lg[k][r] for k in range(G + 1)])
        err = np.abs(got - olog[P - 1:]).max()
        print(f'one-pass attention row {r}: max logit error {err:.2e}', flush=True)
        assert err < LOGIT_TOL, r
        nxt = np.array([ins[k][r] for k in range(G + 1)])
        _tokens_match(f'one-pass attention row {r}', nxt, onx[P - 1:], marg[P - 1:], err)


@pytest.mark.parametrize('B,engine', [(64, 'layered'), (8, 'persistent')])
def test_xl_widths_match_oracle(B, engine):
    """GPT-2 XL widths (d 1600, 25 heads, f 6400), two layers to keep the
    oracle quick. At 64 rows the engine 'auto' picks (the layered one, faster
    at every row count at these widths); at 8 rows the persistent kernel,
    asked for, on the matrix cores. Two rows against the oracle."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.gpt2_program import gpt2_program
    from vesta.weights import GPT2Shape, RandomGPT2, random_prompts, stacked
    shape = GPT2Shape(2, 1600, 25, 6400)
    hf = RandomGPT2(shape, 4)
    m = VestaGPT2(hf, batch=B, tmax=16, engine='auto' if engine == 'layered' else engine)
    assert m.engine == engine, m.why_layered
    if engine == 'layered':
        assert m.why_layered.startswith(f'{B} rows'), m.why_layered
    P, G = 4, 3
    pr = random_prompts(B, P, 50257, seed=22)
    m.reset()
    m.prefill(torch.from_numpy(pr).to('cuda', torch.int32))
    lg, ins = [m.logits().float().cpu().numpy().copy()], [m.x.cpu().numpy().copy()]
    for _ in range(G):
        m.step()
        torch.cuda.synchronize()
        lg.append(m.logits().float().cpu().numpy().copy())
        ins.append(m.x.cpu().numpy().copy())
    W = decode.oracle_weights(stacked(hf.numpy_state(), 2))
    text = gpt2_program(2, 1600, 25, 6400, 50257, 'custom')
    for r in (0, B - 1):
        seq = np.concatenate([pr[r], [ins[k][r] for k in range(G)]])
        onx, olog, marg = decode.teacher_forced(text, W, seq, 16)
        got = np.stack([lg[k][r] for k in range(G + 1)])
        err = np.abs(got - olog[P - 1:]).max()
        assert err < LOGIT_TOL, r
        nxt = np.array([ins[k][r] for k in range(G + 1)])
        _tokens_match(f'XL widths B={B} row {r}', nxt, onx[P - 1:], marg[P - 1:], err)


def _grammar_cases():
    return json.load(open(os.path.join(GOLD, 'grammar_cases.json')))


@pytest.mark.parametrize('name', sorted(_grammar_cases()))
def test_grammar_programs_match_reference_golden(name):
    """Each language form through the GPU compiler against the reference
    interpreter's values (index arithmetic NumPy does in int64/float64 is
    compared at fp32 tolerance)."""
    torch = _torch()
    from vesta.launch import Kernel
    from vesta.lower import lower
    case = _grammar_cases()[name]
    gold = np.load(os.path.join(GOLD, 'grammar_cases.npz'))
    R, spec = {}, {}
    for k, v in case['inputs'].items():
        if isinstance(v, dict):
            arr = np.array(v['values'], dtype={'f32': np.float32, 'f16': np.float16}[v['dtype']])
            R[k] = torch.from_numpy(arr).to('cuda')
            spec[k] = (arr.shape, v['dtype'])
        else:
            R[k] = torch.tensor(int(v), dtype=torch.int32, device='cuda')
            spec[k] = ((), 'i32')
    outs = tuple(r for r in case['record'] if r in case.get('axes', {}))
    low = lower(case['text'], spec, {}, outputs=outs)
    k = Kernel(low)
    k(R)
    torch.cuda.synchronize()
    for r in case['record']:
        want = gold[f'{name}/{r}']
        got = (k.view(r) if r in outs else R[r]).float().cpu().numpy()
        if r in outs:                       # values carry the batch axis (extent 1) in front
            assert got.shape == (1,) + want.shape, (r, got.shape)
            got = got.reshape(want.shape)
        assert got.shape == want.shape, r
        assert np.allclose(got, want.astype(np.float64), rtol=1e-6, atol=1e-6), (r, got, want)


@pytest.mark.slow
def test_config1_greedy_tokens_match_oracle(small):
    """B=1, 128-token uniform-random prompt, 256 greedy
    tokens. Tokens must equal the oracle's (which follows the reference
    interpreter bit for bit on the golden vectors)."""
    torch = _torch()
    from oracle import decode
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import random_prompts
    hf, W, text = small
    P, G = 128, 256
    prompt = random_prompts(1, P, 50257, seed=1)
    m = VestaGPT2(hf, batch=1, tmax=P + G)
    m.reset()
    hist = torch.zeros(G, dtype=torch.int32, device='cuda')
    m.prefill(torch.from_numpy(prompt).to('cuda', torch.int32))
    torch.cuda.synchronize()
    first = int(m.x.item())
    m.step(G - 1, hist)
    torch.cuda.synchronize()
    gpu = [first] + hist[:G - 1].cpu().tolist()
    ref = decode.greedy(text, W, prompt[0], G, P + G)
    mism = [k for k in range(G) if gpu[k] != int(ref['tokens'][k])]
    assert not mism, f'first mismatch at {mism[0]}: margin there {ref["margins"][mism[0]]:.2e}'
