"""Weights: the seeded random-init recipe, and local checkpoints (HF
``save_pretrained`` directories, bare ``GPT2Model`` safetensors files) read
into the names the decode API stacks (reference ``vesta/gpt2.py:18-25``).

The GPT-2 arithmetic of the oracle is also pinned here against an independent
implementation: the ``transformers`` GPT-2 forward pass (eager attention, fp32)
on the same fp16-valued weights.
"""
import numpy as np
import pytest
import torch

from oracle import decode
from vesta.gpt2_program import gpt2_program
from vesta.weights import (GPT2Shape, LocalGPT2, RandomGPT2, normalize_state, random_state, read_checkpoint,
                           stacked)

transformers = pytest.importorskip('transformers')

TINY = dict(vocab_size=37, n_positions=32, n_embd=16, n_layer=2, n_head=4, n_inner=64)


def _hf_tiny(seed=0, wscale=1.0):
    """A random-init ``GPT2LMHeadModel`` (no download) with fp16-valued weights
    and non-trivial LayerNorm gains and biases; ``wscale`` widens the matrices
    (N(0, 0.02 * wscale)) so that every term of the step moves the logits."""
    torch.manual_seed(seed)
    cfg = transformers.GPT2Config(**TINY, attn_implementation='eager')
    m = transformers.GPT2LMHeadModel(cfg).eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if 'ln_' in name:
                p.copy_(1.0 + 0.1 * torch.randn_like(p) if name.endswith('weight') else 0.1 * torch.randn_like(p))
            elif name.endswith('bias'):
                p.copy_(0.02 * torch.randn_like(p))
            else:
                p.mul_(wscale)
            p.copy_(p.half().float())
    return m


def _params(sd):
    return {k: v for k, v in sd.items() if not k.endswith(('.attn.bias', '.attn.masked_bias')) and k != 'lm_head.weight'}


def test_random_state_recipe_is_seeded_and_fp16():
    cfg = GPT2Shape(2, 16, 4, 64, vocab=37, n_positions=32)
    a, b = random_state(cfg, 5), random_state(cfg, 5)
    assert all(np.array_equal(a[k], b[k]) for k in a)
    assert all(v.dtype == np.float16 for v in a.values())
    assert np.all(a['transformer.h.1.ln_2.weight'] == 1) and np.all(a['transformer.ln_f.bias'] == 0)
    assert not np.array_equal(random_state(cfg, 6)['transformer.wte.weight'], a['transformer.wte.weight'])


def test_save_pretrained_directory_round_trip(tmp_path):
    m = _hf_tiny()
    m.save_pretrained(tmp_path, safe_serialization=True)
    local = LocalGPT2(tmp_path)
    assert local.config.n_head == 4 and local.config.n_layer == 2
    got = local.state_dict()
    want = _params(m.state_dict())
    assert set(got) == set(want)
    for k in want:
        assert torch.equal(got[k], want[k]), k
    res = stacked({k: v.numpy() for k, v in got.items()}, 2)
    assert res['qkvw'].shape == (2, 16, 48) and res['pw'].shape == (2, 64, 16)


def test_bare_gpt2model_file_with_mask_buffers(tmp_path):
    """Hub GPT-2 checkpoints store ``GPT2Model`` names and the mask buffers."""
    from safetensors.torch import save_file
    sd = {k[len('transformer.'):]: v.clone() for k, v in _params(_hf_tiny(1).state_dict()).items()}
    sd['h.0.attn.bias'] = torch.tril(torch.ones(1, 1, 32, 32))
    path = tmp_path / 'model.safetensors'
    save_file(sd, str(path))
    got = LocalGPT2(path).state_dict()
    assert 'transformer.h.0.attn.c_attn.weight' in got and not any(k.endswith('.attn.bias') for k in got)
    assert LocalGPT2(path).config is None
    assert len(got) == len(sd) - 1


def test_sharded_index_and_bin(tmp_path):
    import json
    from safetensors.torch import save_file
    sd = _params(_hf_tiny(2).state_dict())
    keys = sorted(sd)
    half = len(keys) // 2
    shards = {'model-00001-of-00002.safetensors': keys[:half], 'model-00002-of-00002.safetensors': keys[half:]}
    for fn, ks in shards.items():
        save_file({k: sd[k].contiguous() for k in ks}, str(tmp_path / fn))
    json.dump({'weight_map': {k: fn for fn, ks in shards.items() for k in ks}},
              open(tmp_path / 'model.safetensors.index.json', 'w'))
    got = read_checkpoint(tmp_path)
    assert set(got) == set(sd) and all(torch.equal(got[k], sd[k]) for k in sd)
    torch.save(sd, tmp_path / 'weights.bin')
    got = LocalGPT2(tmp_path / 'weights.bin').state_dict()
    assert all(torch.equal(got[k], sd[k]) for k in sd)


def test_untied_head_and_missing_table_are_errors():
    sd = _params(_hf_tiny().state_dict())
    bad = dict(sd)
    bad['lm_head.weight'] = sd['transformer.wte.weight'] + 1
    with pytest.raises(ValueError, match='ties the output head'):
        normalize_state(bad)
    tied = dict(sd)
    tied['lm_head.weight'] = sd['transformer.wte.weight'].clone()
    assert 'lm_head.weight' not in normalize_state(tied)
    with pytest.raises(KeyError):
        normalize_state({k: v for k, v in sd.items() if 'wte' not in k})


def test_random_model_state_dict_is_hf_named():
    sd = RandomGPT2(GPT2Shape(2, 16, 4, 64, vocab=37, n_positions=32), seed=0).state_dict()
    assert normalize_state(sd).keys() == sd.keys()


def test_oracle_agrees_with_transformers_forward():
    """The program's answers (logits at every position, greedy tokens) against
    the transformers GPT-2 forward pass over the whole sequence. The oracle
    rounds cache rows to fp16 as the kernel does, so agreement is within a
    tolerance, not bit for bit: 1.0e-4 measured, against 8e-4 to 7e-3 for a
    wrong LayerNorm eps (1e-4), score scale (1/2.2), or either GELU constant
    (0.04, 0.79) planted in the program."""
    m = _hf_tiny(3, wscale=5.0)
    sd = {k: v.numpy().astype(np.float16) for k, v in _params(m.state_dict()).items()}
    W = decode.oracle_weights(stacked(sd, 2))
    text = gpt2_program(2, 16, 4, 64, 37, 'tiny')
    toks = np.array([5, 9, 3, 30, 1, 36, 0, 17, 22, 8, 11, 4, 29, 33])
    nexts, logits, margins = decode.teacher_forced(text, W, toks, 16)
    with torch.no_grad():
        hf = m(torch.from_numpy(toks)[None]).logits[0].numpy()
    assert np.abs(hf).max() > 1.0
    assert np.abs(logits - hf).max() < 4e-4
    sure = margins > 1e-2
    assert sure.sum() >= 10
    assert np.array_equal(nexts[sure], hf.argmax(-1)[sure])
