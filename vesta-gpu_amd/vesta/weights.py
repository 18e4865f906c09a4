"""Seeded random-init GPT-2 weights with Hugging Face names.

There is no network for checkpoints, so the benchmark and the tests run on
random-init weights of the real architecture. The reference's decode API only
needs an object with ``.state_dict()`` carrying HF GPT-2 names
(reference ``vesta/gpt2.py:18-25``); ``RandomGPT2`` is that object.

Recipe (fixed, so every run and the CPU oracle see the same numbers):
  * ``rng = numpy.random.default_rng(seed)`` (PCG64);
  * tensors are visited in HF ``state_dict`` order: ``wte``, ``wpe``, then per
    layer ``ln_1.{weight,bias}``, ``attn.c_attn.{weight,bias}``,
    ``attn.c_proj.{weight,bias}``, ``ln_2.{weight,bias}``,
    ``mlp.c_fc.{weight,bias}``, ``mlp.c_proj.{weight,bias}``, then ``ln_f``;
  * every non-LayerNorm tensor (linear biases included) is drawn
    ``rng.standard_normal(shape, float32) * 0.02`` and rounded to fp16
    (round to nearest even); LayerNorm gains are 1 and biases 0.
  * Conv1D weights are stored ``[in, out]`` as in HF GPT-2.
Prompts come from a separate generator: ``default_rng(seed).integers(0, vocab, (B, P))``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class GPT2Shape:
    n_layer: int
    n_embd: int
    n_head: int
    n_inner: int
    vocab: int = 50257
    n_positions: int = 1024

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head


SHAPES = {
    'small': GPT2Shape(12, 768, 12, 3072),
    'medium': GPT2Shape(24, 1024, 16, 4096),
    'xl': GPT2Shape(48, 1600, 25, 6400),
}


def layer_tensors(cfg: GPT2Shape):
    """(suffix, shape, is_layernorm) of one block's tensors, HF order."""
    d, f = cfg.n_embd, cfg.n_inner
    return [('ln_1.weight', (d,), True), ('ln_1.bias', (d,), True),
            ('attn.c_attn.weight', (d, 3 * d), False), ('attn.c_attn.bias', (3 * d,), False),
            ('attn.c_proj.weight', (d, d), False), ('attn.c_proj.bias', (d,), False),
            ('ln_2.weight', (d,), True), ('ln_2.bias', (d,), True),
            ('mlp.c_fc.weight', (d, f), False), ('mlp.c_fc.bias', (f,), False),
            ('mlp.c_proj.weight', (f, d), False), ('mlp.c_proj.bias', (d,), False)]


def random_state(cfg: GPT2Shape, seed: int = 0) -> dict[str, np.ndarray]:
    """HF-named fp16 numpy arrays drawn by the recipe in the module docstring."""
    rng = np.random.default_rng(seed)

    def draw(shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float16)

    sd = {'transformer.wte.weight': draw((cfg.vocab, cfg.n_embd)),
          'transformer.wpe.weight': draw((cfg.n_positions, cfg.n_embd))}
    for layer in range(cfg.n_layer):
        for suffix, shape, is_ln in layer_tensors(cfg):
            if is_ln:
                val = np.ones(shape, np.float16) if suffix.endswith('weight') else np.zeros(shape, np.float16)
            else:
                val = draw(shape)
            sd[f'transformer.h.{layer}.{suffix}'] = val
    sd['transformer.ln_f.weight'] = np.ones((cfg.n_embd,), np.float16)
    sd['transformer.ln_f.bias'] = np.zeros((cfg.n_embd,), np.float16)
    return sd


def random_prompts(batch: int, length: int, vocab: int = 50257, seed: int = 1) -> np.ndarray:
    """Uniform random token ids, int64 [batch, length]."""
    return np.random.default_rng(seed).integers(0, vocab, (batch, length))


class RandomGPT2:
    """Stand-in for ``GPT2LMHeadModel``: only ``state_dict()`` and ``config`` are used."""

    def __init__(self, shape: str | GPT2Shape = 'small', seed: int = 0):
        self.config = SHAPES[shape] if isinstance(shape, str) else shape
        self.seed = seed
        self._sd = None

    def numpy_state(self) -> dict[str, np.ndarray]:
        if self._sd is None:
            self._sd = random_state(self.config, self.seed)
        return self._sd

    def state_dict(self):
        import torch
        return {k: torch.from_numpy(v) for k, v in self.numpy_state().items()}


def stacked(sd: dict, n_layer: int) -> dict[str, np.ndarray]:
    """HF state dict -> the program's residues, per-layer tensors stacked along a
    leading layer axis (reference ``vesta/gpt2.py:18-25``). Works on numpy arrays."""
    def st(suffix):
        return np.stack([np.asarray(sd[f'transformer.h.{i}.{suffix}']) for i in range(n_layer)])
    return dict(wte=np.asarray(sd['transformer.wte.weight']), wpe=np.asarray(sd['transformer.wpe.weight']),
                ln1w=st('ln_1.weight'), ln1b=st('ln_1.bias'), qkvw=st('attn.c_attn.weight'), qkvb=st('attn.c_attn.bias'),
                ow=st('attn.c_proj.weight'), ob=st('attn.c_proj.bias'), ln2w=st('ln_2.weight'), ln2b=st('ln_2.bias'),
                fcw=st('mlp.c_fc.weight'), fcb=st('mlp.c_fc.bias'), pw=st('mlp.c_proj.weight'), pb=st('mlp.c_proj.bias'),
                lnfw=np.asarray(sd['transformer.ln_f.weight']), lnfb=np.asarray(sd['transformer.ln_f.bias']))
