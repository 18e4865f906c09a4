"""Seeded random-init GPT-2 weights with Hugging Face names.

The reference's decode API only needs an object with ``.state_dict()``
carrying HF GPT-2 names (reference ``vesta/gpt2.py:18-25``). Two such objects
live here: ``RandomGPT2`` (seeded random init of the real architecture: there
is no network for checkpoints, so the benchmark and the tests run on it) and
``LocalGPT2`` (a checkpoint already on disk: a ``save_pretrained`` directory
or a single ``.safetensors`` / ``.bin`` file, with or without the
``transformer.`` prefix).

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


# Non-parameter entries some GPT-2 checkpoints carry (the causal mask buffers).
_BUFFER_SUFFIXES = ('.attn.bias', '.attn.masked_bias')


def normalize_state(sd: dict) -> dict:
    """Checkpoint entries -> ``GPT2LMHeadModel`` names (``transformer.`` prefix).

    Accepts both the LM-head model's names and the bare ``GPT2Model`` names
    of hub checkpoints (``h.0.attn.c_attn.weight``, ``wte.weight``), drops the
    attention mask buffers, and checks that an ``lm_head.weight`` present is
    the word table: the program's output head is tied to ``wte`` (gpt2.vst
    Q9), so an untied head cannot be run and is an error."""
    out = {}
    head = None
    for k, v in sd.items():
        if k == 'lm_head.weight':
            head = v
            continue
        name = k if k.startswith('transformer.') else 'transformer.' + k
        if name.endswith(_BUFFER_SUFFIXES):
            continue
        out[name] = v
    if 'transformer.wte.weight' not in out:
        raise KeyError('checkpoint has no word table (wte.weight)')
    if head is not None:
        a, b = np.asarray(_host(head), np.float32), np.asarray(_host(out['transformer.wte.weight']), np.float32)
        if a.shape != b.shape or not np.array_equal(a, b):
            raise ValueError('lm_head.weight differs from wte.weight: the program ties the output head to wte')
    return out


def _host(v):
    """A tensor or array as a host array (bf16 tensors widened to fp32)."""
    if isinstance(v, np.ndarray):
        return v
    import torch
    t = v.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


def read_checkpoint(path) -> dict:
    """Tensors of a checkpoint on disk, as torch CPU tensors keyed as stored.

    ``path``: a ``.safetensors`` file, a ``.bin``/``.pt`` file (read with
    ``torch.load(weights_only=True)``, which executes nothing from the file),
    or a directory holding ``model.safetensors``, a sharded
    ``model.safetensors.index.json`` or ``pytorch_model.bin``."""
    import json
    import os
    import torch
    path = os.fspath(path)
    if os.path.isdir(path):
        index = os.path.join(path, 'model.safetensors.index.json')
        if os.path.exists(index):
            with open(index, encoding='utf-8') as fh:
                shards = sorted(set(json.load(fh)['weight_map'].values()))
            out = {}
            for sh in shards:
                out.update(read_checkpoint(os.path.join(path, sh)))
            return out
        for name in ('model.safetensors', 'pytorch_model.bin'):
            if os.path.exists(os.path.join(path, name)):
                return read_checkpoint(os.path.join(path, name))
        raise FileNotFoundError(f'no model.safetensors or pytorch_model.bin in {path}')
    if path.endswith('.safetensors'):
        from safetensors.torch import load_file
        return load_file(path)
    if path.endswith(('.bin', '.pt', '.pth')):
        sd = torch.load(path, map_location='cpu', weights_only=True)
        return sd.get('state_dict', sd) if isinstance(sd, dict) else sd
    raise ValueError(f'unknown checkpoint format: {path}')


class _Config:
    """The GPT-2 hyper-parameters ``VestaGPT2`` reads (``n_head``), from a
    ``config.json`` when there is one."""

    def __init__(self, d: dict):
        self.__dict__.update(d)


class LocalGPT2:
    """A GPT-2 checkpoint on local disk, as the object ``VestaGPT2`` takes.

        m = VestaGPT2(LocalGPT2('/models/gpt2'), batch=8, tmax=1024)

    ``state_dict()`` returns ``GPT2LMHeadModel``-named torch tensors in the
    checkpoint's dtype (``VestaGPT2`` converts them); ``config`` carries
    ``config.json``'s fields (``n_head`` among them) when the directory has
    one, else None (the head count then follows from the width)."""

    def __init__(self, path):
        import json
        import os
        self.path = os.fspath(path)
        self.config = None
        cfg = os.path.join(self.path if os.path.isdir(self.path) else os.path.dirname(self.path), 'config.json')
        if os.path.exists(cfg):
            with open(cfg, encoding='utf-8') as fh:
                self.config = _Config(json.load(fh))
        self._sd = None

    def state_dict(self):
        if self._sd is None:
            self._sd = normalize_state(read_checkpoint(self.path))
        return self._sd
