"""gpt2.vst on the GPU: GPT-2 weights as residues, lowered to one kernel per step.

    m = VestaGPT2(hf, dtype='f16', batch=8, tmax=1024)
    m.reset(); m.x.copy_(tok); m.t.fill_(p); m.step()     # one decode step
    m.logits(), m.next()                                    # views, no sync
    m.check()                                               # raises if a launch failed (syncs)

The object keeps a host copy of the position to refuse steps past the last
cache row. It is known after ``reset()``, ``prefill()`` and ``seek(p)`` and
advanced by each step; a caller that writes ``t`` itself (as above) should
say so with ``seek(p)``, else the check is off until the next ``reset`` or
``prefill``.

With feedback on, each step writes its chosen token into x and advances t,
so generation is back-to-back launches with nothing from the host between.

Same surface as the reference decode API (reference ``vesta/gpt2.py:1-55``:
``gpt2_weights``, ``VestaGPT2`` with ``x``/``t``/``keys``/``vals``/``W``/
``low``/``k``/``weight_bytes`` and ``reset``/``step``/``logits``/``next``/
``kv_bytes``). ``hf`` only needs ``state_dict()`` with Hugging Face GPT-2 names
(a ``transformers`` GPT-2 model, or ``vesta.weights.RandomGPT2``). Extents
come from the state dict, so GPT-2 small, medium and XL all work; the program
defaults to the committed one for those shapes.
"""
from __future__ import annotations

from . import PROGRAMS
from .gpt2_program import gpt2_program
from .launch import TORCH_DT, Kernel, code_spills, compile_code, lower_fitted
from .lower import GRID_FEW_ROWS, GRID_WIDE, lower

LDS_PER_CU = 160 * 1024      # bytes of LDS one block of the persistent kernel may use
SPILLS_LAYERED = 64          # spilled registers beyond which 'auto' takes the layered engine
LAYERED_ROWS = {768: 11, 1024: 9, 1600: 1}   # rows from which 'auto' takes the layered engine, by model
LAYERED_ROWS_OTHER = 9        # width (same box, ms per step, persistent / layered: GPT-2 small 8 rows 0.283 /
                              # 0.395, 10 rows 0.372 / 0.399, 11 rows 0.545 / 0.398, 16 rows 0.594 / 0.403, 32
                              # rows with a 1024-position cache 0.867 / 0.546; medium 8 rows 0.744 / 0.893, 9
                              # rows 1.253 / 0.903, 16 rows 1.246 / 0.919; XL 2 rows 2.601 / 2.124, 8 rows
                              # 3.182 / 2.099, 64 rows 7.321 / 3.070)

FEW_ROWS_REPLICAS = 12       # below 4 rows the persistent kernel's grid gives each attention head this many
                              # replica blocks (at least the lowering's 144 blocks, at most one per CU):
                              # GPT-2 small 144, medium 192 (same box, ms per step, medium at
                              # one row: 0.598 on 144 blocks, 0.582 on 128, 0.553 on 160, 0.544-0.562 on 192,
                              # 0.545 on 208, 0.550 on 224, 0.602 on 256; small: 0.199 on 144, 0.207 on 160,
                              # 0.213 on 192, and on another box 0.195 on 144, 0.201 on 132, 0.203 on 120,
                              # 0.218 on 108, 0.211 on 96)


def persistent_grid(batch, heads):
    """The persistent kernel's grid for ``batch`` rows of a model with
    ``heads`` attention heads: FEW_ROWS_REPLICAS blocks per head below 4 rows,
    else the lowering's own choice (None)."""
    return min(GRID_WIDE, max(GRID_FEW_ROWS, FEW_ROWS_REPLICAS * heads)) if batch < 4 else None


SHAPE_PROGRAMS = {(12, 768, 12): 'gpt2.vst', (24, 1024, 16): 'gpt2_medium.vst', (48, 1600, 25): 'gpt2_xl.vst'}


def _n_layer(sd):
    n = 0
    while f'transformer.h.{n}.ln_1.weight' in sd:
        n += 1
    return n


def gpt2_weights(hf):
    """HF state dict -> the program's residues: per-layer tensors stacked along
    a leading layer axis (reference gpt2.py:18-25)."""
    import torch
    sd = hf.state_dict()
    L = _n_layer(sd)

    def st(n):
        return torch.stack([sd[f'transformer.h.{i}.{n}'] for i in range(L)])
    return dict(wte=sd['transformer.wte.weight'], wpe=sd['transformer.wpe.weight'],
                ln1w=st('ln_1.weight'), ln1b=st('ln_1.bias'), qkvw=st('attn.c_attn.weight'), qkvb=st('attn.c_attn.bias'),
                ow=st('attn.c_proj.weight'), ob=st('attn.c_proj.bias'), ln2w=st('ln_2.weight'), ln2b=st('ln_2.bias'),
                fcw=st('mlp.c_fc.weight'), fcb=st('mlp.c_fc.bias'), pw=st('mlp.c_proj.weight'), pb=st('mlp.c_proj.bias'),
                lnfw=sd['transformer.ln_f.weight'], lnfb=sd['transformer.ln_f.bias'])


def _n_head(hf, d):
    cfg = getattr(hf, 'config', None)
    for attr in ('n_head', 'num_attention_heads'):
        if cfg is not None and getattr(cfg, attr, None):
            return int(getattr(cfg, attr))
    return {768: 12, 1024: 16, 1280: 20, 1600: 25}[d]


class VestaGPT2:
    def __init__(self, hf, dtype='f16', batch=1, tmax=1024, feedback=True, program=None, timing=False,
                 blocks_per_sm=None, engine='auto'):
        """``engine``: 'persistent' lowers the program to one persistent kernel
        per launch (the reference design); 'layered' runs each step as a
        sequence of ordinary per-layer launches (``vesta.prefill``: the
        multi-token prefill kernels with one position per row); 'auto' takes
        the layered engine from ``LAYERED_ROWS[d]`` rows (``LAYERED_ROWS_OTHER``
        for widths not listed; where it is faster) and
        the persistent kernel below, unless that does not fit the device (LDS
        beyond a CU's 160 KB, or more than ``SPILLS_LAYERED`` spilled
        registers), as for GPT-2 XL at one row. With the layered engine ``low`` and ``k``
        are None."""
        import torch
        if engine not in ('auto', 'persistent', 'layered'):
            raise ValueError(f'unknown engine {engine!r}')
        tdt = TORCH_DT[dtype]
        self.W = {k: v.detach().to('cuda', tdt).contiguous() for k, v in gpt2_weights(hf).items()}
        L = self.W['qkvw'].shape[0]
        D = self.W['wte'].shape[1]
        H = _n_head(hf, D)
        E = D // H
        F = self.W['fcw'].shape[2]
        V = self.W['wte'].shape[0]
        if tmax > self.W['wpe'].shape[0]:
            raise ValueError(f'tmax {tmax} exceeds the {self.W["wpe"].shape[0]} learned positions')
        self.L, self.H, self.E, self.D = L, H, E, D
        self.B, self.tmax = batch, tmax
        self.keys = torch.zeros(batch, L, tmax, H, E, device='cuda', dtype=tdt)
        self.vals = torch.zeros_like(self.keys)
        self.x = torch.zeros(batch, dtype=torch.int32, device='cuda')
        self.t = torch.zeros(1, dtype=torch.int32, device='cuda')
        R = {'x': self.x, 't': self.t, **self.W, 'keys': self.keys, 'vals': self.vals}
        dts = {torch.int32: 'i32', torch.float16: 'f16', torch.float32: 'f32'}
        spec = {n: ((), 'i32') if n == 't' else (tuple(v.shape), dts[v.dtype]) for n, v in R.items()}
        if program is None:
            name = SHAPE_PROGRAMS.get((L, D, H))
            text = (PROGRAMS / name).read_text(encoding='utf-8') if name and F == 4 * D and V == 50257 \
                else gpt2_program(L, D, H, F, V, 'custom')
        else:
            text = open(program, encoding='utf-8').read()
        grid = persistent_grid(batch, H)
        self._lower_args = (text, spec, dict(axis_max={'s': tmax}, batch=batch, per_token=('x', 'keys', 'vals'),
                                             outputs=('logit', 'next'),
                                             feedback={'x': 'next', 't': 1} if feedback else None, grid=grid))
        self._R, self._bps, self._timing = R, blocks_per_sm, timing
        self.low, self.k, self._pf = None, None, None
        self._variants = {}
        self._know_pos(0)
        self.engine, self.why_layered = 'persistent', None
        from .prefill import supported
        if engine == 'layered':
            self.why_layered = 'asked for'
        elif engine == 'auto' and batch >= (rows := LAYERED_ROWS.get(D, LAYERED_ROWS_OTHER)) and supported(D, H, F):
            self.why_layered = f'{batch} rows (layered is faster from {rows} rows)'
        else:
            self.why_layered = self._persistent(text, spec, batch, timing, blocks_per_sm, strict=engine == 'persistent')
        if self.k is None:
            from .prefill import Prefill
            if not supported(D, H, F):
                raise ValueError(f'the persistent kernel does not fit ({self.why_layered}) and the layered '
                                 f'engine needs 64-wide heads and widths that are multiples of 32')
            self.engine = 'layered'
            self._logit = torch.zeros(batch, V, dtype=torch.float32, device='cuda')
            self._next = torch.zeros(batch, dtype=torch.float32, device='cuda')
            self._pf = Prefill(self)
        self.weight_bytes = sum(v.numel() * v.element_size() for n, v in self.W.items() if n != 'wpe') \
            + D * self.W['wpe'].element_size()

    def _persistent(self, text, spec, batch, timing, blocks_per_sm, strict):
        """Build the persistent kernel; returns None, or (when it does not fit
        and ``strict`` is off) why not."""
        kw = dict(**self._lower_args[2], timing=timing, kernel_name=f'vesta_step_b{batch}')
        if not strict:
            lds = lower(text, spec, **kw).shared_bytes
            if lds > LDS_PER_CU:
                return f'{lds} bytes of LDS per block'
        low = lower_fitted(lower, text, spec, **kw)
        spills = code_spills(compile_code(low.src))
        if not strict and spills > SPILLS_LAYERED:
            return f'{spills} spilled registers'
        self.low = low
        self.k = Kernel(low, blocks_per_sm=blocks_per_sm)
        self.k.bind(self._R)
        return None

    def reset(self):
        self.keys.zero_()
        self.vals.zero_()
        self.t.zero_()
        self._know_pos(0)

    def _know_pos(self, pos):
        """The host's copy of the position is ``pos``, as of ``t``'s present
        in-place version: a later host write to ``t`` (``fill_``, ``copy_``)
        bumps torch's version counter of the tensor, while the kernels'
        own advances of ``t`` do not."""
        self._pos = pos
        self._t_version = self.t._version if pos is not None else None

    def _advance(self, n, what):
        """Keep the host's copy of the position (known after ``reset``,
        ``seek`` and ``prefill``, advanced by every step this object runs;
        unknown once the caller writes ``t`` itself, until the next ``reset``,
        ``seek`` or ``prefill``) and refuse steps past the last cache row: the
        engines must never be asked for a position the cache does not hold."""
        pos = getattr(self, '_pos', None)
        if pos is not None and getattr(self, '_t_version', None) != self.t._version:
            self._know_pos(None)             # the caller wrote t: the host no longer knows the position
            pos = None
        if pos is not None:
            if pos + n > self.tmax:
                raise ValueError(f'{what}: positions {pos}..{pos + n - 1} exceed the cache (tmax {self.tmax})')
            self._pos = pos + n

    def seek(self, pos):
        """Set the position to ``pos`` (device and host copies)."""
        if not 0 <= pos < self.tmax:
            raise ValueError(f'position {pos} outside the cache (tmax {self.tmax})')
        self.t.fill_(int(pos))
        self._know_pos(int(pos))

    def step(self, n=1, tokens=None):
        """One decode step (the reference API); ``n`` > 1 runs n steps in one
        launch, writing each step's tokens into ``tokens`` (contiguous int32,
        e.g. [n, B]; step k at flat offsets k * B ..) if given."""
        if tokens is not None:
            if not (tokens.is_cuda and tokens.dtype == self.x.dtype and tokens.is_contiguous()):
                raise TypeError('tokens must be a contiguous int32 device tensor')
            if tokens.numel() < n * self.B:
                raise ValueError(f'tokens holds {tokens.numel()} ids, {n * self.B} needed')
        self._advance(n, 'step')
        if self.k is None:
            self._pf.decode(n, tokens)
            return
        self.k.launch(n, tokens)

    def check(self):
        """Raise if an earlier launch reported a failure: a grid barrier of the
        persistent kernel that gave up waiting, or an activation beyond the
        fp16 range on a matrix-core product (one device synchronisation)."""
        for k in [self.k, *self._variants.values()]:
            if k is not None:
                k.check()
        if self._pf is not None:
            self._pf.check()

    def variant(self, name):
        """The persistent kernel of this model's program under another symbol
        (the source is otherwise the same), bound to the same residues: for
        launches that should show apart in kernel profiles (prompt feeding,
        warm-up, a one-launch-per-step timing). Built once per name."""
        if self.k is None:
            raise RuntimeError('the layered engine has no persistent kernel')
        v = self._variants.get(name)
        if v is None:
            text, spec, kw = self._lower_args
            low = lower_fitted(lower, text, spec, **kw, timing=self._timing, kernel_name=name)
            v = Kernel(low, blocks_per_sm=self._bps)
            v.bind(self._R)
            self._variants[name] = v
        return v

    def _prefill_kernel(self):
        """The program under its own symbol for prompt feeding and warm-up (so
        profiles of the decode kernel hold decode launches only)."""
        return self.variant(f'vesta_prefill_b{self.B}')

    def prefill(self, prompt, tokens=None, mode='auto'):
        """Feed a prompt [B, P] (int32 device tensor) at positions t .. t + P - 1;
        afterwards x holds the token chosen after the last prompt token and t
        has advanced by P (as after P reference-style steps).

        ``mode``: 'batched' runs all positions through each layer together
        (matrix-core products, ``vesta.prefill``); 'steps' runs P decode steps
        in one launch and can write each step's chosen token into ``tokens``;
        'auto' takes 'batched' when no per-step tokens are asked for and the
        shapes allow it."""
        P = prompt.shape[1]
        if prompt.shape[0] != self.B:
            raise ValueError(f'prompt has {prompt.shape[0]} rows, the model {self.B}')
        if P < 1:
            raise ValueError('empty prompt')
        if mode not in ('auto', 'batched', 'steps'):
            raise ValueError(f'unknown prefill mode {mode!r}')
        from .prefill import supported
        fits = supported(self.D, self.H, self.W['fcw'].shape[2])
        if mode == 'batched' and (tokens is not None or not fits):
            raise ValueError('batched prefill writes no per-step tokens and needs 64-wide heads and widths '
                             'that are multiples of 32')
        if tokens is not None and not (tokens.is_cuda and tokens.dtype == self.x.dtype and tokens.is_contiguous()
                                       and tokens.numel() >= P * self.B):
            raise TypeError(f'tokens must be a contiguous int32 device tensor of at least {P * self.B} ids')
        self.check()
        t0 = int(self.t.item())
        if t0 + P > self.tmax:
            raise ValueError(f'positions {t0}..{t0 + P - 1} exceed the cache (tmax {self.tmax})')
        self._know_pos(t0 + P)
        if mode == 'batched' or (mode == 'auto' and tokens is None and fits):
            if self._pf is None:
                from .prefill import Prefill
                self._pf = Prefill(self)
            self._pf.run(prompt.to(dtype=self.x.dtype))
            return
        ins = prompt.t().contiguous().to(dtype=self.x.dtype)
        if self.k is None:
            flat = None if tokens is None else tokens.view(-1)
            for i in range(P):
                self.x.copy_(ins[i])
                self._pf.decode(1, None if flat is None else flat[i * self.B:(i + 1) * self.B])
            return
        self.x.copy_(ins[0])
        self._prefill_kernel().launch(P, tokens, ins)
        self._take_outputs()

    def warm(self, n):
        """n decode steps through the prefill kernel (untimed warm-up)."""
        if n > 0:
            self._advance(n, 'warm')
        if n > 0 and self.k is None:
            self._pf.decode(n)
        elif n > 0:
            self._prefill_kernel().launch(n)
            self._take_outputs()

    def _take_outputs(self):
        """The prefill kernel's last logits and tokens into the decode
        kernel's scratch, so ``logits()``/``next()`` answer for the last step
        whichever kernel ran it (a device copy on the current stream)."""
        kp = self._prefill_kernel()
        for name in ('logit', 'next'):
            self.k.view(name).copy_(kp.view(name))

    def logits(self):
        return self._logit if self.k is None else self.k.view('logit')

    def next(self):
        return self._next if self.k is None else self.k.view('next')

    def kv_bytes(self, n_ctx):
        return 2 * self.L * self.B * n_ctx * self.D * self.keys.element_size()
