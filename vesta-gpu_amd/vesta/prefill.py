"""Multi-token prefill: a prompt's positions go through each layer together.

The reference feeds a prompt one token per launch (reference
``bench/g0_bench.py:172-173``): P decode steps, each reading every weight.
Here the B rows' P positions form one M = B * P row batch and each layer is
a handful of ordinary launches (``hip/prefill.hip``): LayerNorm, the qkv
product writing the key/value cache rows, causal attention over the cache,
the out-projection with its residual, LayerNorm, the widening product with
GELU, the narrowing product with its residual. The products run on the
matrix cores. Only the last position of each row goes through the final
LayerNorm and the tied output head; its argmax becomes the next input.

Afterwards the model is in the state P decode steps would leave: cache rows
t0 .. t0 + P - 1 written, ``x`` the token chosen after the last prompt token,
``t`` advanced by P, ``logits()`` that step's logits.

The same launch sequence with one position per row is the layered decode
engine (``Prefill.decode``, replayed from a captured HIP graph). Up to 64
rows its products are ``pf_mgemm*``, which read weights packed once in the
matrix cores' operand order (``frag_weights``) and activations that the
LayerNorms, attention and the widening product's GELU write in that order.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from .launch import compile_code, lib, ok, track, unload

PREFILL_SRC = Path(__file__).resolve().parent / 'hip' / 'prefill.hip'
PRELUDE_SRC = Path(__file__).resolve().parent / 'hip' / 'prelude.h'
BLOCK = 256
TILE = 64
CHUNK = 64                    # fold depth one product step stages in LDS
HEAD = 64
KERNELS = ('pf_embed', 'pf_ln', 'pf_gemm', 'pf_reduce', 'pf_reduce_ln', 'pf_attn', 'pf_attn1', 'pf_argmax_part',
           'pf_argmax', 'pf_mgemm1', 'pf_mgemm2', 'pf_mgemm4', 'pf_mgemm1n', 'pf_mgemm2n', 'pf_mgemm4n',
           'pf_reduce_frag', 'pf_attn1s', 'pf_mhead1', 'pf_mhead2', 'pf_mhead4', 'pf_embed_ln')
ARGMAX_SPLIT = 32             # blocks per row of the output-head argmax (same box, 16 -> 32: GPT-2 small 32 rows
                              # 547.6 -> 545.8 us per step, 8 rows 396.3 -> 395.5, XL 64 rows even)
SPLIT_BLOCKS = 384            # a product with fewer output tiles than this splits its fold over blocks ...
                              # (XL B=64 decode: 4.95 ms per step at 320-384, 5.18 at 256, 5.42 at 512)
SPLIT_MIN_CHUNKS = 4          # ... into parts of at least this many 64-deep chunks
FUSE_REDUCE_LN = True         # (prefill products) a split residual product's reduction makes the LayerNorm
                              # that follows (one launch instead of two; same box, decode on these products:
                              # GPT-2 small B=32 1.073 -> 1.055 ms per step, XL B=64 5.194 -> 5.212)
MODE_PLAIN, MODE_RESID, MODE_GELU, MODE_QKV = 0, 1, 2, 3
DECODE_ROWS = 64              # decode passes of up to this many rows run the fragment-order products (pf_mgemm*)
MG_WAVES = 8                  # waves of a pf_mgemm block ...
MG_TILES = {1: 1, 2: 1, 4: 2}  # ... and the 16-column tiles it makes, by 16-row tiles (pf_mgemm1/2/4's MN)
MG_BLOCKS = 200               # a decode product splits its fold so that it has about this many blocks, ...
MG_MIN_STEPS = 16             # ... each part at least this many 32-deep k-steps (two per wave)
MG_MIN_STEPS_LN = 8           # ... or this many for a residual product whose reduction makes the next LayerNorm
                              # (its split adds no launch; same box, 16 / 12 / 8: XL B=64 3.089 / 3.057 / 3.059
                              # ms per step, small B=32 with 1024 positions 0.620 / 0.610 / 0.608)
MEM_CACHE_BYTES = 256 << 20   # the device's memory-side cache: decode products of a model whose weights are
                              # larger load them nontemporal (same box: XL B=64 3.000 -> 2.944 ms per step,
                              # medium B=16 0.958 -> 0.916; GPT-2 small's 247 MB stay in that cache between
                              # steps, nontemporal there: 32 rows 0.548 -> 0.553)
FRAG_DECODE = True            # decode passes on the fragment-order products (else the prefill products)
HEAD_SPLIT_N = True           # the decode pass's output head on pf_mhead* (waves split the columns)
ATTN_ONE_PASS_BLOCKS = 1024   # decode passes with at most this many (row, head) blocks read each cache row in
                              # one pass (pf_attn1s), more in two (pf_attn1: keys, then values; fewer
                              # registers, more blocks resident). Same box, two -> one pass: small 16 / 24 rows
                              # (192 / 288 blocks, 448 positions) 0.450 -> 0.436 / 0.479 -> 0.466 ms per step,
                              # 32 rows (384, 1024 positions) 0.666 -> 0.637; XL 64 rows (1600) 3.110 -> 3.128


def supported(D, H, F):
    """Shapes the prefill kernels take: 64-wide heads and products whose fold
    lengths are multiples of the 64-deep chunk a product stages at a time."""
    return H * HEAD == D and D % CHUNK == 0 and F % CHUNK == 0 and D <= 8 * BLOCK


def _mtiles(rows: int) -> int:
    """16-row tiles of a decode product's kernel (pf_mgemm1 / 2 / 4)."""
    t = -(-rows // 16)
    return 1 if t <= 1 else 2 if t == 2 else 4


def frag_weights(Wt):
    """Weights [.., N, K] (row n: output n's K weights) in the decode
    products' fragment order [.., N/16, K/32, 64, 8]: element (n, k) at
    n-tile n // 16, k-step k // 32, lane 16 * ((k % 32) // 8) + n % 16,
    position k % 8 (the B operand of v_mfma_f32_16x16x32_f16 as a lane
    holds it). N is padded with zero rows to a multiple of 16."""
    import torch
    *lead, N, K = Wt.shape
    Np = -(-N // 16) * 16
    if Np != N:
        Wt = torch.cat([Wt, Wt.new_zeros(*lead, Np - N, K)], dim=-2)
    f = Wt.reshape(*lead, Np // 16, 16, K // 32, 4, 8)
    n = len(lead)
    return f.permute(*range(n), n, n + 2, n + 3, n + 1, n + 4).reshape(*lead, Np // 16, K // 32, 64, 8)


def frag_offset(M16: int, K: int, plane: int, m: int, k: int) -> int:
    """Half index of activation element (m, k) in fragment order (the
    layout pf_frag_put8 writes: plane, m-tile, k-step, lane, 8; M16 rows in
    16-row tiles)."""
    MT, KT = M16 // 16, K // 32
    return (((plane * MT + m // 16) * KT + k // 32) * 64 + ((k % 32) // 8) * 16 + m % 16) * 8 + k % 8


def prefill_source(tmax: int) -> str:
    return (f'#define VBLOCK {BLOCK}\n#define PF_TMAX {tmax}\n' + PRELUDE_SRC.read_text() + '\n'
            + PREFILL_SRC.read_text())


class _Args:
    """A kernel argument array for the C-ABI launch: pointers to each value."""

    def __init__(self, vals):
        self.vals = vals
        ptrs = [ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals]
        self.array = (ctypes.c_void_p * len(ptrs))(*ptrs)


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _i(v):
    return ctypes.c_int(int(v))


class Prefill:
    """The prefill kernels bound to one ``VestaGPT2``'s weights and cache."""

    def __init__(self, model, graphs=True):
        self.m = model
        self.graphs = graphs           # layered decode steps replay a captured HIP graph
        if not supported(model.D, model.H, model.W['fcw'].shape[2]):
            raise ValueError(f'prefill kernels need 64-wide heads and widths that are multiples of 32 '
                             f'(d={model.D}, H={model.H})')
        self.code = compile_code(prefill_source(model.tmax))
        L = lib()
        mod = ctypes.c_void_p()
        ok(L.vh_module_load(self.code, ctypes.byref(mod)), 'prefill module load')
        self.mod = mod
        track(self)
        self.fn = {}
        for name in KERNELS:
            fn = ctypes.c_void_p()
            ok(L.vh_module_get_function(mod, name.encode(), ctypes.byref(fn)), name)
            self.fn[name] = fn
        import torch
        self.err = torch.zeros(1, dtype=torch.int32, device='cuda')   # raised by a product that met an
                                                                     # activation beyond the fp16 range
        self._bufs = {}
        self._own = {}
        self._ws = None
        self._grew = False
        self._graph = None
        self._plans = {}
        self._plan = []

    def check(self):
        """Raise if a product of an earlier launch met an activation beyond the
        fp16 range its matrix-core path can carry (one synchronisation); the
        word is cleared first."""
        if int(self.err.item()):
            self.err.zero_()
            raise RuntimeError('layered engine: an activation beyond the fp16 range (65504) reached a matrix-core '
                               'product; the results are invalid')

    def close(self):
        if getattr(self, 'mod', None) is not None and self.mod.value:
            try:
                self._graph = None          # a captured graph holds launches of this module
                unload(self.mod)
            except Exception:
                pass
            self.mod = None

    def __del__(self):
        self.close()

    def _launch(self, name, grid, vals, block=BLOCK):
        """Record one launch of the plan being built."""
        self._plan.append((name, self.fn[name], int(grid), _Args(vals), int(block)))

    def _buffers(self, M):
        """Activation buffers for M rows (one set per row count, kept)."""
        import torch
        if M not in self._bufs:
            m = self.m
            F = m.W['fcw'].shape[2]
            f32 = dict(dtype=torch.float32, device='cuda')
            self._bufs[M] = dict(Z=torch.empty(M, m.D, **f32), A=torch.empty(M, m.D, **f32),
                                 Q=torch.empty(M, m.D, **f32), G=torch.empty(M, F, **f32),
                                 C=torch.empty(m.B, m.D, **f32),
                                 tok=torch.empty(M, dtype=torch.int32, device='cuda'),
                                 apv=torch.empty(m.B * ARGMAX_SPLIT, **f32),
                                 api=torch.empty(m.B * ARGMAX_SPLIT, dtype=torch.int32, device='cuda'))
        return self._bufs[M]

    def _decode_buffers(self, B):
        """Fragment-order activations of a decode pass of B rows: AF for the
        products over d (LayerNorm and attention outputs), GF for the one over
        the feed-forward width (GELU outputs). Zeroed once: rows past B are
        never written."""
        import torch
        key = ('frag', B)
        if key not in self._bufs:
            m = self.m
            rows = 16 * _mtiles(B)
            F = m.W['fcw'].shape[2]
            h16 = dict(dtype=torch.float16, device='cuda')
            self._bufs[key] = dict(AF=torch.zeros(2 * rows * m.D, **h16), GF=torch.zeros(2 * rows * F, **h16))
        return self._bufs[key]

    def _frag(self, name):
        """Weight ``name`` in the decode products' fragment order
        ([L,] n-tile, k-step, lane, 8; see hip/prefill.hip), made on first use
        and held. Layer weights are stored [L, in, out]; the output head
        ``wte`` [V, d] is already [out, in] and gets zero rows up to a
        multiple of 16."""
        key = name + '__f'
        if key not in self._own:
            W = self.m.W[name]
            self._own[key] = frag_weights(W) if name == 'wte' else frag_weights(W.transpose(1, 2))
        return self._own[key]

    def _mgemm(self, Af, K, wname, layer, N, mode, bias=None, out=None, ldo=0, F=None, ln=None, M=1):
        """One decode product (``pf_mgemm*``) over M rows: A in fragment order
        (Af), weights ``wname`` (layer ``layer``) in fragment order. With a
        split fold the parts are added by a second launch: ``pf_reduce_ln``
        for a residual product followed by the LayerNorm ``ln`` = (w, b, F_out)
        (returns True: that LayerNorm is done), ``pf_reduce_frag`` for the
        GELU product, ``pf_reduce`` otherwise."""
        m = self.m
        KT, NT = K // 32, -(-N // 16)
        mt = _mtiles(M)
        nb = -(-NT // MG_TILES[mt])
        steps = MG_MIN_STEPS_LN if mode == MODE_RESID and ln is not None else MG_MIN_STEPS
        ks = max(1, min(round(MG_BLOCKS / nb), KT // steps))
        ws = self._workspace(ks * M * N) if ks > 1 else None
        Wf = self._frag(wname)
        Wf = Wf[layer] if layer is not None else Wf
        # the extents pf_mgemm* indexes, checked before the launch is recorded
        if K % 32 or M > 16 * mt or mt > 4:
            raise ValueError(f'decode product: K={K} must be a multiple of 32 and M={M} at most 64')
        if Af.numel() < 2 * 16 * mt * K or Wf.numel() < NT * KT * 512:
            raise ValueError(f'decode product {wname}: operands smaller than {M}x{K} activations / {N}x{K} weights')
        if mode == MODE_GELU and (N % 32 or F is None or F.numel() < 2 * 16 * mt * N):
            raise ValueError(f'decode product {wname}: GELU output needs a fragment buffer of {M}x{N}, N % 32 == 0')
        if mode in (MODE_PLAIN, MODE_RESID, MODE_QKV) and out.numel() < M * ldo:
            raise ValueError(f'decode product {wname}: output smaller than {M} rows of {ldo}')
        t_args = [_p(m.keys), _p(m.vals), _p(m.t), _i(layer or 0), _i(m.L), _i(m.tmax)]
        self._launch(f'pf_mgemm{mt}' + ('n' if self._weights_nt() else ''), nb * ks,
                     [_p(Af), _p(Wf), _i(KT), _i(NT), _i(ks), _p(bias), _i(M), _i(N), _i(mode), _p(out), _i(ldo)]
                     + t_args + [_p(ws), _p(F), _p(self.err)], block=MG_WAVES * 64)
        if ks == 1:
            return False
        if mode == MODE_RESID and ln is not None:
            w, b, Fo = ln
            self._launch('pf_reduce_ln', M, [_p(ws), _i(ks), _p(bias), _i(M), _i(N), _p(out), _p(w), _p(b), _p(None),
                                             _p(Fo), _i(mt), _p(self.err)])
            return True
        if mode == MODE_GELU:
            self._launch('pf_reduce_frag', -(-M * (N // 8) // BLOCK), [_p(ws), _i(ks), _p(bias), _i(M), _i(N), _p(F),
                                                                       _i(mt), _p(self.err)])
        else:
            self._launch('pf_reduce', -(-M * N // BLOCK), [_p(ws), _i(ks), _p(bias), _i(M), _i(N), _i(mode), _p(out),
                                                            _i(ldo), _p(m.keys), _p(m.vals), _i(1), _p(m.t),
                                                            _i(layer or 0), _i(m.L), _i(m.tmax)])
        return False

    def _weights_nt(self):
        """Whether the decode products load their weights nontemporal
        (``pf_mgemm*n``): when the model's weights do not fit the memory-side
        cache."""
        return getattr(self.m, 'weight_bytes', 0) > MEM_CACHE_BYTES

    def _mhead(self, Af, K, N, out, M):
        """The output head over M rows (``pf_mhead*``): logits [M, N] = A wte^T,
        A in fragment order (Af), the packed head weights; a block of
        MG_WAVES waves per 2 MG_WAVES column tiles, each wave over the whole
        fold."""
        KT, NT = K // 32, -(-N // 16)
        Wf = self._frag('wte')
        mt = _mtiles(M)
        if K % 32 or M > 16 * mt or mt > 4 or Af.numel() < 2 * 16 * mt * K or Wf.numel() < NT * KT * 512 \
                or out.numel() < M * N:
            raise ValueError(f'output head: operands do not cover {M}x{K} activations, {N}x{K} weights')
        self._launch(f'pf_mhead{mt}', -(-NT // (2 * MG_WAVES)),
                     [_p(Af), _p(Wf), _i(KT), _i(NT), _i(M), _i(N), _p(out), _i(N)], block=MG_WAVES * 64)

    def _build_decode(self, buf, B, tok):
        """One decode pass (one position per row, B <= DECODE_ROWS) on the
        fragment-order products: LayerNorm and attention write their outputs
        as the next product's fragment-order activations, the widening
        product writes its GELU outputs as the narrowing one's."""
        m = self.m
        D, H, L = m.D, m.H, m.L
        F = m.W['fcw'].shape[2]
        V = m.W['wte'].shape[0]
        W = m.W
        mt = _mtiles(B)
        Z, Q = buf['Z'], buf['Q']
        fb = self._decode_buffers(B)
        AF, GF = fb['AF'], fb['GF']
        err = self.err
        self._launch('pf_embed_ln', B, [_p(tok), _p(m.t), _p(W['wte']), _p(W['wpe']), _p(Z), _i(D), _i(V),
                                        _i(W['wpe'].shape[0]), _p(W['ln1w'][0]), _p(W['ln1b'][0]), _p(AF), _i(mt),
                                        _p(err)])
        for layer in range(L):
            def lw(name, layer=layer):
                return W[name][layer]
            self._mgemm(AF, D, 'qkvw', layer, 3 * D, MODE_QKV, bias=lw('qkvb'), out=Q, ldo=D, M=B)
            self._launch(self._attn1(), B * H, [_p(Q), _p(m.keys), _p(m.vals), _p(None), _p(m.t), _i(layer),
                                                _i(L), _i(m.tmax), _i(H), _p(AF), _i(mt), _p(err)])
            if not self._mgemm(AF, D, 'ow', layer, D, MODE_RESID, bias=lw('ob'), out=Z, ldo=D,
                               ln=(lw('ln2w'), lw('ln2b'), AF), M=B):
                self._launch('pf_ln', B, [_p(Z), _i(0), _i(1), _p(lw('ln2w')), _p(lw('ln2b')), _p(None), _i(D),
                                          _p(AF), _i(mt), _p(err)])
            self._mgemm(AF, D, 'fcw', layer, F, MODE_GELU, bias=lw('fcb'), F=GF, M=B)
            nw, nb_ = (lw('ln1w', layer + 1), lw('ln1b', layer + 1)) if layer + 1 < L else (W['lnfw'], W['lnfb'])
            if not self._mgemm(GF, F, 'pw', layer, D, MODE_RESID, bias=lw('pb'), out=Z, ldo=D, ln=(nw, nb_, AF),
                               M=B):
                self._launch('pf_ln', B, [_p(Z), _i(0), _i(1), _p(nw), _p(nb_), _p(None), _i(D), _p(AF), _i(mt),
                                          _p(err)])
        logit, nxt = m.logits(), m.next()
        if HEAD_SPLIT_N:
            self._mhead(AF, D, V, logit, B)
        else:
            self._mgemm(AF, D, 'wte', None, V, MODE_PLAIN, out=logit, ldo=V, M=B)
        self._launch('pf_argmax_part', B * ARGMAX_SPLIT, [_p(logit), _i(V), _i(ARGMAX_SPLIT), _p(buf['apv']),
                                                           _p(buf['api'])])
        self._launch('pf_argmax', B, [_p(buf['apv']), _p(buf['api']), _i(ARGMAX_SPLIT), _p(m.x), _p(nxt), _p(m.t),
                                      _i(1)])

    def _attn1(self):
        """The decode attention kernel for this model's rows and heads."""
        return 'pf_attn1s' if self.m.B * self.m.H <= ATTN_ONE_PASS_BLOCKS else 'pf_attn1'

    def _transposed(self, name):
        """The weight copy ``name`` (``<w>__t``: [L, out, in]); the decode
        kernel's own when it binds one, else made here. Held here from first
        use on, so launch plans never point at freed memory."""
        if name not in self._own:
            packed = getattr(self.m.k, '_packed', {})
            self._own[name] = packed[name] if name in packed else \
                self.m.W[name[:-3]].transpose(-1, -2).contiguous()
        return self._own[name]

    def _gemm(self, A, lda, Wt, bias, M, N, K, mode, out, ldo, layer=0, P=1, ln=None):
        """One product launch; with few output tiles, or a long fold, the fold
        is split over blocks too (partial tiles into a workspace, then
        ``pf_reduce`` adds them in order and applies the epilogue). ``ln``
        (w, b, Y) for a residual product: the LayerNorm of all M rows of
        ``out`` into Y that comes next; a split product then does it in the
        launch that adds its parts (``pf_reduce_ln``). Returns whether it did."""
        m = self.m
        tiles = -(-M // TILE) * -(-N // TILE)
        ks = max(1, min(-(-SPLIT_BLOCKS // tiles), (K // CHUNK) // SPLIT_MIN_CHUNKS))
        ws = self._workspace(ks * M * N) if ks > 1 else None
        tail = [_p(m.keys), _p(m.vals), _i(P), _p(m.t), _i(layer), _i(m.L), _i(m.tmax)]
        self._launch('pf_gemm', tiles * ks, [_p(A), _i(lda), _p(Wt), _p(bias), _i(M), _i(N), _i(K), _i(mode),
                                             _p(out), _i(ldo)] + tail + [_i(ks), _p(ws), _p(self.err)])
        if FUSE_REDUCE_LN and ks > 1 and ln is not None and mode == MODE_RESID and ldo == N:
            w, b, Y = ln
            self._launch('pf_reduce_ln', M, [_p(ws), _i(ks), _p(bias), _i(M), _i(N), _p(out), _p(w), _p(b), _p(Y),
                                             _p(None), _i(0), _p(self.err)])
            return True
        if ks > 1:
            self._launch('pf_reduce', -(-M * N // BLOCK), [_p(ws), _i(ks), _p(bias), _i(M), _i(N), _i(mode),
                                                            _p(out), _i(ldo)] + tail)
        return False

    def _workspace(self, n):
        """Partial tiles of split products: one buffer, grown to the largest
        need (launches on one stream run one after another)."""
        import torch
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(n, dtype=torch.float32, device='cuda')
            self._plans = {}            # plans hold the old pointer
            self._grew = True
        return self._ws

    def _plan_for(self, key, buf, B, P, tok):
        """The launch plan ``key``, built on first use (twice when the build
        grew the workspace, so that no launch keeps the old pointer)."""
        if key not in self._plans:
            for _ in range(2):
                self._plan, self._grew = [], False
                self._build(buf, B, P, tok)
                if not self._grew:
                    break
            self._plans[key] = self._plan
        return self._plans[key]

    def _replay(self, plan):
        import torch
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        L = lib()
        for name, fn, grid, a, block in plan:
            ok(L.vh_launch(fn, grid, block, 0, stream, a.array), name)

    def run(self, prompt):
        """Prefill ``prompt`` (int32 device tensor [B, P]) at positions t .. t + P - 1
        (t the model's position counter, read and advanced on the device).

        The launch sequence with its argument arrays is built once per P and
        replayed: every pointer it holds (weights, cache, this object's
        activation buffers and prompt copy) stays fixed."""
        B, P = prompt.shape
        buf = self._buffers(B * P)
        buf['tok'].copy_(prompt.reshape(-1))
        self._replay(self._plan_for(P, buf, B, P, buf['tok']))

    def decode(self, n, tokens=None):
        """``n`` greedy decode steps, each one pass with P = 1 over the
        model's input ``x`` (the last pass's argmax): the layer-at-a-time
        path for shapes the persistent kernel does not fit. ``tokens`` (a
        contiguous int32 device tensor of at least n * B ids, any shape, e.g.
        [n, B]) receives each step's chosen tokens, step k at flat offsets
        k * B .. k * B + B - 1."""
        m = self.m
        flat = None
        if tokens is not None:
            if not (tokens.is_cuda and tokens.dtype == m.x.dtype and tokens.is_contiguous()):
                raise TypeError('tokens must be a contiguous int32 device tensor')
            if tokens.numel() < n * m.B:
                raise ValueError(f'tokens holds {tokens.numel()} ids, {n * m.B} needed')
            flat = tokens.view(-1)
        buf = self._buffers(m.B)
        plan = self._plan_for('decode', buf, m.B, 1, m.x)
        step = lambda: self._replay(plan)       # noqa: E731
        if self.graphs:
            if self._graph is None or self._graph[0] is not plan:
                self._graph = (plan, self._capture(plan))
            step = self._graph[1].replay
        for k in range(n):
            step()
            if flat is not None:
                flat[k * m.B:(k + 1) * m.B].copy_(m.x)

    def _capture(self, plan):
        """One decode pass recorded as a HIP graph: a step is then one graph
        launch instead of some hundred kernel launches from the host. The pass
        has no memory sets or host reads, and every pointer it holds stays
        fixed (the position is read on the device)."""
        import torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._replay(plan)
        return g

    def _build(self, buf, B, P, tok):
        if P == 1 and B <= DECODE_ROWS and FRAG_DECODE:
            return self._build_decode(buf, B, tok)
        m = self.m
        M, D, H, L = B * P, m.D, m.H, m.L
        F = m.W['fcw'].shape[2]
        V = m.W['wte'].shape[0]
        W = m.W
        Z, A, Q, G, C = buf['Z'], buf['A'], buf['Q'], buf['G'], buf['C']
        self._launch('pf_embed', M, [_p(tok), _i(P), _p(m.t), _p(W['wte']), _p(W['wpe']), _p(Z), _i(D), _i(V),
                                     _i(W['wpe'].shape[0])])
        normed = False                  # A holds LN1 of Z already (made by the last product's reduction)
        for layer in range(L):
            def lw(name, layer=layer):
                return W[name][layer]

            def lt(name):
                return self._transposed(name)[layer]
            if not normed:
                self._launch('pf_ln', M, [_p(Z), _i(0), _i(1), _p(lw('ln1w')), _p(lw('ln1b')), _p(A), _i(D),
                                          _p(None), _i(0), _p(self.err)])
            self._gemm(A, D, lt('qkvw__t'), lw('qkvb'), M, 3 * D, D, MODE_QKV, Q, D, layer, P)
            if P == 1:      # a decode pass: a block per (row, head) (GPT-2 small, 32 rows, 1024
                            # positions: 1.32 -> 1.07 ms per step against a wave per (row, head))
                self._launch(self._attn1(), M * H, [_p(Q), _p(m.keys), _p(m.vals), _p(A), _p(m.t), _i(layer),
                                                    _i(L), _i(m.tmax), _i(H), _p(None), _i(0), _p(self.err)])
            else:
                self._launch('pf_attn', -(-M * H // (BLOCK // 64)),
                             [_p(Q), _p(m.keys), _p(m.vals), _p(A), _i(M), _i(P), _p(m.t), _i(layer), _i(L),
                              _i(m.tmax), _i(H)])
            if not self._gemm(A, D, lt('ow__t'), lw('ob'), M, D, D, MODE_RESID, Z, D,
                              ln=(lw('ln2w'), lw('ln2b'), A)):
                self._launch('pf_ln', M, [_p(Z), _i(0), _i(1), _p(lw('ln2w')), _p(lw('ln2b')), _p(A), _i(D),
                                          _p(None), _i(0), _p(self.err)])
            self._gemm(A, D, lt('fcw__t'), lw('fcb'), M, F, D, MODE_GELU, G, F)
            if layer + 1 < L:
                nxt = (lw('ln1w', layer + 1), lw('ln1b', layer + 1), A)
            else:
                nxt = (W['lnfw'], W['lnfb'], C) if P == 1 else None   # the final norm: each row's last position
            normed = self._gemm(G, F, lt('pw__t'), lw('pb'), M, D, F, MODE_RESID, Z, D, ln=nxt)
        if not normed:
            self._launch('pf_ln', B, [_p(Z), _i(P - 1), _i(P), _p(W['lnfw']), _p(W['lnfb']), _p(C), _i(D),
                                      _p(None), _i(0), _p(self.err)])
        logit, nxt = m.logits(), m.next()
        self._gemm(C, D, W['wte'], None, B, V, D, MODE_PLAIN, logit, V)
        self._launch('pf_argmax_part', B * ARGMAX_SPLIT, [_p(logit), _i(V), _i(ARGMAX_SPLIT), _p(buf['apv']),
                                                           _p(buf['api'])])
        self._launch('pf_argmax', B, [_p(buf['apv']), _p(buf['api']), _i(ARGMAX_SPLIT), _p(m.x), _p(nxt), _p(m.t),
                                      _i(P)])
