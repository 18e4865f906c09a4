"""The gfx950 lowering on the CPU: analyses, placements, barrier counts, and
hipRTC compilation of the generated kernels (hipRTC needs no GPU).

Reference behaviour being mirrored: batch lift (reference vesta/lower.py:109-132),
hoist/alias/inline (:187-310), placement classes (:543-561), Lowered fields
(:69-79) and lower() (:1294-1329).
"""
import os
import re

import pytest

from vesta import stream
from vesta import launch, mfma
from vesta.gpt2_program import gpt2_program
from vesta.interp import parse
from vesta.lower import LowerError, Lowering, batch_lift, lower

from conftest import PKG, REPO


def gpt2_spec(B, tmax, L=12, D=768, H=12, F=3072, V=50257, npos=1024):
    E = D // H
    return {'x': ((B,), 'i32'), 't': ((), 'i32'), 'wte': ((V, D), 'f16'), 'wpe': ((npos, D), 'f16'),
            'ln1w': ((L, D), 'f16'), 'ln1b': ((L, D), 'f16'), 'qkvw': ((L, D, 3 * D), 'f16'),
            'qkvb': ((L, 3 * D), 'f16'), 'ow': ((L, D, D), 'f16'), 'ob': ((L, D), 'f16'), 'ln2w': ((L, D), 'f16'),
            'ln2b': ((L, D), 'f16'), 'fcw': ((L, D, F), 'f16'), 'fcb': ((L, F), 'f16'), 'pw': ((L, F, D), 'f16'),
            'pb': ((L, D), 'f16'), 'lnfw': ((D,), 'f16'), 'lnfb': ((D,), 'f16'),
            'keys': ((B, L, tmax, H, E), 'f16'), 'vals': ((B, L, tmax, H, E), 'f16')}


def lower_gpt2(B=1, tmax=384, shape=(12, 768, 12, 3072, 50257), **kw):
    L, D, H, F, V = shape
    text = gpt2_program(L, D, H, F, V)
    return lower(text, gpt2_spec(B, tmax, L, D, H, F, V), {'s': tmax}, batch=B, per_token=('x', 'keys', 'vals'),
                 outputs=('logit', 'next'), feedback={'x': 'next', 't': 1}, **kw)


def placements(low):
    out = {}
    for st, pl in low.plan:
        name = st.split('[')[0].split(' ')[0] if not st.startswith('residue') else st.split('[')[0]
        out[name] = pl
    return out


def test_batch_lift_adds_token_axis():
    stmts = batch_lift(parse('residue x\nresidue w[n]\naxis n = 3\ny[n] = w[n] + x\nz = fold sum n: y[n]\n'), 4, {'x'})
    assert stmts[0] == ('axis', 'bt', ('num', 4))
    let_y = [s for s in stmts if s[0] == 'let' and s[1] == 'y'][0]
    assert let_y[2] == ['bt', 'n']
    assert ('idx', 'x', [('name', 'bt')]) in [n for n in _nodes(let_y[3])]
    let_z = [s for s in stmts if s[0] == 'let' and s[1] == 'z'][0]
    assert let_z[2] == ['bt'] and let_z[3][3] == ('idx', 'y', [('name', 'bt'), ('name', 'n')])


def _nodes(e):
    from vesta.lower import nodes
    return list(nodes(e))


def test_gpt2_small_b1_plan():
    low = lower_gpt2(1)
    p = placements(low)
    # two projections stream rows of a transposed weight copy, no split-K; the
    # attention's blocks do the out-projection (12 of the 144 blocks per head) and add it
    # into z1, a fixed-point sum whose base z + ob is stored in the phase before
    for name in ('qkv', 'u'):
        assert p[name].startswith('stream (transposed copy)'), (name, p[name])
    assert p['oo'] == 'attention[bt, h] projection x12'
    assert p['z1'].startswith('fixed-point sum')
    # the down-projection folds each block's own 22 widened values in the widening's
    # phase, from pw's rows in their own layout, into z kept in 4 fixed-point copies
    assert p['z2'] == 'local fold over the points of u (22 per block), fixed-point sum in 4 copies'
    assert low.packs == {'qkvw__t': 'qkvw', 'ow__t': 'ow', 'fcw__t': 'fcw'}
    assert 'stage_fxc<4>' in low.src and 'clear the copies of z' in low.src
    # attention: scores, softmax statistics and weighted values in one block per (bt, h)
    assert p['sc'] == p['mx'] == p['_h1'] == p['o'] == 'attention[bt, h]'
    assert p['logit'] == 'stream'
    # argmax over each block's own logits, combined by every block; the embedding
    # (the layer loop's first residual) is evaluated where layer 0 reads it
    assert p['best'] == 'argmax (own points)' and p['next'] == 'argmax'
    assert p['z0'] == 'first value of z, made where read'
    assert p['m1'] == p['v1'] == p['a'] == 'private'
    assert p['residue keys'] == 'epilogue of qkv' and p['residue vals'] == 'epilogue of qkv'
    assert p['g'] == 'epilogue of u'
    # softmax denominator hoisted, q / ex / w inlined
    assert '_h1' in p and 'q' not in p and 'w' not in p and 'ex' not in p
    # three grid barriers per layer: the down-projection folds in the widening's phase
    assert low.barriers_per_launch == 3 * 12 + 1
    assert set(low.scratch) >= {'logit', 'next'} and low.scratch['logit'][2] == (1, 50257)
    # fixed-point, block-local and elided values are not host-visible
    assert not {'z1', 'oo', 'o', 'g', 'z'} & set(low.scratch)


def test_attention_readiness_flags_lower_to_two_barriers_per_layer(monkeypatch):
    """With READY_ATTN the attention waits for the blocks that made its query,
    key and value rows instead of a grid barrier: two grid barriers per layer
    at B=1 and B=8; the projection's sum and the layer carry alternate
    between two buffers (cleared once a launch, then a layer ahead). Off by
    default (slower on the MI355X); it must still lower and compile."""
    from vesta import attn
    monkeypatch.setattr(attn, 'READY_ATTN', True)
    for B in (1, 8):
        low = lower_gpt2(B, 448)
        assert low.barriers_per_launch == 2 * 12 + 1, B
        assert low.src.count('flag_publish(bar') == (1 if B == 1 else 2)
        assert 'both layer buffers of z1, cleared once a launch' in low.src
        assert "clear the next layer's z1" in low.src and 'clear the buffer of z read before' in low.src
        assert launch.code_spills(launch.compile_code(low.src)) <= 16


def test_gpt2_small_b8_plan():
    low = lower_gpt2(8)
    p = placements(low)
    assert p['mx'] == p['_h1'] == p['o'] == 'attention[bt, h]'
    # several rows: the streams with 8+ points per block run on the matrix cores
    assert p['qkv'] == 'stream (transposed copy) mfma +2 fused' and p['logit'] == 'stream mfma'
    assert p['u'].endswith('mfma +1 fused')
    # few points per block: the fold is split over blocks too, partial tiles added
    # into a fixed-point residual
    # (point groups of two 16-column tiles at 8 rows: 24 groups, the fold in 8 slices)
    assert p['z2'].startswith('stream (transposed copy) mfma, fold in 8 slices, fixed-point sum')
    assert low.barriers_per_launch <= 75
    assert low.scratch['logit'][2] == (8, 50257) and low.scratch['next'][2] == (8,)


@pytest.mark.parametrize('B,tiles', [(4, 2), (8, 2), (12, 4)])
def test_fold_split_point_groups_by_rows(B, tiles, monkeypatch):
    """A fold split's point groups take at most two 16-column tiles at 8 rows
    or fewer and four up to 16 rows (``SPLIT_TILES_PACKED``, ``SPLIT_TILES``),
    and the cost model goes up to that bound here."""
    chosen = []
    orig = mfma.MfmaMixin.split_of

    def spy(self, s):
        r = orig(self, s)
        if r is not None:
            chosen.append(r['NTS'])
        return r
    monkeypatch.setattr(mfma.MfmaMixin, 'split_of', spy)
    lower_gpt2(B)
    assert chosen and max(chosen) == tiles


def test_layer_norm_square_roots_per_thread_at_one_row():
    """At one row every wave folds the LayerNorm statistics itself, so each
    thread makes sqrt(v + eps) and its reciprocal in registers (no LDS slot,
    no block sync); from two rows one thread per row makes them into LDS."""
    one = lower_gpt2(1).src
    assert 'once per leading point' not in one
    assert len(re.findall(r'const float (hv\d+_0)r = 1\.0f / \1;', one)) == 3     # LN1, LN2, final LN
    assert lower_gpt2(8).src.count('once per leading point') == 3


def test_local_fold_adds_cover_each_element_once_per_block():
    """The local fold's rotated adds (blocks sharing a fixed-point copy start
    apart): read the rotation and the loop out of the generated B=1 source
    and evaluate them for every block and thread; each block adds every
    element of its row exactly once, and blocks of one copy do start apart."""
    src = lower_gpt2(1).src
    rot = re.search(r'const int ro_ = \(int\)\(\(blockIdx\.x / (\d+)u\) \* (\d+)u % (\d+)u\);', src)
    loop = re.search(r'for \(int i_ = tid; i_ < (\d+); i_ \+= (\d+)\) \{\s*'
                     r'const int e_ = i_ \+ ro_ < (\d+) \? i_ \+ ro_ : i_ \+ ro_ - (\d+);', src)
    assert rot and loop
    copies, step, n = map(int, rot.groups())
    lim, stride, lt, sub = map(int, loop.groups())
    assert n == lim == lt == sub == 768 and stride == 512
    starts = set()
    for b in range(144):
        ro = (b // copies) * step % n
        got = sorted(i + ro if i + ro < lt else i + ro - sub for t in range(512) for i in range(t, lim, stride))
        assert got == list(range(n)), b
        starts.add((b % copies, ro))
    assert len(starts) > copies


def test_params_and_abi():
    low = lower_gpt2(1)
    names = [n for n, _, _ in low.params]
    spec = list(gpt2_spec(1, 384))
    # transposed copies for the streams (the down-projection's local fold reads pw as it is)
    assert names[:len(spec)] == spec and sorted(names[len(spec):]) == ['fcw__t', 'ow__t', 'qkvw__t']
    written = {n for n, _, w in low.params if w}
    assert written == {'x', 't', 'keys', 'vals'}
    sig = re.search(r'vesta_step\((.*?)\) \{', low.src).group(1)
    assert sig.endswith('const int nsteps, int* __restrict__ tok_out, const int* __restrict__ tok_in')
    assert 'const vh_half* __restrict__ R_wte' in sig and 'vh_half* __restrict__ R_keys' in sig


def test_kernel_has_no_cache_maintenance_fences():
    """Cross-block data goes through coherent loads/stores: no agent fences."""
    src = lower_gpt2(1).src
    assert '__builtin_amdgcn_fence' not in src.split('extern "C"')[1]


@pytest.mark.parametrize('B', [1, 8])
def test_gpt2_small_compiles_for_gfx950(B):
    low = lower_gpt2(B)
    code = launch.compile_code(low.src, cache=False)
    assert code[:4] == b'\x7fELF'


def test_tiny_and_medium_compile():
    tiny = lower_gpt2(1, 20, (2, 16, 4, 64, 37))
    assert launch.compile_code(tiny.src, cache=False)[:4] == b'\x7fELF'
    med = lower_gpt2(1, 512, (24, 1024, 16, 4096, 50257))
    assert placements(med)['qkv'].startswith('stream')
    assert launch.compile_code(med.src, cache=False)[:4] == b'\x7fELF'


def test_fitted_kernels_take_the_deepest_mfma_pipeline_that_fits(monkeypatch):
    """lower_fitted tries each prefetch budget with two k-blocks per register
    set of an unprefetched matrix-core stream, then one, and keeps the first
    try within SPILLS_OK."""
    tries = []

    class Low:
        def __init__(self, b, d):
            self.src = (b, d)

    def fake_lower(text, res, prefetch_vgprs, mfma_pipe, **kw):
        tries.append((prefetch_vgprs, mfma_pipe))
        return Low(prefetch_vgprs, mfma_pipe)
    spills = {(64, 2): launch.SPILLS_OK + 1, (64, 1): launch.SPILLS_OK}     # just beyond, then at the limit
    with monkeypatch.context() as mp:
        mp.setattr(launch, 'compile_code', lambda src: src)
        mp.setattr(launch, 'code_spills', lambda code: spills.get(code, 99))
        assert launch.lower_fitted(fake_lower, '', {}).src == (64, 1)
        assert tries == [(64, 2), (64, 1)]
        spills.clear()
        tries.clear()
        last = launch.lower_fitted(fake_lower, '', {}).src
        assert tries == [(b, d) for b in launch.PREFETCH_BUDGETS for d in (2, 1)] and last == tries[-1]
        # 4 to 8 rows start from their own budgets, other row counts from the default ones
        for batch, budgets in ((4, launch.PREFETCH_BUDGETS_PACKED), (8, launch.PREFETCH_BUDGETS_PACKED),
                               (3, launch.PREFETCH_BUDGETS), (9, launch.PREFETCH_BUDGETS)):
            tries.clear()
            launch.lower_fitted(fake_lower, '', {}, batch=batch)
            assert tries == [(b, d) for b in budgets for d in (2, 1)], batch
    # GPT-2 small B=8: the first try within the limit, every earlier one beyond it
    small = launch.lower_fitted(lower, gpt2_program(12, 768, 12, 3072, 50257), gpt2_spec(8, 448),
                                axis_max={'s': 448}, batch=8, per_token=('x', 'keys', 'vals'),
                                outputs=('logit', 'next'), feedback={'x': 'next', 't': 1})
    for b, d in [(b, d) for b in launch.PREFETCH_BUDGETS_PACKED for d in (2, 1)]:
        src = lower_gpt2(8, 448, prefetch_vgprs=b, mfma_pipe=d).src
        if src == small.src:
            assert launch.code_spills(launch.compile_code(src)) <= launch.SPILLS_OK
            break
        assert launch.code_spills(launch.compile_code(src)) > launch.SPILLS_OK, (b, d)
    else:
        raise AssertionError('the fitted kernel is none of the tries')


def test_errors():
    with pytest.raises(NameError):
        lower('residue q[i]\naxis i = 2\ny[i] = q[i]\n', {}, {})
    with pytest.raises(LowerError):
        lower('residue q[s]\naxis s = t + 1\nresidue t\ny[s] = q[s]\n', {'q': ((4,), 'f32'), 't': ((), 'i32')}, {})
    with pytest.raises(NameError):
        lower('residue q[i]\naxis i = 2\ny[i] = q[i]\n', {'q': ((2,), 'f32')}, {}, outputs=('nope',))


def test_hiprtc_error_carries_log():
    with pytest.raises(RuntimeError, match='hipRTC failed'):
        launch.compile_code('extern "C" __global__ void vesta_step() { undeclared_thing(); }', cache=False)


def test_generic_programs_lower_and_compile():
    """Small programs of every form lower to kernels that compile."""
    import json
    cases = json.load(open(os.path.join(REPO, 'tests', 'golden', 'grammar_cases.json')))
    for name, case in cases.items():
        res = {}
        for k, v in case['inputs'].items():
            if isinstance(v, dict):
                import numpy as np
                res[k] = (tuple(np.array(v['values']).shape), v['dtype'])
            else:
                res[k] = ((), 'i32')
        outs = [r for r in case['record'] if r in case.get('axes', {})]
        low = lower(case['text'], res, {}, outputs=tuple(outs))
        assert launch.compile_code(low.src, cache=False)[:4] == b'\x7fELF', name


def test_c_abi_exports_every_declared_symbol():
    import ctypes
    header = open(os.path.join(REPO, 'include', 'vesta_hip.h')).read()
    declared = set(re.findall(r'^(?:int|void|const char\*)\s+(vh_\w+)\(', header, re.M))
    assert {'vh_compile', 'vh_module_load', 'vh_launch_cooperative', 'vh_occupancy'} <= declared
    lib = ctypes.CDLL(launch.LIB_PATH)
    for sym in declared:
        assert hasattr(lib, sym), sym
    lib.vh_error_string.restype = ctypes.c_char_p
    assert lib.vh_error_string(0) == b'success'


@pytest.mark.parametrize('budget', [16, 32, 64])
def test_chunked_attention_loads_every_slot(budget):
    """Long caches run the softmax over chunks of slots; whatever the prefetch
    register budget, every slot's key and value rows are loaded somewhere:
    the first chunk's into kq / vq (at the barrier before, or at the start),
    each later chunk's by the run-time chunk loop one iteration ahead."""
    import re as _re
    from vesta.attn import ATTN_CHUNK
    from vesta.lower import lower
    text = open(os.path.join(PKG, 'vesta', 'programs', 'gpt2.vst')).read()
    low = lower(text, gpt2_spec(1, 512), {'s': 512}, batch=1, per_token=('x', 'keys', 'vals'),
                outputs=('logit', 'next'), feedback={'x': 'next', 't': 1}, prefetch_vgprs=budget)
    nchunks = int(_re.search(r'for \(int c_ = 0; c_ < (\d+); \+\+c_\)', low.src).group(1))
    for arr, nxt in (('kq', 'kn_'), ('vq', 'vn_')):
        name = _re.search(arr + r'_\w+\[10\];', low.src).group(0).split('[')[0]
        first = {int(k) for k in _re.findall(_re.escape(name) + r'\[(\d+)\] = ldc16_h', low.src)}
        assert first == set(range(ATTN_CHUNK)), (arr, sorted(first))
        later = {int(j) for j in _re.findall(_re.escape(nxt) + r'\[(\d+)\] = ldc16_h', low.src)}
        assert later == set(range(ATTN_CHUNK))
        covered = first | {(c + 1) * ATTN_CHUNK + j for c in range(nchunks - 1) for j in later}
        assert set(range(10)) <= covered
    assert _re.search(r'const int sn0_ = \(\(c_ \+ 1\) \* 4 \+ 0\) \* 56', low.src)


def test_prefill_kernels_compile_for_gfx950():
    """The multi-token prefill / layered-engine kernels: one code object per
    cache length, every kernel the host launches present, no spills."""
    from vesta.prefill import KERNELS, prefill_source, supported
    for tmax in (384, 1024):
        code = launch.compile_code(prefill_source(tmax), cache=False)
        assert code[:4] == b'\x7fELF'
        for name in KERNELS:
            assert name.encode() in code, name
        assert launch.code_spills(code) == 0
    assert supported(768, 12, 3072) and supported(1600, 25, 6400)
    assert not supported(16, 4, 64) and not supported(768, 16, 3072)


def test_weight_cache_policy(monkeypatch):
    """Weights kept in the caches (temporal loads): all of them below 4 rows;
    from 4 rows the output head (outside the layer loop), the fold-split
    down-projection, and the attention out-projection fused into the
    attention while its copies over all layers fit the bound (GPT-2 small
    14 MB, medium 50 MB); past the bound it is streamed."""
    import re as _re

    def policy(B, shape=(12, 768, 12, 3072, 50257)):
        src = lower_gpt2(B, 64, shape).src.split('extern "C"')[1]
        got = set(_re.findall(r'ldg16_t\(mk_rsrc\((R_\w+)', src))
        streamed = set(_re.findall(r'ldg16_nt\(mk_rsrc\((R_\w+)', src))
        assert not got & streamed, (B, got & streamed)
        return got
    assert policy(1) == {'R_qkvw__t', 'R_ow__t', 'R_fcw__t', 'R_pw', 'R_wte'}
    assert policy(8) == {'R_pw__t', 'R_wte', 'R_ow__t'}
    assert policy(8, (24, 1024, 16, 4096, 50257)) == {'R_pw__t', 'R_wte', 'R_ow__t'}
    monkeypatch.setattr(stream, 'PROJ_KEPT_BYTES', 12 * 768 * 768 * 2 - 1)
    assert policy(8) == {'R_pw__t', 'R_wte'}


def test_grid_choice():
    """144 blocks below 4 rows, 192 from 4 rows; the full 256 when the default
    grid would overflow LDS (XL widths at 8 rows) or starve the attention
    projection of replicas (16 heads x 8 rows)."""
    assert lower_gpt2(1).grid_max == 144
    assert lower_gpt2(8).grid_max == 192
    assert lower_gpt2(8, 16, (2, 1600, 25, 6400, 50257)).grid_max == 256
    assert lower_gpt2(8, 64, (2, 1024, 16, 4096, 50257)).grid_max == 256
    assert lower_gpt2(8, grid=160).grid_max == 160


def test_xl_widths_at_64_rows_fit_a_cu_of_lds():
    """GPT-2 XL widths at 64 rows fit a CU's LDS on the widest grid: the
    products stage their other factor through LDS in fold chunks (before,
    a row stream staged 8 rows x 6400 floats, 206,592 bytes per block)."""
    from vesta.lower import LDS_BYTES
    low = lower_gpt2(64, 16, (2, 1600, 25, 6400, 50257))
    assert low.grid_max == 256 and low.shared_bytes <= LDS_BYTES


def test_matrix_core_streams_beyond_16_rows():
    """From 17 to 64 rows the products stay on the matrix cores: 16-row tiles
    per weight fragment, the fold staged through LDS in chunks when the
    halves of all rows do not fit, and fold splits over blocks whose tiles
    go only to the seven compute waves (the eighth polls barriers and holds
    no prefetched weights). GPT-2 XL at 64 rows fits a CU's LDS."""
    from vesta.lower import LDS_BYTES
    from vesta.mfma import MfmaMixin, MFMA_HALVES_MAX
    assert MfmaMixin.mfma_rows(16, 24) == (1, 24, 1)
    RT, CB, NC = MfmaMixin.mfma_rows(64, 50)
    assert RT == 4 and CB * NC >= 50 and 2 * 64 * (CB * 64 + 16) <= MFMA_HALVES_MAX
    for B, tmax, shape in ((32, 64, (2, 768, 12, 3072, 50257)), (64, 16, (2, 1600, 25, 6400, 50257))):
        low = lower_gpt2(B, tmax, shape)
        assert low.shared_bytes <= LDS_BYTES
        pl = placements(low)
        for name in ('qkv', 'oo', 'u', 'z2', 'logit'):
            assert 'mfma' in pl[name], (B, name, pl[name])
        waves = [min(int(w) for w in re.findall(r'wave < (\d+)', m))
                 for m in re.findall(r'const bool mok_ = [^;]*;', low.src)]
        assert waves and max(waves) <= 7, waves
