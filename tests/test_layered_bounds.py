"""Host bounds checks of the layered engine's decode products, on the CPU.

``Prefill._mgemm`` and ``Prefill._mhead`` check every extent the
``pf_mgemm*`` / ``pf_mhead*`` kernels index (fold depth, row tiles, operand,
fragment and output sizes, the output pitch) before a launch is recorded in
the plan, so a mis-sized operand is a ValueError on the host and never an
out-of-bounds access on the device. A launch with a wrong output pitch (the
pitch of the 3*d qkv columns given for a d-column output buffer) is one such
case. No GPU and no kernel are involved: the plan is only recorded."""
import types

import pytest
import torch

from vesta import prefill as pf

D, F, V, L, B = 64, 256, 97, 2, 8


def _engine(frag_numel=None):
    """A Prefill with its host state only: a plan list, weights in fragment
    order of the right (or the given) size, a CPU workspace."""
    e = pf.Prefill.__new__(pf.Prefill)
    e._plan, e._own, e._bufs = [], {}, {}
    e.fn = {n: None for n in ('pf_mgemm1', 'pf_mgemm2', 'pf_mgemm4', 'pf_mgemm1n', 'pf_mgemm2n', 'pf_mgemm4n',
                              'pf_reduce_ln', 'pf_reduce_frag', 'pf_reduce',
                              'pf_mhead1', 'pf_mhead2', 'pf_mhead4')}
    e.err = torch.zeros(1, dtype=torch.int32)
    e.m = types.SimpleNamespace(keys=torch.zeros(1), vals=torch.zeros(1), t=torch.zeros(1, dtype=torch.int32),
                                L=L, tmax=16, B=B, D=D)

    def frag(name):
        n_out, k = {'qkvw': (3 * D, D), 'ow': (D, D), 'fcw': (F, D), 'pw': (D, F), 'wte': (V, D)}[name]
        n = frag_numel if frag_numel is not None else -(-n_out // 16) * (k // 32) * 512
        return torch.zeros(n if name == 'wte' else (L, n), dtype=torch.float16)
    e._frag = frag
    e._workspace = lambda n: torch.zeros(n)
    return e


def _af(rows, k):
    return torch.zeros(2 * 16 * pf._mtiles(rows) * k, dtype=torch.float16)


def test_a_well_formed_product_is_recorded():
    e = _engine()
    e._mgemm(_af(B, D), D, 'qkvw', 0, 3 * D, pf.MODE_QKV, bias=torch.zeros(3 * D), out=torch.zeros(B, D), ldo=D,
             M=B)
    assert e._plan and e._plan[0][0] == 'pf_mgemm1'
    e._mhead(_af(B, D), D, V, torch.zeros(B, V), B)
    assert e._plan[-1][0] == 'pf_mhead1'


@pytest.mark.parametrize('case', ['fold', 'rows', 'activations', 'weights', 'pitch', 'gelu'])
def test_mis_sized_products_are_refused_before_anything_is_recorded(case):
    e = _engine(frag_numel=100 if case == 'weights' else None)
    kw = dict(Af=_af(B, D), K=D, wname='qkvw', layer=0, N=3 * D, mode=pf.MODE_QKV, bias=torch.zeros(3 * D),
              out=torch.zeros(B, D), ldo=D, M=B)
    if case == 'fold':
        kw['K'] = D - 16                         # not a multiple of 32
    elif case == 'rows':
        kw['M'] = 65                             # beyond four 16-row tiles
    elif case == 'activations':
        kw['Af'] = _af(B, D)[:-1]                # one value short of 16 x K in two planes
    elif case == 'pitch':
        kw['ldo'] = 3 * D                        # the qkv columns' pitch for a d-column output
    elif case == 'gelu':
        kw.update(wname='fcw', N=F, mode=pf.MODE_GELU, bias=torch.zeros(F), out=None, ldo=0,
                  F=torch.zeros(2 * 16 * F - 1, dtype=torch.float16))
    with pytest.raises(ValueError):
        e._mgemm(**kw)
    assert e._plan == []


@pytest.mark.parametrize('case', ['fold', 'activations', 'weights', 'output'])
def test_mis_sized_output_heads_are_refused(case):
    e = _engine(frag_numel=100 if case == 'weights' else None)
    Af, K, out = _af(B, D), D, torch.zeros(B, V)
    if case == 'fold':
        K = D + 8
    elif case == 'activations':
        Af = Af[:100]
    elif case == 'output':
        out = torch.zeros(B * V - 1)
    with pytest.raises(ValueError, match='output head'):
        e._mhead(Af, K, V, out, B)
    assert e._plan == []


@pytest.mark.parametrize('weight_bytes,kernel', [(247_000_000, 'pf_mgemm1'), (707_000_000, 'pf_mgemm1n')])
def test_products_load_weights_nontemporal_beyond_the_memory_side_cache(weight_bytes, kernel):
    """A model whose weights fit the device's memory-side cache keeps the
    default policy for the products' weight loads; a larger one gets the
    nontemporal variant of the same kernel."""
    e = _engine()
    e.m.weight_bytes = weight_bytes
    e._mgemm(_af(B, D), D, 'qkvw', 0, 3 * D, pf.MODE_QKV, bias=torch.zeros(3 * D), out=torch.zeros(B, D), ldo=D,
             M=B)
    assert e._plan[0][0] == kernel


@pytest.mark.parametrize('rows,tiles', [(8, 1), (32, 1), (64, 2)])
def test_products_take_one_column_tile_per_block_up_to_32_rows(rows, tiles):
    """A decode product's block makes one 16-column tile up to 32 rows (two
    row tiles) and two at 64 rows (four): the grid is the column tiles over
    that, times the fold parts."""
    e = _engine()
    e.m.B = rows
    e._mgemm(_af(rows, D), D, 'qkvw', 0, 3 * D, pf.MODE_QKV, bias=torch.zeros(3 * D), out=torch.zeros(rows, D),
             ldo=D, M=rows)
    name, _, grid, args, _ = e._plan[0]
    ks = args.vals[4].value
    assert name == f'pf_mgemm{pf._mtiles(rows)}'
    assert grid == -(-(3 * D // 16) // tiles) * ks
