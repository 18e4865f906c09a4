"""The phase emulator (``vesta.phases``) on the CPU: the lowered GPT-2 plans
order every cross-block access under the weak memory model (grid barriers,
readiness-flag waits, local folds and fixed-point adds, parity buffers), and
a deliberately dropped barrier or a readiness-flag range one block short is
caught. Reference behaviour being checked: the barrier placement of
reference ``vesta/lower.py:563-600`` (its static hazard table), here for the
gfx950 lowering and the barriers it removes."""
import pytest

from vesta import attn, phases
from vesta import lower as LM
from vesta.chain import ChainError
from vesta.gpt2_program import gpt2_program

from test_lower import gpt2_spec

TINY = (2, 128, 2, 512, 97)
SMALL = (12, 768, 12, 3072, 50257)


def lowering(shape, B, tmax=64):
    """The Lowering behind ``LM.lower``'s kernel: the same fallback without
    local folds and the same switch to the wide grid."""
    L, D, H, F, V = shape
    args = (gpt2_program(L, D, H, F, V), gpt2_spec(B, tmax, L, D, H, F, V), {'s': tmax}, B,
            ('x', 'keys', 'vals'), ('logit', 'next'), {'x': 'next', 't': 1}, False, 'k')
    out, low = LM._lower(*args, None, None, None)
    if low.grid_auto and low.grid != LM.GRID_WIDE and (low.proj_wider or out.shared_bytes > LM.LDS_BYTES):
        out, low = LM._lower(*args, LM.GRID_WIDE, None, None)
    return low


@pytest.fixture(params=[False, True], ids=['barriers', 'ready_attn'])
def ready_attn(request, monkeypatch):
    monkeypatch.setattr(attn, 'READY_ATTN', request.param)
    return request.param


@pytest.mark.parametrize('shape', [TINY, SMALL], ids=['tiny', 'small'])
@pytest.mark.parametrize('B', [1, 4, 8])
def test_lowered_plans_order_every_access(shape, B, ready_attn):
    low = lowering(shape, B)
    races = phases.check(low, steps=2)
    assert not races, '\n'.join(map(str, races[:8]))
    assert not phases.flag_range_gaps(low)
    waits = {e[1] for e in low.trace if e[0] == 'flagrange'}
    if shape == SMALL:
        # what the emulator had to get through: the split's and (READY_ATTN) the
        # attention's readiness flags, the local fold, the parity buffers
        assert ('split' in waits) == (B >= 4)
        assert ('attention' in waits) == ready_attn
        assert bool(low.fx_parity) == ready_attn
        assert any(e[0] == 'clear' for e in low.trace)


@pytest.mark.parametrize('shape,B,tmax', [
    (SMALL, 32, 1024),                          # configuration 3: 16-row tiles, runtime attention chunks
    ((24, 1024, 16, 4096, 50257), 8, 512),      # configuration 4
    ((24, 1024, 16, 4096, 50257), 1, 512),      # configuration 4, one row
    ((48, 1600, 25, 6400, 50257), 64, 256),     # configuration 5: 64 rows, fold chunks
], ids=['c3', 'c4', 'c4b1', 'c5'])
def test_benchmark_configurations_order_every_access(shape, B, tmax):
    """The persistent kernels of the benchmark configurations, at their real
    cache lengths and widths, as ``lower`` builds them."""
    low = lowering(shape, B, tmax)
    assert not phases.check(low, steps=2)
    assert not phases.flag_range_gaps(low)


def _barrier_labels(shape, B, monkeypatch):
    seen = []
    orig = LM.Lowering.barrier

    def spy(self, out, ind, what='', pre_wait=()):
        seen.append(what)
        return orig(self, out, ind, what, pre_wait)
    with monkeypatch.context() as m:
        m.setattr(LM.Lowering, 'barrier', spy)
        lowering(shape, B)
    return list(dict.fromkeys(seen))


@pytest.mark.parametrize('B', [1, 8])
def test_a_dropped_barrier_is_caught(B, monkeypatch):
    """Each grid barrier of the plan in turn is left out of the kernel (the
    lowering's own bookkeeping is not told): the emulator reports a race for
    every one. (Where the lowering's local-fold checks refuse such a plan,
    ``lower`` falls back to the plan without local folds, and it is that
    plan, still one barrier short, that the emulator sees.)"""
    orig = LM.Lowering.barrier
    labels = _barrier_labels(SMALL, B, monkeypatch)
    caught = {}
    for drop in labels:
        def skip(self, out, ind, what='', pre_wait=(), drop=drop):
            if what != drop:
                return orig(self, out, ind, what, pre_wait)
        with monkeypatch.context() as m:
            m.setattr(LM.Lowering, 'barrier', skip)
            try:
                low = lowering(SMALL, B)
            except ChainError:
                caught[drop] = 'lowering'
                continue
        races = phases.check(low, steps=2)
        assert races, f'barrier before {drop} dropped, no race found'
        caught[drop] = 'emulator'
    print(f'B={B}: {caught}')
    assert caught and all(v == 'emulator' for v in caught.values()), caught


def test_a_flag_range_one_block_short_is_caught():
    """The fold split's wait, with its last producer block left out of the
    range, leaves consumer blocks reading values nobody waited for."""
    low = lowering(SMALL, 8)
    i = next(i for i, e in enumerate(low.trace) if e[0] == 'flagrange')
    kind, ranges, active, setup, info = low.trace[i][1:]
    short = [(lo, f'({hi}) - 1') for lo, hi in ranges]
    low.trace[i] = ('flagrange', kind, short, active, setup, info)
    gaps = phases.flag_range_gaps(low)
    assert gaps and all(k == 'split' for k, _, _ in gaps)


def test_a_clear_moved_into_the_phase_of_its_readers_is_caught():
    """The local fold's sum cleared one barrier too early (in the phase where
    the first LayerNorm still reads it) is a write-after-read race."""
    low = lowering(SMALL, 1)
    clears = [i for i, e in enumerate(low.trace) if e[0] == 'clear' and e[2] is not None]
    assert clears
    i = clears[0]
    _, z, slot, ahead = low.trace[i]
    low.trace[i] = ('clear', z, slot - 1, ahead)
    races = phases.check(low, steps=2)
    assert any(r.kind in ('WAR', 'RAW', 'WAW') and r.value.startswith(z) for r in races)
