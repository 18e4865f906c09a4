"""Host-side logic of the boundary, on the CPU: the barrier error word the
host checks, the reference's default block size, unloading modules at exit,
and the position checks that keep every engine inside its cache."""
import types

import pytest
import torch

from vesta import launch
from vesta.gpt2 import VestaGPT2
from vesta.lower import BAR_ERROR, BAR_WORDS


def _kernel_stub(err):
    k = launch.Kernel.__new__(launch.Kernel)
    k.bar = torch.zeros(BAR_WORDS, dtype=torch.int32)
    k.bar[BAR_ERROR] = err
    k.bar[0] = 7                      # an arrival counter left behind by the failed launch
    k.lowered = types.SimpleNamespace(name='vesta_step_b1')
    k.grid = 144
    return k


def test_error_word_sits_in_the_barrier_block():
    # the device's VH_BAR_ERROR: line 9 (after 8 per-XCD counters and the exit counter), word 1
    assert BAR_ERROR == 32 * 9 + 1 and BAR_ERROR < BAR_WORDS


def test_check_raises_on_a_failed_barrier_and_clears_the_words():
    k = _kernel_stub(1)
    with pytest.raises(RuntimeError, match='grid barrier gave up'):
        k.check()
    assert int(k.bar.abs().sum()) == 0
    k.check()                         # cleared: the next check passes


def test_check_names_an_out_of_range_activation():
    k = _kernel_stub(2)
    with pytest.raises(RuntimeError, match='beyond the fp16 range'):
        k.check()
    assert int(k.bar.abs().sum()) == 0


def test_check_passes_when_no_barrier_failed():
    k = _kernel_stub(0)
    k.check()
    assert int(k.bar[0]) == 7         # nothing touched


def test_reference_default_block_maps_to_the_lowered_block():
    assert launch.REFERENCE_BLOCK == 256
    assert launch.resolve_block(256, 512) == 512
    assert launch.resolve_block(None, 512) == 512
    assert launch.resolve_block(512, 512) == 512
    with pytest.raises(ValueError, match='lowered for 512'):
        launch.resolve_block(128, 512)


def test_exit_hook_closes_every_live_module_owner(monkeypatch):
    closed = []

    class Owner:
        def __init__(self, n):
            self.n = n

        def close(self):
            closed.append(self.n)

    registered = []
    monkeypatch.setattr(launch, '_live', launch.weakref.WeakSet())
    monkeypatch.setattr(launch, '_hook', [])
    monkeypatch.setattr(launch.atexit, 'register', registered.append)
    a, b = Owner(1), Owner(2)
    launch.track(a)
    launch.track(b)
    assert registered == [launch._close_all]       # one hook, registered once
    launch._close_all()
    assert sorted(closed) == [1, 2]


def _model_stub(tmax, pos):
    m = VestaGPT2.__new__(VestaGPT2)
    m.tmax, m._pos = tmax, pos
    return m


def test_steps_past_the_cache_are_refused():
    m = _model_stub(384, 380)
    m._advance(4, 'step')             # positions 380..383: the last rows
    assert m._pos == 384
    with pytest.raises(ValueError, match='exceed the cache'):
        m._advance(1, 'step')
    assert m._pos == 384              # a refused step does not move the position


def test_unknown_position_skips_the_check():
    m = _model_stub(384, None)
    m._advance(1000, 'step')
    assert m._pos is None
