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
    m.tmax = tmax
    m.t = torch.zeros(1, dtype=torch.int32)
    m._know_pos(pos)
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


def test_a_caller_write_of_t_makes_the_position_unknown():
    """The reference's usage ``reset(); t.fill_(p); step()``: the host copy
    cannot know p, so the check is off (no false refusal when t is rewound,
    none based on a stale count) until reset / seek / prefill set it again."""
    m = _model_stub(384, 0)                # as after reset()
    m._advance(380, 'step')
    m.t.fill_(5)                           # the caller rewinds t itself
    m._advance(10, 'step')                 # would be 390 > 384 on the stale count: not refused
    assert m._pos is None
    m.t.fill_(383)
    m._know_pos(383)                       # what seek(383) leaves
    m._advance(1, 'step')
    with pytest.raises(ValueError, match='exceed the cache'):
        m._advance(1, 'step')


# ---------------------------------------------------------------- launch arguments and the no-alloc error word
def _bound_stub(history=8, device=0):
    """A Kernel with its argument slots filled (as after bind), on the CPU."""
    import ctypes
    k = _kernel_stub(0)
    k.device = device
    k.lowered = types.SimpleNamespace(name='vesta_step_b8', history=history)
    k.args = object()
    k._nsteps, k._tok, k._tok_in = ctypes.c_int(1), ctypes.c_void_p(0), ctypes.c_void_p(0)
    return k


class _FakeDev:
    """Stands in for an int32 device tensor (the checks look at is_cuda, dtype,
    contiguity, device and size only)."""
    def __init__(self, n, dtype=torch.int32, contiguous=True, index=0):
        self.is_cuda, self.dtype, self._c, self._n = True, dtype, contiguous, n
        self.device = types.SimpleNamespace(index=index)

    def is_contiguous(self):
        return self._c

    def numel(self):
        return self._n

    def data_ptr(self):
        return 0x1000


@pytest.mark.parametrize('bad, err, match', [
    (torch.zeros(64, dtype=torch.int32), TypeError, 'int32 device tensor'),      # host memory
    (_FakeDev(64, dtype=torch.int64), TypeError, 'int32 device tensor'),
    (_FakeDev(64, contiguous=False), TypeError, 'int32 device tensor'),
    (_FakeDev(64, index=1), ValueError, 'on device 1'),
    (_FakeDev(8 * 4 - 1), ValueError, 'need 32'),                                   # one token short
])
@pytest.mark.parametrize('which', ['tokens', 'inputs'])
@pytest.mark.parametrize('entry', ['launch', 'launch_noalloc'])
def test_bad_token_buffers_are_refused_before_anything_is_enqueued(monkeypatch, bad, err, match, which, entry):
    k = _bound_stub()
    monkeypatch.setattr(launch, 'lib', lambda: pytest.fail('the shim was called'))
    with pytest.raises(err, match=match):
        getattr(k, entry)(4, **{which: bad})


def test_good_token_buffers_pass_the_checks():
    k = _bound_stub()
    k._steps_and_tokens(4, _FakeDev(32), _FakeDev(40), 'launch')
    assert (k._nsteps.value, k._tok.value, k._tok_in.value) == (4, 0x1000, 0x1000)
    k._steps_and_tokens(2, None, None, 'launch')
    assert k._nsteps.value == 2 and not k._tok.value and not k._tok_in.value      # null pointers


def test_tokens_for_a_kernel_without_token_feedback_are_refused():
    k = _bound_stub(history=0)
    with pytest.raises(ValueError, match='records no tokens'):
        k._steps_and_tokens(1, _FakeDev(8), None, 'launch')
    with pytest.raises(ValueError, match='at least 1'):
        k._steps_and_tokens(0, None, None, 'launch')


def test_check_after_a_noalloc_launch_reads_the_static_error_word(monkeypatch):
    """check() after launch_noalloc reads the error word at the static scratch's
    barrier block (vh_noalloc_read at bar_off + 4 * BAR_ERROR), not the
    object's own bar, and raises on it."""
    import ctypes
    k = _bound_stub()
    static = {}

    class FakeLib:
        def vh_noalloc_read(self, dst, offset, n, stream):
            static['read'] = (offset.value if hasattr(offset, 'value') else offset, n)
            ctypes.memmove(dst.value, ctypes.byref(ctypes.c_int(static.get('word', 0))), 4)
            return 0

    fake_torch = types.SimpleNamespace(
        zeros=torch.zeros, int32=torch.int32,
        cuda=types.SimpleNamespace(current_stream=lambda: types.SimpleNamespace(cuda_stream=0)))
    monkeypatch.setattr(launch, 'lib', FakeLib)
    monkeypatch.setattr(launch, '_torch', lambda: fake_torch)
    k._noalloc_bar = 4096                         # as launch_noalloc leaves it
    k.check()                                     # word 0: passes
    assert static['read'] == (4096 + 4 * BAR_ERROR, 4)
    static['word'] = 1
    with pytest.raises(RuntimeError, match='grid barrier gave up'):
        k.check()
    assert k._noalloc_bar is None                 # the next check reads the object's own (cleared) bar
    k.check()


@pytest.mark.parametrize('plain', [False, True])
def test_profiling_launch_switch_picks_the_ordinary_launch(monkeypatch, plain):
    """VESTA_PLAIN_LAUNCH=1 (profiling only) issues the same kernel, grid and
    arguments through vh_launch instead of vh_launch_cooperative."""
    calls = []

    class FakeLib:
        def vh_launch(self, *a):
            calls.append(('vh_launch', a[1], a[2]))
            return 0

        def vh_launch_cooperative(self, *a):
            calls.append(('vh_launch_cooperative', a[1], a[2]))
            return 0

    fake_torch = types.SimpleNamespace(
        cuda=types.SimpleNamespace(current_stream=lambda: types.SimpleNamespace(cuda_stream=0)))
    monkeypatch.setattr(launch, 'lib', FakeLib)
    monkeypatch.setattr(launch, '_torch', lambda: fake_torch)
    monkeypatch.setattr(launch, 'PLAIN_LAUNCH', plain)
    k = _bound_stub()
    k.fn, k.block, k.smem = None, 512, 0
    k.launch(2)
    assert calls == [('vh_launch' if plain else 'vh_launch_cooperative', 144, 512)]
    if plain:
        with pytest.raises(RuntimeError, match='cooperative only'):
            k.launch_noalloc(1)
