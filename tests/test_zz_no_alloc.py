"""The allocation-free cooperative launch (``vh_launch_cooperative_noalloc``,
the library's static per-device scratch in place of the kernel's S, bar and
TS buffers) against the ordinary one (``vh_launch_cooperative``): the same
tokens, cache rows and logits, bit for bit, on two calls in a row, the second
with a smaller batch; the same launch captured in a HIP graph and replayed;
and a kernel whose buffers exceed the static scratch is refused before
anything is enqueued."""
import ctypes

import numpy as np
import pytest

def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('no GPU visible: -m gpu tests need an MI355X')
    return torch


def _model(B, tmax):
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2
    return VestaGPT2(RandomGPT2('small', 0), batch=B, tmax=tmax, engine='persistent')


def _decode(m, steps, noalloc):
    """Prefill 24 prompt positions (batched prefill), then ``steps`` decode steps
    in one cooperative launch; returns tokens, cache and the last logits."""
    torch = _torch()
    from vesta.weights import random_prompts
    m.reset()
    m.prefill(torch.from_numpy(random_prompts(m.B, 24, 50257, seed=3)).to('cuda', torch.int32))
    toks = torch.zeros(steps * m.B, dtype=torch.int32, device='cuda')
    logit = torch.zeros(m.B * 50257, dtype=torch.float32, device='cuda')
    if noalloc:
        m.k.launch_noalloc(steps, toks)
        m.k.read_noalloc('logit', logit)
    else:
        m.k.launch(steps, toks)
        logit.copy_(m.k.view('logit').reshape(-1))
    torch.cuda.synchronize()
    m.check()
    return (toks.cpu().numpy(), m.keys.cpu().numpy(), m.vals.cpu().numpy(), int(m.t.item()),
            logit.cpu().numpy())


@pytest.mark.gpu
def test_noalloc_launch_matches_the_ordinary_launch():
    _torch()
    big, small = _model(8, 64), _model(2, 64)
    want_big = _decode(big, 6, False)
    want_small = _decode(small, 4, False)
    got_big = _decode(big, 6, True)             # first call on the static scratch
    got_small = _decode(small, 4, True)         # second call, smaller batch and scratch
    for want, got in ((want_big, got_big), (want_small, got_small)):
        for a, b in zip(want, got):
            assert np.array_equal(np.asarray(a), np.asarray(b))
    assert len(set(want_big[0].tolist())) > 1


@pytest.mark.gpu
def test_noalloc_refuses_buffers_beyond_the_static_scratch():
    _torch()
    from vesta import launch
    m = _model(8, 64)                           # claim an S one word larger than the whole static scratch
    n_bytes = ctypes.c_size_t()
    base = ctypes.c_void_p()
    launch.ok(launch.lib().vh_noalloc_scratch(ctypes.byref(base), ctypes.byref(n_bytes)), 'static scratch')
    assert base.value and n_bytes.value == 8 << 20
    saved = m.k.S
    m.k.S = saved.new_empty(((8 << 20) // 4) + 1)
    try:
        with pytest.raises(RuntimeError, match='exceed the static scratch'):
            m.k.launch_noalloc(1)
    finally:
        m.k.S = saved


def test_static_scratch_layout_and_limit():
    """Host arithmetic of the static scratch, on the CPU: S at 0, bar and TS at
    256-byte boundaries after it, and a clear refusal past 8 MiB."""
    from vesta import launch
    L = launch.lib()
    bar, ts = ctypes.c_size_t(), ctypes.c_size_t()
    assert L.vh_noalloc_layout(1000, 1280, 4096, ctypes.byref(bar), ctypes.byref(ts)) == 0
    assert (bar.value, ts.value) == (1024, 1024 + 1280)
    assert L.vh_noalloc_layout(2215552, 1280, 294912, ctypes.byref(bar), ctypes.byref(ts)) == 0   # B=8 kernel
    st = L.vh_noalloc_layout((8 << 20) - 256, 1280, 0, ctypes.byref(bar), ctypes.byref(ts))
    assert st == 20004 and b'exceed the static scratch' in L.vh_error_string(st)


@pytest.mark.gpu
def test_noalloc_launch_replays_from_a_hip_graph():
    """After one eager call (which looks up the static scratch's address), the
    fill kernel, the cooperative launch and the logits read of
    ``launch_noalloc`` are captured on torch's capture stream and replayed
    three times, each from the same restored state, with eager work and a
    synchronisation between replays; every replay's tokens, cache rows,
    position and logits equal the ordinary launch's bit for bit."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts
    print('noalloc graph: GPT-2 small B=2 tmax 64, 4 steps per launch', flush=True)
    m = VestaGPT2(RandomGPT2('small', 0), batch=2, tmax=64, engine='persistent')
    m.reset()
    m.prefill(torch.from_numpy(random_prompts(2, 24, 50257, seed=5)).to('cuda', torch.int32))
    torch.cuda.synchronize()
    saved = [t.clone() for t in (m.x, m.t, m.keys, m.vals)]

    def restore():
        for dst, src in zip((m.x, m.t, m.keys, m.vals), saved):
            dst.copy_(src)

    steps = 4
    tok_ref = torch.zeros(steps * 2, dtype=torch.int32, device='cuda')
    m.k.launch(steps, tok_ref)
    torch.cuda.synchronize()
    m.check()
    want = [tok_ref.cpu().numpy(), m.k.view('logit').reshape(-1).cpu().numpy(), m.keys.cpu().numpy(),
            m.vals.cpu().numpy(), int(m.t.item())]

    toks = torch.zeros(steps * 2, dtype=torch.int32, device='cuda')
    logit = torch.zeros(2 * 50257, dtype=torch.float32, device='cuda')
    restore()
    m.k.launch_noalloc(steps, toks)                  # eager call: the scratch address is looked up here
    torch.cuda.synchronize()
    m.check()
    restore()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        m.k.launch_noalloc(steps, toks)
        m.k.read_noalloc('logit', logit)
    torch.cuda.synchronize()
    for r in range(3):
        restore()
        toks.zero_()
        logit.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        m.check()
        got = [toks.cpu().numpy(), logit.cpu().numpy(), m.keys.cpu().numpy(), m.vals.cpu().numpy(), int(m.t.item())]
        for a, b in zip(want, got):
            assert np.array_equal(np.asarray(a), np.asarray(b)), f'replay {r}'
        print(f'replay {r}: tokens {got[0].tolist()} equal the ordinary launch', flush=True)
