"""GPU tests of the decode API's instrumented and failure paths (run on an
MI355X with -m gpu): timing builds (reference ``timing=True``), the PyTorch
comparison arms' token agreement (reference ``bench/g0_bench.py:244-245``),
the matrix-core range guard, and token buffers of either layout."""
import os
import sys

import numpy as np
import pytest

from conftest import REPO

sys.path.insert(0, REPO)
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('no GPU visible: -m gpu tests need an MI355X')
    return torch


def _decode(m, prompts, n):
    """Prefill, then n steps one launch each; tokens [n, B] and logits [n, B, V]."""
    torch = _torch()
    m.reset()
    m.prefill(torch.from_numpy(prompts).to('cuda', torch.int32))
    toks, lg = [], []
    for _ in range(n):
        m.step()
        toks.append(m.x.clone())
        lg.append(m.logits().clone())
    torch.cuda.synchronize()
    m.check()
    return torch.stack(toks).cpu().numpy(), torch.stack(lg).cpu().numpy()


@pytest.mark.parametrize('timing', [True, 'trace'])
def test_timing_builds_match_the_untimed_kernel(timing):
    """A timed build decodes exactly as the untimed one (the clock reads change
    no arithmetic), and its per-site sums fit in the measured time."""
    from vesta import profile
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2
    B, n = 8, 6
    prompts = bench.bench_prompts(B)[:, :16]
    hf = RandomGPT2('small', 0)
    plain = VestaGPT2(hf, batch=B, tmax=64)
    want_t, want_l = _decode(plain, prompts, n)
    del plain
    m = VestaGPT2(hf, batch=B, tmax=64, timing=timing)
    got_t, got_l = _decode(m, prompts, n)
    assert np.array_equal(got_t, want_t)
    assert np.array_equal(got_l, want_l)
    if timing is True:
        labels, us, wall = profile.site_times(m, 16)
        assert len(labels) == us.shape[0] > 10
        assert (us >= 0).all()
        # every block's sites cover its time in the launch: never more than the wall time
        assert us.sum(axis=0).max() <= wall * 1.05 + 5.0, (us.sum(axis=0).max(), wall)
        assert us[:, 0].sum() > 0.5 * wall
    else:
        rows = profile.barrier_trace(m, 8)
        assert len(rows) == m.low.barriers_per_launch
        assert all(rel >= 0 and spread >= 0 for _, _, spread, rel in rows)
        assert rows[0][0] == profile.barrier_labels(m)[0]


def test_graph_arm_tokens_equal_eager():
    """The PyTorch comparison arms: a HIP-graph replay of the eager step gives
    the eager step's tokens (reference g0_bench.py:244-245)."""
    _, eager = bench.run_arm('torch_eager', 8, 12, 2)
    _, graph = bench.run_arm('torch_graph', 8, 12, 2)
    assert np.array_equal(eager.numpy(), graph.numpy())


def _big_gain_checkpoint(tmp_path):
    """GPT-2 small (seed 0) with layer 0's first LayerNorm gain at 60000: the
    normalised activations entering the qkv product reach ~2e5, beyond fp16."""
    import torch
    from safetensors.torch import save_file
    from vesta.weights import RandomGPT2
    sd = {k: torch.from_numpy(v) for k, v in RandomGPT2('small', 0).numpy_state().items()}
    sd['transformer.h.0.ln_1.weight'] = torch.full_like(sd['transformer.h.0.ln_1.weight'], 60000.0)
    path = os.path.join(tmp_path, 'model.safetensors')
    save_file({k: v.contiguous() for k, v in sd.items()}, path)
    return path


@pytest.mark.parametrize('engine', ['persistent', 'layered'])
def test_matrix_core_path_refuses_activations_beyond_fp16(tmp_path, engine):
    """At 8 rows the products run on the fp16 matrix cores with activations as
    fp16 halves; an activation beyond 65504 cannot go in, and the launch is
    reported instead of returning silently wrong tokens."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import LocalGPT2
    m = VestaGPT2(LocalGPT2(_big_gain_checkpoint(tmp_path)), batch=8, tmax=bench.BENCH_TMAX, engine=engine)
    m.reset()
    m.x.fill_(11)
    m.step()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match='beyond the fp16 range'):
        m.check()
    m.check()                       # reported once, then cleared


def test_layered_engine_accepts_token_buffers_of_either_layout():
    """Per-step tokens into a [n, B] buffer and into a flat one agree (each
    step k lands at flat offsets k * B ..)."""
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2
    B, n = 8, 5
    m = VestaGPT2(RandomGPT2('small', 0), batch=B, tmax=64, engine='layered')
    prompts = torch.from_numpy(bench.bench_prompts(B)[:, :8]).to('cuda', torch.int32)
    outs = []
    for buf in (torch.zeros(n, B, dtype=torch.int32, device='cuda'),
                torch.zeros(n * B, dtype=torch.int32, device='cuda')):
        m.reset()
        m.prefill(prompts)
        m.step(n, buf)
        outs.append(buf.view(-1).cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    assert len(set(outs[0][:B].tolist())) > 1 or len(set(outs[0].tolist())) > 1
    # ... and equal the tokens of steps taken one at a time
    m.reset()
    m.prefill(prompts)
    one = []
    for _ in range(n):
        m.step()
        one.append(m.x.clone())
    assert np.array_equal(torch.stack(one).view(-1).cpu().numpy(), outs[0])


def test_steps_past_the_cache_are_refused_on_the_device_model():
    torch = _torch()
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2
    m = VestaGPT2(RandomGPT2('small', 0), batch=1, tmax=64)
    m.reset()
    m.prefill(torch.from_numpy(bench.bench_prompts(1)[:, :60]).to('cuda', torch.int32))
    m.step(4)                        # positions 60..63
    with pytest.raises(ValueError, match='exceed the cache'):
        m.step()
    torch.cuda.synchronize()
    assert int(m.t.item()) == 64
